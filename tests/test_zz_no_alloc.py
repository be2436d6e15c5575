"""bt_attention_noalloc through the C ABI: the same results as bt_attention with a caller's workspace, bit for bit, over
two calls in a row on one runtime (the second smaller, so its partial sums land in a working memory that still holds
the first call's), and a clear refusal of a plan larger than its static working memory. Needs a GPU."""
import ctypes
import numpy as np
import pytest

from baretile_amd import _lib
from helpers import up, down, bits_to_float
from oracle import bfp as B, ops

pytestmark = pytest.mark.gpu


def args_for(rt, q, k, v, places, parts=0):
  E, rows, hd = q.shape
  kvh, keys, _ = k.shape
  dq, dk, dv = (up(rt, B.bf16_bits(t)) for t in (q, k, v))
  outs = [rt.dram_alloc(E * rows * hd * 2) for _ in range(2)]
  for o in outs: rt.upload(o, b"\xff" * (E * rows * hd * 2))  # NaN bits until a call writes them
  dp = up(rt, np.asarray(places, np.int32))
  make = lambda o: _lib.AttentionArgs(dq, dk, dv, o, dp, rows * hd, hd, keys * hd, hd, keys * hd, hd, rows * hd, hd,
                                      rows, E, E // kvh, rows, keys, hd, 0, parts, 0, 0, 0)
  return make(outs[0]), make(outs[1]), outs


# (heads, rows, head width, keys, heads per key head): a decode split into 32 parts of 16384 keys, then a smaller one
CALLS = [(32, 4, 128, 16384, 4), (8, 1, 64, 1000, 4)]


def test_noalloc_attention_equals_attention_with_a_workspace(rt):
  rng = np.random.default_rng(11)
  for e, rows, hd, keys, rep in CALLS:
    q = B.bf16(rng.normal(0, 1, (e, rows, hd)) / np.sqrt(hd))
    k, v = (B.bf16(rng.normal(0, 1, (e // rep, keys, hd))) for _ in range(2))
    places = rng.integers(keys - 80, keys, (e, rows))
    with_ws, noalloc, (o1, o2) = args_for(rt, q, k, v, places)
    need = ctypes.c_uint64()
    _lib.call("attention_scratch", ctypes.byref(with_ws), ctypes.byref(need))
    assert 0 < need.value <= 8 << 20, need.value  # split into parts, within the static working memory
    with_ws.scratch, with_ws.scratch_bytes = rt.dram_alloc(need.value), need.value
    rt.run("attention", "attention", ctypes.byref(with_ws))
    rt.run("attention", "attention_noalloc", ctypes.byref(noalloc))
    want = down(rt, o1, (e, rows, hd), np.uint16)
    got = down(rt, o2, (e, rows, hd), np.uint16)
    assert np.array_equal(got, want), (e, keys)
    ref = ops.attention(q, k, v, places[..., None], 0, rep)
    assert np.allclose(bits_to_float(got), ref, rtol=0.011, atol=0.011), (e, keys)


def test_noalloc_attention_refuses_a_plan_beyond_its_working_memory(rt):
  # 8 key heads x 4 tiles of 16 query rows x 64 parts x 8320 bytes = 17 MB > 8 MiB: refused before any launch
  rng = np.random.default_rng(12)
  q = B.bf16(rng.normal(0, 1, (32, 16, 128)))
  k = B.bf16(rng.normal(0, 1, (8, 16384, 128)))
  _, noalloc, _ = args_for(rt, q, k, k, np.full((32, 16), 16383), parts=64)
  with pytest.raises(ValueError, match="working memory"):
    rt.run("attention", "attention_noalloc", ctypes.byref(noalloc))
  from baretile_amd.tensor import Tensor
  assert Tensor.of(rt, [[1.0, 2.0]]).relu().tolist() == [[1.0, 2.0]]  # the runtime goes on working
