"""Writes, aliasing, replays and the runtime's promises on the GPU, as the reference's tests state them
(test/test_kernels.py:1022-1079, test/test_device.py:486, 962; docs/api.md:38-63). Needs a GPU."""
import numpy as np
import pytest

from baretile_amd.runtime import Runtime
from baretile_amd.tensor import Tensor, jit
from oracle import bfp as B

pytestmark = pytest.mark.gpu


def value(t): return np.array(t.tolist()).reshape(t.shape)


def test_block_float_views_as_b_use_their_own_tiles(rt):
  # x @ W[0] then x @ W[1] on a plain bfp8 batch: each product reads its own matrix (the tiles columns() makes are kept
  # per view), bit for bit the product with the matrix's bf16 values
  rng = np.random.default_rng(1)
  w = Tensor.of(rt, rng.normal(0, 1, (2, 64, 48)).tolist()).cast("bfp8")
  x = Tensor.of(rt, rng.normal(0, 1, (4, 64)).tolist())
  wv = value(w.cast("bf16"))
  for i in (0, 1, 0):
    got = value(x @ w[i])
    want = value(x @ Tensor.of(rt, wv[i].tolist()))
    assert np.array_equal(got, want), i
  assert value(x @ w).shape == (2, 4, 48)  # the whole batch after its views


def test_writes_drop_cached_tiles(rt):
  # matmul, then a write into the block float (assign, put), then matmul again: the second product sees the new values
  rng = np.random.default_rng(2)
  a, b = rng.normal(0, 1, (64, 32)), rng.normal(0, 1, (64, 32))
  w = Tensor.of(rt, a.tolist()).cast("bfp8")
  x = Tensor.of(rt, np.eye(64).tolist())
  assert np.array_equal(value(x @ w)[0], B.bfp(a, "bfp8"))
  w.assign(Tensor.of(rt, b.tolist()).cast("bfp8"))
  assert np.array_equal(value(x @ w)[0], B.bfp(b, "bfp8"))
  rows = Tensor.of(rt, a[:3].tolist())
  w.put(Tensor.of(rt, [[0, 1, 2]], "int32"), rows)
  want = B.bfp(b, "bfp8")
  want[:3] = B.bfp(a[:3], "bfp8")
  assert np.array_equal(value(x @ w)[0], want)


def test_assign(rt):
  # test_kernels.py:1022-1038: assign writes in place, so a view sees it; w @ tm into w goes through a copy and equals
  # the product on a fresh copy; a jit step that assigns updates the weight on every call, replays included
  rng = np.random.default_rng(17)
  w0, m = (B.bf16(rng.uniform(-1, 1, shape)) for shape in ((64, 96), (96, 96)))
  w, tm = Tensor.of(rt, w0.tolist()), Tensor.of(rt, m.tolist())
  addr, view = w.addr, w[:, 32:64]
  w.assign(w * 2 + 1)
  assert w.addr == addr and np.allclose(value(view)[0], (w0 * 2 + 1)[:, 32:64], rtol=1e-2)
  fresh = value(Tensor.of(rt, value(w)[0].tolist()) @ tm)
  w.assign(w @ tm)
  assert w.addr == addr and np.array_equal(value(w), fresh)
  step = jit(lambda x: w.assign(w + x))
  for _ in range(4): step(Tensor.of(rt, np.ones((64, 96)).tolist()))
  assert np.allclose(value(w), fresh + 4, rtol=1e-2, atol=0.05)


def test_assign_overlapping_views(rt):
  # test_kernels.py:1040-1057: a copy reads the source as it was, whichever way the views overlap, for plain copies,
  # fused expressions and block floats
  a = np.arange(64 * 640, dtype=np.float32).reshape(64, 640)
  for left, right in ((slice(32, None), slice(None, -32)), (slice(None, -32), slice(32, None))):
    for add in (False, True):
      x = Tensor.of(rt, a.tolist(), "fp32")
      source, want = x[:, right], a.copy()
      x[:, left].assign(source + 1 if add else source)
      want[:, left] = a[:, right] + int(add)
      assert np.array_equal(value(x)[0], want), (left, add)
  # a block float's view takes the values of an overlapping view of itself, both ways (decoded whole first, then put
  # row by row, each run rounded as a cast rounds it, which leaves values already on a block float's grid as they are)
  for fmt in ("bfp8", "bfp4"):
    for left, right in ((slice(32, None), slice(None, -32)), (slice(None, -32), slice(32, None))):
      x = Tensor.of(rt, a.tolist()).cast(fmt).realize()
      want = value(x)[0]
      x[:, left].assign(x[:, right])
      want[:, left] = want[:, right].copy()
      assert np.array_equal(value(x)[0], want), (fmt, left)
  # a strided block-float view reads back and casts as its values
  x = Tensor.of(rt, a.tolist()).cast("bfp8").realize()
  whole = value(x)[0]
  assert np.array_equal(value(x[8:40:2, 16:208])[0], whole[8:40:2, 16:208])
  assert np.array_equal(value(x[:, 48:112].cast("bf16"))[0], whole[:, 48:112])


def test_realize_overlapping_destination(rt):
  # test_kernels.py:1068-1079: a product realized into its own operand, and an expression into a shifted view of its
  # source, both as if the source were read first
  a, b = (Tensor.full(rt, 256, 256, 1.0) for _ in range(2))
  out = (a @ b).realize(b)
  assert out.addr == b.addr and np.all(value(b) == 256) and np.all(value(out) == 256)
  data = np.arange(64 * 96, dtype=np.float32).reshape(64, 96)
  x = Tensor.of(rt, data.tolist(), "fp32")
  (x[:, :-32] + 1).realize(x[:, 32:])
  want = data.copy()
  want[:, 32:] = data[:, :-32] + 1
  assert np.array_equal(value(x)[0], want)


def test_jit_with_block_float_and_written_inputs(rt):
  # a jit whose input is a bfp8 matrix, over three calls with different matrices (the third replayed): each equals
  # eager; and a jit that writes into an input (put) leaves the write in the caller's tensor after every call
  rng = np.random.default_rng(3)
  x = Tensor.of(rt, rng.normal(0, 1, (8, 64)).tolist())
  f = jit(lambda w: (x @ w).relu())
  for i in range(3):
    w = Tensor.of(rt, rng.normal(0, 1, (64, 32)).tolist()).cast("bfp8")
    assert np.array_equal(value(f(w)), value((x @ w).relu())), i
  put = jit(lambda cache, rows, ids: cache.put(ids, rows) * 1)
  for i in range(3):
    cache = Tensor.zeros(rt, 16, 32, dtype="fp32")
    rows = rng.normal(0, 1, (2, 32)).astype(np.float32)
    put(cache, Tensor.of(rt, rows.tolist(), "fp32"), Tensor.of(rt, [[i, 5 + i]], "int32"))
    want = np.zeros((16, 32), np.float32)
    want[[i, 5 + i]] = rows
    assert np.array_equal(value(cache)[0], want), i
  # a view of a larger block float can't be copied byte for byte into the recording's input (the first call runs
  # eagerly; the second, which records, refuses it)
  g, pair = jit(lambda w: x @ w), Tensor.of(rt, rng.normal(0, 1, (2, 64, 32)).tolist()).cast("bfp8")
  g(pair[1])
  with pytest.raises(ValueError, match="whole tensor"): g(pair[1])


def test_wait_times_out_and_the_stream_drains(rt):
  # test_device.py:962: wait(timeout) raises TimeoutError while a launch is still running; here the launch keeps the
  # device busy for two seconds and then ends by itself, so the stream drains and later work runs
  import time
  rt.sleep(2.0)
  t0 = time.perf_counter()
  with pytest.raises(TimeoutError): rt.wait(timeout=0.2)
  assert time.perf_counter() - t0 < 1.5
  rt.wait(timeout=30)
  assert Tensor.of(rt, [[1.0, 2.0]]).relu().tolist() == [[1.0, 2.0]]
  with pytest.raises(ValueError): rt.sleep(11)


def test_freed_blocks_are_reused_in_stream_order(rt):
  # runtime.py:814-820's stream-ordered free, with the runtime keeping freed blocks for its next allocations of their
  # size: the block comes back at once, a second free of it is refused, and a tensor whose block is handed out again
  # while a launch that reads it is still queued (behind a two-tenths-of-a-second sleep) still gives that launch its
  # old values
  p = rt.dram_alloc(1000)
  rt.dram_free(p)
  assert rt.dram_alloc(1000) == p  # 1000 bytes round to 1024: the same block
  q = rt.dram_alloc(5000)
  assert q != p
  rt.dram_free(q)
  rt.dram_free(p)
  with pytest.raises(ValueError, match="twice"): rt.dram_free(p)
  rt.dram_alloc(1024), rt.dram_alloc(5120)  # both kept blocks taken again
  vals = np.arange(-32, 32, dtype=np.float32).reshape(1, 64)
  x = Tensor.of(rt, vals.tolist(), "fp32")
  rt.sleep(0.2)
  y = x.relu().realize()
  del x
  z = Tensor.of(rt, np.full((1, 64), 7.0).tolist(), "fp32")
  assert np.array_equal(value(y)[0], np.maximum(vals, 0)) and np.array_equal(value(z)[0], np.full((1, 64), 7.0))


def test_open_device(chip):
  # test_device.py:69 and docs/api.md:43-45: while a Chip holds the GPU, a second opener gets RuntimeError, so two live
  # runtimes never share one device (nor the device's static working memory); a GPU that isn't there is a ValueError.
  # A runtime made without a chip shares the open one.
  from baretile_amd import pci
  with pytest.raises(RuntimeError, match="already open"): pci.open_device()
  with pytest.raises(ValueError, match="GPUs"): pci.open_device(64)
  r = Runtime()
  assert r.chip is chip
  r.close()


def test_takeover_and_closed_runtime(chip):
  # test_device.py:486 and docs/api.md:38-63: a new runtime on the chip takes over, and the old one's tensors and
  # recordings then raise RuntimeError, as does a closed runtime's
  first = Runtime(chip)
  t = Tensor.of(first, [[1.0, 2.0]])
  f = jit(lambda a: a * 2)
  for _ in range(3): f(t)
  second = Runtime(chip)
  assert first.closed and not second.closed
  with pytest.raises(RuntimeError): t.tolist()
  with pytest.raises(RuntimeError): (t + 1).realize()
  with pytest.raises(RuntimeError): f(t)
  with pytest.raises(RuntimeError): Tensor.of(first, [[1.0]])
  assert Tensor.of(second, [[3.0]]).tolist() == [[3.0]]
  second.close()
  with pytest.raises(RuntimeError): second.wait()


def test_profile_reports_time_and_bytes(chip):
  # runtime.py:773-786: (name, launches, time, bytes) by name, longest first; bytes are what the launches read
  rt = Runtime(chip, timing=True)
  try:
    w = Tensor.of(rt, np.ones((576, 1536)).tolist()).cast("bfp8").columns()
    x = Tensor.of(rt, np.ones((4, 576)).tolist())
    base = rt.launches
    for _ in range(3): (x @ w).realize()
    rows = {name: (n, us, nbytes) for name, n, us, nbytes in rt.profile(base)}
    n, us, nbytes = rows["matmul"]
    assert n == 3 and us > 0 and nbytes == 3 * (4 * 576 * 2 + 1536 // 16 * 576 // 64 * 1088)
    assert list(rows) == [r[0] for r in sorted(rt.profile(base), key=lambda r: -r[2])]
  finally:
    rt.close()


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_matmul_refuses_exponents_it_cannot_read(rt, fmt):
  # a run whose exponent the matmul kernels can't read (bfp8: a top exponent field of 1, the smallest normal bf16;
  # bfp4: 248, values near 2^121) makes columns() raise instead of multiplying wrong; a run of zeros under exponent 0
  # is fine, and readback stays exact either way
  a = np.full((64, 32), 0.5, np.float32)
  a[3, :16] = 2.0 ** -126 if fmt == "bfp8" else 2.0 ** 121
  a[9, 16:] = 0
  w = Tensor.of(rt, a.tolist()).cast(fmt)
  assert np.array_equal(value(w)[0], B.bfp(a, fmt))
  with pytest.raises(ValueError, match="exponent"): w.columns()
  with pytest.raises(ValueError, match="exponent"): (Tensor.of(rt, np.ones((2, 64)).tolist()) @ w).realize()
  bad = w
  a[3, :16] = 1.0
  w = Tensor.of(rt, a.tolist()).cast(fmt).columns()
  assert np.array_equal(value(Tensor.of(rt, np.eye(64).tolist()) @ w)[0], B.bfp(a, fmt))
  # a jit input used as B is checked on every call, the recorded and replayed ones too, which lay it out inside a
  # capture that can't read the count back
  x = Tensor.of(rt, np.eye(64).tolist())
  good = Tensor.of(rt, a.tolist()).cast(fmt)
  f = jit(lambda b: x @ b)
  for i in range(4):
    assert np.array_equal(value(f(good))[0], B.bfp(a, fmt)), i
    with pytest.raises(ValueError, match="exponent"): f(bad)


def test_jit_copies_back_a_cache_written_by_rope_put(rt):
  # rope_put writes key and value rows into its cache: a jit whose input is that cache leaves the rows in the caller's
  # tensor after each call, the replays included, as eager calls do
  rng = np.random.default_rng(9)
  heads, kv, d, size = 2, 1, 64, 16
  nh = heads + 2 * kv
  cos, sin = Tensor.of(rt, np.ones((1, nh * d)).tolist()), Tensor.of(rt, np.zeros((1, nh * d)).tolist())
  f = jit(lambda x, cache, at: x.rope_put(cos, sin, cache, at, heads, kv))
  for i in range(3):
    rows = B.bf16(rng.normal(0, 1, (1, nh * d)))
    cache = Tensor.zeros(rt, size, d, batch=2 * kv)
    q = f(Tensor.of(rt, rows.tolist()), cache, Tensor.of(rt, [[i + 3]], "int32"))
    want = np.zeros((2 * kv, size, d))
    want[:, i + 3] = rows[0, heads * d:].reshape(2 * kv, d)
    assert np.array_equal(value(cache), want), i
    assert np.array_equal(value(q)[0], rows[:, :heads * d]), i
