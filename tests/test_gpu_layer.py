"""BASELINE config 5 on the GPU: one Llama-3-8B-shaped block (hidden 4096, SwiGLU 14336, 32 query and 8 key heads of
128) with every projection N(0, 0.02) in bfp4, against the NumPy oracle (oracle/llama_ref.layer) on the same block
floats: a causal prefill from position 0, and one batch-32 decode step at position 4095 of each slot's 4096-row cache.
The tolerance is the reference's for a block, 3% of the largest change the block makes to x
(test/test_models.py:818-833), checked per slot for the batch as test_batched_decode does (test_models.py:1629-1650).
Needs a GPU."""
import numpy as np
import pytest

from baretile_amd.models import llama
from baretile_amd.runtime import Runtime
from baretile_amd.tensor import Tensor
from oracle import bfp as B, llama_ref as L

pytestmark = pytest.mark.gpu

DIM, HEADS, KV, HD, FFN = 4096, 32, 8, 128, 14336
SHAPES = {"qkv_proj": (DIM, (HEADS + 2 * KV) * HD), "o_proj": (HEADS * HD, DIM), "gate_up_proj": (DIM, 2 * FFN),
          "down_proj": (FFN, DIM)}


def values(t, shape):  # a tensor's values read back, as float32
  return B.bf16_floats(np.frombuffer(t.tobytes(), np.uint16).reshape(shape))


@pytest.fixture(scope="module")
def block(chip):
  """The block on the device and in the oracle. The oracle's weights are the device's block floats read back, after a
  slice of each is checked bit for bit against the oracle's own cast."""
  rt = Runtime(chip)
  rng = np.random.default_rng(0)
  c = llama.model(dim=DIM, heads=HEADS, kv=KV, layers=1, eps=1e-5, theta=500000.0, ffn=FFN, head_dim=HD)
  c.precision = {(op, 0): ("bfp4", 4) for op in ("qkv", "o", "gate_up", "down")}
  rc = L.model(dim=DIM, heads=HEADS, kv=KV, layers=1, eps=1e-5, theta=500000.0, ffn=FFN, head_dim=HD)
  dev, ref = {}, {}
  for name, shape in SHAPES.items():
    a = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)
    t = Tensor.of(rt, a).cast("bfp4").columns()
    dev[name] = t
    ref[name] = values(t, shape)
    assert np.array_equal(ref[name][:128], B.bfp(a[:128], "bfp4").astype(np.float32)), name
    del a
  for name in ("input_layernorm", "post_attention_layernorm"):
    n = B.bf16(rng.normal(1, 0.1, (1, DIM)))
    dev[name], ref[name] = Tensor.of(rt, n), n
  size = 4096
  cos, sin, turn = llama.rotary(c, size)
  dev["cos"], dev["sin"], dev["turn"] = Tensor.of(rt, cos), Tensor.of(rt, sin), Tensor.of(rt, turn).columns()
  rot = L.rotary(rc, size)
  assert all(np.array_equal(a, b) for a, b in zip((cos, sin, turn), rot))
  yield rt, c, rc, dev, ref, rot
  rt.close()


def test_prefill_matches_numpy(block):
  rt, c, rc, dev, ref, (cos, sin, turn) = block
  n, size = 256, 512
  x = np.random.default_rng(1).standard_normal((n, DIM), dtype=np.float32)
  cache = Tensor.zeros(rt, size, HD, batch=2 * KV)
  places = Tensor.of(rt, [list(range(n))], "int32")
  rot = (dev["cos"].gather(places), dev["sin"].gather(places), dev["turn"])
  got = np.array(llama.layer(Tensor.of(rt, x[None], "fp32"), dev, c, rot, places.reshape(1, n, 1), cache,
                             places).tolist()).reshape(n, DIM)
  mask = np.where(np.arange(size) > np.arange(n)[:, None], np.float32(-1e9), np.float32(0))
  kv = np.zeros((2 * KV, size, HD))
  want = L.layer(x, ref, rc, (cos[:n], sin[:n], turn), mask, kv, range(n))
  change, err = np.abs(want - x).max(), np.abs(got - want).max()
  assert change > 0.5 and err < 0.03 * change, (err, change)
  # the keys and values the block put into its cache
  got_kv = np.array(cache.tolist()).reshape(2 * KV, size, HD)
  assert np.abs(got_kv[:, :n] - kv[:, :n]).max() < 0.03 * np.abs(kv[:, :n]).max() and not got_kv[:, n:].any()


def test_prefill_2048_matches_numpy_on_rows(block):
  # BASELINE config 5's prefill at its configured 2048 tokens: from 512 rows up the bfp4 products run on the GEMM that
  # decodes B in registers (qkv on 128 x 384 blocks, o and down with the residual on 128 x 256, gate_up with SiLU x up
  # on 256 x 256 and a 128-row tail), at the full K of 4096 and 14336. The oracle's layer gives the rows asked for
  # (every row's keys and values still go into its cache); each within 3% of the block's change, and the cache rows
  # the block put, all 2048 of them, within 3% of their largest.
  rt, c, rc, dev, ref, (cos, sin, turn) = block
  n = size = 2048
  x = np.random.default_rng(4).standard_normal((n, DIM), dtype=np.float32)
  cache = Tensor.zeros(rt, size, HD, batch=2 * KV)
  places = Tensor.of(rt, [list(range(n))], "int32")
  rot = (dev["cos"].gather(places), dev["sin"].gather(places), dev["turn"])
  y = llama.layer(Tensor.of(rt, x[None], "fp32"), dev, c, rot, places.reshape(1, n, 1), cache, places)
  got = np.frombuffer(y.tobytes(), np.float32).reshape(n, DIM)
  rows = [0, 1, 255, 511, 512, 1024, 1500, 2047]
  mask = np.where(np.arange(size) > np.arange(n)[:, None], np.float32(-1e9), np.float32(0))
  kv = np.zeros((2 * KV, size, HD))
  want = L.layer(x, ref, rc, (cos[:n], sin[:n], turn), mask, kv, range(n), only=rows)
  change, err = np.abs(want - x[rows]).max(), np.abs(got[rows] - want).max()
  assert change > 0.5 and err < 0.03 * change, (err, change)
  got_kv = B.bf16_floats(np.frombuffer(cache.tobytes(), np.uint16)).reshape(2 * KV, size, HD)
  assert np.abs(got_kv - kv).max() < 0.03 * np.abs(kv).max()


def test_batch32_decode_matches_numpy_per_slot(block):
  rt, c, rc, dev, ref, (cos, sin, turn) = block
  S, size, place = 32, 4096, 4095
  rng = np.random.default_rng(2)
  K = B.bf16(rng.standard_normal((S * KV, size, HD), dtype=np.float32))
  V = B.bf16(rng.standard_normal((S * KV, size, HD), dtype=np.float32))
  K[:, place:], V[:, place:] = 0, 0  # the step writes row 4095 of each slot
  x = rng.standard_normal((S, DIM), dtype=np.float32)
  keys, values_ = Tensor.of(rt, K), Tensor.of(rt, V)
  at = Tensor.of(rt, [[place] * S], "int32")
  rot = (dev["cos"].gather(at), dev["sin"].gather(at), dev["turn"])
  got = np.array(llama.slots_layer(Tensor.of(rt, x[None], "fp32"), dev, c, rot, keys, values_,
                                   Tensor.of(rt, [[place]], "int32")).tolist()).reshape(S, DIM)
  new_k = np.array(keys[:, place:place + 1, :].contiguous().tolist()).reshape(S * KV, HD)
  new_v = np.array(values_[:, place:place + 1, :].contiguous().tolist()).reshape(S * KV, HD)
  mask = np.zeros((1, size), np.float32)
  for s in range(S):
    cache = np.concatenate([K[s * KV:(s + 1) * KV], V[s * KV:(s + 1) * KV]]).astype(np.float64)
    want = L.layer(x[s:s + 1], ref, rc, (cos[[place]], sin[[place]], turn), mask, cache, [place])[0]
    change, err = np.abs(want - x[s]).max(), np.abs(got[s] - want).max()
    assert change > 0.5 and err < 0.03 * change, (s, err, change)
    for g, w in ((new_k[s * KV:(s + 1) * KV], cache[:KV, place]), (new_v[s * KV:(s + 1) * KV], cache[KV:, place])):
      assert np.abs(g - w).max() < 0.03 * np.abs(w).max(), s


def test_llama31_block_at_tt_precision_matches_numpy(block):
  # test_models.py:1375-1395: one block in Llama-3.1-8B's shapes at tt_transformers' performance precision (gate_up
  # bfp4, the other matrices and the output layer bfp8, a bfp8 KV cache), Llama 3's RoPE scaling, a 2048 vocabulary:
  # a 64-token prompt, then two decode steps, each with NumPy's pick and logits within 2% of their span
  rt = block[0]
  rope = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
  kw = dict(dim=DIM, heads=HEADS, kv=KV, layers=1, eps=1e-5, theta=500000.0, ffn=FFN, vocab=2048, rope=rope)
  c, rc = llama.model(**kw), L.model(**kw)
  c.precision, rc.precision = llama.precision(c, "tt"), L.precision(rc, "tt")
  rng = np.random.default_rng(8)
  bits = lambda shape, scale, mean=0.0: B.bf16_bits(rng.normal(mean, scale, shape))
  w = {"layers.0.input_layernorm": bits((1, DIM), 0.1, 1), "layers.0.post_attention_layernorm": bits((1, DIM), 0.1, 1),
       **{f"layers.0.{name}": bits(shape, 0.02) for name, shape in SHAPES.items()},
       "norm": bits((1, DIM), 0.1, 1), "embed": bits((2048, DIM), 1.0)}
  w["embed.T"] = np.ascontiguousarray(w["embed"].T)
  dw = llama.upload(rt, {k: llama.Weight(lambda v=v: v) for k, v in w.items()}, c, places=96)
  assert {k: t.dtype for k, t in dw.items() if k.endswith("_proj")} == \
      {f"layers.0.{n}": "bfp4" if n == "gate_up_proj" else "bfp8" for n in SHAPES}
  ref = {}
  for k, v in w.items():  # the device's block floats, read back; a slice of each checked against the oracle's cast
    if k in dw and dw[k].layout == "columns":
      ref[k] = values(dw[k], v.shape)
      fmt = L.weight_format(k, rc.precision)
      assert np.array_equal(ref[k][:64], B.bfp(B.bf16_floats(v[:64]), fmt).astype(np.float32)), k
    else:
      ref[k] = B.bf16_floats(v)
  ref["cos"], ref["sin"], ref["turn"] = L.rotary(rc, 96)
  kv, np_kv = llama.kv_cache(rt, c, 96), L.kv_cache(rc, 96)
  assert kv[0].dtype == "bfp8"
  prompt = [int(i) for i in rng.integers(0, 2048, 64)]
  for new, places in ((prompt, list(range(64))), ([5], [64]), ([9], [65])):
    got = np.frombuffer(llama.forward(Tensor.of(rt, [new], "int32"), Tensor.of(rt, [places], "int32"), dw, c,
                                      kv).tobytes(), np.float32)
    want = L.forward(new, places, ref, rc, np_kv)[0]
    assert got.argmax() == want.argmax() and np.abs(got - want).max() < 0.02 * np.ptp(want), \
        (places[0], np.abs(got - want).max(), np.ptp(want))
