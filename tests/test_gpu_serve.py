"""Serving on the GPU: heads (top-k and log-sum-exp) against NumPy, and the slot engine's greedy streams against
single-sequence decode. Needs a GPU."""
import math
import numpy as np
import pytest

from baretile_amd.models import llama, serve
from baretile_amd.tensor import Tensor
from oracle import llama_ref as L

pytestmark = pytest.mark.gpu


def numpy_head(x, t, k=64):
  """The k largest of a row, largest first with equal values in column order (a stable sort), and
  log(sum(exp((x - max) * t))) in float64."""
  ids = np.argsort(-x, kind="stable")[:k]
  return x[ids], ids, math.log(np.exp((x.astype(np.float64) - x.max()) * t).sum())


def test_heads_match_numpy(rt):
  # serve.py:43-63: the 64 largest of each row with their ids, and lse at each row's inverse temperature
  rng = np.random.default_rng(3)
  x = rng.normal(0, 4, (3, 49152)).astype(np.float32)
  x[1, 7] = x[1, 40000] = x[1].max() + 1  # a tie across parts
  ts = [1.0, 0.5, 2.0]
  values, ids, lse = serve.heads(Tensor.of(rt, x[None], "fp32"), Tensor.of(rt, [[t] for t in ts], "fp32"))
  values, ids = np.array(values.tolist()).reshape(3, 64), np.array(ids.tolist()).reshape(3, 64)
  lse = np.array(lse.tolist()).reshape(3)
  for i, t in enumerate(ts):
    want_v, want_i, want_lse = numpy_head(x[i], t)
    assert np.array_equal(ids[i], want_i) and np.array_equal(values[i], want_v), i
    assert abs(lse[i] - want_lse) <= 1e-4 * max(1.0, abs(want_lse)), (i, lse[i], want_lse)


def model(rt, vocab=512, layers=2, places=64, seed=12):
  rng = np.random.default_rng(seed)
  c, w = L.smol(rng, layers, vocab=vocab, places=places)
  dc = llama.model(dim=576, heads=9, kv=3, layers=layers, eps=1e-5, theta=10000.0, vocab=vocab, ffn=1536,
                   precision=llama.precision(llama.model(layers=layers, dim=576), "bfp8"))
  host = {k: v for k, v in w.items() if k not in ("cos", "sin", "turn", "embed.T")}
  return dc, llama.upload(rt, host, dc, places=places)


def test_engine_greedy_matches_single_sequence_decode(rt):
  # three streams of different lengths decode together in three slots, one replayed step for all; each equals the same
  # prompt decoded alone (llama.generate)
  dc, dw = model(rt)
  prompts = [[7, 200, 31, 64, 5], [3, 1, 4, 1, 5, 9, 2, 6, 5], [42, 43]]
  engine = serve.Engine(rt, dw, dc, slots=3, places=64, chunk=4)
  streams = [engine.submit(serve.Stream(p, limit=8)) for p in prompts]
  for _ in range(40):
    engine.step()
    if all(s.ended for s in streams): break
  for p, s in zip(prompts, streams):
    want, _ = llama.generate(dw, dc, p, 8, 64)
    assert s.ended == "limit" and s.tokens == want, (p, s.tokens, want)
  # a fourth stream reuses a free slot's cache rows for its prompt's shared prefix
  s = engine.submit(serve.Stream(prompts[1][:6] + [100], limit=4))
  for _ in range(20):
    engine.step()
    if s.ended: break
  want, _ = llama.generate(dw, dc, prompts[1][:6] + [100], 4, 64)
  assert s.tokens == want and s.reused == 6
  # a stream that runs out of rows ends with "full" after the last token its slot can feed
  s = engine.submit(serve.Stream(list(range(1, 59)), limit=50))
  while not s.ended: engine.step()
  assert s.ended == "full" and len(s.tokens) == 64 - 1 - 58 + 1
  with pytest.raises(ValueError): engine.submit(serve.Stream(list(range(63))))
