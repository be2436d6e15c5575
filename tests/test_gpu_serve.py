"""Serving on the GPU: heads (top-k and log-sum-exp) against NumPy, and the slot engine's greedy streams against
single-sequence decode. Needs a GPU."""
import numpy as np
import pytest

from baretile_amd.models import llama, serve
from baretile_amd.tensor import Tensor
from oracle import llama_ref as L

pytestmark = pytest.mark.gpu


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
    want = serve.Head.of(x[i], t)
    assert np.array_equal(ids[i], want.ids) and np.array_equal(values[i], want.values), i
    assert abs(lse[i] - want.lse) <= 1e-4 * max(1.0, abs(want.lse)), (i, lse[i], want.lse)


def model(rt, vocab=512, layers=2, places=64, seed=12):
  rng = np.random.default_rng(seed)
  c, w = L.smol(rng, layers, vocab=vocab, places=places)
  dc = llama.model(dim=576, heads=9, kv=3, layers=layers, eps=1e-5, theta=10000.0, vocab=vocab, ffn=1536,
                   precision=llama.precision(llama.model(layers=layers, dim=576), "bfp8"))
  host = {k: v for k, v in w.items() if k not in ("cos", "sin", "turn", "embed.T")}
  return dc, llama.upload(rt, host, dc, places=places)


def test_engine_greedy_matches_single_sequence_decode(rt):
  # three requests of different lengths decode together in three slots, one replayed step for all; each stream equals
  # the same prompt decoded alone (llama.generate)
  dc, dw = model(rt)
  prompts = [[7, 200, 31, 64, 5], [3, 1, 4, 1, 5, 9, 2, 6, 5], [42, 43]]
  engine = serve.Engine(rt, dw, dc, slots=3, places=64, chunk=4)
  reqs = [serve.Request(p, max_tokens=8, temperature=0) for p in prompts]
  for r in reqs: assert engine.offer(r)
  for _ in range(40):
    engine.step()
    if all(r.finish for r in reqs): break
  for p, r in zip(prompts, reqs):
    want, _ = llama.generate(dw, dc, p, 8, 64)
    assert r.finish == "length" and r.made == want, (p, r.made, want)
  # a fourth request reuses a free slot, and its prompt's shared prefix
  r = serve.Request(prompts[1][:6] + [100], max_tokens=4, temperature=0)
  assert engine.offer(r)
  for _ in range(20):
    engine.step()
    if r.finish: break
  want, _ = llama.generate(dw, dc, prompts[1][:6] + [100], 4, 64)
  assert r.made == want and r.cached == 6
