"""Serving: heads of logits on the device, the slot engine against single-sequence decode, and the host sampler."""
import numpy as np
import pytest

from baretile_amd.models import serve


def test_sampling_from_a_head_matches_the_row():
  # serve.py:143-188: where the head decides the pick (greedy, a top_k or top_p cut within it), a pick from the head
  # equals the pick from the whole row with the same seed
  rng = np.random.default_rng(0)
  for trial in range(40):
    logits = rng.normal(0, 3, 1000)
    for kw in (dict(temperature=0), dict(temperature=0.7, top_k=20), dict(temperature=0.5, top_p=0.9)):
      a, b = serve.Request([1], seed=trial, **kw), serve.Request([1], seed=trial, **kw)
      head = serve.Head.of(logits, serve.scale(a), k=64)
      assert a.pick(head) == b.draw(logits), (trial, kw)


def test_sampling_without_a_cut_keeps_every_probability():
  # with no cut a draw may land past the head's mass and then reads the row back: every token keeps its probability
  rng = np.random.default_rng(1)
  logits = rng.normal(0, 1, 50)
  r = serve.Request([1], seed=5, temperature=1.5)
  head = serve.Head.of(logits, serve.scale(r), k=10)
  n = 40000
  counts = np.bincount([r.pick(head) for _ in range(n)], minlength=50)
  p = np.exp(logits / 1.5 - (logits / 1.5).max())
  assert np.abs(counts / n - p / p.sum()).max() < 0.01


def test_request_ends():
  r = serve.Request([1, 2], max_tokens=2, temperature=0, eos=(5,))
  assert not r.take(np.array([0.0, 3.0, 1.0, 0.0, 0.0, 0.0]), True) and r.made == [1]
  assert r.take(np.array([0.0, 0.0, 1.0, 0.0, 0.0, 9.0]), True) and r.finish == "stop" and r.made == [1]
  r = serve.Request([1], max_tokens=1, temperature=0)
  assert r.take(np.array([0.0, 3.0]), True) and r.finish == "length"
  with pytest.raises(ValueError): serve.Request([1], temperature=-1)
  with pytest.raises(ValueError): serve.Request([1], top_p=0)
