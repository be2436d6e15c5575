"""Serving's host logic, on the CPU: how a stream takes tokens and ends, and which prompt tokens a slot can skip."""
import pytest

from baretile_amd.models import serve


def test_stream_ends_at_limit_stop_or_full_slot():
  s = serve.Stream([1, 2], limit=3, stop=(5,))
  assert not s.offer(7, True) and s.tokens == [7] and s.ended is None
  assert s.offer(5, True) and s.ended == "stop" and s.tokens == [7] and s.finished.is_set()
  s = serve.Stream([1], limit=2)
  assert not s.offer(4, True) and s.offer(4, True) and s.ended == "limit" and s.wait(0) == [4, 4]
  s = serve.Stream([1], limit=9)
  assert s.offer(3, False) and s.ended == "full" and s.tokens == [3]  # the token is kept; no row is left to feed it
  with pytest.raises(TimeoutError): serve.Stream([1]).wait(0)
  for bad in (dict(prompt=[], limit=2), dict(prompt=[1], limit=0), dict(prompt=[1], limit=1.5)):
    with pytest.raises(ValueError): serve.Stream(**bad)


def test_shared_prefix_keeps_the_last_prompt_token():
  assert serve.shared([], [1, 2, 3]) == 0
  assert serve.shared([1, 2, 9, 9], [1, 2, 3]) == 2
  assert serve.shared([1, 2, 3, 4], [1, 2, 3]) == 2  # all of it is kept, but the last token runs again for its logits
  assert serve.shared([1, 2, 3], [1, 2, 3, 4, 5]) == 3
  assert serve.shared([5], [1]) == 0
