"""Serving on baretile_amd: greedy token streams decoded together, one cache slot each, on one model.

What this keeps of baretile/models/serve.py is its hot path: `heads` (serve.py:43-63), the top-k and log-sum-exp of
rows of logits found on the device so only a few values per row come back, and `Engine.decode` (serve.py:455-457), one
forward over every slot recorded once and replayed each step. Around them sits the least a greedy stream needs:
slots that each own a region of every block's KV cache, prompts prefilled in chunks into their slot, a prompt's shared
prefix reused from a free slot's cache rows, and one replayed decode step for all slots.

Out of scope: sampling (temperature, top-k/top-p/min-p draws), the HTTP server, chat templates, tokenizers and text,
stop strings, saved sessions, speculative decoding and Qwen's recurrent state. Streams speak token ids.
"""
import queue, threading
import numpy as np
from baretile_amd.tensor import Tensor, jit
from baretile_amd.models import llama


def heads(logits, t=None, k=64):
  """The head of each row of fp32 logits, on the device: (values, ids[, lse]) realized (serve.py:43-63).

  values and ids are each row's k largest logits and their columns, largest first, equal values in column order.
  topk runs on equal parts of each row, 4096 columns or fewer, then on the parts' winners by their labels. Given t,
  a column with each row's inverse temperature, lse = log(sum(exp((x - max) * t))) over the row comes from one
  reduction. Returns None for a row that doesn't split so."""
  cols = logits.cols
  parts = next((p for p in range(1, 126) if cols % p == 0 and cols // p <= 4096), None)
  if parts is None or k > cols // parts: return None
  best, ids = logits.topk(k, parts)
  values, ids = best.topk(k, labels=ids) if parts > 1 else (best, ids)
  values, ids = values.realize(), ids.realize()
  if t is None: return values, ids
  m = values[:, :, 0:1]  # the row's largest: the first of its head
  lse = ((logits - m) * t).exp().sum(2).log()
  return values, ids, lse.realize()


class Stream:
  """A prompt of token ids, decoded greedily. `tokens` collects the new ids as they come. It ends after `limit`
  tokens ("limit"), at a token in `stop`, which is not kept ("stop"), when its slot has no row left for the next
  token ("full"), or on an error ("error"); `ended` says which, and `finished` is set then. `reused` counts the
  prompt's leading tokens whose cache rows were found in its slot and not computed again."""
  def __init__(self, prompt, limit=16, stop=()):
    if type(limit) is not int or limit < 1: raise ValueError("a stream's limit must be a positive integer")
    self.prompt, self.limit, self.stop = [int(i) for i in prompt], limit, frozenset(stop)
    if not self.prompt: raise ValueError("a stream needs at least one prompt token")
    self.tokens, self.ended, self.reused, self.finished = [], None, 0, threading.Event()

  def wait(self, timeout=None):
    """The new tokens, once the stream has ended (TimeoutError if it hasn't within timeout seconds)."""
    if not self.finished.wait(timeout): raise TimeoutError("the stream is still decoding")
    return self.tokens

  def offer(self, token, room):
    """Takes the next token; room says whether the slot can still hold it. True once the stream has ended."""
    if token in self.stop: return self.end("stop")
    self.tokens.append(token)
    if len(self.tokens) == self.limit: return self.end("limit")
    return False if room else self.end("full")

  def end(self, why):
    self.ended = why
    self.finished.set()
    return True


def shared(kept, prompt):
  """How many of prompt's leading tokens a slot holding `kept` can skip: their common prefix, but never the prompt's
  last token, whose logits pick the first new token."""
  n = 0
  for a, b in zip(kept, prompt):
    if a != b: break
    n += 1
  return min(n, len(prompt) - 1)


class Slot:
  """A region of `places` rows in every block's cache. `kept` lists the tokens whose keys and values fill its first
  rows, `stream` is the stream it decodes (or None when free), and `stamp` orders slots by last use."""
  def __init__(self, caches):
    self.caches, self.kept, self.stream, self.stamp = caches, [], None, 0

  @property
  def prefilled(self): return self.stream is not None and len(self.kept) >= len(self.stream.prompt)


class Engine:
  """Greedy streams decoded together on one runtime (serve.py:228-522, reduced to its decode path). Every block's cache
  is cut into `slots` regions of `places` rows. step() admits waiting streams into free slots, prefills one chunk of
  one prompt, then decodes one token for every slot past its prompt in a single replayed forward. A free slot still
  runs through that forward: its token sits at its region's last row, which no stream uses, and sees only its
  region's first row."""
  def __init__(self, rt, w, c, slots=4, places=512, chunk=None):
    if slots < 1 or places < 4: raise ValueError("an engine needs at least one slot of at least 4 rows")
    self.rt, self.w, self.c, self.places, self.chunk = rt, w, c, places, chunk or places
    self.kv = llama.kv_cache(rt, c, slots * places)
    self.slots = [Slot([cache[:, u * places:(u + 1) * places, :] for cache in self.kv]) for u in range(slots)]
    self.waiting, self.clock, self.made = queue.Queue(), 0, None
    self.step_replay = jit(self._recorded)
    self.error, self.halt = None, threading.Event()

  def submit(self, stream):
    """Queues a stream; it starts once a slot is free. ValueError for a prompt its slot can't hold."""
    if self.error is not None: raise RuntimeError(f"the engine stopped: {self.error}")
    if len(stream.prompt) > self.places - 2:
      raise ValueError(f"a prompt of {len(stream.prompt)} tokens doesn't fit a slot of {self.places} rows")
    self.waiting.put(stream)
    return stream

  def row(self, values, dtype="int32"): return Tensor.of(self.rt, [list(values)], dtype)

  def decode(self, ids, places, t=None):
    """The next logits of every slot, and their heads at t (serve.py:455-457): llama.forward over the slots, then heads.
    ids and places are int32 rows with one entry per slot."""
    logits = llama.forward(ids, places, self.w, self.c, self.kv, slots=len(self.slots)).realize()
    return logits, heads(logits, t, k=1)

  def _recorded(self, ids, places):  # what the replay runs: decode, keeping its heads where the next call reads them
    logits, self.made = self.decode(ids, places)
    return logits

  def admit(self):
    """Moves waiting streams into free slots: each to the free slot whose kept tokens share the longest prefix with
    its prompt, the least recently used of equals."""
    while not self.waiting.empty():
      free = [s for s in self.slots if s.stream is None]
      if not free: return
      stream = self.waiting.get_nowait()
      slot = max(free, key=lambda s: (shared(s.kept, stream.prompt), -s.stamp))
      n = shared(slot.kept, stream.prompt)
      self.clock += 1
      slot.kept, slot.stream, slot.stamp, stream.reused = slot.kept[:n], stream, self.clock, n

  def fill(self, slot):
    """Prefills the next chunk of the slot's prompt into its rows; the last chunk's logits give the first token."""
    at, prompt = len(slot.kept), slot.stream.prompt
    ids = prompt[at:at + self.chunk]
    logits = llama.forward(self.row(ids), self.row(range(at, at + len(ids))), self.w, self.c, slot.caches)
    slot.kept += ids
    if slot.prefilled: self.settle(slot, llama.argmax(logits))

  def advance(self):
    """One token for every slot past its prompt, from one replay of the decode step over all slots."""
    live = [s if s.prefilled and s.stream.tokens else None for s in self.slots]
    if not any(live): return
    ids = [s.stream.tokens[-1] if s else 0 for s in live]
    places = [len(s.kept) if s else self.places - 1 for s in live]
    self.step_replay(self.row(ids), self.row(places))
    picks = np.asarray(self.made[1].tolist()).reshape(len(self.slots), -1)[:, 0]
    for s, pick in zip(live, picks):
      if s is None: continue
      s.kept.append(s.stream.tokens[-1])
      self.settle(s, int(pick))

  def settle(self, slot, token):
    """Gives the slot's stream its next token, and frees the slot when the stream ends. The token will be fed at row
    len(kept), which must leave the region's last row free."""
    if slot.stream.offer(token, len(slot.kept) < self.places - 1): slot.stream = None

  def step(self):
    """Admit, prefill one chunk, decode one token for every decoding slot."""
    self.admit()
    filling = [s for s in self.slots if s.stream is not None and not s.prefilled]
    if filling: self.fill(filling[0])
    self.advance()

  def busy(self): return not self.waiting.empty() or any(s.stream is not None for s in self.slots)

  def run(self, idle=0.01):
    """The engine's loop, for a thread of its own: steps while there is work, until stop(). An error ends every
    stream it holds with "error" and stops the engine."""
    try:
      while not self.halt.is_set():
        if self.busy(): self.step()
        else: self.halt.wait(idle)
    except BaseException as e:
      self.error = f"{type(e).__name__}: {e}"
      for s in self.slots:
        if s.stream is not None: s.stream.end("error"); s.stream = None
      while not self.waiting.empty(): self.waiting.get_nowait().end("error")
      raise

  def stop(self): self.halt.set()
