"""Serving on baretile_amd: requests decode together in cache slots of one model, a replayed step for all slots and the
heads of the logits (top-k and log-sum-exp) found on the device. The hot path of baretile/models/serve.py:
Engine.decode, heads and Engine.advance (serve.py:43-63, 417-426, 455-457), with the host side it needs to run:
Head, Request's sampling from a head, and the Engine's admit / fill / advance loop.

Out of scope here: the HTTP server, chat templates, tokenizers and text, stop strings, penalties, output constraints,
saved sessions, speculative decoding and Qwen's recurrent state. Requests speak token ids.
"""
import math, queue, threading
import numpy as np
from baretile_amd.tensor import Tensor, jit
from baretile_amd.models import llama


class Head:
  """The largest logits of a row with their token ids, in descending order, and lse = log(sum(exp((x - max(x)) * t)))
  over the whole row for the inverse temperature t (serve.py:19-31). row() reads the full row when sampling needs it.
  Head.of makes the same from NumPy logits."""
  def __init__(self, values, ids, lse, row):
    self.values, self.ids, self.lse, self.row = np.asarray(values, np.float64), np.asarray(ids), float(lse), row

  @staticmethod
  def of(logits, t=1.0, k=64):
    """From a NumPy row: the k largest, the first of equals first (stable), and lse at t."""
    logits = finite(np.asarray(logits, np.float64))
    ids = np.argsort(-logits, kind="stable")[:k]
    m = float(logits[ids[0]])
    return Head(logits[ids], ids, math.log(np.exp((logits - m) * t).sum()), lambda: logits)


def finite(logits):
  """Logits sampling can use: a nonempty row whose maximum is finite (serve.py:33-36)."""
  if logits.ndim != 1 or not logits.size or not np.isfinite(logits.max()):
    raise ValueError("sampling needs a nonempty logit row with a finite maximum and no NaN")
  return logits


def scale(r):
  """The inverse temperature of a request; any value serves greedy picks (serve.py:41)."""
  return 1 / r.temperature if r and r.temperature > 0 else 1.0


def heads(logits, t=None, k=64):
  """The head of each row of fp32 logits, on the device: (values, ids[, lse]) realized (serve.py:43-63).

  topk runs on equal parts of each row, 4096 columns or fewer, then on the best of the parts by their labels. Given t,
  a column with each row's inverse temperature, lse = log(sum(exp((x - max) * t))) comes from one reduction over the
  row. Returns None for a row that doesn't split so, and the host then finds the heads in NumPy."""
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


class Request:
  """A prompt of token ids and its sampling settings; made collects the new tokens. Ends at an eos id, max_tokens or
  a full slot; finish records why (serve.py:65-101). out receives each token id, then None at the end."""
  def __init__(self, ids, max_tokens=16, temperature=1.0, top_p=1.0, eos=(), seed=None, top_k=0, min_p=0.0):
    if type(max_tokens) is not int or max_tokens < 1: raise ValueError("max_tokens must be a positive integer")
    if type(top_k) is not int or top_k < 0: raise ValueError("top_k must be a nonnegative integer")
    for name, v in (("temperature", temperature), ("top_p", top_p), ("min_p", min_p)):
      if not isinstance(v, (int, float)) or isinstance(v, bool) or not math.isfinite(v): raise ValueError(f"{name} must be a finite number")
    if temperature < 0: raise ValueError("temperature must be nonnegative")
    if not 0 < top_p <= 1 or not 0 <= min_p <= 1: raise ValueError("top_p must be in (0, 1] and min_p in [0, 1]")
    self.ids, self.max_tokens, self.temperature, self.top_p, self.top_k, self.min_p = list(ids), max_tokens, temperature, top_p, top_k, min_p
    self.eos, self.rng = set(eos), np.random.default_rng(seed)
    self.made, self.out, self.finish, self.gone, self.cached, self.room = [], queue.Queue(), None, False, 0, None

  def sample(self, head):
    """The token draw would pick, from the head alone where it decides it (serve.py:143-170); None where a top_k or
    a top_p / min_p cut reaches past the head. With no cut, a draw past the head's mass reads the row back."""
    finite(head.values)
    if self.temperature == 0: return int(head.ids[0])
    if not math.isfinite(head.lse) or head.lse < 0: return self.draw(head.row())
    t, k = 1 / self.temperature, len(head.ids)
    p, total = np.exp((head.values - head.values[0]) * t), math.exp(head.lse)
    keep = None
    if self.top_k or self.top_p < 1:
      if self.top_k > k: return None
      run = np.cumsum(p[:self.top_k or k])
      if self.top_p < 1 and not self.top_k and run[-1] < self.top_p * total: return None
      keep = np.arange(np.searchsorted(run, self.top_p * (run[-1] if self.top_k else total)) + 1 if self.top_p < 1 else len(run))
    if self.min_p:
      if keep is None and p[-1] >= self.min_p: return None
      keep = np.flatnonzero(p >= self.min_p) if keep is None else keep[p[keep] >= self.min_p]
    if keep is None:
      run, u = np.cumsum(p), self.rng.random() * total
      if u < run[-1]: return int(head.ids[min(int(np.searchsorted(run, u, side="right")), k - 1)])
      rest = np.exp((np.float64(head.row()) - head.values[0]) * t)
      rest[head.ids] = 0
      cum = np.cumsum(rest)
      return min(int(np.searchsorted(cum, (u - run[-1]) / max(total - run[-1], 1e-300) * cum[-1], side="right")), len(rest) - 1)
    w = np.cumsum(p[keep])
    return int(head.ids[keep[min(int(np.searchsorted(w, self.rng.random() * w[-1], side="right")), len(keep) - 1)]])

  def draw(self, logits):
    """From a whole row: the largest at temperature 0, else a sample after the top_k, top_p and min_p cuts
    (serve.py:172-188)."""
    logits = finite(np.asarray(logits, np.float64))
    if self.temperature == 0: return int(logits.argmax())
    p, keep = np.exp((logits - logits.max()) / self.temperature), None
    if self.top_k or self.top_p < 1:
      keep = np.argsort(-p, kind="stable")[:self.top_k or len(p)]
      if self.top_p < 1: keep = keep[:np.searchsorted(np.cumsum(p[keep]), self.top_p * (p[keep] if self.top_k else p).sum()) + 1]
    if self.min_p: keep = np.flatnonzero(p >= self.min_p * p.max()) if keep is None else keep[p[keep] >= self.min_p * p.max()]
    w = p if keep is None else p[keep]
    i = min(int(np.searchsorted(np.cumsum(w), self.rng.random() * w.sum(), side="right")), len(w) - 1)
    return i if keep is None else int(keep[i])

  def pick(self, head):
    token = self.sample(head)
    return token if token is not None else self.draw(head.row())

  def take(self, head, room):
    """The next token from a Head or a NumPy row; room tells whether the slot can hold it. True when the request
    ends."""
    if self.gone: self.finish = "gone"; return True
    head = head if isinstance(head, Head) else Head.of(head, scale(self))
    token = self.pick(head)
    if token in self.eos:
      self.finish = "stop"
      return True
    self.made.append(token)
    self.out.put(token)
    if len(self.made) == self.max_tokens or not room:
      self.finish = "length"
      return True
    return False

  def end(self):
    if self.room: self.room.release(); self.room = None
    self.out.put(None)


class Engine:
  """Decodes requests together, one cache slot each, on one runtime (serve.py:228-522, reduced). Each slot owns
  `places` rows of every block's cache; a step decodes one token for every slot in a recorded, replayed forward, and
  the heads of its logits come back instead of the logits where they decide the pick. A free slot's token sits at its
  region's last row, which is kept for it."""
  def __init__(self, rt, w, c, slots=4, places=512, chunk=None):
    if slots < 1 or places < 4: raise ValueError("an engine needs a slot and room for a prompt")
    self.rt, self.w, self.c, self.slots, self.places = rt, w, c, slots, places
    self.chunk = chunk or places
    self.kv = llama.kv_cache(rt, c, slots * places)
    self.slot = [[cache[:, u * places:(u + 1) * places, :] for cache in self.kv] for u in range(slots)]
    self.held, self.busy, self.used = [[] for _ in range(slots)], [None] * slots, [0] * slots
    self.replays, self.made = {}, {}
    self.waiting, self.prefilled = queue.Queue(), 0
    self.room = threading.BoundedSemaphore(slots)
    self.lock, self.failed = threading.Lock(), False

  def on(self, row, dtype="int32"): return Tensor.of(self.rt, [row], dtype)

  def column(self, ts): return Tensor.of(self.rt, [[x] for x in ts], "fp32")

  def offer(self, r):
    """Queues r if a slot is free and holds the slot until r ends; False without waiting otherwise."""
    with self.lock:
      if self.failed: raise RuntimeError("the engine stopped on an error")
      if not 0 < len(r.ids) < self.places - 1: raise ValueError(f"a prompt needs 1 to {self.places - 2} tokens, not {len(r.ids)}")
      if not self.room.acquire(blocking=False): return False
      r.room = self.room
      self.waiting.put(r)
      return True

  def reach(self, held, ids):
    """The reusable prefix of ids in held; the prompt's last token always runs again."""
    return min(next((i for i, (a, b) in enumerate(zip(held, ids)) if a != b), min(len(held), len(ids))), len(ids) - 1)

  def admit(self, r):
    """The free slot with the longest reusable prefix of r's prompt, least recently used first."""
    if r.gone: return r.end()
    free = [u for u, b in enumerate(self.busy) if b is None]
    u = max(free, key=lambda u: (self.reach(self.held[u], r.ids), -self.used[u]))
    self.used[u], self.busy[u] = max(self.used) + 1, r
    n = self.reach(self.held[u], r.ids)
    self.held[u], r.cached = r.ids[:n], n

  def fill(self, u):
    """Prefills the next chunk of slot u's prompt in its region of the caches; the last chunk picks the first token."""
    r, at = self.busy[u], len(self.held[u])
    if r.gone: return self.take(u, None)
    ids = r.ids[at:at + self.chunk]
    out = llama.forward(self.on(ids), self.on(list(range(at, at + len(ids)))), self.w, self.c, self.slot[u])
    self.held[u] += ids
    self.prefilled += len(ids)
    if len(self.held[u]) == len(r.ids):
      row = np.frombuffer(out.tobytes(), np.float32).astype(np.float64)
      if self.take(u, Head.of(row, scale(r)), 1, end=False): self.release(u)

  def replay(self, f):
    """The replay (jit) of f; made keeps what its last call made."""
    if f not in self.replays:
      def run(*xs):
        self.made[f] = f(*xs)
        return self.made[f][0]
      self.replays[f] = jit(run)
    return self.replays[f]

  def decode(self, ids, places, t):
    """Replayed: the next logits of every slot, and their heads at t (serve.py:455-457)."""
    logits = llama.forward(ids, places, self.w, self.c, self.kv, slots=self.slots).realize()
    return logits, heads(logits, t)

  def rows(self, f):
    """Heads for the rows of the last call of f, read back; a row's logits are read only if sampling needs them."""
    logits, made = self.made[f]
    whole = {}
    def row(i):
      if "all" not in whole: whole["all"] = np.frombuffer(logits.tobytes(), np.float32).reshape(self.slots, -1).astype(np.float64)
      return whole["all"][i]
    if made is None: return [row(i) for i in range(self.slots)]
    values, ids, lse = (np.array(x.tolist(), np.float64).reshape(self.slots, -1) for x in made)
    return [Head(values[i], ids[i].astype(np.int64), lse[i, 0], lambda i=i: row(i)) for i in range(self.slots)]

  def advance(self):
    """Decodes one token for every occupied slot."""
    live = [r if r and r.made else None for r in self.busy]
    if not any(live): return
    ids = [r.made[-1] if r else 0 for r in live]
    places = [len(h) if r else self.places - 1 for h, r in zip(self.held, live)]
    self.replay(self.decode)(self.on(ids), self.on(places), self.column([scale(r) for r in live]))
    for u, (r, head) in enumerate(zip(live, self.rows(self.decode))):
      if r:
        self.held[u].append(r.made[-1])
        self.take(u, head)

  def take(self, u, head, room=1, end=True):
    r = self.busy[u]
    try: done = head is None or r.take(head, len(self.held[u]) + room < self.places - 1)
    except Exception as e:
      r.finish, r.error, done = "error", f"{type(e).__name__}: {e}", True
    if done and end: self.release(u)
    return done

  def release(self, u):
    r = self.busy[u]
    self.busy[u] = None
    r.end()

  def step(self):
    """One turn of the engine's loop: admit while a slot is free, prefill a chunk, decode a token for all slots."""
    while None in self.busy and not self.waiting.empty(): self.admit(self.waiting.get())
    if filling := [u for u, r in enumerate(self.busy) if r and not r.made]: self.fill(filling[0])
    self.advance()

  def run(self):
    """The engine's thread: steps until an error, which ends every request (serve.py:507-521)."""
    try:
      while True:
        if not any(self.busy): self.admit(self.waiting.get())
        self.step()
    except BaseException:
      with self.lock:
        self.failed = True
        pending = [r for r in self.busy if r]
        while not self.waiting.empty(): pending.append(self.waiting.get_nowait())
        for r in pending: r.finish = "error"; r.end()
      raise
