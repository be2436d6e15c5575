"""The Llama decoder in NumPy, restating the reference's NumPy branch — TEST INFRASTRUCTURE ONLY.

Not imported by the product. Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline. This is the
parity oracle for models.llama on the device: same weights (block floats rounded by oracle.bfp), float32 weights
with full products, and a float64 KV cache, as the reference's NumPy path has (llama.py:686 passes np.zeros).

Reference sources restated here (Llama family only; Qwen/gpt-oss extras are out of scope):
  models/llama.py:48-83    precision(c, mode, kv)
  models/llama.py:91-95    rms: x * rsqrt(mean(x^2) + eps) * w (bf16 rounding is the identity in NumPy, llama.py:27)
  models/llama.py:103-104  rope: x * cos + (x @ turn) * sin
  models/llama.py:106-183  layer / attention / mlp / glu (NumPy branch: full scores, softmax(s + mask) @ v)
  models/llama.py:151-154  attention's put: rows going into a block-float (bfp8/bfp4) cache are rounded by gpt2.bfp first
  models/llama.py:187-227  frequencies (default RoPE and Llama 3's scaling) and rotary: fp32 angles, bf16 tables
                           repeated across heads, q's rows carrying 1/sqrt(head width), v's cos 1 and sin 0
  models/llama.py:238-291  fuse: q, k, v side by side; gate and up side by side
  models/llama.py:293-316  around (no slots): rows = places, rotary rows, mask over the cache's rows
  models/llama.py:325-363  forward (fp32 residual, last row's logits) and prefill in chunks
  models/llama.py:365-373  kv_cache: (2 * kv, size, head) zeros per block
  models/llama.py:464-510  weight_format and arrays: block-float weights rounded 1024 rows at a time
  models/gpt2.py:101-114   masked: -1e9 for keys past a token's place
  test/test_models.py:639-645  smol(): SmolLM-135M shapes with random weights

How it is pinned (tests/test_oracle.py):
  forward        against transformers' LlamaForCausalLM (an independent implementation) on the CPU in float64
                 with the same weights, to a tolerance that covers the bf16 rounding of the RoPE tables
  kv cache       a decode step after a prompt equals the full-prompt forward at the last position (the reference's
                 own check, test_models.py:851), and prefill in chunks equals one forward (test_models.py:1539)
  precision      the reference's known answers (test_models.py:1549-1556 for the "tt" and "bf16" keys)
  frequencies    Llama 3's scaled frequencies against transformers' own llama3 RoPE initialisation (rtol 1e-6, as
                 test_models.py:676-688), with its known answers: short wavelengths kept, long ones slowed by the factor
  kv rounding    a block-float cache holds, row for row, bfp() of what a bf16 cache holds after the same step, every
                 row is a fixed point of bfp(), and the logits move by less than the rounding can explain
"""
import math
from types import SimpleNamespace
import numpy as np
from oracle import bfp as B


def model(**kw):
  """A config: dim, heads, kv, layers, eps, theta, plus vocab, ffn, head_dim, precision and rope, the RoPE scaling
  parameters or None (llama.py:392-394, 418-425)."""
  base = dict(head_dim=None, vocab=None, ffn=None, precision=None, places=None, rope=None)
  return SimpleNamespace(**(base | kw))


def head(c): return c.head_dim or c.dim // c.heads


def precision(c, mode="bf16", kv=None):
  """{(op, block): (format, phases)} for the Llama family (llama.py:48-83). Phases are kept as data only: the
  device always computes exact bf16 products (fidelity 4)."""
  if mode not in ("bf16", "bfp8", "bfp4", "tt"): raise ValueError(f"unknown precision mode: {mode}")
  if kv is not None and kv not in ("bf16", "bfp8", "bfp4"): raise ValueError(f"unknown KV cache format: {kv}")
  def entry(op):
    if mode in ("bf16", "bfp8"): return (mode, 4)
    fmt = "bfp4" if op == "gate_up" else "bfp8"
    if mode == "tt": return (fmt, 1 if fmt == "bfp4" else 2)
    return (fmt, 4)
  p = {(op, l): entry(op) for l in range(c.layers) for op in ("qkv", "o", "gate_up", "down")}
  if mode == "tt" and (c.layers, c.dim) == (32, 4096): p["gate_up", 31] = ("bfp8", 2)
  p["head", None] = entry("head")
  p["attention", "decode"] = (None, 2 if mode == "tt" else 4)
  p["attention", "prefill"] = (None, 4)
  p["kv", None] = (kv or ("bfp8" if mode == "tt" else "bf16"), None)
  return p


def weight_format(name, prec):
  """A weight's storage format (llama.py:464-474): block matrices and the output layer from prec, else bf16."""
  if not prec: return "bf16"
  if name == "embed.T": key = ("head", None)
  elif name.startswith("layers.") and name.endswith("_proj"):
    key = (name.split(".")[-1].removesuffix("_proj"), int(name.split(".")[1]))
  else: return "bf16"
  return prec[key][0] if key in prec else "bf16"


def frequencies(c):
  """RoPE inverse frequencies in float32 (llama.py:187-200). Llama 3's scaling (rope_type "llama3") divides the
  frequencies of wavelengths longer than original / low_freq_factor by the factor, keeps those shorter than
  original / high_freq_factor, and in between blends the two linearly in original / wavelength."""
  hd = head(c)
  inv = (1 / c.theta ** (np.arange(0, hd, 2, dtype=np.float32) / hd)).astype(np.float32)
  r = getattr(c, "rope", None)
  if r and r.get("rope_type") == "llama3":
    factor, lo, hi = r["factor"], r["low_freq_factor"], r["high_freq_factor"]
    span = r["original_max_position_embeddings"]
    wave = np.float32(2 * math.pi) / inv
    slow = inv / np.float32(factor)
    t = (np.float32(span) / wave - np.float32(lo)) / np.float32(hi - lo)  # 0 at the long end of the blend, 1 at the short
    inv = np.where(wave > span / lo, slow, np.where(wave < span / hi, inv, (1 - t) * slow + t * inv)).astype(np.float32)
  return inv


def rotary(c, n):
  """(cos, sin, turn) for positions 0..n-1 (llama.py:209-227). Tables are bf16-rounded float32 of shape
  (n, (heads + 2 kv) * hd): q's heads carry hd^-0.5, k's are plain, v's have cos 1 and sin 0. turn maps a head to
  (-x2, x1)."""
  hd = head(c)
  inv = frequencies(c)
  ang = np.arange(n, dtype=np.float32)[:, None] * inv[None]
  def table(g, still):
    t = np.concatenate([g(ang), g(ang)], 1).astype(np.float32)
    rows = [t * np.float32(hd ** -0.5)] * c.heads + [t] * c.kv + [np.full_like(t, still)] * c.kv
    return B.bf16(np.concatenate(rows, 1))
  turn = np.zeros((hd, hd), np.float32)
  half = np.arange(hd // 2)
  turn[half + hd // 2, half] = -1
  turn[half, half + hd // 2] = 1
  return table(np.cos, 1.0), table(np.sin, 0.0), turn


def fuse(w, c):
  """q, k, v become qkv_proj and gate, up become gate_up_proj (llama.py:238-291), for each block."""
  w = dict(w)
  for l in range(c.layers):
    p = f"layers.{l}."
    w[p + "qkv_proj"] = np.concatenate([w.pop(p + n) for n in ("q_proj", "k_proj", "v_proj")], 1)
    w[p + "gate_up_proj"] = np.concatenate([w.pop(p + n) for n in ("gate_proj", "up_proj")], 1)
  return w


def smol(rng, layers, vocab=256, places=64):
  """SmolLM-135M's config and random weights in its shapes, bf16-rounded float32 (test_models.py:639-645):
  linears N(0, 0.02) laid out for x @ w, norms N(1, 0.1), embedding N(0, 1), tied output layer."""
  c = model(dim=576, heads=9, kv=3, layers=layers, eps=1e-5, theta=10000.0, vocab=vocab, ffn=1536)
  shapes = {"input_layernorm": (1, 576, 1), "post_attention_layernorm": (1, 576, 1), "q_proj": (576, 576, 0),
            "k_proj": (576, 192, 0), "v_proj": (576, 192, 0), "o_proj": (576, 576, 0), "gate_proj": (576, 1536, 0),
            "up_proj": (576, 1536, 0), "down_proj": (1536, 576, 0)}
  w = {}
  for l in range(layers):
    for k, (r, n, mean) in shapes.items():
      w[f"layers.{l}.{k}"] = B.bf16(rng.normal(mean, 0.1 if r == 1 else 0.02, (r, n)))
  w["norm"] = B.bf16(rng.normal(1, 0.1, (1, 576)))
  w["embed"] = B.bf16(rng.normal(0, 1, (vocab, 576)))
  w["embed.T"] = np.ascontiguousarray(w["embed"].T)
  w["cos"], w["sin"], w["turn"] = rotary(c, places)
  return c, fuse(w, c)


def arrays(w, prec):
  """The weights as the device holds them: block-float matrices rounded by oracle.bfp, 1024 rows at a time
  (llama.py:500-510), as float32."""
  out = {}
  for name, v in w.items():
    f = weight_format(name, prec)
    if f == "bf16": out[name] = v
    else:
      rows = v.reshape(-1, v.shape[-1])
      out[name] = np.concatenate([B.bfp(rows[i:i + 1024], f) for i in range(0, len(rows), 1024)]).astype(np.float32).reshape(v.shape)
  return out


def kv_cache(c, size):
  """A (2 * kv, size, head) float64 zeros cache per block (llama.py:365-373 with np.zeros)."""
  return [np.zeros((2 * c.kv, size, head(c))) for _ in range(c.layers)]


def rms(x, w, eps):
  return x * (1 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)) * w


def rope(x, cos, sin, turn):
  return x * cos + (x @ turn) * sin


def split(a, n):  # (rows, n * w) -> (n, rows, w)
  return a.reshape(a.shape[0], n, -1).transpose(1, 0, 2)


def merge(a):  # (n, rows, w) -> (rows, n * w)
  return a.transpose(1, 0, 2).reshape(a.shape[1], -1)


def cache_format(c):
  """The KV cache's format, precision's kv entry (llama.py:74-83); bf16 without a precision table."""
  return ((c.precision or {}).get(("kv", None)) or ("bf16", None))[0] or "bf16"


def attention(h, p, c, rot, mask, cache, rows, only=None):
  """One block's attention on the NumPy branch (llama.py:132-172). The new key and value rows go into the cache as a
  cache of c's format holds them: a block-float cache rounds each run of 16 along a row by bfp (llama.py:151-154).
  only, a list of row indices, returns those query rows alone (every row's keys and values still go into the cache);
  a row's attention reads no other query row, so this is the full result's rows."""
  hd, rep, nh = head(c), c.heads // c.kv, c.heads + 2 * c.kv
  qkv = split(h @ p["qkv_proj"], nh)
  qkv = merge(rope(qkv, split(rot[0], nh), split(rot[1], nh), rot[2]))
  heads = split(qkv, nh)
  kv, fmt = heads[c.heads:c.heads + 2 * c.kv], cache_format(c)
  cache[:, list(rows)] = B.bfp(kv, fmt) if fmt != "bf16" else kv
  q, k, v = heads[:c.heads], cache[:c.kv], cache[c.kv:]
  if only is not None: q, mask = q[:, only], mask[only]
  m = mask.shape[-1]
  if m < k.shape[-2]: k, v = k[:, :m], v[:, :m]
  k, v = np.repeat(k, rep, 0), np.repeat(v, rep, 0)
  s = q @ k.swapaxes(-1, -2) + mask
  e = np.exp(s - s.max(-1, keepdims=True))
  o = (e / e.sum(-1, keepdims=True)) @ v
  return merge(o) @ p["o_proj"]


def mlp(h, p):
  m = p["down_proj"].shape[-2]
  gu = h @ p["gate_up_proj"]
  g, u = gu[:, :m], gu[:, m:]
  return (g / (1 + np.exp(-g)) * u) @ p["down_proj"]


def layer(x, p, c, rot, mask, cache, rows, only=None):
  """Attention then the SwiGLU MLP, each after an RMSNorm and added to the residual (llama.py:106-130). only: just
  those rows of the result (see attention)."""
  a = attention(rms(x, p["input_layernorm"], c.eps), p, c, rot, mask, cache, rows, only)
  x = (x if only is None else x[only]) + a
  return x + mlp(rms(x, p["post_attention_layernorm"], c.eps), p)


def block(w, l):
  pre = f"layers.{l}."
  return {k[len(pre):]: v for k, v in w.items() if k.startswith(pre)}


def forward(ids, places, w, c, caches, every=False):
  """Logits after ids at places, updating caches (llama.py:325-354, no slots). Returns (1, vocab) for the last row,
  or (n, vocab) with every."""
  places = np.asarray(list(places))
  size = caches[0].shape[-2]
  x = w["embed"][list(ids)].astype(np.float32)
  rot = (w["cos"][places], w["sin"][places], w["turn"])
  k = np.arange(size)
  mask = np.where(k > places[:, None], np.float32(-1e9), np.float32(0))
  for l in range(c.layers):
    x = layer(x, block(w, l), c, rot, mask, caches[l], places)
  h = rms(x, w["norm"], c.eps)
  return (h if every else h[-1:]) @ w["embed.T"]


def prefill(ids, w, c, caches, tokens):
  """A prompt from position 0 in chunks of `tokens` (llama.py:356-363)."""
  if not len(ids) or tokens < 1: raise ValueError("prefill needs a nonempty prompt and a chunk of at least one token")
  for i in range(0, len(ids), tokens):
    out = forward(ids[i:i + tokens], range(i, min(i + tokens, len(ids))), w, c, caches)
  return out


def greedy(prompt, steps, w, c, size):
  """Autonomous greedy decode: the prompt, then `steps` tokens each fed back. Returns (tokens, per-step logits)."""
  caches = kv_cache(c, size)
  logits = forward(prompt, range(len(prompt)), w, c, caches)[0]
  toks, outs = [], []
  for i in range(steps):
    t = int(logits.argmax())
    toks.append(t)
    outs.append(logits)
    if i + 1 < steps: logits = forward([t], [len(prompt) + i], w, c, caches)[0]
  return toks, outs
