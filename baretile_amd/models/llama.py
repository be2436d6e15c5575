"""Llama-family decoders on baretile_amd tensors: the device side of baretile/models/llama.py.

The functions keep the reference's names and meaning (llama.py:48-373): precision, rms, rope, rotary, fuse, layer,
attention, mlp, forward, prefill, kv_cache, upload. They run on Tensor only. The NumPy twin that the reference keeps
in the same functions is this repository's CPU oracle (oracle/llama_ref.py), which the tests compare against.

The numbers follow the reference's device path (llama.py:88-183):
  - the residual stream is fp32 and each half of a block adds onto it in its last matmul's kernel;
  - RMSNorm reads the stream rounded to bf16, then rounds each step in bf16;
  - RoPE takes bf16 tables that carry 1/sqrt(head width) for q's heads (llama.py:209-227);
  - the MLP is silu(gate) * up with gate and up side by side (llama.py:174-183);
  - attention runs in one kernel from each token's place.
Llama-family only: Qwen's DeltaNet and experts, gpt-oss sinks and sliding windows other than the plain causal one
are outside this backend's scope.
"""
import collections.abc
import json
import math
import operator
import os
from types import SimpleNamespace
import numpy as np
from baretile_amd.tensor import Tensor, jit


def model(**kw):
  """A config: dim, heads, kv, layers, eps, theta, vocab, ffn, and optionally head_dim, precision and rope (RoPE
  scaling parameters, or None)."""
  base = dict(head_dim=None, vocab=None, ffn=None, precision=None, rope=None)
  return SimpleNamespace(**(base | kw))


def smol(layers=30, vocab=49152):
  """SmolLM-135M's shapes (test/test_models.py:639-645): 576 wide, 9 query and 3 KV heads of 64, FFN 1536."""
  return model(dim=576, heads=9, kv=3, layers=layers, eps=1e-5, theta=10000.0, vocab=vocab, ffn=1536)


def head(c): return c.head_dim or c.dim // c.heads


def precision(c, mode="bf16", kv=None):
  """{(op, block): (format, phases)}, as llama.py:48-83 gives for the Llama family. bf16 and bfp8 put every matrix
  and the output layer in that format; bfp4 puts gate_up in bfp4 and the rest in bfp8; tt is tt_transformers'
  performance mode. Phases are kept as data: the matrix cores multiply bf16 exactly at any count."""
  if mode not in ("bf16", "bfp8", "bfp4", "tt"): raise ValueError(f"unknown precision mode: {mode}")
  if kv is not None and kv not in ("bf16", "bfp8", "bfp4"): raise ValueError(f"unknown KV cache format: {kv}")
  def entry(op):
    if mode in ("bf16", "bfp8"): return mode, 4
    fmt = "bfp4" if op == "gate_up" else "bfp8"
    return fmt, (1 if fmt == "bfp4" else 2) if mode == "tt" else 4
  table = {(op, l): entry(op) for l in range(c.layers) for op in ("qkv", "o", "gate_up", "down")}
  if mode == "tt" and (c.layers, c.dim) == (32, 4096): table["gate_up", 31] = ("bfp8", 2)
  table["head", None] = entry("head")
  table["attention", "decode"] = (None, 2 if mode == "tt" else 4)
  table["attention", "prefill"] = (None, 4)
  table["kv", None] = (kv or ("bfp8" if mode == "tt" else "bf16"), None)
  return table


def weight_format(name, prec):
  """A weight's storage format (llama.py:464-474): the block matrices and the output layer from prec, else bf16."""
  if not prec: return "bf16"
  if name == "embed.T": key = ("head", None)
  elif name.startswith("layers.") and name.endswith("_proj"):
    key = (name.split(".")[-1][:-len("_proj")], int(name.split(".")[1]))
  else: return "bf16"
  return prec.get(key, ("bf16", 4))[0]


def _bf16(a):  # float32 rounded to bf16 (nearest even) and back
  b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
  return (((b + 0x7FFF + (b >> 16 & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def frequencies(c):
  """RoPE's inverse frequencies in fp32, as Hugging Face computes them (llama.py:187-200). With Llama 3's scaling
  (c.rope["rope_type"] == "llama3"), frequencies whose wavelength passes original / low_freq_factor are divided by the
  factor, those under original / high_freq_factor are kept, and the ones between blend the two, linearly in
  original / wavelength."""
  hd = head(c)
  base = (1 / c.theta ** (np.arange(0, hd, 2, dtype=np.float32) / hd)).astype(np.float32)
  r = getattr(c, "rope", None) or {}
  if r.get("rope_type") != "llama3": return base
  span = r["original_max_position_embeddings"]
  lo, hi, factor = r["low_freq_factor"], r["high_freq_factor"], r["factor"]
  wave = np.float32(2 * math.pi) / base
  slowed = base / np.float32(factor)
  mix = (np.float32(span) / wave - np.float32(lo)) / np.float32(hi - lo)
  blended = (1 - mix) * slowed + mix * base
  return np.select([wave > span / lo, wave < span / hi], [slowed, base], blended).astype(np.float32)


def rotary(c, n):
  """(cos, sin, turn) for positions 0 .. n-1 (llama.py:209-227). The tables are bf16 and repeat a head's row across
  the heads of q, k and v: q's carry 1/sqrt(head width), v's have cos 1 and sin 0. x @ turn is (-x2, x1)."""
  hd = head(c)
  angles = np.arange(n, dtype=np.float32)[:, None] * frequencies(c)[None]
  def table(g, still):
    t = np.concatenate([g(angles), g(angles)], 1).astype(np.float32)
    heads = [t * np.float32(hd ** -0.5)] * c.heads + [t] * c.kv + [np.full_like(t, still)] * c.kv
    return _bf16(np.concatenate(heads, 1))
  turn = np.zeros((hd, hd), np.float32)
  half = np.arange(hd // 2)
  turn[half + hd // 2, half], turn[half, half + hd // 2] = -1, 1
  return table(np.cos, 1.0), table(np.sin, 0.0), turn


class Weight:
  """One matrix of a checkpoint, read only when asked for, so the host never holds a whole model (llama.py:229-233).
  Made from a function of no arguments that returns the matrix's bf16 bits laid out for x @ w; bits() calls it and
  values() gives the same as float32."""
  __slots__ = ("read",)

  def __init__(self, read): self.read = read
  def bits(self): return self.read()
  def values(self): return (np.asarray(self.bits(), np.uint32) << 16).view(np.float32)


def fuse(w, c):
  """q, k, v side by side as qkv_proj, and gate, up as gate_up_proj, in each block (llama.py:238-291). Takes NumPy
  arrays or Weights (joined when read)."""
  def join(xs):
    if isinstance(xs[0], Weight): return Weight(lambda: np.ascontiguousarray(np.concatenate([x.bits() for x in xs], 1)))
    return np.concatenate(xs, 1)
  w = dict(w)
  for l in range(c.layers):
    p = f"layers.{l}."
    if p + "q_proj" in w:
      w[p + "qkv_proj"] = join([w.pop(p + n) for n in ("q_proj", "k_proj", "v_proj")])
    if p + "gate_proj" in w:
      w[p + "gate_up_proj"] = join([w.pop(p + n) for n in ("gate_proj", "up_proj")])
  return w


TYPES = ("llama",)


class Shards:
  """The tensors of a safetensors checkpoint in one file or several: each file starts with an 8-byte little-endian
  header length and a JSON header giving every tensor's dtype, shape and byte range after the header. Nothing but the
  headers is read until a tensor is asked for, and then only its own bytes."""
  def __init__(self, paths):
    self.entries = {}
    for path in paths:
      with open(path, "rb") as f:
        size = int.from_bytes(f.read(8), "little")
        header = json.loads(f.read(size))
      for name, entry in header.items():
        if name != "__metadata__": self.entries[name] = (path, 8 + size, entry)

  def bf16(self, name, transposed=False):
    """Tensor `name` as bf16 bits: BF16 as stored, F32 rounded to nearest even. A vector comes back as one row, and a
    matrix transposed when asked (a linear layer's weight, stored (out, in), used as x @ w)."""
    path, start, e = self.entries[name]
    kind = {"BF16": np.uint16, "F32": np.float32}.get(e["dtype"])
    if kind is None: raise ValueError(f"{name} is {e['dtype']}: checkpoint tensors are read from BF16 or F32")
    lo, hi = e["data_offsets"]
    a = np.fromfile(path, kind, (hi - lo) // np.dtype(kind).itemsize, offset=start + lo)
    if kind is np.float32: a = (_bf16(a).view(np.uint32) >> 16).astype(np.uint16)
    a = a.reshape(e["shape"] if len(e["shape"]) > 1 else (1, -1))
    return np.ascontiguousarray(a.T) if transposed else a


def config(folder, places=4096):
  """A config from a Hugging Face config.json (llama.py:400-427), Llama family. places, capped at the model's maximum,
  sizes the RoPE tables. RoPE scaling may be Llama 3's (rope_type "llama3", kept in c.rope); ValueError for another
  model type or another scaling."""
  with open(os.path.join(folder, "config.json")) as f: j = json.load(f)
  j = j.get("text_config", j)
  if j.get("model_type") not in TYPES:
    raise ValueError(f"{folder}: model type {j.get('model_type')!r} isn't supported; this backend runs {', '.join(TYPES)}")
  rope = dict(j.get("rope_parameters") or j.get("rope_scaling") or {})  # transformers 5 names it rope_parameters
  theta = float(rope.pop("rope_theta", j.get("rope_theta", 10000.0)))
  kind = rope.pop("rope_type", None) or rope.get("type") or "default"  # older configs name it type
  rope.pop("type", None)
  if kind not in ("default", "llama3"): raise ValueError(f"RoPE scaling {kind!r} ({rope}) isn't supported")
  return model(dim=j["hidden_size"], heads=j["num_attention_heads"], kv=j.get("num_key_value_heads", j["num_attention_heads"]),
               layers=j["num_hidden_layers"], eps=j["rms_norm_eps"], theta=theta, vocab=j["vocab_size"],
               ffn=j.get("intermediate_size"), head_dim=j.get("head_dim"),
               places=min(j.get("max_position_embeddings", places), places), tied=j.get("tie_word_embeddings", False),
               rope={"rope_type": kind, **rope} if kind == "llama3" else None)


def load(folder, places=4096):
  """(config, {name: Weight}) from model.safetensors or the shards model.safetensors.index.json lists
  (llama.py:429-462). Names drop "model.", "self_attn." and "mlp."; linear layers are transposed for x @ w and vectors
  become one-row matrices; the output layer is lm_head, or the embedding's transpose when tied; fuse joins q/k/v and
  gate/up. Nothing is read until a Weight's bits() are."""
  c = config(folder, places)
  index = os.path.join(folder, "model.safetensors.index.json")
  if os.path.exists(index):
    with open(index) as f: files = sorted(set(json.load(f)["weight_map"].values()))
  else:
    files = ["model.safetensors"]
  shards = Shards([os.path.join(folder, f) for f in files])
  out = {}
  for full, (_, _, e) in shards.entries.items():
    name = full.removeprefix("model.").removesuffix(".weight").replace("self_attn.", "").replace("mlp.", "")
    if name.startswith("layers.") and int(name.split(".")[1]) >= c.layers: continue
    linear = (name.endswith("_proj") or name == "lm_head") and len(e["shape"]) == 2
    out[name] = Weight(lambda full=full, linear=linear: shards.bf16(full, linear))
  out["embed"] = out.pop("embed_tokens")
  tied = Weight(lambda e=out["embed"]: np.ascontiguousarray(e.bits().T))
  out["embed.T"] = out.pop("lm_head", None) or tied
  return c, fuse(out, c)


def upload(rt, w, c, places=None):
  """Weights (NumPy float arrays, or Weights from load: their bf16 bits go up as they are) laid out for x @ w with
  q/k/v and gate/up fused, to the device (llama.py:479-495), one at a time. Matrices go to their precision's format
  and into the matmul's tiles once; norms and the embedding stay bf16; the tied output layer is embed.T in the head's
  format. Adds the RoPE tables for `places` positions: cos and sin are the two halves of the rows of one table,
  cos_sin."""
  prec = c.precision
  out = {}
  for name, a in w.items():
    if name in ("cos", "sin", "turn"): continue
    if isinstance(a, Weight):
      bits = a.bits()
      t = Tensor.frombytes(rt, *bits.shape[-2:], np.ascontiguousarray(bits).tobytes())
    else:
      a = np.asarray(a, np.float32)
      if a.ndim == 1: a = a[None]
      t = Tensor.of(rt, a)
    if name.endswith("_proj") or name == "embed.T":
      fmt = weight_format(name, prec)
      t = (t.cast(fmt) if fmt != "bf16" else t).columns()
    out[name] = t
  if "embed.T" not in out: out["embed.T"] = Tensor.of(rt, np.ascontiguousarray(np.asarray(w["embed"], np.float32).T)).cast(
    weight_format("embed.T", prec) if weight_format("embed.T", prec) != "bf16" else "bf16").columns()
  if places:
    cos, sin, turn = rotary(c, places)
    both = Tensor.of(rt, np.concatenate([cos, sin], 1))  # a place's cos row, then its sin row: one gather for both
    out["cos_sin"], out["cos"], out["sin"] = both, both[:, :cos.shape[1]], both[:, cos.shape[1]:]
    out["turn"] = Tensor.of(rt, turn).columns()
  return out


def kv_cache(rt, c, size):
  """A (2 * kv, size, head) cache of zeros per block: key heads, then value heads (llama.py:365-373), in the format
  c.precision gives the KV cache (bf16, or a block float: bfp8, bfp4)."""
  fmt = (c.precision or {}).get(("kv", None), ("bf16", None))[0] or "bf16"
  return [Tensor.zeros(rt, size, head(c), batch=2 * c.kv).cast(fmt).realize() for _ in range(c.layers)]


_aranges = {}


def _arange(rt, n):  # an int32 row 0 .. n-1, made once per runtime (a recording finds it made)
  key = (id(rt), n)
  if key not in _aranges or _aranges[key].rt is not rt: _aranges[key] = Tensor.of(rt, [list(range(n))], "int32")
  return _aranges[key]


def rope_into(qkv, cos, sin, cache, rows, c):
  """RoPE of each token's heads with the key and value heads put into the cache at rows (llama.py:132-160): one
  kernel for a bf16 cache (rope_put); a block-float cache takes the rows from a bf16 stage through put, which rounds
  each run of 16 as a cast does (kernels.py:1083-1168). Returns the query heads, (tokens, heads * head)."""
  if cache.dtype == "bf16": return qkv.rope_put(cos, sin, cache, rows, c.heads, c.kv)
  n = qkv.rows
  stage = Tensor(qkv.rt, n, head(c), batch=2 * c.kv)
  q = qkv.rope_put(cos, sin, stage, _arange(qkv.rt, n), c.heads, c.kv)
  cache.put(rows, stage)
  return q


def rms(x, w, c):
  """RMSNorm of the stream rounded to bf16, scaled by w (llama.py:88-95): for fp32 rows of one matrix, one kernel
  (Tensor.rms_rows, in fp32, rounded once); otherwise the lazy graph, which rounds each step in bf16."""
  if x.dtype == "fp32" and x.batch == 1 and w.dtype == "bf16" and len(x.shape) <= 3:
    return x.rms_rows(w, c.eps)
  x = x.bfloat16()
  return x * ((x * x).mean(2) + c.eps).rsqrt() * w


def rope(x, cos, sin, turn):
  """x cos + (x @ turn) sin (llama.py:103-104); the matmul runs the rest as its epilogue."""
  return x * cos + (x @ turn) * sin


def attention(h, p, c, rot, places, cache, rows, firsts=None):
  """One block's attention over its cache (llama.py:132-172): qkv, then RoPE with the new keys and values put into
  the cache at rows in one kernel (x cos + (x @ turn) sin, worked out in fp32 from the turn's pairs), then one
  attention kernel from each token's place (and, with slots, from its slot's first row)."""
  rep = c.heads // c.kv
  qkv = h.matmul(p["qkv_proj"])
  n = qkv.rows
  q = rope_into(qkv.reshape(n, qkv.cols), rot[0].reshape(n, rot[0].cols), rot[1].reshape(n, rot[1].cols), cache,
                rows, c).split(c.heads)
  k, v = cache[:c.kv, :, :], cache[c.kv:, :, :]
  o = q.attend(k.repeat_interleave(rep), v.repeat_interleave(rep), places, firsts=firsts, merged=True)
  return o.matmul(p["o_proj"], "fp32")


def mlp(h, p):
  """SwiGLU: silu(h @ gate) * (h @ up), then down, with gate and up side by side (llama.py:174-183)."""
  m = p["down_proj"].rows
  if h.batch == 1 and m % 16 == 0 and h.cols % 32 == 0:  # SiLU-mul as the product's epilogue
    return h.matmul_swiglu(p["gate_up_proj"]).matmul(p["down_proj"], "fp32")
  gate_up = h.matmul(p["gate_up_proj"])
  return (gate_up[:, :m].silu() * gate_up[:, m:]).matmul(p["down_proj"], "fp32")


def block(w, l):
  pre = f"layers.{l}."
  return {k[len(pre):]: v for k, v in w.items() if k.startswith(pre)}


def blocks(w, layers):
  """block(w, l) for every l < layers, from one pass over the weights (not one a layer)."""
  out = [{} for _ in range(layers)]
  for k, v in w.items():
    if k.startswith("layers."):
      l, _, name = k[7:].partition(".")
      if l.isdigit() and int(l) < layers: out[int(l)][name] = v
  return out


def layer(x, p, c, rot, places, cache, rows, firsts=None):
  """Attention, then the MLP, each after an RMSNorm and added onto the fp32 stream in its own kernel (llama.py:106-130)."""
  x = (x + attention(rms(x, p["input_layernorm"], c), p, c, rot, places, cache, rows, firsts)).realize()
  return (x + mlp(rms(x, p["post_attention_layernorm"], c), p)).realize()


def row_fits(w, c):
  """Whether one-token steps can take the fused row kernels (row_layer): the widths bt_matmul_row takes, heads
  attend() takes, bf16 norms, matrices by columns."""
  hd, ffn = head(c), c.ffn or 4 * c.dim
  widths = (c.dim, c.heads * hd, ffn)
  return (all(k <= 4096 and k % 8 == 0 for k in widths) and hd in (64, 128) and w["norm"].dtype == "bf16" and
          all(w[f"layers.{l}.{n}"].layout == "columns" for l in range(c.layers)
              for n in ("qkv_proj", "o_proj", "gate_up_proj", "down_proj")) and w["embed.T"].layout == "columns")


def row_layer(x, p, c, rot, places, cache, rows):
  """One block for a single token, as layer() computes it, in five kernels: the norm inside the qkv and gate_up
  products, RoPE with the cache put inside the qkv product, attention, the residual adds inside the o and down
  products, and silu(gate) * up inside the down product (bt_matmul_row, bt_matmul_row_rope). Each fused step rounds
  once, in fp32, where the lazy graph rounds each operation to bf16."""
  rep = c.heads // c.kv
  if cache.dtype == "bf16":
    q = x.matmul_row(p["qkv_proj"], norm=p["input_layernorm"], eps=c.eps,
                     rope=(rot[0], rot[1], cache, rows, c.heads, c.kv)).split(c.heads)
  else:  # a block-float cache: the rows go in through put
    qkv = x.matmul_row(p["qkv_proj"], "bf16", norm=p["input_layernorm"], eps=c.eps)
    q = rope_into(qkv, rot[0].reshape(1, rot[0].cols), rot[1].reshape(1, rot[1].cols), cache, rows, c).split(c.heads)
  o = q.attend(cache[:c.kv, :, :].repeat_interleave(rep), cache[c.kv:, :, :].repeat_interleave(rep), places)
  x = o.matmul_row(p["o_proj"], "fp32", residual=x)
  gate_up = x.matmul_row(p["gate_up_proj"], "bf16", norm=p["post_attention_layernorm"], eps=c.eps)
  return gate_up.matmul_row(p["down_proj"], "fp32", swiglu=True, residual=x)


def slots_layer(x, p, c, rot, keys, values, place, h=None, then=None):
  """One block for a batch of slots, each with its own cache and one new token, all at one place: the batched decode
  of llama.forward(slots=...) (llama.py:293-354). x is (1, S, dim), the stream of the S slots; keys and values are
  (S * kv, size, head) bf16, slot s's key heads at s * kv .. s * kv + kv - 1; rot holds the tables at the place for
  each slot's row; place is a (1, 1) int32 row. The slots' query heads become S * heads attention heads of one row.
  RoPE and the cache puts run as one kernel (bt_rope_put), in fp32 with one rounding. The qkv product feeds that kernel
  its split-K partial sums, and the o product feeds the residual add and the MLP's norm likewise (matmul_rope_put,
  matmul_residual_rms), with the same results as the separate steps.

  h: x's input norm when it is already made (by the block before, with `then`). then: the norm weights that the next
  step applies to the new x (the next block's input norm, or the model's final norm); with them the down product
  feeds the residual add and that norm as the o product does, and (x, the next step's h) comes back."""
  S, hd, rep = x.rows, head(c), c.heads // c.kv
  if keys.dtype != "bf16": raise ValueError("slots_layer takes bf16 caches")
  if h is None: h = rms(x, p["input_layernorm"], c)
  q = h.matmul_rope_put(p["qkv_proj"], rot[0], rot[1], keys, place, c.heads, c.kv, values=values)
  o = q.reshape(S * c.heads, 1, hd).attend(keys.repeat_interleave(rep), values.repeat_interleave(rep),
                                           place.reshape(1, 1, 1)).reshape(1, S, c.heads * hd)
  norm = p["post_attention_layernorm"]
  fused = x.dtype == "fp32" and x.batch == 1
  if fused and norm.dtype == "bf16":
    x, h = o.matmul_residual_rms(p["o_proj"], x, norm, c.eps)
  else:
    x = (x + o.matmul(p["o_proj"], "fp32")).realize()
    h = rms(x, norm, c)
  if then is None: return (x + mlp(h, p)).realize()
  m = p["down_proj"].rows
  if fused and then.dtype == "bf16" and h.batch == 1 and m % 16 == 0 and h.cols % 32 == 0:
    return h.matmul_swiglu(p["gate_up_proj"]).matmul_residual_rms(p["down_proj"], x, then, c.eps)
  x = (x + mlp(h, p)).realize()
  return x, rms(x, then, c)


def starts(w, n, slots, part):
  """The first cache row of each token's slot, for n tokens of `slots` sequences in turn, as an int32 row
  (llama.py:320-323's firsts). Kept with the weights, so a recorded step finds it made."""
  made = w.setdefault("starts", {})
  if (n, slots, part) not in made:
    made[n, slots, part] = Tensor.of(w["norm"].rt, [[i // (n // slots) * part for i in range(n)]], "int32")
  return made[n, slots, part]


def forward(ids, places, w, c, caches, every=False, slots=None):
  """Logits after ids (an int32 row) at places (an int32 row), updating each block's cache (llama.py:325-354):
  the last token's, or every token's with every, in fp32.

  slots: decode that many sequences together, each with an equal run of consecutive tokens and a region of its own
  of size / slots rows in every cache (llama.py:293-318); places count from each region's start, and the logits of
  every token come back. A free slot's token sits at its region's last row, which is kept for it, and sees only the
  region's first row."""
  n = ids.cols
  x = w["embed"].gather(ids).float()
  row = n == 1 and not slots and w.setdefault("row_fits", row_fits(w, c))  # one token: the fused row kernels
  if row and "cos_sin" in w:  # both tables' rows in one launch
    both = w["cos_sin"].gather(places).reshape(2, w["cos"].cols)
    rot = (both[0:1, :], both[1:2, :], w["turn"])
  else:
    rot = (w["cos"].gather(places), w["sin"].gather(places), w["turn"])
  firsts = None
  if not slots:
    rows, column = places, places.reshape(1, n, 1)
  else:
    size = caches[0].rows
    if n % slots or size % slots: raise ValueError(f"{n} tokens and {size} cache rows don't split into {slots} slots")
    part = size // slots
    first = starts(w, n, slots, part)
    rows = (places + first).realize()  # each token's cache row
    column = (first + places * (places < part - 1)).realize().reshape(1, n, 1)  # a free slot's token: its first row
    firsts = first.reshape(1, n, 1)
  ps = blocks(w, c.layers)
  if row:
    x = x.reshape(1, c.dim)
    for l in range(c.layers): x = row_layer(x, ps[l], c, rot, column, caches[l], rows)
    return x.matmul_row(w["embed.T"], "fp32", norm=w["norm"], eps=c.eps).reshape(1, 1, w["embed.T"].cols)
  for l in range(c.layers): x = layer(x, ps[l], c, rot, column, caches[l], rows, firsts)
  h = rms(x, w["norm"], c)
  if not (every or slots) and n > 1: h = h[:, n - 1:n, :]  # the last token's row
  return h.matmul(w["embed.T"], "fp32")


def prefill(ids, w, c, caches, tokens):
  """A prompt from position 0 in chunks of `tokens` (llama.py:356-363); the logits after its last token."""
  if not len(ids) or tokens < 1: raise ValueError("prefill needs a nonempty prompt and a chunk of at least one token")
  rt = w["norm"].rt
  for i in range(0, len(ids), tokens):
    out = forward(Tensor.of(rt, [list(ids[i:i + tokens])], "int32"),
                  Tensor.of(rt, [list(range(i, min(i + tokens, len(ids))))], "int32"), w, c, caches)
  return out


def argmax(logits):
  """The index of the largest of one row of fp32 logits, read back once."""
  return int(np.argmax(np.frombuffer(logits.tobytes(), np.float32)))


def generate(w, c, prompt, steps, size, feed=None, clock=None, replay=True):
  """Greedy decode: prefill the prompt, then `steps` tokens. Each step after the first replays the recorded forward
  (jit); on its own (no feed, replay), a step also picks its token on the device and feeds it, with the next place,
  to the next step (greedy_steps), so the steps follow each other with no trip to the host; the picks come back once
  at the end, and those steps' logits stay on the device until one of them is asked for (Logits). With feed, step i
  is fed feed[i] instead of its own pick (the reference's NumPy-fed protocol, gpt2.py:147-161), and each step's
  logits come back to the host before the next. With clock (a list), the time.perf_counter() at which each pick is
  known on the host is appended to it (on the device path, every pick after the prompt's at the end). replay=False
  runs every step eagerly, one launch per kernel, as the first call of a jit does. Returns (picks, per-step logits as
  float32 arrays, in a list or a Logits sequence)."""
  import time
  rt = w["norm"].rt
  caches = kv_cache(rt, c, size)
  logits = prefill(prompt, w, c, caches, len(prompt))
  row = np.frombuffer(logits.tobytes(), np.float32).copy()
  picks, outs = [int(np.argmax(row))], [row]
  if clock is not None: clock.append(time.perf_counter())
  if steps > 1 and feed is None and replay:
    more, rows = greedy_steps(w, c, caches, picks[0], len(prompt), steps - 1)
    if clock is not None: clock.extend([time.perf_counter()] * (steps - 1))
    return picks + more, Logits(outs, rows)
  step = (jit if replay else lambda f: f)(lambda i, p: forward(i, p, w, c, caches))
  for s in range(steps - 1):
    tok = picks[-1] if feed is None else feed[s]
    logits = step(Tensor.of(rt, [[tok]], "int32"), Tensor.of(rt, [[len(prompt) + s]], "int32"))
    row = np.frombuffer(logits.tobytes(), np.float32).copy()
    outs.append(row)
    picks.append(int(np.argmax(row)))
    if clock is not None: clock.append(time.perf_counter())
  return picks, outs


def argmax_parts(vocab):
  """The equal parts an on-device argmax splits a row of logits into: a block each, then one over their winners."""
  return max(p for p in range(1, 257) if vocab % p == 0)


def greedy_steps(w, c, caches, pick, place, n, stats=None):
  """n greedy one-token steps after `pick` at `place`, chained on the device: each step's forward, the argmax of its
  logits (topk over up to 256 equal parts of the row, then over the parts' winners, which keeps the first of equal
  values, as numpy's argmax does) written as the next step's token, the logits into rows kept by place, and the next place, all
  as launches; the picks are made again from the kept rows at the end, in one pass, by the same kernels. On the
  fused row kernels (row_fits), which keep nothing made on first use, the step is recorded into a graph at once and
  every step is a replay of it; otherwise, or should the capture refuse something the step makes the first time (an
  upload), the first step runs eagerly, as jit's first call does, and the recording follows it. Nothing comes back
  to the host until the last step is done.
  Returns (the n picks, their logits: an (n, vocab) fp32 view of a device tensor); stats (a dict), if given, gets
  the recorded step's kernel count as "kernels"."""
  from baretile_amd.tensor import Recording
  rt, vocab = w["norm"].rt, w["embed.T"].cols
  end = place + n
  if n < 1 or place < 0: raise ValueError(f"greedy_steps takes at least one step from a place of 0 or more: {n}, {place}")
  if end > caches[0].rows: raise ValueError(f"{n} steps from place {place} run past the cache's {caches[0].rows} rows")
  ids, at = Tensor.of(rt, [[pick]], "int32"), Tensor.of(rt, [[place]], "int32")
  best, rows = Tensor(rt, 1, 1, dtype="fp32"), Tensor(rt, end, vocab, dtype="fp32")
  parts = argmax_parts(vocab)

  def argmax(x, out=None):  # the first largest of each row, as x.rows x 1 (values, ids)
    if parts == 1: return x.topk(1, out=out)
    top, i = x.topk(1, parts=parts)
    return top.topk(1, labels=i, out=out)

  def step():  # the pick goes straight into the next step's token
    logits = forward(ids, at, w, c, caches).reshape(1, vocab)
    argmax(logits, out=(best, ids))
    rows.put(at, logits)
    at.assign(at + 1)

  ran = 0
  if not w.setdefault("row_fits", row_fits(w, c)):  # other kernels keep a block-float B's tiles from a first call
    step()
    ran = 1
  rec = Recording(rt)
  try:
    with rec: step()
  except RuntimeError:  # the step makes something the first time that a capture can't (an upload): run it first
    if ran: raise
    step()
    rec, ran = Recording(rt), 1
    with rec: step()
  for _ in range(n - ran): rec.send()
  if stats is not None: stats["kernels"] = rec.kernels
  kept = rows[place:end, :]
  got = np.frombuffer(argmax(kept)[1].tobytes(), np.int32)  # the same picks, made again from the kept logits at once
  return [int(t) for t in got], kept


class Logits(collections.abc.Sequence):
  """Per-step logits as float32 arrays: those made on the host, then the rows of an fp32 device tensor (greedy_steps'
  logits, kept on the device), read back whole the first time one is asked for (so the runtime must still be open)."""
  def __init__(self, host, rows):
    self.host, self.rows, self.read = list(host), rows, None

  def __len__(self): return len(self.host) + self.rows.rows

  def __getitem__(self, i):
    if isinstance(i, slice): return [self[j] for j in range(*i.indices(len(self)))]
    i = operator.index(i)
    if i < 0: i += len(self)
    if not 0 <= i < len(self): raise IndexError(f"step {i} of {len(self)}")
    if i < len(self.host): return self.host[i]
    if self.read is None:
      t = self.rows
      self.read = np.frombuffer(t.rt.download(t.addr, 4 * t.rows * t.cols), np.float32).reshape(t.rows, t.cols)
    return self.read[i - len(self.host)]
