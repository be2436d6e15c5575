"""Pins the CPU oracle (oracle/) before anything is checked against it. CPU only.

Each check is chosen so a plausible mistake in the restatement (a dropped term, a wrong shift, sign or index, a
transposed operand) fails it: known answers from the reference's own tests, closed forms computed another way
(exact rationals, float arithmetic instead of bit manipulation), and independent libraries (torch, transformers).
"""
from fractions import Fraction
import os

import numpy as np
import pytest
import torch

from oracle import bfp as B
from oracle import ops, llama_ref as L


# ---- bf16 -------------------------------------------------------------------------------------------------------

def test_bf16_rounding_matches_torch():
  rng = np.random.default_rng(0)
  a = (rng.normal(0, 1, 100000) * np.exp(rng.normal(0, 8, 100000))).astype(np.float32)
  a[:8] = [0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 3.0e38, 1e-40, -1e-40]  # ties, huge, denormal
  want = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
  assert np.array_equal(B.bf16_bits(a), want)
  assert np.array_equal(B.round_bf16_bits(a), want)
  nan = np.array([np.float32("nan")]).view(np.uint32) | 0x12345
  assert B.round_bf16_bits(nan.view(np.float32))[0] == (nan[0] >> 16 | 0x40)


# ---- block floats: known answers ------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", B.FORMATS)
def test_bfp_known_answers(fmt):
  # test_kernels.py:2096-2103: [2, 3] in a run of zeros decodes to bf16 0x4000, 0x4040 in both formats
  row = np.zeros((1, 16), np.float32)
  row[0, :2] = [2, 3]
  top, q = B.bfp_fields(row, fmt)
  assert list(B.decode_fields(top, q, fmt)[0, :2]) == [0x4000, 0x4040]
  assert list(B.bfp(row, fmt)[0, :2]) == [2.0, 3.0]


def test_bfp8_small_integers_exact():
  # ramps/1_tensors.py:71-80: (r * c) % 3 and (r + c) % 2 fit exactly in bfp8
  bm = np.array([[float(r * c % 3) for c in range(32)] for r in range(64)])
  am = np.array([[float((r + c) % 2) for c in range(64)] for r in range(32)])
  assert np.array_equal(B.bfp(bm, "bfp8"), bm) and np.array_equal(B.bfp(am, "bfp8"), am)
  assert np.array_equal(ops.matmul(am, B.bfp(bm, "bfp8")), ops.matmul(am, bm))


def _brute(values, fmt):
  """A run's block-float values by exact rationals: each bf16 value goes to the nearest multiple of the run's step,
  ties away from zero, saturated at 127 (bfp8) or 7 (bfp4) steps. The step is 2^(top - 133) or 2^(top - 129), where
  top is the largest bf16 exponent field. Denormals are excluded (e = 0 drops the hidden bit, as restated)."""
  bits = B.bf16_bits(values).astype(np.int64)
  top = int((bits >> 7 & 255).max())
  step = Fraction(2) ** (top - (133 if fmt == "bfp8" else 129))
  cap = 127 if fmt == "bfp8" else 7
  out = []
  for v in B.bf16_floats(bits):
    x = abs(Fraction(float(v)))
    n = x / step
    q = int(n) + (1 if n - int(n) >= Fraction(1, 2) else 0)
    out.append(float(min(q, cap) * step) * (-1.0 if v < 0 or (v == 0 and np.signbit(v)) else 1.0))
  return np.array(out)


@pytest.mark.parametrize("fmt", B.FORMATS)
def test_bfp_against_exact_rationals(fmt):
  rng = np.random.default_rng(1)
  for trial in range(400):
    spread = [0, 1, 3, 9][trial % 4]  # exponent gaps up to and past the shift clamp of 8
    run = rng.normal(0, 1, 16) * 2.0 ** rng.integers(-spread, spread + 1, 16)
    if trial % 7 == 0: run[rng.integers(0, 16)] = 0.0
    if trial % 11 == 0: run[:] = np.round(run * 8) / 8  # exact ties
    run = run.astype(np.float32)
    got = B.bfp(run[None], fmt)[0]
    assert np.array_equal(got, _brute(run, fmt)), (trial, run, got)
  # saturation: 255/128 * 2^k with the run's top at the same exponent is one step past 127 (bfp8) / 7 (bfp4)
  run = np.full(16, 1.9921875, np.float32)
  assert B.bfp(run[None], "bfp8")[0, 0] == 127 * 2.0 ** -6 and B.bfp(run[None], "bfp4")[0, 0] == 7 * 2.0 ** -2


@pytest.mark.parametrize("fmt", B.FORMATS)
def test_fields_decode_to_values(fmt):
  rng = np.random.default_rng(5)  # test_models.py:587-593's input: N(0,1) * e^N(0,2)
  a = B.bf16(rng.normal(0, 1, (64, 96)) * np.exp(rng.normal(0, 2, (64, 96))))
  top, q = B.bfp_fields(a, fmt)
  got = B.bf16_floats(B.decode_fields(top, q, fmt))
  want = B.bfp(a, fmt)
  assert np.array_equal(got, want)  # -0.0 == 0.0: a zero never carries a sign in the fields
  assert q.min() >= (-127 if fmt == "bfp8" else -7) and q.max() <= (127 if fmt == "bfp8" else 7)


def test_decode_bits_against_float_arithmetic():
  # every bfp8 byte x every exponent: the unpacker's bits are the bf16 of +-mag * 2^(e - 133), whenever that is a
  # normal bf16 (exponent field e - shift in 1..254)
  e, x = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
  bits = B.decode_bits(e, x, "bfp8")
  mag, sign = x & 127, x >> 7
  val = np.where(sign == 1, -1.0, 1.0) * mag * 2.0 ** (e.astype(np.float64) - 133)
  shift = 8 - np.floor(np.log2(np.maximum(mag, 1) * 2)).astype(np.int64) - 1
  normal = (mag > 0) & (e - shift >= 1) & (e - shift <= 254)
  assert np.array_equal(B.bf16_floats(bits)[normal], val[normal].astype(np.float32))
  assert np.all(bits[(mag == 0) & (sign == 0)] == 0) and np.all(bits[(mag == 0) & (sign == 1)] == 0xFF80)
  # bfp4: nibble s<<3|m reads as the byte m<<4 with the sign on top, so mag3 * 2^(e - 129)
  n = np.arange(16)
  b4 = B.decode_bits(np.full(16, 130), n, "bfp4")
  assert np.array_equal(B.bf16_floats(b4)[1:8], (np.arange(1, 8) * 2.0).astype(np.float32))
  assert np.array_equal(B.bf16_floats(b4)[9:16], (-np.arange(1, 8) * 2.0).astype(np.float32))


def test_decode_bits_against_the_reference_unpacker():
  # the whole domain, edge rules included (a zero magnitude with its sign set reads -inf, exponents wrap mod 256),
  # against the reference unpacker's own output (tests/golden/make_unpacker_vectors.py ran tensor.py's `_bf16s`):
  # every bfp8 byte and every bfp4 nibble at every exponent byte
  g = np.load(os.path.join(os.path.dirname(__file__), "golden", "unpacker_bf16s.npz"))
  e, x = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
  assert np.array_equal(B.decode_bits(e, x, "bfp8"), g["bits8"])
  e, n = np.meshgrid(np.arange(256), np.arange(16), indexing="ij")
  assert np.array_equal(B.decode_bits(e, n, "bfp4"), g["bits4"])


# ---- matmul and elementwise -------------------------------------------------------------------------------------

def test_matmul_known_answers():
  x, w = np.array([[1.0, 2.0], [3.0, 4.0]]), np.array([[2.0, 0.0], [0.0, 3.0]])
  assert np.maximum(ops.matmul(x, w), 0).tolist() == [[2.0, 6.0], [6.0, 12.0]]  # README.md:82-83
  assert np.maximum(ops.matmul(x, x), 0).tolist() == [[7.0, 10.0], [15.0, 22.0]]  # ramps/1_tensors.py:27-31
  a = np.array([[float((r * 7 + c * 3) % 3 - 1) for c in range(64)] for r in range(32)])
  b = np.array([[float((r * 5 + c) % 3 - 1) for c in range(32)] for r in range(64)])
  brute = [[sum(a[i][k] * b[k][j] for k in range(64)) for j in range(32)] for i in range(32)]
  assert ops.matmul(a, b).tolist() == brute  # test_kernels.py:637-642
  assert np.array_equal(ops.matmul(a, np.eye(64)), a)


def test_silu_gelu_match_torch():
  x = np.linspace(-9, 9, 1001)
  t = torch.from_numpy(x)
  assert np.allclose(ops.silu(x), torch.nn.functional.silu(t).numpy(), rtol=1e-12, atol=1e-12)
  assert np.allclose(ops.gelu(x), torch.nn.functional.gelu(t, approximate="tanh").numpy(), rtol=1e-12, atol=1e-12)


# ---- attention ----------------------------------------------------------------------------------------------------

def test_attention_matches_torch_sdpa():
  rng = np.random.default_rng(43)
  for e, rows, hd, keys, rep, window in ((4, 8, 64, 96, 2, 0), (2, 40, 128, 200, 1, 50), (8, 1, 128, 512, 4, 0)):
    q, k, v = rng.normal(0, 1, (e, rows, hd)), rng.normal(0, 1, (e // rep, keys, hd)), rng.normal(0, 1, (e // rep, keys, hd))
    places = rng.integers(max(0, keys - rows - 60), keys, (e, rows, 1))
    got = ops.attention(q, k, v, places, window, rep)
    kk, vv = np.repeat(k, rep, 0), np.repeat(v, rep, 0)
    allowed = torch.from_numpy(ops.mask(places, keys, window) == 0)
    want = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(kk), torch.from_numpy(vv),
                                                            attn_mask=allowed, scale=1.0).numpy()
    assert np.allclose(got, want, rtol=1e-10, atol=1e-10)


def test_mask_brute_force():
  places = np.array([[[0], [3], [7]]])
  m = ops.mask(places, 8, window=3)
  for r, p in enumerate([0, 3, 7]):
    for k in range(8): assert (m[0, r, k] == 0) == (p - 3 < k <= p)


def test_attention_extremes():
  # test_kernels.py:1323-1337: scores beyond bf16's precision, keys 32-63 masked -> all ones; 101 > 100 -> all twos
  for query, key in ((100, 100), (100, -100), (10000, 10000), (10000, -10000)):
    q = np.full((1, 3, 64), float(query))
    k = np.full((1, 64, 64), float(key))
    v = np.concatenate([np.ones((1, 32, 64)), np.full((1, 32, 64), 5.0)], 1)
    assert np.array_equal(ops.attention(q, k, v, np.full((1, 3, 1), 31)), np.ones((1, 3, 64)))
  q = np.full((1, 1, 64), 100.0)
  k = np.concatenate([np.full((1, 32, 64), 100.0), np.full((1, 32, 64), 101.0)], 1)
  v = np.concatenate([np.ones((1, 32, 64)), np.full((1, 32, 64), 2.0)], 1)
  assert np.array_equal(ops.attention(q, k, v, np.array([[[63]]])), np.full((1, 1, 64), 2.0))


# ---- the Llama decoder ----------------------------------------------------------------------------------------------

def _hf_logits(c, w, ids):
  from transformers import LlamaConfig, LlamaForCausalLM
  cfg = LlamaConfig(vocab_size=w["embed"].shape[0], hidden_size=c.dim, intermediate_size=c.ffn, num_hidden_layers=c.layers,
                    num_attention_heads=c.heads, num_key_value_heads=c.kv, rms_norm_eps=c.eps, rope_theta=c.theta,
                    max_position_embeddings=64, tie_word_embeddings=True, attention_bias=False, mlp_bias=False)
  m = LlamaForCausalLM(cfg).double().eval()
  sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm"][0], "lm_head.weight": w["embed"]}
  q, kv, f = c.heads * 64, c.kv * 64, c.ffn
  for l in range(c.layers):
    p, h = L.block(w, l), f"model.layers.{l}."
    qkv, gu = p["qkv_proj"], p["gate_up_proj"]
    sd |= {h + "self_attn.q_proj.weight": qkv[:, :q].T, h + "self_attn.k_proj.weight": qkv[:, q:q + kv].T,
           h + "self_attn.v_proj.weight": qkv[:, q + kv:].T, h + "self_attn.o_proj.weight": p["o_proj"].T,
           h + "mlp.gate_proj.weight": gu[:, :f].T, h + "mlp.up_proj.weight": gu[:, f:].T,
           h + "mlp.down_proj.weight": p["down_proj"].T, h + "input_layernorm.weight": p["input_layernorm"][0],
           h + "post_attention_layernorm.weight": p["post_attention_layernorm"][0]}
  m.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(v, np.float64)) for k, v in sd.items()}, strict=False)
  with torch.no_grad(): return m(torch.tensor([ids])).logits[0].numpy()


def test_llama_forward_matches_transformers():
  rng = np.random.default_rng(12)
  c, w = L.smol(rng, 2)
  ids = [7, 200, 31, 64, 5, 9, 100, 3]
  got = L.forward(ids, range(len(ids)), w, c, L.kv_cache(c, 32), every=True)
  want = _hf_logits(c, w, ids)
  # the oracle's RoPE tables are bf16 (llama.py:219), transformers' are exact: a few 1e-3 of the logit scale
  good = np.abs(got - want).max()
  assert good < 1e-3 * np.abs(want).max(), good
  assert (got.argmax(-1) == want.argmax(-1)).all()
  # a mistake in the RoPE turn (its transpose), the GQA grouping or the residual is far outside that agreement
  for mistake in ("turn", "gqa", "residual"):
    w2, c2 = dict(w), L.model(**vars(c))
    if mistake == "turn": w2["turn"] = w["turn"].T
    if mistake == "gqa": c2.kv, c2.heads = 3, 9; w2 = {k: (v[:, :576 + 192 + 192] if k.endswith("qkv_proj") else v) for k, v in w.items()}
    if mistake == "residual": w2 = {k: (v * 2 if k.endswith("o_proj") else v) for k, v in w.items()}
    if mistake == "gqa":  # swap the key heads' order: a wrong query->key grouping
      for l in range(c.layers):
        q = w2[f"layers.{l}.qkv_proj"].copy()
        k = q[:, 576:768].reshape(576, 3, 64)[:, ::-1].reshape(576, 192)
        q[:, 576:768] = k
        w2[f"layers.{l}.qkv_proj"] = q
    bad = L.forward(ids, range(len(ids)), w2, c2, L.kv_cache(c2, 32), every=True)
    assert np.abs(bad - want).max() > 100 * good, mistake


def test_llama_kv_cache_and_chunked_prefill():
  rng = np.random.default_rng(13)
  c, w = L.smol(rng, 2, places=96)
  ids = [int(i) for i in rng.integers(0, 256, 70)]
  caches = L.kv_cache(c, 96)
  full = L.forward(ids, range(70), w, c, L.kv_cache(c, 96))[0]
  chunked = L.prefill(ids, w, c, caches, 32)[0]
  assert np.allclose(full, chunked, atol=1e-3)  # test_models.py:1539
  step = L.forward([5], [70], w, c, caches)[0]
  again = L.forward(ids + [5], range(71), w, c, L.kv_cache(c, 96))[0]
  assert np.allclose(step, again, atol=1e-3)  # test_models.py:851
  with pytest.raises(ValueError, match="prefill"): L.prefill([], w, c, caches, 32)


def test_precision_known_answers():
  big = L.model(layers=32, dim=4096, heads=32, kv=8, eps=1e-5, theta=5e5)
  tt = L.precision(big, "tt")
  assert tt["gate_up", 31] == ("bfp8", 2) and tt["gate_up", 30] == ("bfp4", 1)  # test_models.py:1552-1553
  assert tt["head", None] == ("bfp8", 2) and L.precision(big, "bf16")["qkv", 0] == ("bf16", 4)
  assert [tt[k] for k in (("attention", "decode"), ("attention", "prefill"), ("kv", None))] == [(None, 2), (None, 4), ("bfp8", None)]
  p8 = L.precision(big, "bfp8")
  assert L.weight_format("embed.T", p8) == "bfp8" and L.weight_format("layers.3.down_proj", p8) == "bfp8"
  assert L.weight_format("layers.3.input_layernorm", p8) == "bf16" and L.weight_format("embed", p8) == "bf16"
  with pytest.raises(ValueError): L.precision(big, "fp8")


def test_llama3_frequencies_match_transformers():
  # test_models.py:676-688: Llama 3.1's scaled frequencies against transformers' own llama3 initialisation, within a
  # relative 1e-6, with the known answers: the shortest wavelength kept, the longest slowed by exactly the factor
  from transformers import LlamaConfig
  from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
  rope = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
  hf = LlamaConfig(hidden_size=4096, num_attention_heads=32, rope_theta=500000.0, rope_scaling=rope,
                   max_position_embeddings=131072)
  want = ROPE_INIT_FUNCTIONS["llama3"](hf, "cpu")[0].numpy()
  c = L.model(dim=4096, heads=32, kv=8, layers=1, eps=1e-5, theta=500000.0, rope=rope)
  got = L.frequencies(c)
  assert got.dtype == np.float32 and np.allclose(got, want, rtol=1e-6, atol=0), np.abs(got / want - 1).max()
  plain = L.frequencies(L.model(dim=4096, heads=32, kv=8, layers=1, eps=1e-5, theta=500000.0))
  assert plain[0] == got[0] and plain[-1] == 8 * got[-1]
  # some frequencies fall in the blend, where a wrong interpolation (its ends swapped) would be far off
  blend = (got != plain) & (got != plain / 8)
  assert blend.sum() >= 3
  swapped = L.model(**vars(c))
  swapped.rope = dict(rope, low_freq_factor=4.0, high_freq_factor=1.0)
  assert not np.allclose(L.frequencies(swapped)[blend], want[blend], rtol=1e-3)


def test_block_float_kv_cache_rounds_its_rows():
  # llama.py:151-154: with a bfp8 or bfp4 cache, the rows NumPy puts are gpt2.bfp of the rows a bf16 cache would get.
  # Checked on one step from the same starting cache: every cached row is bfp() of the bf16 run's row (so a fixed point
  # of bfp), rows not written stay as they were, and the logits move by no more than the rounding explains.
  rng = np.random.default_rng(21)
  c, w = L.smol(rng, 1, vocab=64, places=16)
  ids, places = [3, 17, 40, 9], range(4)
  plain = L.kv_cache(c, 16)
  want_logits = L.forward(ids, places, w, c, plain, every=True)
  for fmt in B.FORMATS:
    cb = L.model(**vars(c))
    cb.precision = L.precision(c, "bf16", kv=fmt)
    assert L.cache_format(cb) == fmt and L.cache_format(c) == "bf16"
    caches = L.kv_cache(cb, 16)
    got_logits = L.forward(ids, places, w, cb, caches, every=True)
    # the first step's rows come from identical inputs in both runs, so they are exactly bfp() of the bf16 run's
    assert np.array_equal(caches[0][:, :4], B.bfp(plain[0][:, :4], fmt))
    assert np.array_equal(B.bfp(caches[0][:, :4], fmt), caches[0][:, :4])
    assert not caches[0][:, 4:].any()
    assert not np.array_equal(caches[0][:, :4], plain[0][:, :4])  # the rounding did something
    err = np.abs(got_logits - want_logits).max()
    assert 0 < err < (0.05 if fmt == "bfp8" else 0.4) * np.abs(want_logits).max(), (fmt, err)


def test_layer_rows_equal_the_full_layer():
  # layer(..., only=rows) is those rows of the full result, and fills the cache the same way
  rng = np.random.default_rng(4)
  c, w = L.smol(rng, 1, vocab=64, places=32)
  x = rng.normal(0, 1, (20, 576)).astype(np.float32)
  rot = (w["cos"][:20], w["sin"][:20], w["turn"])
  mask = np.where(np.arange(32) > np.arange(20)[:, None], np.float32(-1e9), np.float32(0))
  full_cache, part_cache = L.kv_cache(c, 32), L.kv_cache(c, 32)
  full = L.layer(x, L.block(w, 0), c, rot, mask, full_cache[0], range(20))
  rows = [0, 7, 19]
  part = L.layer(x, L.block(w, 0), c, rot, mask, part_cache[0], range(20), only=rows)
  assert np.allclose(part, full[rows], rtol=1e-6, atol=1e-6) and np.array_equal(part_cache[0], full_cache[0])
