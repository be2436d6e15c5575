"""The Llama decoder on the GPU against the NumPy oracle (oracle/llama_ref.py), with SmolLM-135M's shapes and random
weights, as test/test_models.py checks its chip path against its NumPy path. Needs a GPU."""
import numpy as np
import pytest

from baretile_amd.models import llama
from baretile_amd.tensor import Tensor
from oracle import bfp as B, llama_ref as L

pytestmark = pytest.mark.gpu


def setup(rt, layers, vocab, mode, places=96, seed=12):
  """An oracle config and weights in SmolLM's shapes, and the same on the device in precision `mode`. The oracle's
  config carries no precision table (a bf16 KV cache) unless a test gives it one."""
  rng = np.random.default_rng(seed)
  c, w = L.smol(rng, layers, vocab=vocab, places=places)
  prec = L.precision(c, mode)
  ref = L.arrays(w, prec)  # the weights as the device holds them: block floats rounded as cast rounds them
  dc = llama.model(dim=576, heads=9, kv=3, layers=layers, eps=1e-5, theta=10000.0, vocab=vocab, ffn=1536,
                   precision=llama.precision(llama.model(layers=layers, dim=576), mode))
  host = {k: v for k, v in w.items() if k not in ("cos", "sin", "turn", "embed.T")}
  dw = llama.upload(rt, host, dc, places=places)
  return c, ref, dc, dw


@pytest.mark.parametrize("mode", ["bf16", "bfp8"])
def test_block_and_logits_match_numpy(rt, mode):
  # test_models.py:818-851: a prompt, then a decode step against the cache, within 3% of the largest logit
  c, ref, dc, dw = setup(rt, 2, 256, mode)
  ids = [7, 200, 31, 64, 5, 9, 100, 3]
  caches = llama.kv_cache(rt, dc, 96)
  got = np.array(llama.forward(Tensor.of(rt, [ids], "int32"), Tensor.of(rt, [list(range(8))], "int32"), dw, dc, caches,
                               every=True).tolist())
  want = L.forward(ids, range(8), ref, c, L.kv_cache(c, 96), every=True)
  assert np.abs(got - want).max() <= 0.03 * np.abs(want).max(), np.abs(got - want).max()
  assert (got.argmax(-1) == want.argmax(-1)).mean() >= 0.75
  rcaches = L.kv_cache(c, 96)
  L.forward(ids, range(8), ref, c, rcaches)
  step = np.array(llama.forward(Tensor.of(rt, [[42]], "int32"), Tensor.of(rt, [[8]], "int32"), dw, dc, caches).tolist())[0]
  want = L.forward([42], [8], ref, c, rcaches)[0]
  assert np.abs(step - want).max() <= 0.03 * np.abs(want).max()


def test_greedy_decode_numpy_fed(rt):
  # gpt2.py:147-161's protocol: both sides are fed the NumPy pick each step; their picks agree where the NumPy top two
  # are apart by more than the device's logit error
  c, ref, dc, dw = setup(rt, 2, 512, "bfp8", places=64, seed=3)
  rng = np.random.default_rng(0)
  prompt = [int(i) for i in rng.integers(0, 512, 16)]
  want_toks, want_logits = L.greedy(prompt, 24, ref, c, 64)
  got_toks, got_logits = llama.generate(dw, dc, prompt, 24, 64, feed=want_toks)
  for s, (g, wl) in enumerate(zip(got_logits, want_logits)):
    top2 = np.sort(wl)[-2:]
    err = np.abs(g - wl).max()
    assert err <= 0.03 * np.abs(wl).max(), (s, err)
    if top2[1] - top2[0] > 2 * err: assert got_toks[s] == want_toks[s], s


def test_smollm_full_size_decode_matches_numpy(rt):
  # BASELINE config 3 at its full size (30 layers, a 49152 vocabulary, bfp8 linears and tied output layer), under the
  # NumPy-fed protocol: every step's logits within 3% of the largest, and the picks equal where NumPy's top two are
  # apart by more than twice the device's logit error
  c, ref, dc, dw = setup(rt, 30, 49152, "bfp8", places=40, seed=0)
  prompt = [int(i) for i in np.random.default_rng(1).integers(0, 49152, 16)]
  want_toks, want_logits = L.greedy(prompt, 8, ref, c, 40)
  got_toks, got_logits = llama.generate(dw, dc, prompt, 8, 40, feed=want_toks)
  for s, (g, wl) in enumerate(zip(got_logits, want_logits)):
    top2 = np.sort(wl)[-2:]
    err = np.abs(g - wl).max()
    assert err <= 0.03 * np.abs(wl).max(), (s, err)
    if top2[1] - top2[0] > 2 * err: assert got_toks[s] == want_toks[s], s


def test_smollm_config3_autonomous_decode_matches_numpy(rt):
  # BASELINE config 3 as configured: a 32-token uniform prompt, then 128 greedy tokens with each side feeding back its
  # own picks (gpt2.py:147-161's autonomous protocol; the device's steps are replays of the recorded step). The
  # device's stream equals the oracle's up to the first step whose NumPy top-2 margin is within twice the device's
  # largest logit error (on this seed no step is that close, so all 128), and under the NumPy-fed protocol every
  # step's logits are within 3% of the largest (test_models.py:849). The autonomous steps pick their tokens on the
  # device: where they picked what the oracle fed, their logits (kept on the device, read back when asked for) are
  # the fed run's bit for bit, as both run the same kernels on the same inputs
  size = 160
  c, ref, dc, dw = setup(rt, 30, 49152, "bfp8", places=size, seed=0)
  prompt = [int(i) for i in np.random.default_rng(1).integers(0, 49152, 32)]
  want_toks, want_logits = L.greedy(prompt, 128, ref, c, size)
  got_toks, got_logits = llama.generate(dw, dc, prompt, 128, size)
  _, fed_logits = llama.generate(dw, dc, prompt, 128, size, feed=want_toks)
  assert len(got_logits) == 128 and len(got_logits[-3:]) == 3
  same = next((s for s in range(128) if got_toks[s] != want_toks[s]), 128)
  assert all(np.array_equal(got_logits[s], fed_logits[s]) for s in range(same)), same
  errs = [np.abs(g - w).max() for g, w in zip(fed_logits, want_logits)]
  assert all(e <= 0.03 * np.abs(w).max() for e, w in zip(errs, want_logits)), max(errs)
  close = [s for s, w in enumerate(want_logits) if np.diff(np.sort(w)[-2:])[0] <= 2 * max(errs)]
  n = close[0] + 1 if close else 128
  assert got_toks[:n] == want_toks[:n], next(s for s in range(n) if got_toks[s] != want_toks[s])


@pytest.mark.parametrize("mode", ["bf16", "bfp8"])
def test_chunked_prefill_matches_numpy(rt, mode):
  # test_models.py:1531-1547: a 70-token prompt in chunks of 32, 32 and 6 (each chunk's scores a chunk by the cache),
  # against the oracle's chunked prefill, then one decode step at place 70 from the caches the chunks filled, each
  # within 3% of the largest logit; bad chunk arguments raise ValueError
  c, ref, dc, dw = setup(rt, 2, 256, mode, places=96, seed=29)
  prompt = [int(i) for i in np.random.default_rng(30).integers(0, 256, 70)]
  for ids, chunk in (([], 32), (prompt, 0), (prompt, -1)):
    with pytest.raises(ValueError, match="prefill"): llama.prefill(ids, dw, dc, llama.kv_cache(rt, dc, 96), chunk)
  rcaches = L.kv_cache(c, 96)
  want = L.prefill(prompt, ref, c, rcaches, 32)[0]
  caches = llama.kv_cache(rt, dc, 96)
  got = np.frombuffer(llama.prefill(prompt, dw, dc, caches, 32).tobytes(), np.float32)
  assert np.abs(got - want).max() < 0.03 * np.abs(want).max(), np.abs(got - want).max()
  nxt = int(want.argmax())
  got = np.frombuffer(llama.forward(Tensor.of(rt, [[nxt]], "int32"), Tensor.of(rt, [[70]], "int32"), dw, dc,
                                    caches).tobytes(), np.float32)
  want = L.forward([nxt], [70], ref, c, rcaches)[0]
  assert np.abs(got - want).max() < 0.03 * np.abs(want).max(), np.abs(got - want).max()


@pytest.mark.parametrize("row", [True, False])
def test_jit_decode_matches_eager(rt, row):
  # generate's steps, picked on the device and replayed from a graph, against a host loop of eager forwards; also
  # with the fused row kernels turned off (the per-operation kernels, a first step run eagerly before the recording)
  c, ref, dc, dw = setup(rt, 2, 256, "bfp8", places=64)
  dw["row_fits"] = row
  prompt = [3, 1, 4, 1, 5, 9, 2, 6]
  a, _ = llama.generate(dw, dc, prompt, 6, 64)
  caches = llama.kv_cache(rt, dc, 64)
  logits = llama.prefill(prompt, dw, dc, caches, len(prompt))
  b = []
  for s in range(6):
    b.append(llama.argmax(logits))
    logits = llama.forward(Tensor.of(rt, [[b[-1]]], "int32"), Tensor.of(rt, [[len(prompt) + s]], "int32"), dw, dc, caches)
  assert a == b


def test_slots_layer_matches_each_slot_in_numpy(rt):
  # batched decode (llama.py:293-354 with slots): S slots, each with its own cache holding `place` earlier rows, one
  # new token each; each slot's row equals the NumPy block run on that slot alone, within the block tolerance
  rng = np.random.default_rng(7)
  S, size, place, dim, heads, kv, hd, ffn = 3, 96, 40, 256, 4, 2, 64, 512
  c = L.model(dim=dim, heads=heads, kv=kv, layers=1, eps=1e-5, theta=10000.0, vocab=None, ffn=ffn, head_dim=hd)
  bf = lambda a: B.bf16(np.asarray(a, np.float32))
  w = {"layers.0.input_layernorm": bf(rng.normal(1, 0.1, (1, dim))),
       "layers.0.post_attention_layernorm": bf(rng.normal(1, 0.1, (1, dim))),
       "layers.0.qkv_proj": bf(rng.normal(0, 0.02, (dim, (heads + 2 * kv) * hd))),
       "layers.0.o_proj": bf(rng.normal(0, 0.02, (heads * hd, dim))),
       "layers.0.gate_up_proj": bf(rng.normal(0, 0.02, (dim, 2 * ffn))),
       "layers.0.down_proj": bf(rng.normal(0, 0.02, (ffn, dim))),
       "norm": bf(rng.normal(1, 0.1, (1, dim))), "embed": bf(rng.normal(0, 1, (64, dim)))}
  ref = L.arrays(w, L.precision(c, "bfp8"))
  ref["cos"], ref["sin"], ref["turn"] = L.rotary(c, size)
  dc = llama.model(dim=dim, heads=heads, kv=kv, layers=1, eps=1e-5, theta=10000.0, ffn=ffn, head_dim=hd,
                   precision=llama.precision(llama.model(layers=1, dim=dim), "bfp8"))
  dw = llama.upload(rt, w, dc, places=size)
  K, V = (bf(rng.normal(0, 1, (S * kv, size, hd))) for _ in range(2))
  K[:, place:], V[:, place:] = 0, 0
  x = rng.normal(0, 1, (S, dim)).astype(np.float32)
  rows = Tensor.of(rt, [[place] * S], "int32")
  rot = (dw["cos"].gather(rows), dw["sin"].gather(rows), dw["turn"])
  keys, values = Tensor.of(rt, K), Tensor.of(rt, V)
  got = np.array(llama.slots_layer(Tensor.of(rt, x[None], "fp32"), llama.block(dw, 0), dc, rot, keys, values,
                                   Tensor.of(rt, [[place]], "int32")).tolist()).reshape(S, dim)
  mask = np.where(np.arange(size) > place, np.float32(-1e9), np.float32(0))[None]
  for s in range(S):
    cache = np.concatenate([K[s * kv:(s + 1) * kv], V[s * kv:(s + 1) * kv]]).astype(np.float64)
    want = L.layer(x[s:s + 1], L.block(ref, 0), c, (ref["cos"][[place]], ref["sin"][[place]], ref["turn"]), mask,
                   cache, [place])[0]
    assert np.abs(got[s] - want).max() <= 0.03 * np.abs(want - x[s]).max(), (s, np.abs(got[s] - want).max())
    # the slot's new key and value rows, as the NumPy block put them into its cache
    new_k = np.array(keys.tolist()).reshape(S * kv, size, hd)[s * kv:(s + 1) * kv, place]
    new_v = np.array(values.tolist()).reshape(S * kv, size, hd)[s * kv:(s + 1) * kv, place]
    for got_r, want_r in ((new_k, cache[:kv, place]), (new_v, cache[kv:, place])):
      assert np.abs(got_r - want_r).max() <= 0.03 * np.abs(want_r).max(), (s, np.abs(got_r - want_r).max())


def test_slots_layer_then_fuses_the_next_norm(rt):
  # slots_layer(h=, then=): the block's input norm given, and the down product's partial sums, the residual add and
  # the next norm in one kernel (bt_matmul_residual_rms) -- bit for bit the block's x and rms_rows of it, in two
  # launches fewer than the block with both norms run on their own. 8 slots and K = ffn = 1024 (16 chunks), the
  # shapes the streaming product takes
  rng = np.random.default_rng(17)
  S, size, place, dim, heads, kv, hd, ffn = 8, 64, 21, 256, 4, 2, 64, 1024
  bf = lambda a: B.bf16(np.asarray(a, np.float32))
  w = {"layers.0.input_layernorm": bf(rng.normal(1, 0.1, (1, dim))),
       "layers.0.post_attention_layernorm": bf(rng.normal(1, 0.1, (1, dim))),
       "layers.0.qkv_proj": bf(rng.normal(0, 0.02, (dim, (heads + 2 * kv) * hd))),
       "layers.0.o_proj": bf(rng.normal(0, 0.02, (heads * hd, dim))),
       "layers.0.gate_up_proj": bf(rng.normal(0, 0.02, (dim, 2 * ffn))),
       "layers.0.down_proj": bf(rng.normal(0, 0.02, (ffn, dim))),
       "norm": bf(rng.normal(1, 0.1, (1, dim))), "embed": bf(rng.normal(0, 1, (64, dim)))}
  dc = llama.model(dim=dim, heads=heads, kv=kv, layers=1, eps=1e-5, theta=10000.0, ffn=ffn, head_dim=hd,
                   precision=llama.precision(llama.model(layers=1, dim=dim), "bfp4"))
  dw = llama.upload(rt, w, dc, places=size)
  p = llama.block(dw, 0)
  K, V = (bf(rng.normal(0, 1, (S * kv, size, hd))) for _ in range(2))
  keys, values = Tensor.of(rt, K), Tensor.of(rt, V)
  rows = Tensor.of(rt, [[place] * S], "int32")
  rot = (dw["cos"].gather(rows), dw["sin"].gather(rows), dw["turn"])
  at = Tensor.of(rt, [[place]], "int32")
  x = Tensor.of(rt, rng.normal(0, 1, (1, S, dim)).astype(np.float32), "fp32")
  then = dw["norm"]
  n0 = rt.launches
  h0 = llama.rms(x, p["input_layernorm"], dc)
  x1 = llama.slots_layer(x, p, dc, rot, keys, values, at, h=h0)
  h1 = llama.rms(x1, then, dc)
  want_x, want_h = x1.tobytes(), h1.tobytes()
  n1 = rt.launches
  x2, h2 = llama.slots_layer(x, p, dc, rot, keys, values, at, h=h0, then=then)
  got_x, got_h = x2.tobytes(), h2.tobytes()
  n2 = rt.launches
  assert got_x == want_x and got_h == want_h
  assert n2 - n1 == (n1 - n0) - 2, (n1 - n0, n2 - n1)
  # without h the block makes its input norm itself, the same one
  x3, h3 = llama.slots_layer(x, p, dc, rot, keys, values, at, then=then)
  assert x3.tobytes() == want_x and h3.tobytes() == want_h


@pytest.mark.parametrize("kv", ["bfp8", "bfp4"])
def test_block_float_kv_cache_matches_numpy(rt, kv):
  # the KV cache in bfp8 or bfp4 (precision's kv entry, tt_transformers' cache format, llama.py:74-83): a prompt's
  # logits and a one-token step (the row kernels, with the rows put through the block-float put), against the oracle,
  # whose cache rounds the rows it puts the same way (llama.py:151-154), within 1% of the logits' span and the same pick
  c, ref, dc, dw = setup(rt, 2, 256, "bfp8")
  dc.precision = llama.precision(llama.model(layers=2, dim=576), "bfp8", kv=kv)
  c.precision = L.precision(c, "bfp8", kv=kv)
  caches = llama.kv_cache(rt, dc, 96)
  assert caches[0].dtype == kv and L.cache_format(c) == kv
  ids = [7, 200, 31, 64, 5, 9, 100, 3]
  got = np.array(llama.forward(Tensor.of(rt, [ids], "int32"), Tensor.of(rt, [list(range(8))], "int32"), dw, dc, caches,
                               every=True).tolist())
  rcaches = L.kv_cache(c, 96)
  want = L.forward(ids, range(8), ref, c, rcaches, every=True)
  assert np.abs(got - want).max() <= 0.01 * np.ptp(want), np.abs(got - want).max()
  assert (got.argmax(-1) == want.argmax(-1)).all()
  step = np.array(llama.forward(Tensor.of(rt, [[42]], "int32"), Tensor.of(rt, [[8]], "int32"), dw, dc, caches).tolist())[0]
  want = L.forward([42], [8], ref, c, rcaches)[0]
  assert np.abs(step - want).max() <= 0.01 * np.ptp(want) and step.argmax() == want.argmax(), np.abs(step - want).max()


@pytest.mark.parametrize("mode", ["bfp4", "tt"])
def test_llama_precision_modes(rt, mode):
  # test_models.py:1549-1583: bfp4 mode puts gate_up in bfp4 and the rest in bfp8; tt also makes the KV cache bfp8.
  # NumPy with the same block-float values and exact products picks the same token, within 1% of the logits' span
  c, ref, dc, dw = setup(rt, 2, 256, mode, seed=5)
  c.precision = L.precision(c, mode)
  formats = {k: t.dtype for k, t in dw.items() if k.endswith("_proj") or k == "embed.T"}
  assert formats == {k: "bfp4" if "gate_up" in k else "bfp8" for k in formats}
  caches = llama.kv_cache(rt, dc, 32)
  assert caches[0].dtype == ("bfp8" if mode == "tt" else "bf16")
  rcaches = L.kv_cache(c, 32)
  for ids, places in (([7, 200, 31], [0, 1, 2]), ([5], [3])):
    got = np.frombuffer(llama.forward(Tensor.of(rt, [ids], "int32"), Tensor.of(rt, [places], "int32"), dw, dc,
                                      caches).tobytes(), np.float32)
    want = L.forward(ids, places, ref, c, rcaches)[0]
    assert got.argmax() == want.argmax() and np.abs(got - want).max() < 0.01 * np.ptp(want), \
        (places, np.abs(got - want).max(), np.ptp(want))


def test_loaded_checkpoint_matches_numpy(rt, tmp_path):
  # llama.load (safetensors, llama.py:429-462) -> upload in bfp8 -> a prompt's logits, against the oracle on the
  # same weights (their bf16 values, block floats rounded by oracle.bfp), within test_models.py:849's 3%
  from test_llama_load import checkpoint
  checkpoint(str(tmp_path), dim=256, heads=4, kv=2, ffn=256, vocab=96, layers=2, tied=False)
  c, w = llama.load(str(tmp_path), places=64)
  c.precision = llama.precision(c, "bfp8")
  dw = llama.upload(rt, w, c, places=c.places)
  rc = L.model(dim=c.dim, heads=c.heads, kv=c.kv, layers=c.layers, eps=c.eps, theta=c.theta, vocab=c.vocab, ffn=c.ffn)
  host = {k: v.values() for k, v in w.items()}
  host["cos"], host["sin"], host["turn"] = L.rotary(rc, 64)
  ref = L.arrays(host, L.precision(rc, "bfp8"))
  ids = [5, 90, 17, 3, 44, 61]
  got = np.array(llama.forward(Tensor.of(rt, [ids], "int32"), Tensor.of(rt, [list(range(6))], "int32"), dw, c,
                               llama.kv_cache(rt, c, 64), every=True).tolist())
  want = L.forward(ids, range(6), ref, rc, L.kv_cache(rc, 64), every=True)
  assert np.abs(got - want).max() <= 0.03 * np.abs(want).max(), np.abs(got - want).max()

