"""llama.config / llama.load (llama.py:400-462) on checkpoints written here in the safetensors format: names,
layouts (linear layers transposed for x @ w, q/k/v and gate/up fused, vectors as one-row matrices), the tied or
separate output layer, BF16 kept bit for bit and F32 rounded to nearest even, shards; and llama.Logits, generate's
per-step logits read back from the device on first use. CPU only."""
import json
import os
import struct

import numpy as np
import pytest

from baretile_amd.models import llama
from oracle import bfp as B


def write_safetensors(path, tensors):
  """tensors: {name: (dtype, array)} with dtype "BF16" (uint16 bits) or "F32"."""
  header, blobs, at = {}, [], 0
  for name, (dtype, a) in tensors.items():
    raw = np.ascontiguousarray(a).tobytes()
    header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [at, at + len(raw)]}
    blobs.append(raw)
    at += len(raw)
  head = json.dumps(header).encode()
  head += b" " * (-len(head) % 8)
  with open(path, "wb") as f:
    f.write(struct.pack("<Q", len(head)) + head + b"".join(blobs))


def checkpoint(folder, dim=64, heads=4, kv=2, ffn=96, vocab=50, layers=2, tied=True, dtype="BF16", shards=1,
               model_type="llama", rope=None):
  rng = np.random.default_rng(3)
  hd = dim // heads
  shapes = {"self_attn.q_proj": (heads * hd, dim), "self_attn.k_proj": (kv * hd, dim), "self_attn.v_proj": (kv * hd, dim),
            "self_attn.o_proj": (dim, heads * hd), "mlp.gate_proj": (ffn, dim), "mlp.up_proj": (ffn, dim),
            "mlp.down_proj": (dim, ffn), "input_layernorm": (dim,), "post_attention_layernorm": (dim,)}
  t = {}
  for l in range(layers):
    for k, s in shapes.items(): t[f"model.layers.{l}.{k}.weight"] = rng.normal(0, 0.05, s).astype(np.float32)
  t["model.norm.weight"] = rng.normal(1, 0.1, dim).astype(np.float32)
  t["model.embed_tokens.weight"] = rng.normal(0, 1, (vocab, dim)).astype(np.float32)
  if not tied: t["lm_head.weight"] = rng.normal(0, 0.05, (vocab, dim)).astype(np.float32)
  stored = {k: ("BF16", B.bf16_bits(v)) if dtype == "BF16" else ("F32", v) for k, v in t.items()}
  names = sorted(stored)
  if shards == 1:
    write_safetensors(os.path.join(folder, "model.safetensors"), stored)
  else:
    parts = [names[i::shards] for i in range(shards)]
    weight_map = {}
    for i, part in enumerate(parts):
      file = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
      write_safetensors(os.path.join(folder, file), {n: stored[n] for n in part})
      weight_map |= {n: file for n in part}
    with open(os.path.join(folder, "model.safetensors.index.json"), "w") as f: json.dump({"weight_map": weight_map}, f)
  cfg = {"model_type": model_type, "hidden_size": dim, "num_attention_heads": heads, "num_key_value_heads": kv,
         "num_hidden_layers": layers, "rms_norm_eps": 1e-5, "rope_theta": 10000.0, "vocab_size": vocab,
         "intermediate_size": ffn, "max_position_embeddings": 128, "tie_word_embeddings": tied}
  if rope: cfg["rope_scaling"] = rope
  with open(os.path.join(folder, "config.json"), "w") as f: json.dump(cfg, f)
  return t


def bits_of(a): return B.bf16_bits(a)


@pytest.mark.parametrize("dtype,shards,tied", [("BF16", 1, True), ("F32", 1, False), ("BF16", 3, False)])
def test_load_lays_out_the_checkpoint(tmp_path, dtype, shards, tied):
  t = checkpoint(str(tmp_path), dtype=dtype, shards=shards, tied=tied)
  c, w = llama.load(str(tmp_path), places=4096)
  assert (c.dim, c.heads, c.kv, c.layers, c.ffn, c.vocab, c.theta, c.places) == (64, 4, 2, 2, 96, 50, 10000.0, 128)
  names = {f"layers.{l}.{n}" for l in range(2) for n in ("qkv_proj", "o_proj", "gate_up_proj", "down_proj",
                                                          "input_layernorm", "post_attention_layernorm")}
  assert set(w) == names | {"norm", "embed", "embed.T"}
  for l in range(2):
    p = f"model.layers.{l}."
    qkv = np.concatenate([t[p + f"self_attn.{n}_proj.weight"].T for n in "qkv"], 1)
    assert np.array_equal(w[f"layers.{l}.qkv_proj"].bits(), bits_of(qkv))
    gu = np.concatenate([t[p + f"mlp.{n}_proj.weight"].T for n in ("gate", "up")], 1)
    assert np.array_equal(w[f"layers.{l}.gate_up_proj"].bits(), bits_of(gu))
    assert np.array_equal(w[f"layers.{l}.o_proj"].bits(), bits_of(t[p + "self_attn.o_proj.weight"].T))
    assert np.array_equal(w[f"layers.{l}.down_proj"].bits(), bits_of(t[p + "mlp.down_proj.weight"].T))
    assert np.array_equal(w[f"layers.{l}.input_layernorm"].bits(), bits_of(t[p + "input_layernorm.weight"][None]))
  assert np.array_equal(w["embed"].bits(), bits_of(t["model.embed_tokens.weight"]))
  head = t["model.embed_tokens.weight"] if tied else t["lm_head.weight"]
  assert np.array_equal(w["embed.T"].bits(), bits_of(head.T))
  assert np.array_equal(w["norm"].values(), B.bf16(t["model.norm.weight"][None]).astype(np.float32))


def test_load_keeps_the_configs_blocks_and_refuses_other_models(tmp_path):
  checkpoint(str(tmp_path), layers=2)
  cfg = json.load(open(tmp_path / "config.json"))
  json.dump(cfg | {"num_hidden_layers": 1}, open(tmp_path / "config.json", "w"))
  c, w = llama.load(str(tmp_path))
  assert c.layers == 1 and not any(k.startswith("layers.1.") for k in w)
  json.dump(cfg | {"model_type": "qwen3_moe"}, open(tmp_path / "config.json", "w"))
  with pytest.raises(ValueError, match="isn't supported"): llama.load(str(tmp_path))
  json.dump(cfg | {"rope_scaling": {"rope_type": "yarn", "factor": 8.0}}, open(tmp_path / "config.json", "w"))
  with pytest.raises(ValueError, match="RoPE scaling"): llama.load(str(tmp_path))


LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


@pytest.mark.parametrize("style", ["rope_scaling", "rope_parameters", "type"])
def test_load_takes_llama3_rope_scaling(tmp_path, style):
  # llama.py:400-427 with Llama 3.1's config: the scaling is kept as c.rope, whichever way transformers wrote it, and
  # the frequencies equal the oracle's (which transformers' own llama3 initialisation pins) bit for bit
  from oracle import llama_ref as L
  checkpoint(str(tmp_path), dim=128, heads=2, kv=1, layers=1)
  cfg = json.load(open(tmp_path / "config.json"))
  cfg.pop("rope_theta")
  if style == "rope_scaling": cfg |= {"rope_scaling": LLAMA3, "rope_theta": 500000.0}
  elif style == "rope_parameters": cfg |= {"rope_parameters": LLAMA3 | {"rope_theta": 500000.0}}
  else:
    old = {k: v for k, v in LLAMA3.items() if k != "rope_type"} | {"type": "llama3"}
    cfg |= {"rope_scaling": old, "rope_theta": 500000.0}
  json.dump(cfg, open(tmp_path / "config.json", "w"))
  c, _ = llama.load(str(tmp_path), places=64)
  assert c.rope == LLAMA3 and c.theta == 500000.0 and c.places == 64
  rc = L.model(dim=c.dim, heads=c.heads, kv=c.kv, layers=c.layers, eps=c.eps, theta=c.theta, rope=c.rope)
  assert np.array_equal(llama.frequencies(c), L.frequencies(rc))
  got, want = llama.rotary(c, 64), L.rotary(rc, 64)
  assert all(np.array_equal(g, w) for g, w in zip(got, want))
  plain = llama.model(**{**vars(c), "rope": None})
  assert not np.array_equal(llama.frequencies(plain), llama.frequencies(c))


def test_logits_read_the_device_rows_once_on_first_use():
  # generate's per-step logits on the device path: the host-made rows first, then the device tensor's rows, read back
  # in one transfer the first time any of them is asked for; indexing as a list's (negative, slices, IndexError)
  data = np.arange(12, dtype=np.float32).reshape(3, 4)
  reads = []

  class Runtime:
    def download(self, addr, nbytes):
      reads.append((addr, nbytes))
      return bytearray(data.tobytes())

  class Rows:  # a (3, 4) fp32 view of a device tensor, as greedy_steps returns it
    rt, addr, rows, cols = Runtime(), 4096, 3, 4

  first = np.full(4, -1.0, np.float32)
  got = llama.Logits([first], Rows())
  assert len(got) == 4 and reads == []
  assert got[0] is first and reads == []
  assert np.array_equal(got[1], data[0]) and np.array_equal(got[-1], data[2])
  assert [r.tolist() for r in got[1:3]] == data[:2].tolist()
  assert reads == [(4096, 48)]
  with pytest.raises(IndexError): got[4]
  with pytest.raises(IndexError): got[-5]
  assert len(list(got)) == 4


def test_blocks_split_the_weights_as_block_does():
  # forward's one pass over the weights gives each layer what block(w, l) gives it (layers past the count left out)
  w = {f"layers.{l}.{n}": (l, n) for l in range(12) for n in ("qkv_proj", "input_layernorm")}
  w.update({"embed": 0, "norm": 1, "layers.x.odd": 2, "layers.12.extra": 3})
  got = llama.blocks(w, 12)
  assert len(got) == 12 and all(got[l] == llama.block(w, l) for l in range(12))
