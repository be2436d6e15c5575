"""Matmul, elementwise and attention as the reference's NumPy checks state them — TEST INFRASTRUCTURE ONLY.

Not imported by the product. Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.

Reference sources restated here:
  tensor.py:737-795, docs/api.md:116-129   matmul: exact bf16 products, fp32 (here float64) sums; a block-float
                                           B is the matmul by its values
  test_kernels.py:653-663                  the error bound |got - a@b| <= 2^-8 * (|a| @ |b|) for a bf16 result
  tensor.py:797-841, test_kernels.py:1252-1297
                                           attend: softmax(q k^T + mask) v, mask from places (and window)
  models/gpt2.py:101-114                   mask: -1e9 where a key is past the place or window positions before it
  tensor.py:652-657                        silu = x * sigmoid(x); gelu tanh form

How each function is pinned (tests/test_oracle.py):
  matmul         exact small-integer known answers (README.md:82-83, test_kernels.py:637-651,
                 ramps/1_tensors.py:27-31) and A @ I == A
  attention      torch.nn.functional.scaled_dot_product_attention in float64 on the CPU (an independent library),
                 and the exact extremes of test_kernels.py:1323-1337 (all-ones / all-twos outputs)
  mask           brute force over positions
  silu, gelu     torch.nn.functional.silu / gelu(approximate="tanh") in float64
"""
import math
import numpy as np


def matmul(a, b):
  """a @ b in float64 (batched by NumPy's rules)."""
  return np.asarray(a, np.float64) @ np.asarray(b, np.float64)


def matmul_bound(a, b):
  """The error a bf16-rounded, fp32-summed result may have: 2^-8 * (|a| @ |b|) (test_kernels.py:653-663)."""
  return 2.0 ** -8 * (np.abs(np.asarray(a, np.float64)) @ np.abs(np.asarray(b, np.float64)))


def mask(places, keys, window=0):
  """-1e9 where key k > place or (with window) k <= place - window, else 0 (gpt2.py:101-114; tensor.py:802-804).

  places: (..., rows, 1) integer positions. Returns (..., rows, keys) float64."""
  places = np.asarray(places)
  k = np.arange(keys)
  hidden = k > places
  if window: hidden = hidden | (k <= places - window)
  return np.where(hidden, -1e9, 0.0)


def softmax(s, axis=-1):
  """max first, so exp stays in range (gpt2.py:52; tensor.py:727-729)."""
  e = np.exp(s - s.max(axis, keepdims=True))
  return e / e.sum(axis, keepdims=True)


def attention(q, k, v, places, window=0, rep=1):
  """softmax(q @ k^T + mask) @ v per head (test_kernels.py:1290-1292).

  q: (E, rows, hd); k, v: (E / rep, keys, hd) (each key head serves rep query heads, repeat_interleave);
  places: (1 | E, rows, 1) int. No scale is applied: RoPE pre-scales q (llama.py:210-216)."""
  q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
  k, v = np.repeat(k, rep, 0), np.repeat(v, rep, 0)
  s = q @ k.transpose(0, 2, 1) + mask(places, k.shape[1], window)
  return softmax(s) @ v


def silu(x):
  x = np.asarray(x, np.float64)
  return x / (1 + np.exp(-x))


def gelu(x):
  x = np.asarray(x, np.float64)
  return 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
