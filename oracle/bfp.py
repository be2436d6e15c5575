"""bf16 rounding and block-float (bfp8 / bfp4) rules, restated in NumPy — TEST INFRASTRUCTURE ONLY.

Not imported by the product. Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.

Reference sources restated here:
  models/gpt2.py:14-17    bf16_bits (round to nearest even) and bf16_floats
  tensix.py:240-242       round_bf16: the upload rounding, with a quiet-NaN payload
  models/gpt2.py:19-30    bfp(a, dtype): the chip's cast, as values
  kernels.py:1074-1081    NIBBLE: the bfp4 rounding, "no sign on a zero"
  kernels.py:1108-1114    put_kernel's bfp8 rounding, same rule, "a 0 loses its sign"
  tensix.py:14-21         a run of 16 values shares one exponent; bfp8 sign+7 bits, bfp4 sign+3 bits read as
                          the top 3 of bfp8's
  tensor.py:1093-1104     _bf16s: the unpacker's exact bfp -> bf16 bits, signed zero -> -inf

How each function is pinned (tests/test_oracle.py):
  bf16_bits      numpy float32 -> bfloat16 via torch (an independent library rounding, RNE)
  bfp            known answers of the reference's tests (test_kernels.py:2096-2103: [2, 3] -> 0x4000, 0x4040;
                 ramps/1_tensors.py:71-80: small integers are exact in bfp8), and a brute-force rational
                 restatement on small blocks: the nearest multiple of the block's step 2^(top-133)
                 (bfp8) / 2^(top-129) (bfp4), ties away from zero, saturated at 127 / 7 steps
  bfp_fields     decode(bfp_fields(a)) == bfp(a) as values, for every element
  decode_bits    every bfp8 byte x 256 exponents against float arithmetic +-mag * 2^(e-133) where that
                 is a normal bf16; the -inf rule for a signed zero and the mod-256 wrap are "as restated"
                 (reachable only through inputs the packers never write)

The reference's 32x32 DRAM tile byte order (tensix.py:6-7) is not restated: the device layouts here are this
library's own, and what crosses the boundary (tobytes, tolist) is bf16 values, which decode_bits pins.
"""
import numpy as np

FORMATS = ("bfp8", "bfp4")
RUN = 16  # values that share an exponent: a run along the last axis (gpt2.py:21-24, tensix.py:15-16)


def bf16_bits(a):
  """float32 -> bf16 bits, round to nearest even, no NaN special case (gpt2.py:14-16)."""
  b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
  return ((b + 0x7FFF + (b >> 16 & 1)) >> 16).astype(np.uint16)


def round_bf16_bits(a):
  """Upload rounding (tensix.py:240-242): RNE, but a NaN keeps its high bits and is made quiet."""
  b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
  rne = (b + 0x7FFF + (b >> 16 & 1)) >> 16
  nan = (b & 0x7FFFFFFF) > 0x7F800000
  return np.where(nan, (b >> 16) | 0x40, rne).astype(np.uint16)


def bf16_floats(bits):
  """bf16 bits -> float32 values (gpt2.py:17)."""
  return (np.asarray(bits).astype(np.uint32) << 16).view(np.float32)


def bf16(a):
  """Round float values to bf16 and back to float32."""
  return bf16_floats(bf16_bits(a))


def _runs(x):
  return x.reshape(*x.shape[:-1], -1, RUN)


def bfp_fields(a, dtype="bfp8"):
  """The integer content of a block float: (top, q).

  top: uint8, one exponent per run of 16 along the last axis, shape (..., n/16).
  q:   int8 signed magnitude at the format's precision, shape a.shape: bfp8 in [-127, 127] worth q * 2^(top-133);
       bfp4 in [-7, 7] worth q * 2^(top-129). A zero never carries a sign (kernels.py:1080, 1114).
  Rounding follows gpt2.py:19-30: first bf16 RNE, m = frac | hidden bit, shift = min(top - e, 8),
  bfp8 q = min((m + (1 << shift)) >> (shift + 1), 127), bfp4 q = min((m + (16 << shift)) >> (shift + 5), 7).
  """
  if dtype not in FORMATS: raise ValueError(f"unknown block-float format {dtype}")
  a = np.asarray(a)
  if a.shape[-1] % RUN: raise ValueError("the last axis must be a multiple of 16")
  bits = bf16_bits(a).astype(np.int32)
  s, e = bits >> 15 & 1, bits >> 7 & 255
  m = (bits & 127) | np.where(e != 0, 128, 0)
  top = _runs(e).max(-1, keepdims=True)
  shift = np.minimum(top - _runs(e), 8)
  if dtype == "bfp8": q = np.minimum((_runs(m) + (1 << shift)) >> (shift + 1), 127)
  else: q = np.minimum((_runs(m) + (16 << shift)) >> (shift + 5), 7)
  q = np.where(_runs(s) == 1, -q, q).reshape(a.shape)
  return top[..., 0].astype(np.uint8), q.astype(np.int8)


def bfp(a, dtype="bfp8"):
  """The values a block-float cast gives, as float64 (gpt2.py:19-30). A negative value that rounds to zero gives -0.0."""
  if dtype not in FORMATS: raise ValueError(f"unknown block-float format {dtype}")
  a = np.asarray(a)
  s = bf16_bits(a) >> 15 & 1
  top, q = bfp_fields(a, dtype)
  scale = 2.0 ** (top.astype(np.int64) - (133 if dtype == "bfp8" else 129))
  mag = np.abs(q.astype(np.int32))
  vals = np.where(_runs(s) == 1, -1.0, 1.0) * _runs(mag) * scale[..., None]
  return vals.reshape(a.shape)


def decode_bits(e, x, dtype="bfp8"):
  """The unpacker's bf16 bits for a stored value (tensor.py:1093-1104).

  e: the run's exponent byte. x: the stored value in the reference's sign-magnitude encoding: a bfp8 byte
  sign<<7 | mag7, or a bfp4 nibble sign<<3 | mag3, which the unpacker reads as the byte nibble << 4.
  Zero magnitude gives 0, or -inf (0xFF80) with the sign set. Otherwise the magnitude is normalized and the
  exponent is (e - shift) mod 256.
  """
  e = np.asarray(e, np.int64)
  x = np.asarray(x, np.int64)
  if dtype == "bfp4": x = (x & 15) << 4
  sign, mag = x >> 7 & 1, x & 127
  m = mag << 1
  bl = np.zeros_like(m)
  for b in range(1, 9): bl = np.where(m >= (1 << (b - 1)), b, bl)  # bit length of m
  shift = 8 - bl
  out = (sign << 15) | (((e - shift) % 256) << 7) | ((m << shift) & 0x7E)
  out = np.where(mag == 0, np.where(sign == 1, 0xFF80, 0), out)
  return out.astype(np.uint16)


def sign_magnitude(q, dtype="bfp8"):
  """A signed q from bfp_fields in the reference's stored encoding: sign<<7|mag (bfp8) or sign<<3|mag (bfp4)."""
  q = np.asarray(q, np.int64)
  s = (q < 0).astype(np.int64)
  return (s << (7 if dtype == "bfp8" else 3)) | np.abs(q)


def decode_fields(top, q, dtype="bfp8"):
  """bf16 bits of a block float given as (top, q) from bfp_fields, via the unpacker rule."""
  e = np.repeat(np.asarray(top), RUN, axis=-1)
  return decode_bits(e, sign_magnitude(q, dtype), dtype)
