"""Test helpers: host <-> device copies through the C ABI, and the shared GPU runtime fixture."""
import numpy as np
import pytest


def gpu_available():
  try:
    from baretile_amd import _lib
    return _lib.device_count() > 0
  except Exception:
    return False


def up(rt, a):
  """Upload a NumPy array; returns its device address (freed with the runtime's pool when the test drops it)."""
  a = np.ascontiguousarray(a)
  addr = rt.dram_alloc(max(a.nbytes, 1))
  rt.upload(addr, a.tobytes())
  return addr


def down(rt, addr, shape, dtype):
  n = int(np.prod(shape)) * np.dtype(dtype).itemsize
  return np.frombuffer(bytes(rt.download(addr, n)), dtype).reshape(shape)


def bf16_bits(a):
  """float -> bf16 bits, round to nearest even (the upload rule)."""
  from oracle import bfp as B
  return B.bf16_bits(a)


def bits_to_float(b):
  return (np.asarray(b).astype(np.uint32) << 16).view(np.float32)
