"""Device discovery, name-compatible with baretile/pci.py:453 (open_device).

baretile opens a Blackhole card over PCIe or its simulator; here a device is a GPU that HIP sees. open_device(n)
checks that GPU n exists and returns a handle that Chip wraps. Only one Chip at a time may hold a device, as in the
reference (docs/api.md:40-42).
"""
from baretile_amd import _lib

_held = set()


class Device:
  """GPU n, as HIP numbers it."""
  def __init__(self, index):
    self.index = index

  def __repr__(self): return f"Device({self.index})"


def device_count():
  return _lib.device_count()


def open_device(n=0):
  """Open GPU n. ValueError if there is no such GPU."""
  found = device_count()
  if not 0 <= n < found: raise ValueError(f"open_device({n}): there are {found} GPUs")
  return Device(n)
