"""The chip: name-compatible with baretile/chip.py:7 (Chip(pci.open_device())).

Holds the device a Runtime opens, and a weak reference to the runtime using it, so that a new Runtime on the chip can
take over from the old one (docs/api.md:42-45). The Blackhole NoC, TLB windows and telemetry have no counterpart.
"""
import weakref
from baretile_amd import pci

_chips = weakref.WeakValueDictionary()  # GPU index: the live Chip holding it in this process


class Chip:
  def __init__(self, device=None):
    if device is None: device = pci.open_device()
    if not isinstance(device, pci.Device): raise ValueError("Chip takes a device from pci.open_device()")
    self.device, self.index, self.runtime = device, device.index, None
    _chips[self.index] = self

  def __repr__(self): return f"Chip({self.device!r})"


def shared(n=0):
  """The live Chip on GPU n in this process, or a new one on it (what Runtime() uses when given no chip)."""
  c = _chips.get(n)
  return c if c is not None else Chip(pci.open_device(n))
