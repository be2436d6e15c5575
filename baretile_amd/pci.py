"""Device discovery, name-compatible with baretile/pci.py:453 (open_device).

baretile opens a Blackhole card over PCIe or its simulator; here a device is a GPU that HIP sees. open_device(n)
checks that GPU n exists, claims it and returns a handle that Chip wraps. One opener at a time may hold a device, in
any process (docs/api.md:43-45, pci.py:355-360): within a process a registry of live handles, across processes an
exclusive flock on a lock file per GPU. The claim goes when the handle is dropped (or its process ends).
"""
import fcntl, gc, os, tempfile, weakref
from baretile_amd import _lib

_held = weakref.WeakValueDictionary()  # GPU index: the live Device that claims it in this process


class Device:
  """GPU n, as HIP numbers it, claimed for one opener."""
  def __init__(self, index, lock):
    self.index, self._lock = index, lock

  def __repr__(self): return f"Device({self.index})"

  def __del__(self):
    try:
      if self._lock is not None: os.close(self._lock)  # closing the descriptor drops the flock
    except Exception:
      pass


def device_count():
  return _lib.device_count()


def lock_path(n):
  """The file whose exclusive flock claims GPU n across processes."""
  return os.path.join(tempfile.gettempdir(), f"baretile_amd-gpu{n}.lock")


def _take(n):
  """Claim GPU n: a new Device, or None when another opener holds it."""
  if _held.get(n) is not None: return None
  fd = os.open(lock_path(n), os.O_RDWR | os.O_CREAT | os.O_CLOEXEC, 0o666)
  try:
    fcntl.flock(fd, fcntl.LOCK_EX | fcntl.LOCK_NB)
  except BlockingIOError:
    os.close(fd)
    return None
  dev = Device(n, fd)
  _held[n] = dev
  return dev


def open_device(n=0):
  """Open GPU n. ValueError if there is no such GPU; RuntimeError if another opener, in this process or another,
  holds it (a Chip dropped in this process releases it)."""
  found = device_count()
  if not 0 <= n < found: raise ValueError(f"open_device({n}): there are {found} GPUs")
  dev = _take(n)
  if dev is None:
    gc.collect()  # a Chip dropped in this process may still hold the device from a reference cycle
    dev = _take(n)
  if dev is None:
    raise RuntimeError(f"GPU {n} is already open, in this process or another. Share its Chip, or close its runtimes "
                       f"and drop it")
  return dev
