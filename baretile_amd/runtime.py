"""The runtime: one GPU and one in-order HIP stream, behind the method names of baretile's Runtime.

Mirrors baretile/runtime.py:476-923 in interface, not in mechanism: launches go to a HIP stream through the C ABI
instead of a Tensix command ring, memory comes from the device's stream-ordered pool instead of DRAM holes, and
wait() polls the stream. Promises kept from docs/api.md:38-63: launches are queued in order and wait() blocks, raising
TimeoutError after `timeout` seconds; a new Runtime on the same chip takes over and the old one's tensors then raise
RuntimeError; a bad argument raises ValueError and a bad state RuntimeError, also under python -O.
"""
import collections, ctypes, time, weakref
from ctypes import byref, c_float, c_uint64, c_void_p
from baretile_amd import _lib


class Bound(int):
  """A launch argument that a replay can replace, such as the address of a jit input (runtime.py:476-482). key names
  it in a binding. Kept for code written against the reference's runtime; this backend's jit needs no bound arguments,
  since a HIP graph's kernel arguments are fixed at capture: a replay copies each input into the recording's own
  buffer instead."""
  def __new__(cls, value, key):
    self = super().__new__(cls, value)
    self.key = key
    return self


class Runtime:
  """Queue work on a GPU. Runtime(chip) opens the chip's device with a stream of its own; a newer Runtime on the same
  chip closes this one. Without a chip, the runtime uses this process's Chip on GPU 0, opening one if there is none.
  start/end (Tensix rectangles) and ring are accepted for compatibility and unused."""
  def __init__(self, chip=None, start=None, end=None, ring=1 << 20, timing=False):
    if ring < 64 or ring & (ring - 1): raise ValueError("ring size must be a power of two, at least 64 bytes")
    if chip is None:
      from baretile_amd.chip import shared
      chip = shared(0)
    self.chip, self.handle, self.closed = chip, None, False
    previous = chip.runtime() if chip.runtime is not None else None
    if previous is not None and not previous.closed: previous.close()
    handle = c_void_p()
    _lib.call("open", chip.index, byref(handle))
    self.handle = handle
    chip.runtime = weakref.ref(self)
    self.launches, self.numbers, self.log, self.written, self.recording = 0, {}, None, None, None
    self.timing = timing  # with timing, every launch is bracketed by events, for profile()
    self.times = []  # (launch, name, start event, end event, bytes read or None) while timing
    self.grid, self.readers = None, None  # kernel-cache key parts of the reference; unused here
    self.cores = [None] * 256  # one "worker" per compute unit, for code that sizes work by len(rt.cores)
    self.deferred = []  # (address, captured) frees asked for during a capture

  def check(self):
    if self.closed: raise RuntimeError("this runtime was closed, or another runtime took over its chip")

  # ---- memory
  def dram_alloc(self, size):
    """Allocate size bytes of device memory (at least 256, aligned to 256): from the stream-ordered pool, or, while
    a jit recording captures, a plain allocation that the recording's graph keeps using."""
    self.check()
    addr = c_uint64()
    _lib.call("alloc", self.handle, int(size), byref(addr))
    return addr.value

  def dram_free(self, addr, captured=False):
    """Release memory once the launches queued so far have finished (runtime.py:814-820). Frees asked for while a
    recording captures wait until the capture has ended; memory allocated during a capture is freed by hipFree."""
    if self.closed or not addr: return
    if self.recording is not None:
      self.deferred.append((addr, captured))
      return
    _lib.call("free", self.handle, int(addr), 1 if captured else 0)

  def release_deferred(self):
    """Frees held back during a capture, now that it has ended."""
    held, self.deferred = self.deferred, []
    for addr, captured in held: self.dram_free(addr, captured)

  def upload(self, addr, data):
    """Copy host bytes to device memory; returns once they have arrived."""
    self.check()
    mv = memoryview(data).cast("B")
    if mv.nbytes:
      buf = (ctypes.c_char * mv.nbytes).from_buffer_copy(mv) if mv.readonly else (ctypes.c_char * mv.nbytes).from_buffer(mv)
      _lib.call("upload", self.handle, int(addr), ctypes.addressof(buf), mv.nbytes)

  def download(self, addr, nbytes):
    """Device bytes to a new bytearray, after the launches queued before it."""
    self.check()
    out = bytearray(nbytes)
    if nbytes:
      buf = (ctypes.c_char * nbytes).from_buffer(out)
      _lib.call("download", self.handle, ctypes.addressof(buf), int(addr), nbytes)
    return out

  def copy(self, dst, src, nbytes):
    self.check()
    _lib.call("copy", self.handle, int(dst), int(src), int(nbytes))

  def fill32(self, addr, value, words):
    self.check()
    self.launched("fill")
    _lib.call("fill32", self.handle, int(addr), value & 0xFFFFFFFF, int(words))

  # ---- launches
  def launched(self, name, reads=None):
    """Counts a launch, and with timing brackets it by events. Returns a callable that ends the bracket. reads is the
    bytes the launch reads from device memory, as its operands' sizes give them, for profile()."""
    self.launches += 1
    if self.log is not None: self.log.append(name)
    if not self.timing or self.recording is not None: return lambda: None
    start, end = c_void_p(), c_void_p()
    _lib.call("event_create", self.handle, byref(start))
    _lib.call("event_create", self.handle, byref(end))
    _lib.call("event_record", self.handle, start)
    n = self.launches
    def done():
      _lib.call("event_record", self.handle, end)
      self.times.append((n, name, start, end, reads))
    return done

  def run(self, name, fn, *args, reads=None):
    """Queue bt_<fn>(handle, *args), counted as launch `name` that reads `reads` bytes (None: not counted)."""
    self.check()
    done = self.launched(name, reads)
    _lib.call(fn, self.handle, *args)
    done()

  def sleep(self, seconds):
    """Queue a launch that keeps the device busy for `seconds` (at most 10) and then ends by itself."""
    self.check()
    done = self.launched("sleep", 0)
    _lib.call("sleep", self.handle, float(seconds))
    done()

  def wait(self, timeout=60, launch=None):
    """Block until the launches queued so far (launch must be one of them) are done. TimeoutError after timeout
    seconds."""
    self.check()
    if launch is not None and launch > self.launches:
      raise ValueError(f"launch {launch} was never queued; the last one queued is {self.launches}")
    _lib.call("wait", self.handle, float(timeout))

  def profile(self, since=0):
    """Wait, then [(name, launches, microseconds, bytes)] for the timed launches after `since`, grouped by name with
    the longest first (runtime.py:773-786, which reports cycles and the NoC bytes read). Here the time is HIP events
    around each launch, and bytes are what the launches read from device memory by their operands' sizes: algorithmic
    bytes, not a hardware counter. bytes is None for a name none of whose launches counted them."""
    self.wait()
    totals = collections.defaultdict(lambda: [0, 0.0, None])
    for n, name, start, end, reads in self.times:
      if n <= since: continue
      ms = c_float()
      _lib.call("event_elapsed", start, end, byref(ms))
      t = totals[name]
      t[0] += 1
      t[1] += ms.value * 1000
      if reads is not None: t[2] = (t[2] or 0) + int(reads)
    return sorted(((name, n, us, nbytes) for name, (n, us, nbytes) in totals.items()), key=lambda r: -r[2])

  def close(self):
    """Finish queued work and release the stream. The runtime's tensors then raise RuntimeError."""
    if self.closed: return
    self.closed = True
    for _, _, start, end, _ in self.times:
      _lib.call("event_destroy", start)
      _lib.call("event_destroy", end)
    self.times = []
    if self.handle:
      _lib.call("close", self.handle)
      self.handle = None

  def __del__(self):
    try:
      if not self.closed and self.handle: self.close()
    except Exception:
      pass
