"""Tensors on MI355X: baretile's lazy Tensor surface, lowered onto the HIP kernels of libbaretile_amd.so.

Mirrors baretile/tensor.py (Tensor at tensor.py:25, jit at tensor.py:1231) in behaviour, not in mechanism. As there,
operations build a lazy graph, and realize() / tobytes() / tolist() compile and run it: an elementwise tree becomes
one bt_program run by one kernel (tensor.py:466-524), a matmul takes the elementwise tree above it as its epilogue
(kernels.py:41-727), a reduction takes the tree below it as its prologue, and bf16 rounds every intermediate result
half up as the reference's packer does, so fused and unfused give the same bits (test_kernels.py:987-1004).

Unlike the reference's 32x32 tiles in eight DRAM banks, a tensor here is a row-major device buffer read through
strides. Slices, splits, transposes and repeats are views, and any slice shares storage. Block-float tensors hold the
plain exponent and value planes of include/baretile_amd.h, and columns() repacks them into the matmul's tiles.

Tensors have up to five dimensions: up to three leading ones fold into the batch in row-major order (tensor.py:25-35).
"""
import array, ctypes, functools, math, operator, struct, weakref
import numpy as np
from baretile_amd import _lib
from baretile_amd.program import Program

FIDELITY = 4  # the reference's default phase count: exact bf16 products, which the matrix cores always give
DIMS = 5
BFP = ("bfp8", "bfp4")
ITEMSIZE = {"bf16": 2, "fp32": 4, "int32": 4}
DTYPES = (*ITEMSIZE, *BFP)
UNARY = ("neg", "relu", "exp", "exp2", "log", "log2", "sqrt", "recip", "rsqrt", "sin", "cos", "sigmoid", "silu", "gelu",
         "tanh", "ftob")
BINARY = ("add", "sub", "mul", "div", "max", "min", "cmplt", "cmple", "cmpne", "cmpeq")
INT32_OPS = ("add", "sub", "max", "min", "cmplt", "cmple", "cmpne", "cmpeq", "neg", "relu", "where", "mul")
ELEMENTWISE = UNARY + BINARY + ("where", "cast")
REDUCE = ("sum", "amax")


def _shape(shape):
  shape = tuple(operator.index(s) for s in shape)
  if not 1 <= len(shape) <= DIMS or any(s <= 0 for s in shape):
    raise ValueError(f"tensor dimensions must be 1 to {DIMS} positive sizes, not {shape}")
  return (1,) * max(0, 3 - len(shape)) + shape


def _broadcast(a, b):
  """numpy broadcasting of two shapes, or None."""
  n = max(len(a), len(b))
  a, b = (1,) * (n - len(a)) + tuple(a), (1,) * (n - len(b)) + tuple(b)
  out = []
  for x, y in zip(a, b):
    if x != y and 1 not in (x, y): return None
    out.append(max(x, y))
  return tuple(out)


def _bf16_bits(values):
  """float32 -> bf16 bits, nearest even, NaNs kept quiet (the reference's upload rule, tensix.py:240-242)."""
  b = np.asarray(values, np.float32).reshape(-1).view(np.uint32).astype(np.uint64)
  rne = (b + 0x7FFF + (b >> 16 & 1)) >> 16
  nan = (b & 0x7FFFFFFF) > 0x7F800000
  return np.where(nan, (b >> 16) | 0x40, rne).astype(np.uint16)


class Storage:
  """Device memory that tensors share, freed when the last tensor using it goes. Memory allocated while a jit
  recording captures belongs to the recording too, which keeps it for as long as its graph can replay.

  columns caches, per block-float view read as a matmul's B, the tiles columns() made of it; any write into the
  storage (realize into, assign, put) drops them."""
  __slots__ = ("rt", "addr", "nbytes", "columns", "captured", "vals", "__weakref__")

  def __init__(self, rt, nbytes):
    self.rt, self.nbytes, self.columns, self.addr, self.vals = rt, nbytes, {}, None, 0
    self.captured = rt.recording is not None
    self.addr = rt.dram_alloc(max(256, nbytes))
    if self.captured: rt.recording.storages.append(self)

  def __del__(self):
    try:
      if self.addr is not None: self.rt.dram_free(self.addr, self.captured)
    except Exception:
      pass


def _written(storage):
  """Notes a write into storage that its readers' caches must see: cached columns tiles go, and a jit recording learns
  which of its inputs the function writes."""
  storage.columns.clear()
  if storage.rt.written is not None: storage.rt.written.add(id(storage))


def _bytes(*ts):
  """The bytes a kernel reads for these realized tensors' values, as stored: a block float counts its exponents, a
  tensor by columns its tiles. What Runtime.profile reports."""
  n = 0
  for t in ts:
    if t is None: continue
    if t.layout == "columns": n += t.batch * _tiles_bytes(t.rows, t.cols, t.dtype)
    elif t.dtype in BFP: n += t.batch * sum(_planes(t.rows, t.cols, t.dtype))
    else: n += t.batch * t.rows * t.cols * ITEMSIZE[t.dtype]
  return n


def _planes(rows, cols, dtype):
  """(exponent bytes, value bytes) of one plain block-float matrix."""
  runs = -(-cols // 16)
  return rows * runs, rows * runs * (16 if dtype == "bfp8" else 8)


def _tiles_bytes(rows, cols, dtype):
  """Bytes of one matrix in the matmul's columns tiles."""
  tb = {"bf16": 2048, "bfp8": 1088, "bfp4": 576}[dtype]
  return -(-cols // 16) * -(-rows // 64) * tb


class Tensor:
  """A batch of matrices (batch, rows, cols), or up to three leading dimensions in place of the batch. Storage
  formats: bf16, fp32, int32, bfp8, bfp4 (tensor.py:25-35). An unrealized tensor holds an op and its operands; a
  realized one holds storage and the strides it is read through."""
  def __init__(self, rt, rows, cols, op=None, srcs=(), batch=1, dtype="bf16", args=()):
    batch, rows, cols = _shape((batch, rows, cols))
    if dtype not in DTYPES: raise ValueError(f"unknown tensor dtype: {dtype}")
    if any(isinstance(s, Tensor) and s.rt is not rt for s in srcs):
      raise ValueError("tensor operands must use the same runtime")
    rt.check()
    self.rt, self.rows, self.cols, self.batch, self.dtype = rt, rows, cols, batch, dtype
    self.op, self.srcs, self.args, self.lead = op, tuple(srcs), args, (batch,)
    self.storage, self.offset, self.sb, self.sr, self.sc, self.rep, self.cyc = None, 0, 0, 0, 0, 1, 0
    self.layout = "plain"
    self.requires_grad, self.grad = False, None
    if op is None: self._alloc()

  # ---- storage
  def _alloc(self, layout="plain"):
    self.layout = layout
    if self.dtype in BFP:
      if layout == "columns": n = self.batch * _tiles_bytes(self.rows, self.cols, self.dtype)
      else:
        e, v = _planes(self.rows, self.cols, self.dtype)
        n = -(-self.batch * e // 256) * 256 + self.batch * v
    elif layout == "columns": n = self.batch * _tiles_bytes(self.rows, self.cols, "bf16")
    else: n = self.batch * self.rows * self.cols * ITEMSIZE[self.dtype]
    self.storage = Storage(self.rt, n)
    if self.dtype in BFP and layout == "plain":  # the value plane follows the exponent plane, 256-byte aligned
      self.storage.vals = -(-self.batch * _planes(self.rows, self.cols, self.dtype)[0] // 256) * 256
    self.offset, self.sb, self.sr, self.sc = 0, self.rows * self.cols, self.cols, 1
    self.rep, self.cyc = 1, 0
    return self

  @property
  def addr(self): return None if self.storage is None else self.storage.addr + self.offset * self.itemsize

  @property
  def itemsize(self): return ITEMSIZE.get(self.dtype, 1)

  def _bfp_planes(self):
    """(exponent plane, value plane) addresses of element (0, 0, 0) of a plain block-float tensor or view: a value's
    exponent byte sits at its index / 16, its q at its index (bfp8) or index / 2 (bfp4); offsets count values."""
    base = self.storage.addr
    return base + self.offset // 16, base + self.storage.vals + (self.offset if self.dtype == "bfp8" else self.offset // 2)

  def _bfp_whole(self):  # a plain block float read as whole, contiguous matrices (for re-laying by columns)
    if not self._contiguous():
      raise ValueError("a block-float view lays out by columns only as whole, contiguous matrices")
    return self

  def _unpacked(self, why):
    """A realized plain block float's values as a new bf16 tensor of its shape, exactly as the unpacker decodes them
    (tensor.py:1093-1104). A view that isn't whole, contiguous matrices is read through its storage unpacked whole:
    its runs are whole runs of the storage (_view keeps them so), so each value sits at the same index there."""
    fmt = _lib.DTYPES[self.dtype]
    if self._contiguous():
      out = Tensor(self.rt, self.rows, self.cols, batch=self.batch, dtype="bf16")
      e, v = self._bfp_planes()
      self.rt.run(why, "bfp_unpack", fmt, e, v, self.batch, self.rows, self.cols, out.storage.addr,
                  reads=_bytes(self))
    else:
      s = self.storage
      n = (s.nbytes - s.vals) * (1 if self.dtype == "bfp8" else 2)  # every value the storage holds
      flat = Tensor(self.rt, n // 16, 16, dtype="bf16")
      self.rt.run(why, "bfp_unpack", fmt, s.addr, s.addr + s.vals, 1, n // 16, 16, flat.storage.addr,
                  reads=s.nbytes)
      out = flat._view(self.rows, self.cols, self.batch, self.offset, self.sb, self.sr, self.sc, self.rep,
                       self.cyc)._copy()
    out.lead = self.lead
    return out

  @property
  def shape(self): return (*self.lead, self.rows, self.cols)

  @property
  def _dims(self): return (self.batch, self.rows, self.cols)

  @property
  def tiles(self): return self.batch * -(-self.rows // 32) * -(-self.cols // 32)  # for code that sizes work in tiles

  def _relabel(self, lead):
    lead = tuple(lead)
    if lead == self.lead: return self
    if math.prod(lead) != self.batch: raise ValueError(f"leading sizes {lead} don't fold into a batch of {self.batch}")
    t = self._copy_header()
    t.lead = lead
    return t

  def _copy_header(self):
    t = Tensor.__new__(Tensor)
    t.__dict__.update(self.__dict__)
    return t

  def _operand(self, out_lead=None, out_rows=None, out_cols=None, expand=True):
    """The bt_operand that reads this realized tensor at the result's (batch, row, col), broadcasting dimensions of
    one. The batch maps through rep and cyc where this tensor's leading sizes are one run of the result's, as the
    reference's spread views do (tensor.py:265-279); other patterns are expanded by a copy first."""
    if self.storage is None or self.dtype in BFP or self.layout != "plain":
      raise ValueError("only a realized bf16, fp32 or int32 tensor is read elementwise")
    out_lead = self.lead if out_lead is None else tuple(out_lead)
    sr = 0 if (out_rows or self.rows) != self.rows and self.rows == 1 else self.sr
    sc = 0 if (out_cols or self.cols) != self.cols and self.cols == 1 else self.sc
    mine = (1,) * (len(out_lead) - len(self.lead)) + self.lead
    if len(mine) > len(out_lead) or any(m not in (1, o) for m, o in zip(mine, out_lead)):
      if self.batch == math.prod(out_lead):  # the same matrices under other leading sizes
        return _lib.Operand(self.addr, self.sb, sr, sc, _lib.DTYPES[self.dtype], self.rep, self.cyc, 0)
      raise ValueError(f"cannot read {self.shape} as {out_lead}")
    big = [k for k, n in enumerate(mine) if n > 1]
    if not big:  # one matrix for every batch entry
      return _lib.Operand(self.addr, 0, sr, sc, _lib.DTYPES[self.dtype], 1, 0, 0)
    if mine == out_lead:
      return _lib.Operand(self.addr, self.sb, sr, sc, _lib.DTYPES[self.dtype], self.rep, self.cyc, 0)
    if big != list(range(big[0], big[-1] + 1)) or self.rep != 1 or self.cyc != 0:
      if not expand: raise ValueError(f"{self.shape} is not one run of {out_lead}")
      return self.expand(*out_lead, self.rows, self.cols)._operand(out_lead, out_rows, out_cols)
    rep = math.prod(out_lead[big[-1] + 1:])
    cyc = math.prod(mine[big[0]:big[-1] + 1]) if big[0] > 0 else 0
    return _lib.Operand(self.addr, self.sb, sr, sc, _lib.DTYPES[self.dtype], rep, cyc, 0)

  # ---- construction and transfer
  @classmethod
  def full(cls, rt, rows, cols, value, dtype="bf16"): return cls.of(rt, [[value] * cols for _ in range(rows)], dtype)

  @classmethod
  def zeros(cls, rt, rows, cols, batch=1, dtype="bf16"):
    """A tensor of zeros in any storage format, written on the device (kernels.py:1436-1453)."""
    t = cls(rt, rows, cols, batch=batch, dtype=dtype)
    rt.fill32(t.storage.addr, 0, -(-t.storage.nbytes // 4))
    return t

  @classmethod
  def of(cls, rt, data, dtype="bf16"):
    """A tensor from rows of numbers, a list of those for a batch, nested again for each leading dimension
    (tensor.py:103-121). bf16 rounds to nearest even."""
    if dtype in BFP: return cls.of(rt, data, "bf16").cast(dtype)
    if dtype not in ITEMSIZE: raise ValueError(f"unknown tensor dtype: {dtype}")
    if isinstance(data, np.ndarray): a = data
    else:
      if not len(data) or not len(data[0]): raise ValueError("tensor data must be nonempty")
      try: a = np.array(data, dtype=np.int64 if dtype == "int32" else np.float64)
      except ValueError: raise ValueError("tensor data must be nonempty rectangular matrices of the same shape") from None
      if a.dtype == object: raise ValueError("tensor data must be rectangular")
    if a.ndim < 2 or a.ndim > DIMS or a.size == 0: raise ValueError(f"tensor data must have 2 to {DIMS} dimensions")
    shape = a.shape
    if dtype == "bf16": raw = _bf16_bits(a.astype(np.float32))
    elif dtype == "fp32": raw = a.astype(np.float32).reshape(-1)
    else: raw = a.astype(np.int64).astype(np.int32).reshape(-1)
    lead = shape[:-2] or (1,)
    t = cls.frombytes(rt, shape[-2], shape[-1], raw.tobytes(), math.prod(lead), dtype)
    return t._relabel(lead) if len(shape) > 3 else t

  @classmethod
  def frombytes(cls, rt, rows, cols, data, batch=1, dtype="bf16"):
    """Upload little-endian values in row-major order, matrices one after another (tensor.py:113-135)."""
    if dtype in BFP: raise ValueError("upload as bf16, then cast on the device to a block-float format")
    if dtype not in ITEMSIZE: raise ValueError(f"unknown tensor dtype: {dtype}")
    batch, rows, cols = _shape((batch, rows, cols))
    data = memoryview(data).cast("B")
    if len(data) != ITEMSIZE[dtype] * batch * rows * cols:
      raise ValueError(f"{len(data)} bytes for {batch} x {rows} x {cols} of {dtype}")
    t = cls(rt, rows, cols, batch=batch, dtype=dtype)
    rt.upload(t.storage.addr, data)
    return t

  def tobytes(self):
    """Row-major bytes in the format frombytes takes; block floats come back as bf16, exactly as the unpacker
    decodes them (tensor.py:159-192)."""
    t = self.realize()
    if t.layout == "columns":
      out = Tensor(self.rt, t.rows, t.cols, batch=t.batch, dtype="bf16")
      self.rt.run("readback", "columns_unpack", _lib.DTYPES[t.dtype], t.storage.addr, t.batch, t.rows, t.cols,
                  out.storage.addr, reads=_bytes(t))
      t = out
    elif t.dtype in BFP:
      t = t._unpacked("readback")
    if not t._contiguous(): t = t._copy()
    return bytes(self.rt.download(t.addr, t.batch * t.rows * t.cols * t.itemsize))

  def tolist(self):
    raw = self.tobytes()
    if self.dtype == "int32": a = np.frombuffer(raw, np.int32).astype(np.int64)
    elif self.dtype == "fp32": a = np.frombuffer(raw, np.float32).astype(np.float64)
    else: a = (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    a = a.reshape(self.shape)
    return a.tolist() if len(self.lead) > 1 or self.batch > 1 else a[0].tolist()

  def numpy(self):  # the values as a NumPy array of the tensor's shape (float64 for floats)
    return np.array(self.tolist()).reshape(self.shape)

  def _contiguous(self):
    return (self.storage is not None and self.layout == "plain" and self.sc == 1 and self.sr == self.cols and
            (self.batch == 1 or self.sb == self.rows * self.cols) and self.rep == 1 and self.cyc == 0)

  # ---- views
  def _view(self, rows, cols, batch, offset, sb, sr, sc, rep=1, cyc=0):
    t = self.realize()
    whole_runs = t.dtype in BFP and cols % 16 == 0 and sc == 1 and offset % 16 == 0 and sr % 16 == 0 and sb % 16 == 0
    if t.layout != "plain" or (t.dtype in BFP and not whole_runs):
      raise ValueError("a tensor by columns can only be a matmul's B, read back, or cast; a block-float view keeps "
                       "whole runs of 16 along its rows")
    v = Tensor.__new__(Tensor)
    v.__dict__.update(t.__dict__)
    v.rows, v.cols, v.batch, v.lead = rows, cols, batch, (batch,)
    v.offset, v.sb, v.sr, v.sc, v.rep, v.cyc = offset, sb, sr, sc, rep, cyc
    v.op, v.srcs, v.args = None, (), ()
    return v

  def __getitem__(self, key):
    """x[b] selects a batch entry (or the first leading index); x[rows, cols] and x[batch, rows, cols] slice with any
    steps. Every slice is a view (tensor.py:281-305)."""
    t = self.realize() if self.op is not None else self
    if len(t.lead) > 1:
      flat = t._relabel((t.batch,))
      if isinstance(key, int):
        n = t.lead[0]
        if not -n <= key < n: raise IndexError(f"index {key} outside a leading size of {n}")
        per = t.batch // n
        return flat[key % n * per:(key % n + 1) * per, :, :]._relabel(t.lead[1:] if len(t.lead) > 2 else (per,))
      if isinstance(key, tuple) and len(key) == len(t.shape) and all(isinstance(k, slice) for k in key):
        idx = np.arange(t.batch).reshape(t.lead)[key[:-2]]
        picked = idx.reshape(-1)
        steps = set(np.diff(picked).tolist())
        if len(steps) <= 1 and min(steps, default=1) > 0:
          step = min(steps, default=1)
          v = flat[int(picked[0]):int(picked[-1]) + 1:step, key[-2], key[-1]]
          return v._relabel(idx.shape)
        return t.contiguous()[key]
      key = key if isinstance(key, tuple) else (key,)
      if len(key) < len(t.shape): return t[key + (slice(None),) * (len(t.shape) - len(key))]
      raise ValueError(f"index {t.shape} with an int or one slice per dimension, not {key!r}")
    if isinstance(key, int):
      if not -t.batch <= key < t.batch: raise IndexError(f"batch index {key} outside a batch of {t.batch}")
      key %= t.batch
      m = (key // t.rep) % t.cyc if t.cyc else key // t.rep
      return t._view(t.rows, t.cols, 1, t.offset + m * t.sb, 0, t.sr, t.sc)
    if not (isinstance(key, tuple) and len(key) in (2, 3) and all(isinstance(k, slice) for k in key)):
      raise ValueError(f"index a tensor as x[b], x[rows, cols] or x[batch, rows, cols] with slices, not x[{key!r}]")
    key = (slice(None),) * (3 - len(key)) + tuple(key)
    ranges = [range(*k.indices(n)) for k, n in zip(key, t._dims)]
    if not all(len(r) for r in ranges): raise ValueError(f"an empty slice of {t.shape}")
    b, r, c = ranges
    if (t.rep != 1 or t.cyc) and (b.step != 1 or len(b) != t.batch): t = t.contiguous()
    if t.rep != 1 or t.cyc:
      return t._view(len(r), len(c), len(b), t.offset + r.start * t.sr + c.start * t.sc, t.sb, t.sr * r.step,
                     t.sc * c.step, t.rep, t.cyc)
    return t._view(len(r), len(c), len(b), t.offset + b.start * t.sb + r.start * t.sr + c.start * t.sc,
                   t.sb * b.step, t.sr * r.step, t.sc * c.step)

  def split(self, n, axis=2):
    """n equal parts along columns (axis 2) or rows (axis 1), as a batch, without copying (tensor.py:426-450)."""
    n, axis = operator.index(n), operator.index(axis)
    if n <= 0: raise ValueError("split needs a positive number of parts")
    if len(self.shape) > 3: raise ValueError(f"split takes three dimensions, not {self.shape}")
    t = self.realize()
    if axis == 2:
      if t.batch != 1 or t.cols % n: raise ValueError("split needs batch 1 and equal parts")
      w = t.cols // n
      return t._view(t.rows, w, n, t.offset, w * t.sc, t.sr, t.sc)
    if axis != 1: raise ValueError(f"split cuts columns (axis 2) or rows (axis 1), not axis {axis}")
    if t.rows % n: raise ValueError("split along rows needs equal parts")
    h = t.rows // n
    if t.batch == 1: return t._view(h, t.cols, n, t.offset, h * t.sr, t.sr, t.sc)
    if t.sb != t.rows * t.sr or t.rep != 1 or t.cyc: t = t.contiguous()
    return t._view(h, t.cols, t.batch * n, t.offset, h * t.sr, t.sr, t.sc)

  def merge(self):
    """Batch matrices side by side, the inverse of split (tensor.py:452-461): the expression (or a copy) is written
    straight into the result's columns."""
    if len(self.shape) > 3: raise ValueError(f"merge takes three dimensions, not {self.shape}")
    out = Tensor(self.rt, self.rows, self.batch * self.cols, dtype=self.dtype)
    (self if self.op is not None else self._copy_op()).realize(out.split(self.batch))
    return out

  def repeat_interleave(self, n):
    """Each matrix n times along the batch, read in place: matrix b reads stored matrix b // n (tensor.py:414-424)."""
    if len(self.shape) > 3: raise ValueError(f"repeat_interleave takes three dimensions, not {self.shape}")
    t = self.realize()
    if t.rep != 1 or t.cyc: t = t.contiguous()
    return t._view(t.rows, t.cols, t.batch * n, t.offset, t.sb, t.sr, t.sc, rep=n)

  @property
  def T(self):
    """Each matrix transposed, as a view (a matmul reads it as B without a copy)."""
    t = self.realize()
    if t.dtype in BFP or t.layout != "plain": raise ValueError("cast a block float to bf16 to transpose it")
    v = t._view(t.cols, t.rows, t.batch, t.offset, t.sb, t.sc, t.sr, t.rep, t.cyc)
    v.lead = t.lead
    return v

  def contiguous(self):
    return self if self.op is None and self._contiguous() else self._copy()

  def _copy(self):
    t = self.realize()
    out = Tensor(self.rt, t.rows, t.cols, batch=t.batch, dtype=t.dtype)
    out.lead = t.lead
    (t._copy_op()).realize(out)
    return out

  def _copy_op(self):  # an unrealized identity of this tensor: a cast to its own dtype
    t = Tensor(self.rt, self.rows, self.cols, "cast", (self,), self.batch, self.dtype)
    t.lead = self.lead
    return t

  def reshape(self, *shape):
    """Up to five sizes; missing leading sizes are 1. A reshape of a row-major tensor is a view."""
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)): shape = tuple(shape[0])
    full = _shape(shape)
    if math.prod(full) != math.prod(self.shape): raise ValueError(f"cannot reshape {self.shape} to {shape}")
    lead = full[:-2] if len(shape) > 3 else (full[0],)
    if tuple(full[-2:]) == (self.rows, self.cols): return self._relabel(lead)
    t = self.realize()
    if not t._contiguous(): t = t._copy()
    v = t._view(full[-2], full[-1], math.prod(full[:-2]), t.offset, full[-2] * full[-1], full[-1], 1)
    v.lead = lead
    return v

  def permute(self, *order):
    n = len(self.shape)
    if sorted(order) != list(range(n)): raise ValueError(f"permute needs an order of the axes 0 to {n - 1}, not {order}")
    if tuple(order) == tuple(range(n)): return self
    t = self.realize()
    if n == 3:
      strides = {0: (t.batch, t.sb), 1: (t.rows, t.sr), 2: (t.cols, t.sc)}
      if t.rep != 1 or t.cyc or (t.batch > 1 and t.sb == 0): t = t.contiguous(); strides = {0: (t.batch, t.sb), 1: (t.rows, t.sr), 2: (t.cols, t.sc)}
      (b, sb), (r, sr), (c, sc) = (strides[k] for k in order)
      return t._view(r, c, b, t.offset, sb, sr, sc)
    # more dimensions: through NumPy on the host would defeat the point; copy the leading axes apart by matrix
    src = t.contiguous()
    lead = src.lead
    axes = list(src.shape)
    out_shape = tuple(axes[k] for k in order)
    out = Tensor(self.rt, out_shape[-2], out_shape[-1], batch=math.prod(out_shape[:-2]), dtype=src.dtype)._relabel(out_shape[:-2])
    strides = [0] * n
    s = 1
    for k in range(n - 1, -1, -1): strides[k] = s; s *= axes[k]
    for idx in np.ndindex(*out_shape[:-2]):
      src_off = sum(i * strides[order[k]] for k, i in enumerate(idx))
      view = src._view(out_shape[-2], out_shape[-1], 1, src.offset + src_off, 0, strides[order[-2]], strides[order[-1]])
      dst = out._relabel((out.batch,))[int(np.ravel_multi_index(idx, out_shape[:-2]))]
      view._copy_op().realize(dst)
    return out

  def expand(self, *shape):
    shape = _shape(shape)
    if _broadcast(self.shape, shape) != shape: raise ValueError(f"cannot expand {self.shape} to {shape}")
    if shape == self.shape: return self
    out = Tensor(self.rt, shape[-2], shape[-1], batch=math.prod(shape[:-2]), dtype=self.dtype)._relabel(shape[:-2])
    src = self.realize()
    try:
      _run_copy(self.rt, src._operand(shape[:-2], shape[-2], shape[-1], expand=False), src.dtype, out)
    except ValueError:  # leading sizes that aren't one run of the result's: a copy per result matrix
      mine = (1,) * (len(shape) - 2 - len(src.lead)) + src.lead
      flat = src._relabel((src.batch,)) if len(src.lead) > 1 else src
      for b, idx in enumerate(np.ndindex(*shape[:-2])):
        m = int(np.ravel_multi_index(tuple(i if n > 1 else 0 for i, n in zip(idx, mine)), mine))
        dst = out._relabel((out.batch,))[b]
        _run_copy(self.rt, flat[m]._operand((1,), shape[-2], shape[-1]), src.dtype, dst)
    return out

  def pad(self, widths):
    """Zeros around, with (before, after) for each of the last len(widths) axes, as NumPy's pad."""
    widths = tuple(tuple(map(operator.index, w)) for w in widths)
    n = len(self.shape)
    if len(widths) > n or any(len(w) != 2 for w in widths): raise ValueError("pad needs (before, after) pairs")
    widths = ((0, 0),) * (n - len(widths)) + widths
    shape = tuple(m + a + b for m, (a, b) in zip(self.shape, widths))
    out = Tensor.zeros(self.rt, shape[-2], shape[-1], batch=math.prod(shape[:-2]), dtype=self.dtype)._relabel(shape[:-2])
    key = tuple(slice(a, a + m) for m, (a, _) in zip(self.shape, widths))
    out[key].assign(self)
    return out

  def cat(self, *xs, axis=0):
    ts = (self, *xs)
    n = len(self.shape)
    axis = operator.index(axis) % n
    if not all(len(t.shape) == n and all(t.shape[a] == self.shape[a] for a in range(n) if a != axis) for t in ts):
      raise ValueError("cat requires matching dimensions outside its axis")
    shape = list(self.shape)
    shape[axis] = sum(t.shape[axis] for t in ts)
    out = Tensor(self.rt, shape[-2], shape[-1], batch=math.prod(shape[:-2]), dtype=self.dtype)._relabel(tuple(shape[:-2]))
    at = 0
    for t in ts:
      key = tuple(slice(at, at + t.shape[a]) if a == axis else slice(None) for a in range(n))
      out[key].assign(t)
      at += t.shape[axis]
    return out

  # ---- elementwise
  def _new(self, op, srcs, shape, dtype, args=()):
    lead, rows, cols = shape[:-2], shape[-2], shape[-1]
    t = Tensor(self.rt, rows, cols, op, srcs, math.prod(lead) if lead else 1, dtype, args)
    t.lead = tuple(lead) if lead else (1,)
    return t

  def _unary(self, op):
    if self.dtype == "int32" and op not in ("relu", "neg"): return self.float()._unary(op)
    if self.dtype in BFP: return self.cast("bf16")._unary(op)
    return self._new(op, (self,), self.shape, self.dtype)

  def _binop(self, op, x, reverse=False):
    """NumPy broadcasting; a number takes this tensor's dtype (fp32 for a float with int32); mixed dtypes meet in
    fp32, as int32 does for ops without an int32 form (tensor.py:567-579)."""
    a = self.cast("bf16") if self.dtype in BFP else self
    if isinstance(x, Tensor):
      b = x.cast("bf16") if x.dtype in BFP else x
      if b.rt is not a.rt: raise ValueError("tensor operands must use the same runtime")
      dtype = a.dtype if a.dtype == b.dtype else "fp32"
      shape = _broadcast(a.shape, b.shape)
      if shape is None: raise ValueError(f"cannot broadcast {a.shape} with {b.shape}")
    else:
      if not isinstance(x, (int, float)): raise ValueError(f"cannot combine a tensor with {type(x).__name__}")
      dtype = "fp32" if a.dtype == "int32" and isinstance(x, float) else a.dtype
      shape, b = a.shape, x
    if dtype == "int32" and op not in INT32_OPS: dtype = "fp32"
    srcs = (b, a) if reverse else (a, b)
    return self._new(op, srcs, shape, dtype)

  def cast(self, dtype):
    """To another storage format. bf16 rounds half up as a packed result does; bfp8/bfp4 round as gpt2.bfp does
    (models/gpt2.py:19-30) and are made now (tensor.py:581-596)."""
    if dtype not in DTYPES: raise ValueError(f"unknown tensor dtype: {dtype}")
    if dtype == self.dtype and self.layout == "plain": return self
    if self.dtype in BFP or self.layout == "columns":
      x = self.realize()
      if x.layout == "columns":
        out = Tensor(self.rt, x.rows, x.cols, batch=x.batch, dtype="bf16")
        out.lead = x.lead
        self.rt.run("storage", "columns_unpack", _lib.DTYPES[x.dtype], x.storage.addr, x.batch, x.rows, x.cols,
                    out.storage.addr, reads=_bytes(x))
      else:
        out = x._unpacked("storage")
      return out.cast(dtype)
    if dtype in BFP:
      x = self if self.dtype in ("bf16", "fp32") else self.float()
      x = x.realize()
      if x.rep != 1 or x.cyc: x = x.contiguous()
      out = Tensor(self.rt, x.rows, x.cols, batch=x.batch, dtype=dtype)
      out.lead = x.lead
      e, v = out._bfp_planes()
      self.rt.run("cast", "bfp_pack", _lib.DTYPES[dtype], x.addr, _lib.DTYPES[x.dtype], x.batch, x.rows, x.cols,
                  x.sb, x.sr, x.sc, e, v, reads=_bytes(x))
      return out
    return self._new("cast", (self,), self.shape, dtype)

  def columns(self):
    """B for a matmul laid out in its tiles, once (tensor.py:597-611). Reads back unchanged; other operations need a
    cast to bf16 first."""
    if len(self.shape) > 3: raise ValueError(f"columns takes three dimensions, not {self.shape}")
    if self.dtype not in ("bf16", *BFP):
      raise ValueError(f"columns lays out a matmul's B, which is bf16 or a block float, not {self.dtype}")
    x = self.realize()
    if x.layout == "columns": return x
    out = Tensor(self.rt, x.rows, x.cols, "view", (), x.batch, x.dtype)
    out.op = None
    out._alloc("columns")
    out.lead = x.lead
    if x.dtype in BFP:
      e, v = x._bfp_whole()._bfp_planes()
      # a matmul reads exponents in a narrower range than a block float can hold: checked now, or, inside a jit
      # recording (which can't read the count back), by the jit before each replay
      if self.rt.recording is None: _check_range(x)
      else: self.rt.recording.unchecked.add(id(x.storage))
      self.rt.run("columns", "bfp_columns", _lib.DTYPES[x.dtype], e, v, x.batch, x.rows, x.cols, out.storage.addr,
                  reads=_bytes(x))
    else:
      if x.rep != 1 or x.cyc: x = x.contiguous()
      self.rt.run("columns", "bf16_columns", x.addr, x.batch, x.rows, x.cols, x.sb, x.sr, x.sc, out.storage.addr,
                  reads=_bytes(x))
    return out

  def float(self): return self.cast("fp32")
  def bfloat16(self): return self.cast("bf16")
  def exp2(self): return self._unary("exp2")
  def log2(self): return self._unary("log2")
  def sin(self): return self._unary("sin")
  def cos(self): return self._unary("cos")
  def sqrt(self): return self._unary("sqrt")
  def reciprocal(self): return self._unary("recip")
  def exp(self): return self._unary("exp")
  def log(self): return self._unary("log")
  def relu(self): return self._unary("relu")
  def tanh(self): return self._unary("tanh")
  def rsqrt(self): return self.sqrt().reciprocal()
  def sigmoid(self): return (1 + (-self).exp()).reciprocal()
  def silu(self): return self * self.sigmoid()
  def gelu(self):  # GPT-2's tanh form, as x / (1 + e^-2z) (tensor.py:654-657)
    k = 2 * math.sqrt(2 / math.pi)
    return self * (1 + (self * (self * self * (-0.044715 * k) - k)).exp()).reciprocal()
  def maximum(self, x): return self._binop("max", x)
  def minimum(self, x): return self._binop("min", x)
  def where(self, x, y):
    """x where this tensor isn't 0, else y, keeping the selected value's bits (tensor.py:614-620)."""
    xs = [v for v in (x, y) if isinstance(v, Tensor)]
    dtype = xs[0].dtype if xs else self.dtype
    shape = self.shape
    for v in xs:
      shape = _broadcast(shape, v.shape)
      if shape is None: raise ValueError("where's operands must broadcast")
    return self._new("where", (self, x, y), shape, dtype if all(v.dtype == dtype for v in xs) else "fp32")
  def __add__(self, x): return self._binop("add", x)
  def __sub__(self, x): return self._binop("sub", x)
  def __mul__(self, x): return self._binop("mul", x)
  def __rsub__(self, x): return self._binop("sub", x, True)
  __radd__, __rmul__ = __add__, __mul__
  def __truediv__(self, x): return self * (1 / x if isinstance(x, (int, float)) else x.reciprocal())
  def __rtruediv__(self, x): return self.reciprocal() * x
  def __neg__(self): return 0 - self if self.dtype == "int32" else self * -1
  def __lt__(self, x): return self._binop("cmplt", x)
  def __gt__(self, x): return self._binop("cmplt", x, True)
  def __ge__(self, x): return self._binop("cmple", x, True)
  def __le__(self, x): return self._binop("cmple", x)
  def ne(self, x): return self._binop("cmpne", x)
  def eq(self, x): return self._binop("cmpeq", x)
  __ne__, __eq__ = ne, eq
  def __hash__(self): return id(self)

  def __bool__(self):
    if math.prod(self.shape) != 1: raise ValueError("the truth value of a tensor with more than one element is ambiguous")
    return bool(self.reshape(1, 1).tolist()[0][0])

  # ---- reductions
  def sum(self, axis=None): return self._reduce("sum", axis)
  def max(self, axis=None): return self._reduce("amax", axis)

  def _reduce(self, f, axis):
    """Reduce like NumPy with keepdims: over a leading dimension, rows (-2), columns (-1), or everything (None)
    (tensor.py:659-676). Sums accumulate in fp32."""
    n = len(self.shape)
    if self.dtype in BFP: return self.cast("bf16")._reduce(f, axis)
    if self.dtype == "int32" and f == "sum": return self.float()._reduce(f, axis).cast("int32")
    if axis is None:
      x = self._relabel((self.batch,))._reduce(f, 0)._reduce(f, 1)._reduce(f, 2)
      return x._relabel((1,) * len(self.lead)) if len(self.lead) > 1 else x
    axis = operator.index(axis)
    if not -n <= axis < n: raise ValueError(f"axis {axis} outside {self.shape}")
    axis %= n
    shape = list(self.shape)
    if shape[axis] == 1: return self
    shape[axis] = 1
    return self._new(f, (self,), tuple(shape), self.dtype, (axis,))

  def mean(self, axis=None):
    s = self.sum(axis)
    return s * (math.prod(s.shape) / math.prod(self.shape))

  def softmax(self, axis=-1):  # max first, so exp stays in range
    e = (self - self.max(axis)).exp()
    return e / e.sum(axis)

  def log_softmax(self, axis=-1):
    m = self - self.max(axis)
    return m - m.exp().sum(axis).log()

  def layernorm(self, axis=-1, eps=1e-5):
    c = self - self.mean(axis)
    return c * ((c * c).mean(axis) + eps).rsqrt()

  # ---- matmul
  def __matmul__(self, x): return self.matmul(x)

  def matmul(self, x, dtype=None, fidelity=None, index=None):
    """Batched matrix product with fp32 sums (tensor.py:737-795). x may be bf16, a block float, or laid out by
    columns. fp32 operands split into bf16 high and low parts, whose three products add in fp32 (tensor.py:775-777).
    Every product is exact, whatever fidelity asks for."""
    if index is not None: raise ValueError("matmul by index (mixture of experts) is outside this backend's scope")
    fidelity = FIDELITY if fidelity is None else operator.index(fidelity)
    if not 1 <= fidelity <= 4: raise ValueError("matmul fidelity must be between one and four phases")
    if not isinstance(x, Tensor) or x.rt is not self.rt: raise ValueError("matmul operands must use the same runtime")
    if len(self.shape) > 3 or len(x.shape) > 3:
      lead = _broadcast(self.lead, x.lead)
      if lead is None: raise ValueError(f"matmul needs leading sizes that broadcast: {self.shape} @ {x.shape}")
      a = self if self.lead == lead else self.expand(*lead, self.rows, self.cols)
      b = x if x.lead == lead or x.batch == 1 else x.expand(*lead, x.rows, x.cols)
      return a._relabel((a.batch,)).matmul(b._relabel((b.batch,)), dtype, fidelity)._relabel(lead)
    if dtype == "int32": return self.matmul(x, "fp32", fidelity).cast("int32")
    if "int32" in (self.dtype, x.dtype): raise ValueError(f"matmul needs floats: {self.dtype} @ {x.dtype}")
    if not (self.cols == x.rows and (self.batch == x.batch or 1 in (self.batch, x.batch))):
      raise ValueError(f"matmul needs A's columns to match B's rows, and batches that match or broadcast: "
                       f"{self.shape} @ {x.shape}")
    dtype = dtype or ("fp32" if "fp32" in (self.dtype, x.dtype) else "bf16")
    if dtype not in ("bf16", "fp32"): raise ValueError(f"a matmul writes bf16 or fp32, not {dtype}")
    if self.dtype == "fp32" or x.dtype == "fp32":
      ah, al = _parts(self)
      bh, bl = _parts(x)
      out = ah.matmul(bh, "fp32")
      for p, q in ((ah, bl), (al, bh)):
        if p is not None and q is not None: out = out + p.matmul(q, "fp32")
      return out.cast(dtype)
    a = self.cast("bf16") if self.dtype in BFP else self
    return a._new("matmul", (a, x), (max(a.batch, x.batch), a.rows, x.cols), dtype)

  def matmul_row(self, w, dtype="bf16", norm=None, eps=1e-5, swiglu=False, residual=None, rope=None):
    """The product of one row with w (by columns) in one kernel, with the operation before it fused (the decode step
    of llama.py's layer at batch 1, llama.py:106-130; bt_matmul_row): with norm, the RMSNorm of self (an fp32 row,
    rounded to bf16 first) scaled by norm (bf16); with swiglu, silu(gate) * up of self (a bf16 row holding the gate
    then the up half); else self (bf16). residual, an fp32 row, is added to the fp32 sum. The row may be any tensor
    whose values lie contiguous in memory (an attention output of one row, say). Returns a (1, n) row of dtype.

    rope, (cos, sin, cache, places, heads, kv): the bf16 product then goes through rope_put's RoPE and cache put in
    the same kernel (bt_matmul_row_rope; with norm, no residual), and the query heads come back as rope_put returns
    them."""
    if rope is not None:
      return self._matmul_row_rope(w, norm, eps, *rope)
    if dtype not in ("bf16", "fp32"): raise ValueError(f"matmul_row writes bf16 or fp32, not {dtype}")
    if not isinstance(w, Tensor) or w.rt is not self.rt or w.layout != "columns" or w.batch != 1:
      raise ValueError("matmul_row needs w laid out by columns, batch 1, on the same runtime")
    a = self.realize()
    kind = _lib.ROW_RMS if norm is not None else _lib.ROW_SWIGLU if swiglu else _lib.ROW_PLAIN
    size = a.batch * a.rows * a.cols
    k = size // 2 if swiglu else size
    want = "fp32" if norm is not None else "bf16"
    flat = a._contiguous() or (a.rows == 1 and a.sc == 1 and a.sb == a.cols and a.rep == 1 and a.cyc == 0)
    if not (a.dtype == want and flat and a.layout == "plain" and k == w.rows and (not swiglu or size == 2 * k)):
      raise ValueError(f"matmul_row needs a contiguous {want} row of {w.rows} values{' (twice, gate then up)' if swiglu else ''}: "
                       f"{a.shape} {a.dtype}")
    nw = None
    if norm is not None:
      nw = norm.realize()
      if not (nw.dtype == "bf16" and nw._contiguous() and nw.batch * nw.rows * nw.cols == k):
        raise ValueError(f"matmul_row's norm weights must be a contiguous bf16 row of {k}: {nw.shape} {nw.dtype}")
    res = None
    if residual is not None:
      res = residual.realize()
      if not (res.dtype == "fp32" and res._contiguous() and res.batch * res.rows * res.cols == w.cols):
        raise ValueError(f"matmul_row's residual must be a contiguous fp32 row of {w.cols}: {res.shape} {res.dtype}")
    out = Tensor(self.rt, 1, w.cols, dtype=dtype)
    args = _lib.RowArgs(a.addr, nw.addr if nw is not None else 0, res.addr if res is not None else 0, out.addr,
                        w.storage.addr, k, w.cols, kind, _lib.DTYPES[w.dtype], _lib.DTYPES[dtype], eps)
    self.rt.run("matmul_row", "matmul_row", ctypes.byref(args), reads=_bytes(a, w, nw, res))
    return out

  def _matmul_row_rope(self, w, norm, eps, cos, sin, cache, places, heads, kv):
    a, nw = self.realize(), norm.realize() if norm is not None else None
    c, sn, cc, pl = cos.realize(), sin.realize(), cache.realize(), places.realize()
    nh = heads + 2 * kv
    if nw is None or not isinstance(w, Tensor) or w.layout != "columns" or w.batch != 1 or w.cols % nh:
      raise ValueError("matmul_row with rope needs the norm and w by columns, (heads + 2 kv) heads wide")
    d = w.cols // nh
    if not (a.dtype == "fp32" and a._contiguous() and a.batch * a.rows * a.cols == w.rows):
      raise ValueError(f"matmul_row with rope needs a contiguous fp32 row of {w.rows}: {a.shape} {a.dtype}")
    if not (nw.dtype == "bf16" and nw._contiguous() and nw.batch * nw.rows * nw.cols == w.rows):
      raise ValueError(f"matmul_row's norm weights must be a contiguous bf16 row of {w.rows}: {nw.shape}")
    if not (c.dtype == sn.dtype == "bf16" and c._contiguous() and sn._contiguous() and c.cols == sn.cols == w.cols
            and c.batch * c.rows == sn.batch * sn.rows == 1):
      raise ValueError(f"matmul_row with rope needs one bf16 row of cos and of sin, {w.cols} wide: {c.shape} {sn.shape}")
    if not (cc.dtype == "bf16" and cc.batch == 2 * kv and cc.cols == d and cc.sc == 1 and cc.rep == 1 and not cc.cyc
            and cc.layout == "plain"):
      raise ValueError(f"matmul_row with rope needs a plain ({2 * kv}, size, {d}) cache: {cc.shape}")
    if not (pl.dtype == "int32" and pl.batch * pl.rows * pl.cols == 1):
      raise ValueError("matmul_row with rope needs the token's place as one int32")
    q = Tensor(self.rt, 1, heads * d)
    _written(cc.storage)
    args = _lib.RowArgs(a.addr, nw.addr, 0, 0, w.storage.addr, w.rows, w.cols, _lib.ROW_RMS, _lib.DTYPES[w.dtype],
                        _lib.DTYPES["bf16"], eps)
    tail = _lib.RopeArgs(0, c.addr, sn.addr, q.addr, cc.addr, pl.addr, 0, 0, q.sr, cc.sb, cc.sr, cc.rows, 1, heads, kv,
                         d, 0, 0, 0, 0)
    self.rt.run("matmul_row_rope", "matmul_row_rope", ctypes.byref(args), ctypes.byref(tail), reads=_bytes(a, w, nw))
    return q

  def rms_rows(self, w, eps=1e-5):
    """RMSNorm of each row of self (fp32, a batch of one) scaled by w (bf16), in one kernel a row apart
    (llama.py:88-95; bt_rms_rows): x rounded to bf16, then x / sqrt(mean(x^2) + eps) * w in fp32, rounded once."""
    x, wt = self.realize(), w.realize()
    if not (x.dtype == "fp32" and x.batch == 1 and x.sc == 1 and x.rep == 1 and not x.cyc and x.layout == "plain"):
      raise ValueError(f"rms_rows needs fp32 rows of one matrix: {x.shape} {x.dtype}")
    if not (wt.dtype == "bf16" and wt._contiguous() and wt.batch * wt.rows * wt.cols == x.cols):
      raise ValueError(f"rms_rows needs bf16 weights, one for each column: {wt.shape} {wt.dtype}")
    out = Tensor(self.rt, x.rows, x.cols)
    out.lead = self.lead
    self.rt.run("rms_rows", "rms_rows", x.addr, x.rows, x.cols, x.sr, wt.addr, eps, out.addr, out.sr, reads=_bytes(x, wt))
    return out

  def matmul_swiglu(self, w):
    """silu(self @ gate) * (self @ up) for w holding gate then up side by side (llama.py:174-183), in one kernel: the
    SiLU-mul runs as the product's epilogue (bt_matmul_swiglu). self is bf16 rows of one matrix; returns bf16
    (rows, w.cols / 2)."""
    if not isinstance(w, Tensor) or w.rt is not self.rt or w.layout != "columns" or w.batch != 1:
      raise ValueError("matmul_swiglu needs w laid out by columns, batch 1, on the same runtime")
    a = self.realize()
    if not (a.dtype == "bf16" and a.batch == 1 and a.sc == 1 and a.rep == 1 and not a.cyc and a.cols == w.rows):
      raise ValueError(f"matmul_swiglu needs bf16 rows of one matrix, {w.rows} wide: {a.shape} {a.dtype}")
    out = Tensor(self.rt, a.rows, w.cols // 2)
    out.lead = self.lead
    self.rt.run("matmul_swiglu", "matmul_swiglu", ctypes.byref(_lib.operand(a.addr, "bf16", 0, a.sr)),
                _lib.DTYPES[w.dtype], w.storage.addr, a.rows, a.cols, w.cols,
                ctypes.byref(_lib.operand(out.addr, "bf16", 0, out.sr)), reads=_bytes(a, w))
    return out

  def rope_put(self, cos, sin, cache, places, heads, kv, values=None):
    """RoPE of each head of self (bf16 rows of heads + 2 kv heads) in fp32, the query heads returned as a
    (rows, heads * d) tensor and the key and value heads put into cache (2 kv, size, d) at places (an int32 row, one
    place for each row or one for all), in one kernel (llama.py:132-160; bt_rope_put). With values, cache and values
    are separate key and value caches of rows * kv heads, row i's at i * kv .. i * kv + kv - 1 (the slots of
    llama.py:293-354, each with a cache of its own). cos and sin are bf16 rows laid out as self; the tables turn x
    into x cos + (-x2, x1) sin, which leaves the value heads (cos 1, sin 0) as they are."""
    x = self.realize()
    if not (x.dtype == "bf16" and x.batch == 1 and x.sc == 1):
      raise ValueError(f"rope_put needs bf16 rows of one matrix: {x.shape} {x.dtype}")
    q, args, tables = _rope_args(self.rt, x.rows, x.cols, cos, sin, cache, places, heads, kv, values)
    args.qkv, args.qkv_sr = x.addr, x.sr
    self.rt.run("rope_put", "rope_put", ctypes.byref(args), reads=_bytes(x, *tables))
    return q

  def matmul_rope_put(self, w, cos, sin, cache, places, heads, kv, values=None):
    """(self @ w).rope_put(cos, sin, cache, places, heads, kv, values): for 5 to 32 rows of bf16 against w by columns
    with a long K (a batched decode step's qkv), the product's split-K partial sums go straight to the RoPE kernel
    (bt_matmul_rope_put), two launches instead of four, bit for bit the same; other shapes take the two calls."""
    a = self.realize()
    if not _stream_fits(a, w): return self.matmul(w).rope_put(cos, sin, cache, places, heads, kv, values)
    q, args, tables = _rope_args(self.rt, a.rows, w.cols, cos, sin, cache, places, heads, kv, values)
    self.rt.run("matmul_rope_put", "matmul_rope_put", ctypes.byref(_lib.operand(a.addr, "bf16", 0, a.sr)),
                _lib.DTYPES[w.dtype], w.storage.addr, a.rows, a.cols, w.cols, ctypes.byref(args),
                reads=_bytes(a, w, *tables))
    return q

  def matmul_residual_rms(self, w, residual, norm, eps=1e-5):
    """(x, h) with x = residual + self @ w in fp32 and h = x.rms_rows(norm, eps): for 5 to 32 rows of bf16 against w by
    columns with a long K (a batched decode step's o product and the MLP's norm), the product's split-K partial sums
    are summed in the norm's kernel (bt_matmul_residual_rms), two launches instead of four, bit for bit the same;
    other shapes take the unfused calls."""
    a, res, nw = self.realize(), residual.realize(), norm.realize()
    if not (res.dtype == "fp32" and res.batch == 1 and res.sc == 1 and res.rep == 1 and not res.cyc and
            res.shape[-2:] == (a.rows, w.cols) and res.layout == "plain"):
      raise ValueError(f"matmul_residual_rms needs fp32 residual rows of one matrix, {a.rows} x {w.cols}: {res.shape}")
    if not (nw.dtype == "bf16" and nw._contiguous() and nw.batch * nw.rows * nw.cols == w.cols):
      raise ValueError(f"matmul_residual_rms needs bf16 norm weights, one for each column: {nw.shape}")
    if not (_stream_fits(a, w) and w.cols <= 8192 and w.cols % 4 == 0 and res.addr % 16 == 0 and res.sr % 4 == 0):
      x = (res + self.matmul(w, "fp32")).realize()
      return x, x.rms_rows(nw, eps)
    x = Tensor(self.rt, a.rows, w.cols, dtype="fp32")
    h = Tensor(self.rt, a.rows, w.cols)
    x.lead = h.lead = res.lead
    self.rt.run("matmul_residual_rms", "matmul_residual_rms", ctypes.byref(_lib.operand(a.addr, "bf16", 0, a.sr)),
                _lib.DTYPES[w.dtype], w.storage.addr, a.rows, a.cols, w.cols, res.addr, res.sr, x.addr, x.sr, nw.addr,
                eps, h.addr, h.sr, reads=_bytes(a, w, res, nw))
    return x, h

  # ---- attention, rows in and out
  def attend(self, k, v, places, window=0, fidelity=None, parts=None, firsts=None, merged=False):
    """softmax(self @ k^T + mask) @ v, with the mask from each query row's place (and window), in one kernel
    (tensor.py:797-841). k and v may be repeat views (grouped-query attention). RoPE scales q beforehand. firsts, an
    int32 column like places, raises each row's first visible key: sequences that share one cache in regions of their
    own (llama.py:293-318's slots). merged writes the result as merge() of it, (rows, heads * width)."""
    if len(self.shape) > 3: raise ValueError(f"attend takes three dimensions, not {self.shape}")
    if window < 0 or parts is not None and parts <= 0: raise ValueError("attention needs a nonnegative window and positive parts")
    if not (self.dtype == "bf16" and k.dtype == v.dtype and k.dtype in ("bf16", *BFP) and self.batch == k.batch == v.batch):
      raise ValueError(f"attend needs bf16 queries, keys and values in bf16 or one block-float format, equal batches: "
                       f"{self.dtype} {k.dtype} {v.dtype}")
    if not (self.cols == k.cols == v.cols and self.cols in (64, 128) and k.rows == v.rows):
      raise ValueError(f"attend needs heads 64 or 128 wide and a value for each key: {self.shape} {k.shape} {v.shape}")
    if not (places.rows == self.rows and places.batch in (1, self.batch) and places.cols == 1 and places.dtype == "int32"):
      raise ValueError(f"attend needs places as an int32 column with a row for each query: {places.shape}")
    q, k, v, places, rep = self._attention_operands(k, v, places)
    if merged:  # the heads side by side in each row, as merge() would give them
      out = Tensor(self.rt, q.rows, q.batch * q.cols)
      osh, osr = q.cols, out.sr
    else:
      out = Tensor(self.rt, q.rows, q.cols, batch=q.batch)
      out.lead = self.lead
      osh, osr = out.sb, out.sr
    args = _lib.AttentionArgs(q.addr, k.addr, v.addr, out.addr, places.addr, q.sb, q.sr, k.sb, k.sr, v.sb, v.sr,
                              osh, osr, q.rows if places.batch > 1 else 0, q.batch, rep, q.rows, k.rows, q.cols,
                              window, parts or 0, 0, 0, 0)
    if k.dtype in BFP:  # a block-float cache, read in place (test_kernels.py:2106-2132)
      (args.k_exps, args.k), (args.v_exps, args.v) = k._bfp_planes(), v._bfp_planes()
      args.kv_fmt = _lib.DTYPES[k.dtype]
    if firsts is not None:
      if not (firsts.rows == self.rows and firsts.batch in (1, self.batch) and firsts.cols == 1 and firsts.dtype == "int32"):
        raise ValueError(f"attend needs firsts as an int32 column with a row for each query: {firsts.shape}")
      firsts = firsts.realize()
      if not firsts._contiguous(): firsts = firsts.contiguous()
      args.firsts, args.firsts_sh = firsts.addr, q.rows if firsts.batch > 1 else 0
    need = ctypes.c_uint64()
    _lib.call("attention_scratch", ctypes.byref(args), ctypes.byref(need))
    scratch = None
    if need.value:  # the parts' partial sums, freed (stream-ordered) once the launches that use them are queued
      scratch = Storage(self.rt, need.value)
      args.scratch, args.scratch_bytes = scratch.addr, need.value
    self.rt.run("attention", "attention", ctypes.byref(args), reads=_bytes(q) + q.batch // rep * 2 * k.rows * k.cols *
                (2 if k.dtype == "bf16" else 17 / 16 if k.dtype == "bfp8" else 9 / 16))
    del scratch
    return out

  def _attention_operands(self, k, v, places):
    q = self.realize()
    k, v, places = k.realize(), v.realize(), places.realize()
    if k.rep != v.rep or k.cyc or v.cyc: raise ValueError("attend needs keys and values repeated alike")
    if q.sc != 1 or q.rep != 1 or q.cyc: q = q.contiguous()
    if k.sc != 1: k = k.contiguous()  # a block-float view keeps whole runs, so its columns are contiguous already
    if v.sc != 1: v = v.contiguous()
    if not places._contiguous(): places = places.contiguous()
    return q, k, v, places, k.rep

  def topk(self, k, parts=1, labels=None, out=None):
    """(values, int32 indices) of the k largest entries of each row, descending, in one kernel (tensor.py:685-706):
    equal values keep column order (numpy's stable argsort of -x) and -0 equals 0; bf16 or fp32, k up to 64. With
    parts, each of that many equal parts of a row gives its k, labelled by original column; topk again with those
    labels combines the parts. out: (values, indices) to write into, realized contiguous tensors of the result's
    shape (self's dtype, then int32), which come back."""
    k, parts = operator.index(k), operator.index(parts)
    if k <= 0 or parts <= 0: raise ValueError("topk needs positive k and parts")
    if labels is not None and labels.rt is not self.rt: raise ValueError("topk's labels must use the same runtime")
    cols = self.cols // parts
    if not (self.dtype in ("bf16", "fp32") and k <= min(cols, 64) and parts * cols == self.cols):
      raise ValueError(f"topk needs bf16 or fp32, k up to 64 and a part's width, "
                       f"and equal parts: {self.dtype}, k={k}, {parts} parts of {self.cols}")
    if labels is not None and not (labels.dtype == "int32" and labels.shape == self.shape and parts == 1):
      raise ValueError("topk's labels need int32, x's shape and parts=1")
    x = self.realize()
    if x.sc != 1 or x.rep != 1 or x.cyc: x = x.contiguous()
    lab = None
    if labels is not None:
      lab = labels.realize()
      if lab.sc != 1 or lab.rep != 1 or lab.cyc: lab = lab.contiguous()
    if out is None:
      values = Tensor(self.rt, x.rows, parts * k, batch=x.batch, dtype=x.dtype)
      ids = Tensor(self.rt, x.rows, parts * k, batch=x.batch, dtype="int32")
      values.lead = ids.lead = self.lead
    else:
      values, ids = out
      fits = lambda t, dt: (isinstance(t, Tensor) and t.rt is self.rt and t.op is None and t._contiguous() and
                            (t.batch, t.rows, t.cols, t.dtype) == (x.batch, x.rows, parts * k, dt))
      if not (fits(values, x.dtype) and fits(ids, "int32")):
        raise ValueError(f"topk's out must be realized contiguous ({x.batch}, {x.rows}, {parts * k}) tensors, "
                         f"{x.dtype} and int32")
      _written(values.storage)
      _written(ids.storage)
    self.rt.run("topk", "topk", _lib.DTYPES[x.dtype], x.addr, x.batch, x.rows, x.cols, x.sb if x.batch > 1 else 0, x.sr,
                parts, k, lab.addr if lab is not None else 0, (lab.sb if lab.batch > 1 else 0) if lab is not None else 0,
                lab.sr if lab is not None else 0, values.addr, ids.addr, reads=_bytes(x, lab))
    return values, ids

  def gather(self, ids):
    """Rows picked by ids: a Python list (bounds-checked) or an int32 row on the device (tensor.py:206-221)."""
    if len(self.shape) > 3 or self.batch != 1: raise ValueError("gather needs batch 1")
    if self.dtype not in ITEMSIZE: raise ValueError("cast block-float storage to bf16 before gathering rows")
    if not isinstance(ids, Tensor):
      ids = list(ids)
      if not all(0 <= i < self.rows for i in ids): raise IndexError(f"gather picks rows of a {self.rows}-row matrix: {ids}")
      ids = Tensor.of(self.rt, [ids], "int32")
    if not (ids.dtype == "int32" and ids.shape[-3:-1] == (1, 1) and ids.batch == 1):
      raise ValueError("gather needs ids as an int32 row")
    t, ids = self.realize(), ids.realize()
    if t.sc != 1: t = t.contiguous()
    if not ids._contiguous(): ids = ids.contiguous()
    out = Tensor(self.rt, ids.cols, t.cols, dtype=t.dtype)
    self.rt.run("gather", "gather", _lib.DTYPES[t.dtype], t.addr, t.rows, t.cols, t.sr, ids.addr, ids.cols,
                out.addr, out.sr, reads=_bytes(ids) + ids.cols * t.cols * t.itemsize)
    return out

  def put(self, ids, x):
    """Write the rows of x at the places in ids, in place; a later duplicate wins (tensor.py:223-241)."""
    if not (ids.dtype == "int32" and ids.shape[-3:-1] == (1, 1) and ids.cols == x.rows):
      raise ValueError("put needs ids as an int32 row, with one position for each row of x")
    want = "bf16" if self.dtype in BFP else self.dtype  # into a block float (a bfp8/bfp4 cache), bf16 rows
    if not ((x.batch, x.cols) == (self.batch, self.cols) and x.dtype == want):
      raise ValueError(f"put needs rows of the cache's batch, width and dtype: {x.shape} {x.dtype} into {self.shape} {self.dtype}")
    dst = self.realize()
    if dst.rep != 1 or dst.cyc or dst.sc != 1: raise ValueError("put requires a plain tensor with rep=1")
    x, ids = x.realize(), ids.realize()
    if x.sc != 1 or x.rep != 1 or x.cyc: x = x.contiguous()
    if not ids._contiguous(): ids = ids.contiguous()
    _written(dst.storage)
    if dst.dtype in BFP:  # each run of 16 rounded as cast rounds it (kernels.py:1083-1168)
      e, v = dst._bfp_planes()
      self.rt.run("put", "put_bfp", _lib.DTYPES[dst.dtype], e, v, dst.batch, dst.rows, dst.cols,
                  dst.sb if dst.batch > 1 else 0, dst.sr, ids.addr, ids.cols, x.addr, x.sb if x.batch > 1 else 0, x.sr,
                  reads=_bytes(x, ids))
      return self
    self.rt.run("put", "put", _lib.DTYPES[dst.dtype], dst.addr, dst.batch, dst.rows, dst.cols,
                dst.sb if dst.batch > 1 else 0, dst.sr, ids.addr, ids.cols, x.addr, x.sb if x.batch > 1 else 0, x.sr,
                reads=_bytes(x, ids))
    return self

  # ---- realize
  def realize(self, into=None):
    """Queue the computation; return this tensor, realized. With into, write into that realized tensor or view of
    the same shape and dtype (tensor.py:466-524)."""
    self.rt.check()
    if into is not None:
      if not (into.op is None and into.rep == 1 and into.cyc == 0 and into.layout == "plain" and
              into._dims == self._dims and into.dtype == self.dtype):
        raise ValueError("realize needs a realized destination of the same shape and dtype, not a repeat or a "
                         "tensor by columns")
      if self.op is None: raise ValueError("realize writes into a destination only from an unrealized tensor; assign copies a realized one")
    if self.op is None: return self
    if into is not None and _reads_into(self, into):
      # a kernel would overwrite what it still reads: a matmul's operand, or the same memory read at other places.
      # Compute into storage of its own first, then copy (tensor.py:513-517).
      into.assign(self.realize())
      self._adopt(into)
      return self
    out = into if into is not None else None
    if self.op == "matmul": _realize_matmul(self, None, out)
    elif self.op in REDUCE: _realize_reduce(self, out)
    elif self.op in ELEMENTWISE: _realize_elementwise(self, out)
    else: raise ValueError(f"cannot realize op {self.op}")
    return self

  def assign(self, x):
    """Write x into this tensor in place (tensor.py:526-541)."""
    if isinstance(x, Tensor) and x.rt is not self.rt: raise ValueError("tensor operands must use the same runtime")
    if not (self.op is None and self.rep == 1 and self.cyc == 0 and x.shape[-2:] == self.shape[-2:] and
            x.batch == self.batch and x.dtype == self.dtype):
      raise ValueError("assign requires a realized tensor with rep=1 and an x of the same shape and dtype")
    if self.dtype in BFP:  # a block float: copied whole, or its values put row by row as a cast rounds them
      if self.layout != "plain": raise ValueError("assign writes a plain tensor, not one by columns")
      x = x.realize()
      try:
        if x.storage is not self.storage: return _copy_whole(x, self) or self
      except ValueError:
        pass
      rows = x.cast("bf16").realize()  # decoded exactly, so the put gives back the same values
      if not rows._contiguous(): rows = rows.contiguous()
      return self.put(_row_ids(self.rt, self.rows), rows)
    if x.op is None and x.storage is self.storage: x = x._copy()  # overlapping storage: read it all first
    src = x if x.op is not None else x._copy_op()
    src.lead = self.lead
    src.realize(self)
    return self

  def _adopt(self, other):
    """Take other's storage and read pattern: this tensor becomes a realized tensor with those values."""
    lead = self.lead
    self.storage, self.offset, self.sb, self.sr, self.sc = other.storage, other.offset, other.sb, other.sr, other.sc
    self.rep, self.cyc, self.layout = other.rep, other.cyc, other.layout
    self.op, self.srcs, self.args, self.lead = None, (), (), lead


def _reads_into(t, into):
  """Whether computing t into `into` in one kernel could read memory that the kernel has already written: t's graph
  reads into's storage as a matmul operand, or elementwise at other positions than the ones it writes there."""
  seen, stack = set(), [(t, False)]
  while stack:
    u, by_matmul = stack.pop()
    if not isinstance(u, Tensor) or (id(u), by_matmul) in seen: continue
    seen.add((id(u), by_matmul))
    if u.op is not None:
      stack.extend((s, by_matmul or u.op == "matmul") for s in u.srcs)
      continue
    if u.storage is not into.storage: continue
    same = (u._dims == into._dims and u.layout == into.layout and
            (u.offset, u.sb if u.batch > 1 else 0, u.sr, u.sc, u.rep, u.cyc) ==
            (into.offset, into.sb if into.batch > 1 else 0, into.sr, into.sc, into.rep, into.cyc))
    if by_matmul or not same: return True
  return False


_ids = weakref.WeakKeyDictionary()


def _row_ids(rt, n):
  """An int32 row 0 .. n-1 on rt, made once (so a recording finds it made)."""
  made = _ids.setdefault(rt, {})
  if n not in made: made[n] = Tensor.of(rt, [list(range(n))], "int32")
  return made[n]


def _parts(t):
  """An fp32 operand as bf16 (high, low), low None for bf16 (tensor.py:1045-1051)."""
  if t.dtype != "fp32": return (t if t.dtype in ("bf16", *BFP) else t.cast("bf16")), None
  hi = t.bfloat16()
  lo = (t - t._unary("ftob")).bfloat16()
  return hi, lo


def _run_copy(rt, operand, dtype, out):
  p = Program(dtype)
  r = p.load(p.input(operand))
  prog = p.build(r)
  rt.run("copy", "elementwise", ctypes.byref(prog), out.batch, out.rows, out.cols, ctypes.byref(out._operand()))


def _dest(t, into):
  """The realized tensor a kernel writes t's value to: into, or new storage."""
  if into is not None:
    _written(into.storage)
    t._adopt(into)
    return into
  t.storage = None
  t._alloc()
  t.op, t.srcs, t.args = None, (), ()
  return t


# ---- lowering an elementwise tree to a program
class _Lowering:
  """Builds one bt_program for the elementwise tree under a root, of the root's shape. Realized tensors, and
  subtrees that can't join (another dtype, a matmul other than the anchor, reductions, movement), become inputs."""
  def __init__(self, root, dtype, anchor=None):
    self.root, self.dtype, self.anchor = root, dtype, anchor
    self.p = Program(dtype, epilogue=anchor is not None)
    self.memo = {}
    self.keep = []  # tensors whose storage the queued kernel reads, kept alive until it is queued

  def leaf(self, t):
    t = t.realize() if t.op is not None else t
    if t.dtype in BFP or t.layout != "plain": t = t.cast("bf16").realize()
    self.keep.append(t)
    op = t._operand(self.root.lead, self.root.rows, self.root.cols)
    key = (op.ptr, op.sb, op.sr, op.sc, op.dtype, op.rep, op.cyc)
    return self.p.load(self.p.input(op, key))

  def emit(self, u):
    if not isinstance(u, Tensor): return self.p.const(u)
    if id(u) in self.memo: return self.memo[id(u)]
    if u is self.anchor: r = self.p.value()
    elif u.op is None: r = self.leaf(u)
    elif u.op == "cast":
      src = u.srcs[0]
      if u is self.root or u.dtype == self.dtype and src.dtype == self.dtype: r = self.emit(src)
      elif u.dtype == self.dtype: r = self.leaf(src)  # loading converts src's dtype exactly as the cast does
      else: r = self.leaf(u)  # another dtype: a kernel of its own
    elif u.op in ELEMENTWISE and u.dtype == self.dtype and _fits_root(u, self.root):
      r = self.p.op(u.op, *(self.emit(s) for s in u.srcs))
    else: r = self.leaf(u)
    self.memo[id(u)] = r
    return r


def _fits_root(u, root):
  """Whether u can be computed inside root's kernel: its shape broadcasts to root's (a broadcast subtree is evaluated
  again at each element it covers, reading its inputs with strides of 0)."""
  return _broadcast(u.shape, root.shape) == tuple(root.shape) and len(u.shape) <= len(root.shape)


def _compute_dtype(t):
  """The dtype t's kernel computes in: a cast at the root computes in its source's dtype."""
  if t.op == "cast" and isinstance(t.srcs[0], Tensor) and t.srcs[0].dtype in ITEMSIZE: return t.srcs[0].dtype
  return t.dtype


def _find_anchor(t, dtype):
  """An unrealized matmul in t's elementwise tree that can run t's tree as its epilogue: t's shape, writing dtype."""
  seen, stack = set(), [t]
  while stack:
    u = stack.pop()
    if not isinstance(u, Tensor) or u.op is None or id(u) in seen: continue
    seen.add(id(u))
    if u.op == "matmul":
      if u.shape == t.shape and u.dtype == dtype and u.srcs[1].dtype != "fp32": return u
      continue
    if u.op in ELEMENTWISE and (u.dtype == dtype or u is t) and u.shape == t.shape:
      stack.extend(s for s in u.srcs if isinstance(s, Tensor))
  return None


def _build(t, dtype, anchor):
  """Lower t's tree; when it needs more than one kernel can hold, realize its largest subtree and try again."""
  while True:
    low = _Lowering(t, dtype, anchor)
    try:
      r = low.emit(t)
      return low, low.p.build(r)
    except ValueError as e:
      if "at most" not in str(e) and "more than" not in str(e): raise
      subs = [s for s in t.srcs if isinstance(s, Tensor) and s.op is not None and s is not anchor]
      if not subs: raise
      big = max(subs, key=_size)
      big.realize()


def _size(t):
  n, stack, seen = 0, [t], set()
  while stack:
    u = stack.pop()
    if not isinstance(u, Tensor) or u.op is None or id(u) in seen: continue
    seen.add(id(u))
    n += 1
    stack.extend(u.srcs)
  return n


def _realize_elementwise(t, into):
  dtype = _compute_dtype(t)
  if dtype in BFP: dtype = "bf16"
  anchor = _find_anchor(t, dtype) if dtype in ("bf16", "fp32") else None
  if anchor is not None:
    _realize_matmul(anchor, t, into)
    return
  low, prog = _build(t, dtype, None)
  out = _dest(t, into)
  t.rt.run(_name(prog), "elementwise", ctypes.byref(prog), out.batch, out.rows, out.cols, ctypes.byref(out._operand()),
           reads=_bytes(*low.keep))


def _name(prog):
  return "elementwise"


def _realize_reduce(t, into):
  """A reduction kernel whose prologue computes the source's elementwise tree (tensor.py:657-676)."""
  src = t.srcs[0]
  axis = t.args[0]
  n = len(src.shape)
  dtype = _compute_dtype(src) if src.op in ELEMENTWISE else src.dtype
  if dtype in BFP: dtype = "bf16"
  low = None
  # the prologue: src's tree at src's shape
  while True:
    low = _Lowering(src, dtype)
    try:
      prog = low.p.build(low.emit(src))
      break
    except ValueError as e:
      if "at most" not in str(e) and "more than" not in str(e): raise
      src.realize()
  if axis >= n - 2: k, sweep, step = axis - (n - 3), 0, 0  # rows (1) or columns (2)
  else: k, sweep, step = 0, src.shape[axis], math.prod(src.shape[axis + 1:n - 2])  # a leading dimension
  kind = _lib.REDUCE_SUM if t.op == "sum" else _lib.REDUCE_MAX  # before _dest, which clears t's op
  out = _dest(t, into)
  t.rt.run("reduce", "reduce", ctypes.byref(prog), kind, k, src.batch, src.rows, src.cols, sweep, step,
           ctypes.byref(out._operand()), reads=_bytes(*low.keep))


def _stream_fits(a, w):
  """Whether a product of a (realized) against w is one the fused decode-step products take: 5 to 32 bf16 rows of one
  matrix, contiguous and 16-byte aligned, against w by columns with K a multiple of 256 over 768."""
  return (isinstance(w, Tensor) and w.rt is a.rt and w.op is None and w.layout == "columns" and w.batch == 1 and
          a.dtype == "bf16" and a.batch == 1 and a.sc == 1 and a.rep == 1 and not a.cyc and a.layout == "plain" and
          5 <= a.rows <= 32 and a.cols == w.rows and w.rows % 256 == 0 and w.rows > 768 and a.addr % 16 == 0 and
          a.sr % 8 == 0)


def _rope_args(rt, rows, cols, cos, sin, cache, places, heads, kv, values):
  """The query tensor and bt_rope_args (qkv left 0) of RoPE and the cache put over `rows` rows of `cols` columns
  (heads + 2 kv heads), after the checks of rope_put; and the tables it reads."""
  c, sn, cc, pl = cos.realize(), sin.realize(), cache.realize(), places.realize()
  vc = values.realize() if values is not None else None
  nh = heads + 2 * kv
  if not (c.dtype == sn.dtype == cc.dtype == "bf16" and cols % nh == 0):
    raise ValueError(f"rope_put needs rows of {nh} heads and bf16 tables and caches: {rows} x {cols}")
  d = cols // nh
  if not (c.shape[-2:] == sn.shape[-2:] == (rows, cols) and c.sc == 1 and sn.sc == 1 and c.sr == sn.sr):
    raise ValueError(f"rope_put needs cos and sin laid out as the rows: {c.shape} {sn.shape} for {rows} x {cols}")
  plain = lambda t: t.cols == d and t.sc == 1 and t.rep == 1 and not t.cyc and t.layout == "plain"
  if vc is None and not (cc.batch == 2 * kv and plain(cc)):
    raise ValueError(f"rope_put needs a plain ({2 * kv}, size, {d}) cache: {cc.shape}")
  if vc is not None and not (cc.batch == vc.batch == rows * kv and vc.dtype == "bf16" and plain(cc) and plain(vc)
                             and cc.rows == vc.rows and cc.sb == vc.sb and cc.sr == vc.sr):
    raise ValueError(f"rope_put needs plain ({rows * kv}, size, {d}) key and value caches: {cc.shape}")
  if not (pl.dtype == "int32" and pl.batch * pl.rows == 1 and pl.cols in (1, rows) and pl.sc == 1):
    raise ValueError("rope_put needs places as an int32 row, one for each row or one for all")
  q = Tensor(rt, rows, heads * d)
  _written(cc.storage)
  if vc is not None: _written(vc.storage)
  args = _lib.RopeArgs(0, c.addr, sn.addr, q.addr, cc.addr, pl.addr, 0, c.sr, q.sr, cc.sb, cc.sr, cc.rows, rows,
                       heads, kv, d, vc.addr if vc is not None else 0, kv * cc.sb if vc is not None else 0,
                       int(pl.cols == 1 and rows > 1), 0)
  return q, args, (c, sn)


def _check_range(x):
  """ValueError if a whole plain block float x holds a nonzero run whose exponent a matmul can't multiply exactly (bfp8
  below 5, bfp4 outside 3..247): one counting launch, its count read back."""
  e, v = x._bfp_whole()._bfp_planes()
  bad = Storage(x.rt, 4)
  x.rt.run("range", "bfp_range", _lib.DTYPES[x.dtype], e, v, x.batch, x.rows, x.cols, bad.addr)
  n = int.from_bytes(x.rt.download(bad.addr, 4), "little")
  if n:
    raise ValueError(f"{n} runs of this {x.dtype} tensor hold values under an exponent outside "
                     f"{'5..255' if x.dtype == 'bfp8' else '3..247'}, which a matmul can't multiply exactly")


def _b_tiles(b):
  """(format, tiles address, batch, keep-alive) for a matmul's B: its columns tiles, made now if it has none. A block
  float's tiles are kept with its storage, per view, until something writes the storage; inside a jit recording they
  are made in the recording, so every replay reads the storage as it is then."""
  x = b.realize()
  if x.layout == "columns": return _lib.DTYPES[x.dtype], x.storage.addr, x.batch, x
  if x.dtype in BFP:
    s, key = x.storage, (x.offset, x.sb if x.batch > 1 else 0, x.sr, x.batch, x.rows, x.cols)
    c = s.columns.get(key) if x.rt.recording is None else None
    if c is None:
      c = x.columns()
      if x.rt.recording is None: s.columns[key] = c
    return _lib.DTYPES[c.dtype], c.storage.addr, c.batch, c
  c = x.columns()
  return _lib.BF16, c.storage.addr, c.batch, c


def _realize_matmul(m, root, into):
  """One matmul kernel for m, with root's elementwise tree (if any) as its epilogue, writing root (or m)."""
  a, b = m.srcs
  a = a.realize()
  if a.dtype != "bf16": a = a.cast("bf16").realize()
  fmt, tiles, b_batch, keep_b = _b_tiles(b)
  target = root if root is not None else m
  prog = None
  keep = []
  if root is not None:
    low, prog = _build(root, m.dtype, m)
    keep = low.keep
  out = _dest(target, into)
  batch = max(a.batch, b_batch)
  if a.rep != 1 or a.cyc or (a.batch == 1 and batch > 1):
    aop = a._operand((batch,), a.rows, a.cols) if a.batch == batch else _lib.Operand(a.addr, 0, a.sr, a.sc, _lib.BF16, 1, 0, 0)
  else: aop = _lib.Operand(a.addr, a.sb, a.sr, a.sc, _lib.BF16, 1, 0, 0)
  m.rt.run("matmul", "matmul", ctypes.byref(aop), fmt, tiles, b_batch, batch, a.rows, a.cols, m.cols,
           ctypes.byref(prog) if prog is not None else None, ctypes.byref(out._operand()),
           reads=_bytes(a, keep_b, *keep))
  if root is not None and m is not root:  # the matmul itself was never stored: a later read recomputes it
    pass
  del keep, keep_b


# ---- jit
class Recording:
  """Launches captured into a HIP graph for replay, holding the memory they allocated (tensor.py:1171-1229)."""
  def __init__(self, rt):
    self.rt, self.graph, self.storages, self.held, self.active = rt, None, [], [], False
    self.unchecked = set()  # ids of block-float storages laid out as a matmul's B with no exponent check
    self.kernels = 0  # launches captured

  def __enter__(self):
    if self.rt.recording is not None: raise RuntimeError("cannot nest recordings on the same runtime")
    self.close()
    self.rt.recording = self
    self.active = True
    _lib.call("graph_begin", self.rt.handle)
    self.kernels = -self.rt.launches
    return self

  def __exit__(self, kind, *_):
    g = ctypes.c_void_p()
    self.kernels += self.rt.launches
    try: _lib.call("graph_end", self.rt.handle, ctypes.byref(g))
    finally:
      # memory let go during the capture may still be read by the graph: it is freed with the graph
      self.rt.recording, self.active = None, False
      self.held, self.rt.deferred = self.held + self.rt.deferred, []
    self.graph = g
    if kind is not None: self.close()

  def send(self):
    """Queue the recorded launches once more."""
    self.rt.check()
    if self.active or self.graph is None: raise RuntimeError("recording is not ready for replay")
    _lib.call("graph_launch", self.rt.handle, self.graph)
    self.rt.launches += 1

  def close(self):
    """Destroy the graph, then let go of its memory: storage no live tensor holds is freed."""
    if self.graph is not None and not self.rt.closed:
      self.rt.wait()
      _lib.call("graph_destroy", self.graph)
    self.graph = None
    self.storages = []
    held, self.held = self.held, []
    for addr, captured in held: self.rt.dram_free(addr, captured)

  def __del__(self):
    try:
      if not self.active: self.close()
    except Exception:
      pass


def jit(f):
  """Run f normally on the first call, record the second call into a HIP graph, and replay it from the third
  (tensor.py:1231-1293). Each call's inputs are copied into the recording's own input buffers first; an input that f
  writes (put, assign, realize into) is copied back after each call. A replay returns the recorded results, which the
  next call overwrites. Keep input shapes, dtypes and layouts fixed; a block-float or by-columns input is taken as a
  whole tensor, not a view."""
  state = {"signature": None, "rec": None, "ins": None, "out": None, "wrote": (), "check": ()}

  @functools.wraps(f)
  def run(*xs):
    if not xs or not all(isinstance(x, Tensor) for x in xs):
      raise ValueError("jit inputs must be tensors, with at least one input")
    rt = xs[0].rt
    if any(x.rt is not rt for x in xs): raise ValueError("jit inputs must use the same runtime")
    rt.check()
    sig = [(x.shape, x.dtype, x.layout) for x in xs]
    if state["signature"] is None:
      state["signature"] = sig
      return f(*xs).realize()
    if sig != state["signature"]:
      raise ValueError(f"a jit input is {sig}, where the first call had {state['signature']}")
    xs = [x.realize() for x in xs]
    if state["rec"] is None:
      ins = [_stand_in(x) for x in xs]
      for x, t in zip(xs, ins): _copy_whole(x, t)
      rt.wait()
      rec = Recording(rt)
      rt.written = set()
      try:
        with rec:
          out = f(*ins).realize()
      finally:
        written, rt.written = rt.written, None
      wrote = [i for i, t in enumerate(ins) if id(t.storage) in written]
      check = [i for i, t in enumerate(ins) if id(t.storage) in rec.unchecked]  # block-float inputs used as a B
      state.update(rec=rec, ins=ins, out=out, wrote=wrote, check=check)
      for i in check: _check_range(xs[i])
      rec.send()
    else:
      ins = state["ins"]
      for i in state["check"]: _check_range(xs[i])
      for x, t in zip(xs, ins):
        if x.storage is not t.storage or x.offset != t.offset: _copy_whole(x, t)
      state["rec"].send()
    for i in state["wrote"]:  # what f wrote into an input goes back to the caller's tensor
      if xs[i].storage is not ins[i].storage: _copy_whole(ins[i], xs[i])
    return state["out"]
  return run


def _stand_in(x):
  """A new tensor laid out as x would be if made anew: a jit recording's own buffer for input x."""
  if x.layout == "columns":
    t = Tensor(x.rt, x.rows, x.cols, "view", (), x.batch, x.dtype)
    t.op = None
    t._alloc("columns")
  else:
    t = Tensor(x.rt, x.rows, x.cols, batch=x.batch, dtype=x.dtype)
  t.lead = x.lead
  return t


def _copy_whole(src, dst):
  """Copies src's values into dst, a tensor of the same shape and format that owns its storage. Plain bf16, fp32 and
  int32 views go through a copy kernel; block floats and tensors by columns are copied byte for byte, which takes
  them whole: a view of a larger block float would bring another tensor's exponents and values."""
  if src.dtype in ITEMSIZE and src.layout == "plain" and dst.layout == "plain":
    if src._contiguous() and dst._contiguous():
      src.rt.copy(dst.addr, src.addr, src.batch * src.rows * src.cols * src.itemsize)
    else:
      src._copy_op().realize(dst)
    return
  whole = lambda t: t.offset == 0 and (t.layout == "columns" or t._contiguous())
  if not (whole(src) and whole(dst) and src.layout == dst.layout and src.storage.nbytes == dst.storage.nbytes and
          src.storage.vals == dst.storage.vals):
    raise ValueError("jit takes a block-float or by-columns input only as a whole tensor, not a view of one")
  src.rt.copy(dst.storage.addr, src.storage.addr, src.storage.nbytes)
  _written(dst.storage)
