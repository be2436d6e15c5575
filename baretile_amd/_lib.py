"""ctypes bindings of libbaretile_amd.so (include/baretile_amd.h), and the status -> exception mapping.

The library is loaded the way baretile's pci.Sim loads its device library (baretile/pci.py:50-60): ctypes.CDLL of a
shared object, with argument types declared here. Every call goes through check(), which raises ValueError,
RuntimeError, TimeoutError or MemoryError with the library's own message (docs/api.md:51-63). Nothing falls back to
another implementation: without the built library, load() raises.
"""
import ctypes, os
from ctypes import POINTER, byref, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_uint8, c_uint32, c_uint64, \
  c_void_p

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "libbaretile_amd.so")

OK, EINVAL, ESTATE, ETIMEOUT, ENOMEM = range(5)
BF16, FP32, INT32, BFP8, BFP4 = range(5)
DTYPES = {"bf16": BF16, "fp32": FP32, "int32": INT32, "bfp8": BFP8, "bfp4": BFP4}
ITEMSIZE = {"bf16": 2, "fp32": 4, "int32": 4}
MAX_INPUTS, MAX_INST, MAX_REGS = 8, 48, 16

OPS = ["load", "const", "mov", "add", "sub", "mul", "div", "max", "min", "cmplt", "cmple", "cmpne", "cmpeq", "where",
       "neg", "relu", "exp", "exp2", "log", "log2", "sqrt", "recip", "rsqrt", "sin", "cos", "sigmoid", "silu", "gelu",
       "tanh", "ftob"]
OP = {name: i for i, name in enumerate(OPS)}
REDUCE_SUM, REDUCE_MAX = 0, 1


class Operand(ctypes.Structure):
  _fields_ = [("ptr", c_uint64), ("sb", c_int64), ("sr", c_int64), ("sc", c_int64), ("dtype", c_int32),
              ("rep", c_int32), ("cyc", c_int32), ("pad_", c_int32)]


class Inst(ctypes.Structure):
  _fields_ = [("op", c_uint8), ("dst", c_uint8), ("a", c_uint8), ("b", c_uint8), ("c", c_uint8),
              ("pad_", c_uint8 * 3), ("imm", c_uint32)]


class Program(ctypes.Structure):
  _fields_ = [("n_inst", c_int32), ("n_inputs", c_int32), ("dtype", c_int32), ("result", c_int32),
              ("inst", Inst * MAX_INST), ("inputs", Operand * MAX_INPUTS)]


class AttentionArgs(ctypes.Structure):
  _fields_ = [("q", c_uint64), ("k", c_uint64), ("v", c_uint64), ("out", c_uint64), ("places", c_uint64),
              ("q_sh", c_int64), ("q_sr", c_int64), ("k_sh", c_int64), ("k_sr", c_int64), ("v_sh", c_int64),
              ("v_sr", c_int64), ("o_sh", c_int64), ("o_sr", c_int64), ("places_sh", c_int64),
              ("heads", c_int32), ("rep", c_int32), ("rows", c_int32), ("keys", c_int32), ("head_dim", c_int32),
              ("window", c_int32), ("parts", c_int32), ("pad_", c_int32), ("scratch", c_uint64),
              ("scratch_bytes", c_uint64), ("firsts", c_uint64), ("firsts_sh", c_int64), ("kv_fmt", c_int32),
              ("pad2_", c_int32), ("k_exps", c_uint64), ("v_exps", c_uint64)]


ROW_PLAIN, ROW_RMS, ROW_SWIGLU = range(3)


class RowArgs(ctypes.Structure):  # bt_row_args
  _fields_ = [("a", c_uint64), ("norm", c_uint64), ("residual", c_uint64), ("out", c_uint64), ("b", c_uint64),
              ("k", c_int64), ("n", c_int64), ("kind", c_int32), ("b_fmt", c_int32), ("out_dtype", c_int32),
              ("eps", c_float)]


class RopeArgs(ctypes.Structure):  # bt_rope_args
  _fields_ = [("qkv", c_uint64), ("cos", c_uint64), ("sin", c_uint64), ("q", c_uint64), ("cache", c_uint64),
              ("places", c_uint64), ("qkv_sr", c_int64), ("cs_sr", c_int64), ("q_sr", c_int64), ("cache_sh", c_int64),
              ("cache_sr", c_int64), ("cache_rows", c_int64), ("rows", c_int32), ("heads", c_int32), ("kv", c_int32),
              ("head_dim", c_int32), ("vcache", c_uint64), ("cache_tsh", c_int64), ("one_place", c_int32),
              ("pad_", c_int32)]


RT = c_void_p
U64, I64 = c_uint64, c_int64
# name: argument types. Every function returns an int status.
SIGNATURES = {
  "bt_version": [], "bt_device_count": [POINTER(c_int)], "bt_open": [c_int, POINTER(c_void_p)], "bt_close": [RT],
  "bt_alloc": [RT, U64, POINTER(c_uint64)], "bt_free": [RT, U64, c_int], "bt_upload": [RT, U64, c_void_p, U64],
  "bt_download": [RT, c_void_p, U64, U64], "bt_copy": [RT, U64, U64, U64], "bt_fill32": [RT, U64, c_uint32, U64],
  "bt_wait": [RT, c_double], "bt_sleep": [RT, c_double], "bt_event_create": [RT, POINTER(c_void_p)], "bt_event_record": [RT, c_void_p],
  "bt_event_elapsed": [c_void_p, c_void_p, POINTER(c_float)], "bt_event_destroy": [c_void_p],
  "bt_graph_begin": [RT], "bt_graph_end": [RT, POINTER(c_void_p)], "bt_graph_launch": [RT, c_void_p],
  "bt_graph_destroy": [c_void_p], "bt_stream": [RT, POINTER(c_void_p)], "bt_stream_read": [RT, U64, U64, U64],
  "bt_bfp_pack": [RT, c_int, U64, c_int, I64, I64, I64, I64, I64, I64, U64, U64],
  "bt_bfp_unpack": [RT, c_int, U64, U64, I64, I64, I64, U64],
  "bt_bfp_columns": [RT, c_int, U64, U64, I64, I64, I64, U64],
  "bt_bfp_range": [RT, c_int, U64, U64, I64, I64, I64, U64],
  "bt_bf16_columns": [RT, U64, I64, I64, I64, I64, I64, I64, U64],
  "bt_columns_unpack": [RT, c_int, U64, I64, I64, I64, U64],
  "bt_elementwise": [RT, POINTER(Program), I64, I64, I64, POINTER(Operand)],
  "bt_reduce": [RT, POINTER(Program), c_int, c_int, I64, I64, I64, I64, I64, POINTER(Operand)],
  "bt_matmul": [RT, POINTER(Operand), c_int, U64, I64, I64, I64, I64, I64, POINTER(Program), POINTER(Operand)],
  "bt_attention": [RT, POINTER(AttentionArgs)],
  "bt_attention_scratch": [POINTER(AttentionArgs), POINTER(c_uint64)],
  "bt_attention_noalloc": [RT, POINTER(AttentionArgs)],
  "bt_matmul_row": [RT, POINTER(RowArgs)], "bt_rope_put": [RT, POINTER(RopeArgs)],
  "bt_put_bfp": [RT, c_int, U64, U64, I64, I64, I64, I64, I64, U64, I64, U64, I64, I64],
  "bt_matmul_row_rope": [RT, POINTER(RowArgs), POINTER(RopeArgs)],
  "bt_matmul_rope_put": [RT, POINTER(Operand), c_int, U64, I64, I64, I64, POINTER(RopeArgs)],
  "bt_matmul_residual_rms": [RT, POINTER(Operand), c_int, U64, I64, I64, I64, U64, I64, U64, I64, U64, c_float, U64,
                             I64],
  "bt_matmul_swiglu": [RT, POINTER(Operand), c_int, U64, I64, I64, I64, POINTER(Operand)],
  "bt_rms_rows": [RT, U64, I64, I64, I64, U64, c_float, U64, I64],
  "bt_gather": [RT, c_int, U64, I64, I64, I64, U64, I64, U64, I64],
  "bt_put": [RT, c_int, U64, I64, I64, I64, I64, I64, U64, I64, U64, I64, I64],
  "bt_topk": [RT, c_int, U64, I64, I64, I64, I64, I64, c_int32, c_int32, U64, I64, I64, U64, U64],
}

_lib = None


def load():
  """The loaded library. Raises RuntimeError when it hasn't been built: there is no other implementation."""
  global _lib
  if _lib is None:
    if not os.path.exists(PATH):
      raise RuntimeError(f"{PATH} is missing: build it with `python -m baretile_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(PATH)
    lib.bt_last_error.restype, lib.bt_last_error.argtypes = c_char_p, []
    for name, args in SIGNATURES.items():
      f = getattr(lib, name)
      f.restype, f.argtypes = c_int, args
    if lib.bt_version() != 1: raise RuntimeError("libbaretile_amd.so has another ABI version; rebuild it")
    _lib = lib
  return _lib


EXCEPTIONS = {EINVAL: ValueError, ESTATE: RuntimeError, ETIMEOUT: TimeoutError, ENOMEM: MemoryError}


def check(status):
  if status != OK:
    message = load().bt_last_error().decode(errors="replace")
    raise EXCEPTIONS.get(status, RuntimeError)(message)


def call(name, *args):
  """Calls bt_<name> and raises on a nonzero status."""
  check(getattr(load(), "bt_" + name)(*args))


def device_count():
  n = c_int(0)
  call("device_count", byref(n))
  return n.value


def operand(ptr, dtype, sb=0, sr=0, sc=1, rep=1, cyc=0):
  return Operand(ptr, sb, sr, sc, DTYPES[dtype] if isinstance(dtype, str) else dtype, rep, cyc, 0)
