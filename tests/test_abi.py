"""The C ABI: the built library loads and exports every function include/baretile_amd.h declares. CPU only: nothing
here calls into a GPU."""
import ctypes, os, re
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "baretile_amd.h")


def declared():
  text = open(HEADER).read()
  text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
  return sorted(set(re.findall(r"\b(bt_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_abi():
  names = declared()
  assert {"bt_open", "bt_close", "bt_alloc", "bt_matmul", "bt_attention", "bt_bfp_pack", "bt_bfp_unpack"} <= set(names)


def test_library_exports_every_declared_symbol():
  from baretile_amd import _lib
  lib = ctypes.CDLL(_lib.PATH)
  missing = [n for n in declared() if not hasattr(lib, n)]
  assert not missing, missing
  # the ctypes table covers the same functions
  assert set(declared()) == set(_lib.SIGNATURES) | {"bt_last_error"}


def test_load_and_version():
  from baretile_amd import _lib
  lib = _lib.load()
  assert lib.bt_version() == 1


def test_errors_map_to_exceptions():
  from baretile_amd import _lib
  lib = _lib.load()
  # a null runtime is a bad argument, whatever the machine has
  with pytest.raises(ValueError, match="no runtime"): _lib.call("wait", None, 1.0)
  with pytest.raises(ValueError, match="no runtime"): _lib.call("alloc", None, 16, ctypes.byref(ctypes.c_uint64()))


def test_struct_sizes_match_the_header():
  from baretile_amd import _lib
  assert ctypes.sizeof(_lib.Operand) == 48 and ctypes.sizeof(_lib.Inst) == 12
  assert ctypes.sizeof(_lib.Program) == 16 + 12 * _lib.MAX_INST + 48 * _lib.MAX_INPUTS
  assert ctypes.sizeof(_lib.AttentionArgs) == 5 * 8 + 9 * 8 + 6 * 4
