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


def test_struct_sizes_match_the_header(tmp_path):
  # the ctypes mirrors against what a C compiler makes of include/baretile_amd.h: sizes and every field's offset
  import shutil, subprocess
  from baretile_amd import _lib
  cc = shutil.which("gcc") or shutil.which("cc")
  if cc is None: pytest.skip("no C compiler")
  structs = {"bt_operand": _lib.Operand, "bt_inst": _lib.Inst, "bt_program": _lib.Program,
             "bt_attention_args": _lib.AttentionArgs, "bt_row_args": _lib.RowArgs, "bt_rope_args": _lib.RopeArgs}
  cname = {("bt_program", "inputs"): "in"}  # Python can't name a field `in`
  lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "baretile_amd.h"', "int main(void) {"]
  for name, cls in structs.items():
    lines.append(f'  printf("{name} %zu\\n", sizeof({name}));')
    for field, *_ in cls._fields_:
      lines.append(f'  printf("{name}.{field} %zu\\n", offsetof({name}, {cname.get((name, field), field)}));')
  lines.append("  return 0; }")
  src = tmp_path / "sizes.c"
  src.write_text("\n".join(lines) + "\n")
  exe = tmp_path / "sizes"
  subprocess.run([cc, "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
  got = dict(l.split() for l in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines())
  for name, cls in structs.items():
    assert int(got[name]) == ctypes.sizeof(cls), name
    for field, *_ in cls._fields_:
      assert int(got[f"{name}.{field}"]) == getattr(cls, field).offset, (name, field)
