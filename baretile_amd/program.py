"""Assembles bt_program structs: the per-element instruction lists that the elementwise, reduction and matmul-epilogue
kernels evaluate (include/baretile_amd.h).

Instructions are built on virtual registers, one per value. build() maps them onto the 16 machine registers by
liveness, so an expression of up to 48 instructions fits as long as no more than 16 values are alive at once.
Register 0 is the matmul value in an epilogue, and is never reused there.
"""
import struct
from baretile_amd import _lib


class Program:
  def __init__(self, dtype, epilogue=False):
    if dtype not in ("bf16", "fp32", "int32"): raise ValueError(f"a program computes in bf16, fp32 or int32, not {dtype}")
    self.dtype, self.epilogue = dtype, epilogue
    self.insts = []  # (op, dst vreg, a, b, c, imm); a/b/c are vregs, or an input index for load
    self.inputs = []  # Operand structs
    self.nv = 1  # vreg 0: the epilogue's value
    self.keys = {}  # input key -> index, and (op, operands) -> vreg, for sharing

  def value(self):
    """The epilogue's incoming value (the matmul result) as a vreg."""
    if not self.epilogue: raise ValueError("only a matmul epilogue has an incoming value")
    return 0

  def _new(self):
    self.nv += 1
    return self.nv - 1

  def input(self, op, key=None):
    """Registers an input Operand; the same key returns the same index."""
    if key is not None and ("in", key) in self.keys: return self.keys["in", key]
    if len(self.inputs) == _lib.MAX_INPUTS: raise ValueError(f"a program has at most {_lib.MAX_INPUTS} inputs")
    self.inputs.append(op)
    if key is not None: self.keys["in", key] = len(self.inputs) - 1
    return len(self.inputs) - 1

  def load(self, index):
    k = ("load", index)
    if k not in self.keys:
      self.keys[k] = v = self._new()
      self.insts.append((_lib.OP["load"], v, index, 0, 0, 0))
    return self.keys[k]

  def const(self, value):
    """A constant in the program's dtype: a float is rounded to bf16 as an upload rounds (nearest even) for bf16."""
    if self.dtype == "int32": bits = int(value) & 0xFFFFFFFF
    else:
      bits = struct.unpack("<I", struct.pack("<f", float(value)))[0]
      if self.dtype == "bf16":
        if bits & 0x7FFFFFFF > 0x7F800000: bits = (bits >> 16 | 0x40) << 16
        else: bits = ((bits + 0x7FFF + (bits >> 16 & 1)) >> 16) << 16
    k = ("const", bits)
    if k not in self.keys:
      self.keys[k] = v = self._new()
      self.insts.append((_lib.OP["const"], v, 0, 0, 0, bits))
    return self.keys[k]

  def op(self, name, a, b=0, c=0):
    k = (name, a, b, c)
    if k not in self.keys:
      self.keys[k] = v = self._new()
      self.insts.append((_lib.OP[name], v, a, b, c, 0))
    return self.keys[k]

  def build(self, result):
    """The bt_program struct, with registers allocated. result is the vreg of the value to store."""
    n = len(self.insts)
    if n > _lib.MAX_INST: raise ValueError(f"a program has at most {_lib.MAX_INST} instructions, not {n}")
    load = _lib.OP["load"]
    last = {}  # vreg -> index of its last reader
    for i, (op, dst, a, b, c, imm) in enumerate(self.insts):
      if op == load: continue
      for s in self._reads(op, a, b, c): last[s] = i
    last[result] = n
    phys, free = {}, [r for r in range(_lib.MAX_REGS - 1, 0 if self.epilogue else -1, -1)]
    if self.epilogue: phys[0] = 0
    p = _lib.Program()
    p.n_inst, p.n_inputs, p.dtype = n, len(self.inputs), _lib.DTYPES[self.dtype]
    for i, op in enumerate(self.inputs): p.inputs[i] = op
    const = _lib.OP["const"]
    for i, (op, dst, a, b, c, imm) in enumerate(self.insts):
      srcs = [] if op in (load, const) else self._reads(op, a, b, c)
      regs = [phys[s] for s in srcs]
      for s in set(srcs):  # a register whose value dies here can take the result
        if last.get(s) == i and not (self.epilogue and s == 0): free.append(phys.pop(s))
      if not free: raise ValueError(f"a program needs more than {_lib.MAX_REGS} live values")
      d = free.pop()
      if dst in last: phys[dst] = d
      else: free.append(d)  # never read
      ra, rb, rc = (a, 0, 0) if op == load else tuple(regs + [0, 0, 0])[:3]
      p.inst[i] = _lib.Inst(op, d, ra, rb, rc, (0, 0, 0), imm)
    p.result = phys[result]
    return p

  UNARY = {"mov", "neg", "relu", "exp", "exp2", "log", "log2", "sqrt", "recip", "rsqrt", "sin", "cos", "sigmoid", "silu",
           "gelu", "tanh", "ftob"}

  def _reads(self, op, a, b, c):
    name = _lib.OPS[op]
    if name == "const": return []
    if name in self.UNARY: return [a]
    if name == "where": return [a, b, c]
    return [a, b]
