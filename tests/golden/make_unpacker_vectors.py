"""Writes unpacker_bf16s.npz: the reference unpacker's bf16 bits (baretile/tensor.py:1093-1104, `_bf16s`) for every
stored bfp8 byte at every exponent byte (65,536 values) and every bfp4 nibble at every exponent byte (4,096), so that
oracle.bfp.decode_bits is pinned to the reference's own code over its whole domain, edge rules included (a zero
magnitude with its sign set, exponents that wrap mod 256), not to a restatement of them.

Run where /root/reference is present: `python tests/golden/make_unpacker_vectors.py`. The reference needs Python >= 3.12
as a package (its kernels.py does not parse under 3.10), so this takes the one function from tensor.py's syntax tree
and runs it alone; it uses only the standard `array` module. Nothing of the reference is kept here but the vectors.
"""
import array
import ast
import os

import numpy as np

SRC = "/root/reference/baretile/tensor.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "unpacker_bf16s.npz")


def reference_unpacker():
  tree = ast.parse(open(SRC).read())
  fn = next(n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name == "_bf16s")
  ns = {"array": array}
  exec(compile(ast.Module(body=[fn], type_ignores=[]), SRC, "exec"), ns)
  return ns["_bf16s"]


def main():
  unpack = reference_unpacker()
  # bfp8: a tile is 64 exponent bytes (one a run of 16 values) then 1024 value bytes. Tile t holds exponents 4t .. 4t+3,
  # each over 16 runs that together carry all 256 value bytes.
  bits8 = np.zeros((256, 256), np.uint16)
  for t in range(64):
    exps = np.repeat(np.arange(4 * t, 4 * t + 4), 16)  # 64 runs
    vals = np.tile(np.arange(256), 4)                  # 1024 values, run r = values 16r .. 16r+15
    tile = bytes(exps.astype(np.uint8)) + bytes(vals.astype(np.uint8))
    out = np.frombuffer(unpack(tile, "bfp8"), np.uint16)
    bits8[4 * t:4 * t + 4] = out.reshape(4, 256)
  # bfp4: 64 exponent bytes then 512 value bytes, value i the nibble (byte i // 2) >> 4 (i % 2). Tile t holds exponents
  # 64t .. 64t + 63, one a run, each run's 16 values the 16 nibbles.
  bits4 = np.zeros((256, 16), np.uint16)
  for t in range(4):
    exps = np.arange(64 * t, 64 * t + 64)
    nib = np.tile(np.arange(16), 64)  # 1024 values
    packed = (nib[0::2] | nib[1::2] << 4).astype(np.uint8)
    tile = bytes(exps.astype(np.uint8)) + bytes(packed)
    out = np.frombuffer(unpack(tile, "bfp4"), np.uint16)
    bits4[64 * t:64 * t + 64] = out.reshape(64, 16)
  # bits8[e, x]: exponent byte e, stored byte x; bits4[e, n]: exponent byte e, stored nibble n
  np.savez_compressed(OUT, bits8=bits8, bits4=bits4)
  print("wrote", OUT)


if __name__ == "__main__":
  main()
