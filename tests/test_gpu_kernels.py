"""Kernel parity through the C ABI, against the CPU oracle (oracle/). Needs a GPU.

Block floats are checked bit for bit (exponent and magnitude planes, decoded bf16 bits); matmuls bit for bit where the
reference's tests are (small integers, A @ I, X @ diag, block float == bf16 of its values, fused == unfused) and
otherwise within the reference's bound 2^-8 * (|a| @ |b|) (test_kernels.py:653-663); attention within 1.1% as
test_kernels.py:1290-1292 allows, and exactly at its extremes (test_kernels.py:1323-1337).
"""
import ctypes
import numpy as np
import pytest

from baretile_amd import _lib
from baretile_amd.program import Program
from helpers import up, down, bits_to_float
from oracle import bfp as B, ops

pytestmark = pytest.mark.gpu
FMT = {"bfp8": _lib.BFP8, "bfp4": _lib.BFP4}


def plain_sizes(batch, rows, cols, fmt):
  runs = -(-cols // 16)
  vals = batch * rows * runs * (16 if fmt == "bfp8" else 8)
  return batch * rows * runs, vals


def pack(rt, x, fmt, src="bf16"):
  """x float array (batch, rows, cols) -> device planes (exps, vals)."""
  x = np.asarray(x)
  if x.ndim == 2: x = x[None]
  b, r, c = x.shape
  data = B.bf16_bits(x) if src == "bf16" else x.astype(np.float32)
  d = up(rt, data)
  ne, nv = plain_sizes(b, r, c, fmt)
  exps, vals = rt.dram_alloc(ne), rt.dram_alloc(nv)
  rt.run("pack", "bfp_pack", FMT[fmt], d, _lib.DTYPES[src], b, r, c, r * c, c, 1, exps, vals)
  return exps, vals


def columns(rt, exps, vals, fmt, b, k, n):
  tb = 1088 if fmt == "bfp8" else 576
  dst = rt.dram_alloc(b * -(-n // 16) * -(-k // 64) * tb)
  rt.run("columns", "bfp_columns", FMT[fmt], exps, vals, b, k, n, dst)
  return dst


def bf16_columns(rt, w):
  w = np.asarray(w)
  if w.ndim == 2: w = w[None]
  b, k, n = w.shape
  d = up(rt, B.bf16_bits(w))
  dst = rt.dram_alloc(b * -(-n // 16) * -(-k // 64) * 2048)
  rt.run("columns", "bf16_columns", d, b, k, n, k * n, n, 1, dst)
  return dst


def matmul(rt, x, bcols, fmt, b_batch, n, out="bf16", prog=None):
  """x float (batch, m, k) bf16-rounded on upload; returns the result as float32 (batch, m, n)."""
  x = np.asarray(x)
  if x.ndim == 2: x = x[None]
  batch, m, k = x.shape
  a = _lib.operand(up(rt, B.bf16_bits(x)), "bf16", m * k, k, 1)
  size = 2 if out == "bf16" else 4
  o = rt.dram_alloc(batch * m * n * size)
  rt.run("matmul", "matmul", ctypes.byref(a), _lib.DTYPES[fmt], bcols, b_batch, batch, m, k, n,
         ctypes.byref(prog) if prog is not None else None, ctypes.byref(_lib.operand(o, out, m * n, n, 1)))
  got = down(rt, o, (batch, m, n), np.uint16 if out == "bf16" else np.float32)
  return bits_to_float(got) if out == "bf16" else got.copy()


def bfp_values(w, fmt):
  """The oracle's block-float values of w, padding the last axis to whole runs of 16 with zeros as the planes do."""
  w = np.asarray(w)
  pad = -w.shape[-1] % 16
  return B.bfp(np.pad(w, [(0, 0)] * (w.ndim - 1) + [(0, pad)]), fmt)[..., :w.shape[-1]]


def packed(v):  # bf16 rounding half up, as a packed result rounds (test/conftest.py:11-13)
  b = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
  return (((b + 0x8000) >> 16) << 16).astype(np.uint32).view(np.float32)


# ---- block floats ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
@pytest.mark.parametrize("src", ["bf16", "fp32"])
def test_pack_matches_oracle_bit_for_bit(rt, fmt, src):
  rng = np.random.default_rng(5)  # test_models.py:587-593: N(0,1) * e^N(0,2), (64, 96)
  for shape in ((64, 96), (3, 33, 40), (1, 7, 16)):
    x = rng.normal(0, 1, shape) * np.exp(rng.normal(0, 2, shape))
    x = x.astype(np.float32)
    if len(shape) == 2: x = x[None]
    b, r, c = x.shape
    exps, vals = pack(rt, x, fmt, src)
    top, q = B.bfp_fields(np.pad(x, ((0, 0), (0, 0), (0, -c % 16))), fmt)
    ne, nv = plain_sizes(b, r, c, fmt)
    got_e = down(rt, exps, (ne,), np.uint8)
    assert np.array_equal(got_e, top.reshape(-1))
    raw = down(rt, vals, (nv,), np.uint8)
    if fmt == "bfp8": got_q = raw.view(np.int8).astype(np.int64)
    else:
      nib = np.stack([raw & 15, raw >> 4], -1).reshape(-1).astype(np.int64)
      got_q = np.where(nib >= 8, nib - 16, nib)
    assert np.array_equal(got_q, q.reshape(-1).astype(np.int64))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_unpack_matches_unpacker_rule(rt, fmt):
  rng = np.random.default_rng(5)
  x = (rng.normal(0, 1, (64, 96)) * np.exp(rng.normal(0, 2, (64, 96)))).astype(np.float32)
  exps, vals = pack(rt, x, fmt)
  out = rt.dram_alloc(64 * 96 * 2)
  rt.run("unpack", "bfp_unpack", FMT[fmt], exps, vals, 1, 64, 96, out)
  got = down(rt, out, (64, 96), np.uint16)
  top, q = B.bfp_fields(x, fmt)
  assert np.array_equal(got, B.decode_fields(top, q, fmt))
  assert np.array_equal(bits_to_float(got), B.bfp(x, fmt).astype(np.float32))
  # test_kernels.py:2096-2103: [2, 3] among zeros reads back as 0x4000, 0x4040
  row = np.zeros((1, 16), np.float32)
  row[0, :2] = [2, 3]
  exps, vals = pack(rt, row, fmt)
  out = rt.dram_alloc(32)
  rt.run("unpack", "bfp_unpack", FMT[fmt], exps, vals, 1, 1, 16, out)
  assert list(down(rt, out, (16,), np.uint16)[:2]) == [0x4000, 0x4040]


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_columns_read_back_unchanged(rt, fmt):
  # like wc.tobytes() == w.tobytes() (test_kernels.py:862, 897): the columns tiles decode to the same bits
  rng = np.random.default_rng(9)
  for b, k, n in ((1, 576, 1536), (2, 100, 40), (1, 64, 16), (1, 130, 33)):
    x = rng.normal(0, 0.02, (b, k, n)).astype(np.float32)
    exps, vals = pack(rt, x, fmt)
    plain = rt.dram_alloc(b * k * n * 2)
    rt.run("unpack", "bfp_unpack", FMT[fmt], exps, vals, b, k, n, plain)
    cols = columns(rt, exps, vals, fmt, b, k, n)
    back = rt.dram_alloc(b * k * n * 2)
    rt.run("unpack", "columns_unpack", FMT[fmt], cols, b, k, n, back)
    assert np.array_equal(down(rt, plain, (b, k, n), np.uint16), down(rt, back, (b, k, n), np.uint16))
  w = B.bf16(rng.normal(0, 1, (2, 70, 50)))
  cols = bf16_columns(rt, w)
  back = rt.dram_alloc(w.size * 2)
  rt.run("unpack", "columns_unpack", _lib.BF16, cols, 2, 70, 50, back)
  assert np.array_equal(down(rt, back, w.shape, np.uint16), B.bf16_bits(w))


# ---- matmul -----------------------------------------------------------------------------------------------------

def test_matmul_exact(rt):
  # test_kernels.py:637-651: small integers with K = 64; A @ I == A; X @ diag(d) is x * d rounded once, half up
  a = np.array([[float((r * 7 + c * 3) % 3 - 1) for c in range(64)] for r in range(32)])
  b = np.array([[float((r * 5 + c) % 3 - 1) for c in range(32)] for r in range(64)])
  assert np.array_equal(matmul(rt, a, bf16_columns(rt, b), "bf16", 1, 32)[0], ops.matmul(a, b))
  rng = np.random.default_rng(1)
  x = B.bf16(rng.uniform(-8, 8, (96, 64)))
  assert np.array_equal(matmul(rt, x, bf16_columns(rt, np.eye(64)), "bf16", 1, 64)[0], x)
  d = B.bf16(rng.uniform(1, 2, 64))
  got = matmul(rt, x, bf16_columns(rt, np.diag(d)), "bf16", 1, 64)[0]
  assert np.array_equal(got, packed((x * d).astype(np.float32)))


def test_matmul_random_within_bound(rt):
  rng = np.random.default_rng(2)
  for m, k, n in ((64, 96, 128), (5, 1000, 77), (1, 576, 960), (130, 200, 48)):
    a, b = B.bf16(rng.uniform(-1, 1, (m, k))), B.bf16(rng.uniform(-1, 1, (k, n)))
    got = matmul(rt, a, bf16_columns(rt, b), "bf16", 1, n)[0]
    assert np.all(np.abs(got - ops.matmul(a, b)) <= ops.matmul_bound(a, b)), (m, k, n)
    got32 = matmul(rt, a, bf16_columns(rt, b), "bf16", 1, n, out="fp32")[0]
    assert np.all(np.abs(got32 - ops.matmul(a, b)) <= 2.0 ** -20 * ops.matmul_bound(a, b) * 256), (m, k, n)


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_bfp_matmul_is_bf16_matmul_of_its_values(rt, fmt):
  # test_kernels.py:709-724, bit for bit, on its shapes
  rng = np.random.default_rng(5)
  for b, m, k, n in ((1, 64, 9000, 40), (1, 1, 768, 2304), (1, 100, 256, 200), (2, 100, 256, 96), (1, 32, 2048, 64)):
    x, w = rng.normal(0, 1, (b, m, k)), rng.normal(0, 1, (b, k, n)).astype(np.float32)
    exps, vals = pack(rt, w, fmt)
    cols = columns(rt, exps, vals, fmt, b, k, n)
    got = matmul(rt, x, cols, fmt, b, n)
    wq = bfp_values(w, fmt)
    want = matmul(rt, x, bf16_columns(rt, wq), "bf16", b, n)
    assert np.array_equal(got, want), (b, m, k, n)
    assert np.all(np.abs(got - ops.matmul(B.bf16(x), wq)) <= ops.matmul_bound(B.bf16(x), wq))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
@pytest.mark.parametrize("rows", [1, 4, 16])
def test_decode_gemv_lm_head_shape(rt, fmt, rows):
  # BASELINE config 2's GEMV at its full size, x [B, 576] @ W [576, 49152]
  rng = np.random.default_rng(0)
  x, w = rng.normal(0, 1, (rows, 576)), rng.standard_normal((576, 49152), dtype=np.float32) * np.float32(0.02)
  exps, vals = pack(rt, w, fmt)
  cols = columns(rt, exps, vals, fmt, 1, 576, 49152)
  got = matmul(rt, x, cols, fmt, 1, 49152)[0]
  xw, wq = B.bf16(x), B.bfp(w, fmt)
  assert np.all(np.abs(got - ops.matmul(xw, wq)) <= ops.matmul_bound(xw, wq))


def test_fused_relu_epilogue_config1(rt):
  # relu(x @ W), x bf16 [128, 576] N(0, 1), W [576, 1536] N(0, 0.02) in bfp8. Fused equals the matmul
  # followed by a relu launch bit for bit, and both are within the bound of the oracle.
  rng = np.random.default_rng(0)
  x, w = rng.normal(0, 1, (128, 576)), rng.normal(0, 0.02, (576, 1536)).astype(np.float32)
  exps, vals = pack(rt, w, "bfp8")
  cols = columns(rt, exps, vals, "bfp8", 1, 576, 1536)
  p = Program("bf16", epilogue=True)
  prog = p.build(p.op("relu", p.value()))
  fused = matmul(rt, x, cols, "bfp8", 1, 1536, prog=prog)[0]
  plain = matmul(rt, x, cols, "bfp8", 1, 1536)[0]
  assert np.array_equal(fused, np.maximum(plain, 0))
  xw, wq = B.bf16(x), B.bfp(w, "bfp8")
  assert np.all(np.abs(fused - np.maximum(ops.matmul(xw, wq), 0)) <= ops.matmul_bound(xw, wq))


@pytest.mark.parametrize("out", ["bf16", "fp32"])
@pytest.mark.parametrize("m", [1, 4, 16, 128, 600])
def test_one_operation_epilogues_equal_the_evaluator(rt, m, out):
  # An epilogue of one operation on the product with no inputs (relu, silu, exp, neg, x * x, x + x) runs as that
  # operation straight on the tile; the same program behind a mov runs
  # through the evaluator. Bit for bit the same, in every kernel the row counts reach (the GEMV, the A-staging kernel,
  # the tiled GEMM) and against the plain product with the operation applied by NumPy where that is exact.
  from baretile_amd.program import Program
  rng = np.random.default_rng(m)
  x, w = rng.normal(0, 1, (m, 576)), rng.normal(0, 0.02, (576, 1536)).astype(np.float32)
  exps, vals = pack(rt, w, "bfp8")
  cols = columns(rt, exps, vals, "bfp8", 1, 576, 1536)
  plain = matmul(rt, x, cols, "bfp8", 1, 1536, out=out)[0]
  for name in ("relu", "silu", "exp", "neg", "mul", "add"):
    p, q = Program(out, epilogue=True), Program(out, epilogue=True)
    if name in ("mul", "add"):
      fast = p.build(p.op(name, p.value(), p.value()))
      slow = q.build(q.op(name, q.op("mov", q.value()), q.value()))
    else:
      fast, slow = p.build(p.op(name, p.value())), q.build(q.op(name, q.op("mov", q.value())))
    assert fast.n_inst == 1 and slow.n_inst == 2
    got = matmul(rt, x, cols, "bfp8", 1, 1536, out=out, prog=fast)[0]
    want = matmul(rt, x, cols, "bfp8", 1, 1536, out=out, prog=slow)[0]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
  relu = matmul(rt, x, cols, "bfp8", 1, 1536, out=out,
                prog=(lambda p: p.build(p.op("relu", p.value())))(Program(out, epilogue=True)))[0]
  assert np.array_equal(relu, np.maximum(plain, 0))
  neg = matmul(rt, x, cols, "bfp8", 1, 1536, out=out,
               prog=(lambda p: p.build(p.op("neg", p.value())))(Program(out, epilogue=True)))[0]
  assert np.array_equal(neg, -plain)


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
@pytest.mark.parametrize("m,k,n", [(16, 576, 49152), (20, 576, 40000), (7, 320, 1000), (32, 768, 4096)])
def test_short_k_rows_with_a_in_lds(rt, fmt, m, k, n):
  # 5 to 32 rows and K of at most 12 chunks: A staged whole in LDS once a block of 4 runs, partial last blocks. Bit for bit the same product 4 rows at a time (the GEMV, same K order), within the
  # reference's bound of the oracle, and with a relu epilogue program.
  rng = np.random.default_rng(m * n + k)
  x, w = rng.normal(0, 1, (m, k)), rng.normal(0, 0.05, (k, n)).astype(np.float32)
  exps, vals = pack(rt, w, fmt)
  cols, wq = columns(rt, exps, vals, fmt, 1, k, n), bfp_values(w, fmt)
  got = matmul(rt, x, cols, fmt, 1, n)[0]
  rows4 = np.concatenate([matmul(rt, x[i:i + 4], cols, fmt, 1, n)[0] for i in range(0, m, 4)])
  assert np.array_equal(got, rows4)
  xw = B.bf16(x)
  assert np.all(np.abs(got - ops.matmul(xw, wq)) <= ops.matmul_bound(xw, wq))
  p = Program("bf16", epilogue=True)
  relu = matmul(rt, x, cols, fmt, 1, n, prog=p.build(p.op("relu", p.value())))[0]
  assert np.array_equal(relu, np.maximum(got, 0))


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bfp4"])
@pytest.mark.parametrize("m,k,n,out", [(32, 4096, 4096, "fp32"), (20, 1024, 1000, "bf16"), (5, 14336, 512, "fp32"),
                                       (17, 896, 3000, "bf16"), (32, 4096, 28672, "bf16"), (12, 2048, 16384, "fp32")])
def test_split_k_rows(rt, fmt, m, k, n, out):
  # 5 to 32 rows against a long K. K a multiple of 512: the streaming kernel, A through a two-stage LDS ring, either
  # one split with the epilogue in the kernel (28672 and 16384 columns: 256 groups of runs or more) or splits of whole
  # stages summed in order by a second launch. Otherwise (896 = 14 chunks) splits of 8 or 16 chunks, each block staging
  # its split of A. Within the reference's bound of the oracle; a block-float product bit for bit the bf16 product of
  # its values (the kernel and splits depend on the shape alone); the epilogue program (relu, or the residual add into
  # fp32) bit for bit the plain result put through it. Partial runs (1000, 3000), one tile of rows (5, 12) and two.
  rng = np.random.default_rng(m * n + k)
  x, w = rng.normal(0, 1, (m, k)), rng.normal(0, 0.05, (k, n)).astype(np.float32)
  if fmt == "bf16":
    cols, wq = bf16_columns(rt, w), B.bf16(w)
  else:
    exps, vals = pack(rt, w, fmt)
    cols, wq = columns(rt, exps, vals, fmt, 1, k, n), bfp_values(w, fmt)
  plain = matmul(rt, x, cols, fmt, 1, n, out=out)[0]
  xw = B.bf16(x)
  assert np.all(np.abs(plain - ops.matmul(xw, wq)) <= ops.matmul_bound(xw, wq))
  if fmt != "bf16":
    assert np.array_equal(plain, matmul(rt, x, bf16_columns(rt, wq), "bf16", 1, n, out=out)[0])
  p = Program(out, epilogue=True)
  if out == "bf16":
    assert np.array_equal(matmul(rt, x, cols, fmt, 1, n, out=out, prog=p.build(p.op("relu", p.value())))[0],
                          np.maximum(plain, 0))
  else:
    res = B.bf16(rng.normal(0, 1, (m, n)))
    prog = p.build(p.op("add", p.value(), p.load(p.input(_lib.operand(up(rt, res.astype(np.float32)), "fp32", m * n, n, 1)))))
    assert np.array_equal(matmul(rt, x, cols, fmt, 1, n, out=out, prog=prog)[0], (plain + res).astype(np.float32))


# (rows, K, N, output): rows > 64 run the tiled GEMM, except up to 256 rows when its 128 x 128 blocks would be fewer
# than 128 (then the skinny kernel: 96 x 1536 here). With bf16 B (block floats unpacked to it from 512 rows up) and
# K in 32s, 2048 x 8192 takes 256 x 256 blocks, 2048 x 4096 (fp32 with the residual) and 1000 x 4096 blocks of 128
# rows; 1000 and 520 leave partial blocks, chunks of K and runs of N. bfp4 B with K in whole chunks (256, 192, 640)
# is read by the GEMM as it is stored from 512 rows up. 2048 x 6144 takes blocks of 256 x 192 (256 of them, one round
# of the CUs, where 256 x 256 would leave a quarter idle).
GEMM_CASES = [(300, 1000, 520, "bf16"), (96, 576, 1536, "fp32"), (2048, 256, 8192, "bf16"), (2048, 192, 4096, "fp32"),
              (160, 320, 8192, "bf16"), (1000, 224, 4096, "bf16"), (520, 640, 1296, "fp32"), (2048, 320, 6144, "bf16"),
              (2048, 192, 6144, "fp32"), (2048, 128, 8192, "fp32")]


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bfp4"])
@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: "m{}k{}n{}{}".format(*c))
def test_gemm_equals_row_slices(rt, fmt, case):
  # The GEMM sums each output in the same order as the decode kernels (64-row chunks of K, lower half then upper), so
  # it equals, bit for bit, the same product computed 64 rows at a time; with a fused epilogue (relu for bf16, a
  # residual add for fp32) as well. And it is within the reference's bound of the oracle.
  m, k, n, out = case
  rng = np.random.default_rng(m + k + n)
  x, w = rng.normal(0, 1, (m, k)), rng.normal(0, 0.05, (k, n)).astype(np.float32)
  if fmt == "bf16":
    cols, wq = bf16_columns(rt, w), B.bf16(w)
  else:
    exps, vals = pack(rt, w, fmt)
    cols, wq = columns(rt, exps, vals, fmt, 1, k, n), bfp_values(w, fmt)
  p = Program(out, epilogue=True)
  if out == "bf16": prog = p.build(p.op("relu", p.value()))
  else:
    res = B.bf16(rng.normal(0, 1, (m, n)))
    prog = p.build(p.op("add", p.value(), p.load(p.input(_lib.operand(up(rt, res.astype(np.float32)), "fp32", m * n, n, 1)))))
  got = matmul(rt, x, cols, fmt, 1, n, out=out, prog=prog)[0]
  plain = matmul(rt, x, cols, fmt, 1, n, out=out)[0]
  sliced = np.concatenate([matmul(rt, x[i:i + 64], cols, fmt, 1, n, out=out)[0] for i in range(0, m, 64)])
  assert np.array_equal(plain, sliced)
  if out == "bf16": assert np.array_equal(got, np.maximum(plain, 0))
  else: assert np.array_equal(got, (plain + res).astype(np.float32))
  xw = B.bf16(x)
  assert np.all(np.abs(plain - ops.matmul(xw, wq)) <= ops.matmul_bound(xw, wq))


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_batched_gemm_block_float_b(rt, fmt):
  # a batch of two products, each against its own block-float B (bfp4: the GEMM reads B's tiles as stored, matrix b
  # at b times a matrix's tile bytes), equals bit for bit the batched product with the bf16 values of B
  rng = np.random.default_rng(31)
  b, m, k, n = 2, 768, 256, 4096
  x, w = rng.normal(0, 1, (b, m, k)), rng.normal(0, 0.05, (b, k, n)).astype(np.float32)
  exps, vals = pack(rt, w, fmt)
  got = matmul(rt, x, columns(rt, exps, vals, fmt, b, k, n), fmt, b, n)
  want = matmul(rt, x, bf16_columns(rt, bfp_values(w, fmt)), "bf16", b, n)
  assert np.array_equal(got, want)
  xw = B.bf16(x)
  for i in range(b):
    assert np.all(np.abs(got[i] - ops.matmul(xw[i], bfp_values(w[i], fmt))) <= ops.matmul_bound(xw[i], bfp_values(w[i], fmt)))


@pytest.mark.parametrize("m,k,n,out", [(520, 640, 1296, "fp32"), (2048, 192, 4096, "bf16")])
def test_gemm_under_capture_reads_bfp4_as_stored(chip, m, k, n, out):
  # A fresh runtime has no scratch, and a capture can't grow it, so a prefill-sized bfp4 product recorded in a graph
  # takes the GEMM that decodes B's tiles as it stages them (128-row blocks here, which the eager product gives to
  # the GEMM on B unpacked to bf16): the replay equals the eager product bit for bit
  from baretile_amd.runtime import Runtime
  rt = Runtime(chip)
  try:
    rng = np.random.default_rng(m + n)
    x, w = rng.normal(0, 1, (m, k)), rng.normal(0, 0.05, (k, n)).astype(np.float32)
    exps, vals = pack(rt, w, "bfp4")
    cols = columns(rt, exps, vals, "bfp4", 1, k, n)
    a = _lib.operand(up(rt, B.bf16_bits(x)), "bf16", m * k, k, 1)
    size = 2 if out == "bf16" else 4
    o = rt.dram_alloc(m * n * size)
    rt.wait()
    g = ctypes.c_void_p()
    _lib.call("graph_begin", rt.handle)
    try:
      _lib.call("matmul", rt.handle, ctypes.byref(a), _lib.BFP4, cols, 1, 1, m, k, n, None,
                ctypes.byref(_lib.operand(o, out, m * n, n, 1)))
    finally:
      _lib.call("graph_end", rt.handle, ctypes.byref(g))
    try:
      for _ in range(2):
        rt.upload(o, b"\xff" * (m * n * size))
        _lib.call("graph_launch", rt.handle, g)
        rt.wait()
        got = down(rt, o, (m, n), np.uint16 if out == "bf16" else np.float32).copy()
        want = matmul(rt, x, cols, "bfp4", 1, n, out=out)[0]
        assert np.array_equal(bits_to_float(got) if out == "bf16" else got, want)
    finally:
      _lib.call("graph_destroy", g)
  finally:
    rt.close()


def test_epilogue_reads_other_inputs(rt):
  # (x @ w + bias) * d - c in one launch equals the unfused chain with bf16 rounding after each op
  rng = np.random.default_rng(3)
  m, k, n = 40, 96, 80
  x, w = B.bf16(rng.uniform(-1, 1, (m, k))), B.bf16(rng.uniform(-1, 1, (k, n)))
  bias, d, c = B.bf16(rng.uniform(-1, 1, (1, n))), B.bf16(rng.uniform(-2, 2, (m, n))), B.bf16(rng.uniform(-1, 1, (m, n)))
  p = Program("bf16", epilogue=True)
  ib = p.load(p.input(_lib.operand(up(rt, B.bf16_bits(bias)), "bf16", 0, 0, 1)))
  idd = p.load(p.input(_lib.operand(up(rt, B.bf16_bits(d)), "bf16", m * n, n, 1)))
  ic = p.load(p.input(_lib.operand(up(rt, B.bf16_bits(c)), "bf16", m * n, n, 1)))
  prog = p.build(p.op("sub", p.op("mul", p.op("add", p.value(), ib), idd), ic))
  got = matmul(rt, x, bf16_columns(rt, w), "bf16", 1, n, prog=prog)[0]
  y = matmul(rt, x, bf16_columns(rt, w), "bf16", 1, n)[0]
  want = packed(packed(packed(y + bias) * d) - c)
  assert np.array_equal(got, want)


# ---- elementwise and reductions --------------------------------------------------------------------------------

def run_elementwise(rt, build, inputs, dtype="bf16", out="bf16"):
  shape = inputs[0].shape
  p = Program(dtype)
  regs = []
  for a in inputs:
    if a.dtype == np.float32 and dtype == "bf16": dev, dt = up(rt, B.bf16_bits(a)), "bf16"
    elif a.dtype == np.int32: dev, dt = up(rt, a), "int32"
    else: dev, dt = up(rt, a.astype(np.float32)), "fp32"
    regs.append(p.load(p.input(_lib.operand(dev, dt, shape[1] * shape[2], shape[2], 1))))
  prog = p.build(build(p, *regs))
  size = 2 if out == "bf16" else 4
  o = rt.dram_alloc(int(np.prod(shape)) * size)
  rt.run("elementwise", "elementwise", ctypes.byref(prog), *shape, ctypes.byref(_lib.operand(o, out, shape[1] * shape[2], shape[2], 1)))
  raw = down(rt, o, shape, np.uint16 if out == "bf16" else (np.int32 if out == "int32" else np.float32))
  return bits_to_float(raw) if out == "bf16" else raw.copy()


def test_elementwise_bf16_rounds_each_result(rt):
  rng = np.random.default_rng(4)
  a, b, c, d = (B.bf16(rng.uniform(-3, 3, (2, 70, 100))).astype(np.float32) for _ in range(4))
  got = run_elementwise(rt, lambda p, a, b, c, d: p.op("sub", p.op("mul", p.op("add", a, b), c), p.op("mul", d, a)), [a, b, c, d])
  want = packed(packed(packed(a + b) * c) - packed(d * a))
  assert np.array_equal(got, want)
  got = run_elementwise(rt, lambda p, a, b, c, d: p.op("relu", p.op("max", a, p.const(0.5))), [a, b, c, d])
  assert np.array_equal(got, np.maximum(a, 0.5))


def test_elementwise_int32_wraps(rt):
  a = np.array([[[2**31 - 1, -2**31, 5, -7]]], np.int32)
  b = np.array([[[1, -1, 9, -7]]], np.int32)
  got = run_elementwise(rt, lambda p, a, b: p.op("add", a, b), [a, b], "int32", "int32")
  assert got.tolist() == [[[-2**31, 2**31 - 1, 14, -14]]]
  got = run_elementwise(rt, lambda p, a, b: p.op("cmplt", a, b), [a, b], "int32", "int32")
  assert got.tolist() == [[[0, 1, 1, 0]]]


def test_reductions(rt):
  rng = np.random.default_rng(8)
  x = rng.normal(0, 1, (3, 50, 300)).astype(np.float32)
  dev = up(rt, x)
  for axis in (0, 1, 2):
    p = Program("fp32")
    prog = p.build(p.load(p.input(_lib.operand(dev, "fp32", 50 * 300, 300, 1))))
    oshape = [3, 50, 300]
    oshape[axis] = 1
    for kind, fn in ((_lib.REDUCE_SUM, np.sum), (_lib.REDUCE_MAX, np.max)):
      o = rt.dram_alloc(int(np.prod(oshape)) * 4)
      rt.run("reduce", "reduce", ctypes.byref(prog), kind, axis, 3, 50, 300, 0, 0,
             ctypes.byref(_lib.operand(o, "fp32", oshape[1] * oshape[2], oshape[2], 1)))
      got = down(rt, o, oshape, np.float32)
      assert np.allclose(got, fn(x.astype(np.float64), axis=axis, keepdims=True), rtol=1e-5, atol=1e-4), (axis, kind)


# ---- attention --------------------------------------------------------------------------------------------------

def attend(rt, q, k, v, places, window=0, parts=0):
  """q (E, rows, hd), k/v (E/rep, keys, hd), places (1|E, rows) -> bf16 result as float32."""
  E, rows, hd = q.shape
  kvh, keys, _ = k.shape
  dq, dk, dv = (up(rt, B.bf16_bits(t)) for t in (q, k, v))
  dp = up(rt, np.asarray(places, np.int32))
  o = rt.dram_alloc(E * rows * hd * 2)
  args = _lib.AttentionArgs(dq, dk, dv, o, dp, rows * hd, hd, keys * hd, hd, keys * hd, hd, rows * hd, hd,
                            rows if np.asarray(places).shape[0] > 1 else 0, E, E // kvh, rows, keys, hd, window, parts,
                            0, 0, 0)
  need = ctypes.c_uint64()
  _lib.call("attention_scratch", ctypes.byref(args), ctypes.byref(need))
  if need.value:
    args.scratch, args.scratch_bytes = rt.dram_alloc(need.value), need.value
  rt.run("attention", "attention", ctypes.byref(args))
  return bits_to_float(down(rt, o, (E, rows, hd), np.uint16))


# (heads, rows, head width, keys, heads per key head, window, parts): decode tiles (rep * rows <= 16) in one part and
# split into parts, prefill tiles, windows, and BASELINE config 4's decode shape; in one part, 256 keys give each of
# a decode block's 4 waves one 64-key block (only its last step) and 320 give the first wave two (a step that fetches
# the next block, then the last); 5 to 8 key blocks with the parts left to the library split into parts of two
# blocks and their combine (320, 384, 450, 500 and 512 keys: an odd block, two tiles, a window, one query head a key
# head)
ATTENTION_CASES = [(4, 8, 64, 96, 2, 0, 0), (2, 40, 128, 200, 1, 50, 0), (8, 1, 128, 512, 4, 0, 0),
                   (8, 1, 64, 256, 4, 0, 1), (8, 1, 128, 320, 4, 0, 1), (8, 1, 64, 320, 4, 0, 0),
                   (16, 3, 64, 384, 8, 0, 0), (8, 2, 128, 450, 4, 60, 0), (4, 1, 128, 500, 1, 0, 0),
                   (32, 1, 128, 4096, 4, 0, 0), (9, 32, 64, 160, 3, 0, 0), (9, 1, 64, 160, 3, 0, 0),
                   (8, 1, 128, 1000, 4, 0, 7), (8, 2, 64, 700, 4, 100, 0), (8, 256, 128, 300, 4, 0, 0),
                   (6, 130, 64, 130, 3, 17, 0), (32, 1, 128, 16384, 4, 0, 0), (16, 600, 128, 600, 4, 0, 0),
                   (6, 333, 64, 400, 3, 0, 0), (8, 1, 128, 512, 4, 0, 8), (8, 2, 64, 300, 4, 30, 5),
                   (16, 1, 64, 640, 4, 0, 16)]


@pytest.mark.parametrize("case", ATTENTION_CASES, ids=lambda c: "e{}r{}d{}k{}rep{}w{}p{}".format(*c))
def test_attention_matches_oracle(rt, case):
  e, rows, hd, keys, rep, window, parts = case
  rng = np.random.default_rng(43 + sum(case))
  q, k, v = (B.bf16(rng.normal(0, 1, s)) for s in ((e, rows, hd), (e // rep, keys, hd), (e // rep, keys, hd)))
  q = B.bf16(q / np.sqrt(hd))
  if rows == keys:  # causal prefill from position 0
    places = np.broadcast_to(np.arange(rows), (e, rows))
  else:
    places = rng.integers(max(0, keys - rows - 60), keys, (e, rows))
  got = attend(rt, q, k, v, places, window, parts)
  want = ops.attention(q, k, v, places[..., None], window, rep)
  assert np.allclose(got, want, rtol=0.011, atol=0.011), (case, np.abs(got - want).max())


@pytest.mark.parametrize("keys", [512, 4096, 16384])
def test_attention_config4_batch8_decode(rt, keys):
  # BASELINE config 4's decode at batch 8 (32 query and 8 key heads of 128 a batch entry, the entries as extra heads
  # of one call, each over its own full cache), against the oracle entry by entry
  rng = np.random.default_rng(keys)
  q = B.bf16(rng.standard_normal((256, 1, 128), dtype=np.float32) / np.float32(np.sqrt(128)))
  k = B.bf16(rng.standard_normal((64, keys, 128), dtype=np.float32))
  v = B.bf16(rng.standard_normal((64, keys, 128), dtype=np.float32))
  places = np.full((256, 1), keys - 1)
  got = attend(rt, q, k, v, places)
  for e in range(8):
    want = ops.attention(q[32 * e:32 * e + 32], k[8 * e:8 * e + 8], v[8 * e:8 * e + 8], places[:32, :, None], 0, 4)
    assert np.allclose(got[32 * e:32 * e + 32], want, rtol=0.011, atol=0.011), (e, np.abs(got[32 * e:32 * e + 32] - want).max())


def test_split_decode_is_the_same_call_after_call(rt):
  # A decode split into parts and combined: the same call again, a call with other parts between (sharing the
  # output), and replays of a recorded graph of two calls all give the first call's bits, within the reference's
  # bound of the oracle
  rng = np.random.default_rng(77)
  E, kvh, keys, hd = 64, 16, 3000, 128  # two batch entries of 32 over 8 key heads
  q = B.bf16(rng.standard_normal((E, 1, hd), dtype=np.float32) / np.float32(np.sqrt(hd)))
  k, v = (B.bf16(rng.standard_normal((kvh, keys, hd), dtype=np.float32)) for _ in range(2))
  places = rng.integers(keys // 2, keys, (E, 1))
  dq, dk, dv = (up(rt, B.bf16_bits(t)) for t in (q, k, v))
  dp = up(rt, np.asarray(places, np.int32))
  o = rt.dram_alloc(E * hd * 2)

  def make(parts):
    args = _lib.AttentionArgs(dq, dk, dv, o, dp, hd, hd, keys * hd, hd, keys * hd, hd, hd, hd, 1, E, E // kvh, 1, keys,
                              hd, 0, parts, 0, 0, 0)
    need = ctypes.c_uint64()
    _lib.call("attention_scratch", ctypes.byref(args), ctypes.byref(need))
    assert need.value > 0  # split into parts
    args.scratch, args.scratch_bytes = rt.dram_alloc(need.value), need.value
    return args

  def result():
    rt.wait()
    return down(rt, o, (E, 1, hd), np.uint16).copy()

  auto, seven = make(0), make(7)
  rt.run("attention", "attention", ctypes.byref(auto))
  first = result()
  want = np.concatenate([ops.attention(q[32 * b:32 * b + 32], k[8 * b:8 * b + 8], v[8 * b:8 * b + 8],
                                       places[32 * b:32 * b + 32, :, None], 0, 4) for b in range(2)])
  assert np.allclose(bits_to_float(first), want, rtol=0.011, atol=0.011)
  for args in (auto, seven, auto):
    rt.upload(o, b"\xff" * (E * hd * 2))
    rt.run("attention", "attention", ctypes.byref(args))
    got = result()
    if args is auto: assert np.array_equal(got, first)
    else: assert np.allclose(bits_to_float(got), want, rtol=0.011, atol=0.011)
  g = ctypes.c_void_p()
  _lib.call("graph_begin", rt.handle)
  try:
    _lib.call("attention", rt.handle, ctypes.byref(auto))
    _lib.call("attention", rt.handle, ctypes.byref(auto))
  finally:
    _lib.call("graph_end", rt.handle, ctypes.byref(g))
  try:
    for _ in range(3):
      rt.upload(o, b"\xff" * (E * hd * 2))
      _lib.call("graph_launch", rt.handle, g)
      assert np.array_equal(result(), first)
  finally:
    _lib.call("graph_destroy", g)


def test_attention_config4_causal_prefill(rt):
  # BASELINE config 4's prefill: 2048 rows over their own 2048 keys, causal, 32 query and 8 key heads of 128, against
  # the oracle one key head (and its 4 query heads) at a time
  rng = np.random.default_rng(2048)
  q = B.bf16(rng.standard_normal((32, 2048, 128), dtype=np.float32) / np.float32(np.sqrt(128)))
  k = B.bf16(rng.standard_normal((8, 2048, 128), dtype=np.float32))
  v = B.bf16(rng.standard_normal((8, 2048, 128), dtype=np.float32))
  places = np.broadcast_to(np.arange(2048), (32, 2048))
  got = attend(rt, q, k, v, places)
  for h in range(8):
    want = ops.attention(q[4 * h:4 * h + 4], k[h:h + 1], v[h:h + 1], places[4 * h:4 * h + 4, :, None], 0, 4)
    assert np.allclose(got[4 * h:4 * h + 4], want, rtol=0.011, atol=0.011), (h, np.abs(got[4 * h:4 * h + 4] - want).max())


@pytest.mark.parametrize("slots,rep,part", [(4, 3, 100), (8, 4, 256), (16, 4, 64)])
def test_attention_firsts_keep_each_slot_in_its_region(rt, slots, rep, part):
  # one query row per slot, the slots' caches side by side in one (kv, slots * part, hd) cache: with each row's first
  # key at its slot's first row, every row sees only its own region (llama.py:293-318). 8 or 16 slots of 4 heads make
  # 2 or 4 tiles of 16 query rows per key head.
  rng = np.random.default_rng(slots * rep)
  kvh, hd = 2, 128
  E = kvh * rep
  q = B.bf16(rng.normal(0, 1, (E, slots, hd)) / np.sqrt(hd))
  k, v = (B.bf16(rng.normal(0, 1, (kvh, slots * part, hd))) for _ in range(2))
  at = rng.integers(0, part, slots)
  places = np.broadcast_to(np.arange(slots) * part + at, (E, slots)).astype(np.int32)
  firsts = np.broadcast_to(np.arange(slots) * part, (E, slots)).astype(np.int32)
  dq, dk, dv = (up(rt, B.bf16_bits(t)) for t in (q, k, v))
  o = rt.dram_alloc(E * slots * hd * 2)
  args = _lib.AttentionArgs(dq, dk, dv, o, up(rt, places.copy()), slots * hd, hd, slots * part * hd, hd,
                            slots * part * hd, hd, slots * hd, hd, slots, E, rep, slots, slots * part, hd, 0, 0, 0, 0, 0,
                            up(rt, firsts.copy()), slots)
  need = ctypes.c_uint64()
  _lib.call("attention_scratch", ctypes.byref(args), ctypes.byref(need))
  if need.value: args.scratch, args.scratch_bytes = rt.dram_alloc(need.value), need.value
  rt.run("attention", "attention", ctypes.byref(args))
  got = bits_to_float(down(rt, o, (E, slots, hd), np.uint16))
  for u in range(slots):
    region = slice(u * part, (u + 1) * part)
    want = ops.attention(q[:, u:u + 1], k[:, region], v[:, region], np.full((E, 1, 1), at[u]), 0, rep)
    assert np.allclose(got[:, u:u + 1], want, rtol=0.011, atol=0.011), (u, np.abs(got[:, u:u + 1] - want).max())


def test_attention_rows_without_keys_are_zero(rt):
  # a place before the first key hides every key: p is zero and so is the output (kernels.py:823-826)
  rng = np.random.default_rng(5)
  for rows, keys in ((1, 200), (40, 64)):
    q, k, v = (B.bf16(rng.normal(0, 1, s)) for s in ((4, rows, 64), (2, keys, 64), (2, keys, 64)))
    places = rng.integers(0, keys, (4, rows))
    places[1] = -1
    got = attend(rt, q, k, v, places)
    assert np.array_equal(got[1], np.zeros_like(got[1]))
    want = ops.attention(q, k, v, places[..., None], 0, 2)
    assert np.allclose(got[[0, 2, 3]], want[[0, 2, 3]], rtol=0.011, atol=0.011)


def test_attention_extremes(rt):
  # test_kernels.py:1323-1337: scores far beyond bf16 precision; keys past the place are never read
  for query, key in ((100, 100), (100, -100), (10000, 10000), (10000, -10000)):
    q = np.full((1, 3, 64), float(query))
    k = np.full((1, 64, 64), float(key))
    v = np.concatenate([np.ones((1, 32, 64)), np.full((1, 32, 64), 5.0)], 1)
    assert np.array_equal(attend(rt, q, k, v, np.full((1, 3), 31)), np.ones((1, 3, 64)))
  q = np.full((1, 1, 64), 100.0)
  k = np.concatenate([np.full((1, 32, 64), 100.0), np.full((1, 32, 64), 101.0)], 1)
  v = np.concatenate([np.ones((1, 32, 64)), np.full((1, 32, 64), 2.0)], 1)
  assert np.array_equal(attend(rt, q, k, v, np.array([[63]])), np.full((1, 1, 64), 2.0))


# ---- gather and put ----------------------------------------------------------------------------------------------

def test_gather_and_put(rt):
  rng = np.random.default_rng(11)
  table = B.bf16_bits(rng.normal(0, 1, (500, 576)))
  dt = up(rt, table)
  ids = np.array([3, 499, 0, 3, 250], np.int32)
  o = rt.dram_alloc(5 * 576 * 2)
  rt.run("gather", "gather", _lib.BF16, dt, 500, 576, 576, up(rt, ids), 5, o, 576)
  assert np.array_equal(down(rt, o, (5, 576), np.uint16), table[ids])
  cache = np.zeros((6, 64, 64), np.uint16)
  dc = up(rt, cache)
  x = B.bf16_bits(rng.normal(0, 1, (6, 3, 64)))
  places = np.array([5, 9, 5], np.int32)  # a later duplicate wins
  rt.run("put", "put", _lib.BF16, dc, 6, 64, 64, 64 * 64, 64, up(rt, places), 3, up(rt, x), 3 * 64, 64)
  got = down(rt, dc, (6, 64, 64), np.uint16)
  want = cache.copy()
  for i, p in enumerate(places): want[:, p] = x[:, i]
  assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [2048, 9000])
def test_put_many_rows_later_duplicate_wins(rt, n):
  # a prefill's worth of rows (the parallel path) and more (the ordered path), with repeats and places outside the
  # cache, in fp32 and with row pieces too narrow for 16-byte moves
  rng = np.random.default_rng(n)
  for dtype, cols, np_t in ((_lib.BF16, 64, np.uint16), (_lib.FP32, 6, np.float32)):
    size = n // 2
    cache = np.zeros((3, size, cols), np_t)
    dc = up(rt, cache)
    x = (B.bf16_bits(rng.normal(0, 1, (3, n, cols))) if np_t is np.uint16
         else rng.normal(0, 1, (3, n, cols)).astype(np.float32))
    places = rng.integers(-3, size + 3, n).astype(np.int32)
    rt.run("put", "put", dtype, dc, 3, size, cols, size * cols, cols, up(rt, places), n, up(rt, x), n * cols, cols)
    want = cache.copy()
    for i, p in enumerate(places):
      if 0 <= p < size: want[:, p] = x[:, i]
    assert np.array_equal(down(rt, dc, (3, size, cols), np_t), want), (dtype, n)
