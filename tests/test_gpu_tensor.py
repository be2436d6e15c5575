"""The Tensor surface on the GPU, checked the way the reference's own tests check it (test/test_kernels.py), against
NumPy and the oracle. Needs a GPU."""
import math
import numpy as np
import pytest

from baretile_amd.tensor import Tensor, jit
from oracle import bfp as B, ops

pytestmark = pytest.mark.gpu


def bf(v): return float(B.bf16(np.float32(v)))


def packed(v):  # half-up bf16 rounding of a computed result (test/conftest.py:11-13)
  b = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
  return (((b + 0x8000) >> 16) << 16).astype(np.uint32).view(np.float32).astype(np.float64)


def value(t): return np.array(t.tolist()).reshape(t.shape)


def test_readme_and_ramp_known_answers(rt):
  # README.md:74-83 and ramps/1_tensors.py:27-31
  x, w = Tensor.of(rt, [[1.0, 2.0], [3.0, 4.0]]), Tensor.of(rt, [[2.0, 0.0], [0.0, 3.0]])
  assert ((x @ w).relu()).tolist() == [[2.0, 6.0], [6.0, 12.0]]
  assert (x @ x).relu().tolist() == [[7.0, 10.0], [15.0, 22.0]]


def test_round_trip_formats(rt):
  rng = np.random.default_rng(0)
  a = rng.normal(0, 3, (3, 5, 7))
  assert value(Tensor.of(rt, a.tolist(), "fp32")).tolist() == a.astype(np.float32).astype(np.float64).tolist()
  assert value(Tensor.of(rt, a.tolist())).tolist() == B.bf16(a).astype(np.float64).tolist()
  i = rng.integers(-2**31, 2**31 - 1, (4, 9))
  assert Tensor.of(rt, i.tolist(), "int32").tolist() == i.tolist()


def test_matmul_exact(rt):
  # test_kernels.py:637-651
  a = [[float((r * 7 + c * 3) % 3 - 1) for c in range(64)] for r in range(32)]
  b = [[float((r * 5 + c) % 3 - 1) for c in range(32)] for r in range(64)]
  assert (Tensor.of(rt, a) @ Tensor.of(rt, b)).tolist() == (np.array(a) @ np.array(b)).tolist()
  rng = np.random.default_rng(1)
  x = [[bf(v) for v in row] for row in rng.uniform(-8, 8, (96, 64))]
  eye = np.eye(64).tolist()
  assert (Tensor.of(rt, x) @ Tensor.of(rt, eye)).tolist() == x
  d = [bf(v) for v in rng.uniform(1, 2, 64)]
  diag = np.diag(d).tolist()
  assert (Tensor.of(rt, x) @ Tensor.of(rt, diag)).tolist() == packed(np.array(x) * np.array(d)).tolist()


def test_matmul_transposed_and_batched(rt):
  rng = np.random.default_rng(2)
  a, b = B.bf16(rng.uniform(-1, 1, (3, 40, 70))), B.bf16(rng.uniform(-1, 1, (3, 50, 70)))
  got = value(Tensor.of(rt, a) @ Tensor.of(rt, b).T)
  want = a @ b.transpose(0, 2, 1)
  assert np.all(np.abs(got - want) <= 2.0 ** -8 * (np.abs(a) @ np.abs(b).transpose(0, 2, 1)))
  one = B.bf16(rng.uniform(-1, 1, (70, 30)))  # a batch of A against one B
  got = value(Tensor.of(rt, a) @ Tensor.of(rt, one))
  assert np.all(np.abs(got - a @ one) <= 2.0 ** -8 * (np.abs(a) @ np.abs(one)))


@pytest.mark.parametrize("dtype", ["bfp8", "bfp4"])
def test_bfp(rt, dtype):
  # test_kernels.py:709-724: a matmul by a block-float B is bit for bit the bf16 matmul by its values; then fused with
  # what follows and with a bf16 matmul
  rng = np.random.default_rng(5)
  on = lambda *shape: Tensor.of(rt, rng.normal(0, 1, shape).tolist())
  for b, m, k, n in ((1, 64, 9000, 40), (1, 1, 768, 2304), (1, 100, 256, 200), (2, 100, 256, 96), (1, 32, 2048, 64)):
    x, w = on(b, m, k), on(b, k, n).cast(dtype)
    assert (x @ w).tolist() == (x @ Tensor.of(rt, w.tolist())).tolist(), (b, m, k, n)
  x, w, v, bias = on(64, 192), on(192, 96).cast(dtype), on(192, 96), on(1, 96)
  assert (x @ w + x @ v + bias).relu().tolist() == (x @ Tensor.of(rt, w.tolist()) + x @ v + bias).relu().tolist()


@pytest.mark.parametrize("dtype", ["bfp8", "bfp4"])
def test_bfp_numpy(rt, dtype):
  # test_models.py:587-593: the device's cast equals the NumPy model's, bit for bit, on N(0,1) * e^N(0,2)
  rng = np.random.default_rng(5)
  a = rng.normal(0, 1, (64, 96)) * np.exp(rng.normal(0, 2, (64, 96)))
  got = np.array(Tensor.of(rt, a.tolist()).cast(dtype).tolist())
  assert np.array_equal(got, B.bfp(B.bf16(a), dtype))
  got = np.array(Tensor.of(rt, a.tolist()).cast(dtype).columns().tolist())  # by columns reads back unchanged
  assert np.array_equal(got, B.bfp(B.bf16(a), dtype))


def test_put_block_float_known_answer(rt):
  # test_kernels.py:2096-2103: [2, 3] cast among zeros reads back as bf16 0x4000, 0x4040
  for dtype in ("bfp8", "bfp4"):
    row = Tensor.of(rt, [[2.0, 3.0] + [0.0] * 30]).cast(dtype)
    bits = np.frombuffer(row.tobytes(), np.uint16)
    assert list(bits[:2]) == [0x4000, 0x4040]


def unfused(t):  # the same tree with one launch per op
  if t.op is None: return t
  srcs = [unfused(s) if isinstance(s, Tensor) else s for s in t.srcs]
  if t.op == "matmul": return (srcs[0] @ srcs[1]).realize()
  out = Tensor(t.rt, t.rows, t.cols, t.op, tuple(srcs), t.batch, t.dtype, t.args)
  out.lead = t.lead
  return out.realize()


def test_fusion(rt):
  # test_kernels.py:987-1004: a fused chain gives the bits of one launch per op
  rng = np.random.default_rng(3)
  a, b, c, d = (Tensor.of(rt, B.bf16(rng.uniform(-3, 3, (128, 96))).tolist()) for _ in range(4))
  for build in (lambda a, b, c, d: (a + b) * c - d * a, lambda a, b, c, d: (a + b) * ((c - d) + a * a)):
    launches = rt.launches
    got = build(a, b, c, d).tolist()
    assert rt.launches - launches == 1, "one kernel"
    assert got == unfused(build(a, b, c, d)).tolist()


def test_matmul_fusion(rt):
  # test_kernels.py:1081-1092
  rng = np.random.default_rng(4)
  rnd = lambda r, c: Tensor.of(rt, B.bf16(rng.uniform(-1, 1, (r, c))).tolist())
  a, b, c, d, e, f = rnd(64, 96), rnd(96, 128), rnd(64, 128), rnd(64, 128), rnd(64, 64), rnd(64, 128)
  for build in (lambda: (a @ b) + c, lambda: (a @ b) * d - c, lambda: (a @ b) + (e @ f)):
    assert build().tolist() == unfused(build()).tolist()


def test_fused_cast(rt):
  # test_kernels.py:1006-1020: a cast at the root is part of the kernel and equals casting the computed value
  rng = np.random.default_rng(16)
  x, y = (Tensor.of(rt, rng.normal(0, 2, (70, 100)).astype(np.float32).tolist(), "fp32") for _ in range(2))
  a, b, c = (Tensor.of(rt, rng.normal(0, 2, s).tolist()) for s in ((70, 100), (70, 100), (100, 40)))
  for build in (lambda: (x * 3 + y).bfloat16(), lambda: (x * 50 + y).cast("int32"), lambda: (x * y).sum(1).bfloat16(),
                lambda: (a * b + a).float(), lambda: a.softmax(-1).float(), lambda: (a @ c).float()):
    fused = build().realize()
    t = build()
    t.srcs[0].realize()
    assert fused.tobytes() == t.realize().tobytes()


def test_reductions_and_softmax(rt):
  rng = np.random.default_rng(8)
  a = rng.normal(0, 1, (2, 3, 50, 70))
  t = Tensor.of(rt, a.tolist(), "fp32")
  for axis in (None, 0, 1, 2, 3, -1):
    want = a.astype(np.float32).astype(np.float64).sum(axis=axis, keepdims=True)
    assert np.allclose(value(t.sum(axis)), want, rtol=1e-5, atol=1e-4), axis
    assert np.allclose(value(t.max(axis)), a.astype(np.float32).max(axis=axis, keepdims=True)), axis
  s = Tensor.of(rt, a[0, 0].tolist(), "fp32").softmax(-1)
  assert np.allclose(value(s), ops.softmax(a[0, 0].astype(np.float32)), rtol=1e-5, atol=1e-6)


def test_elementwise_ops_against_numpy(rt):
  rng = np.random.default_rng(9)
  a = rng.uniform(0.5, 3, (40, 70)).astype(np.float32)
  t = Tensor.of(rt, a.tolist(), "fp32")
  checks = [(t.exp(), np.exp(a)), (t.log(), np.log(a)), (t.sqrt(), np.sqrt(a)), (t.reciprocal(), 1 / a),
            (t.rsqrt(), 1 / np.sqrt(a)), (t.sigmoid(), 1 / (1 + np.exp(-a))), (t.silu(), a / (1 + np.exp(-a))),
            (t.gelu(), ops.gelu(a)), (t.maximum(1.5), np.maximum(a, 1.5)), (t.minimum(1.5), np.minimum(a, 1.5)),
            ((t > 1.5).where(t, -t), np.where(a > 1.5, a, -a)), (t.sin(), np.sin(a)), (t.cos(), np.cos(a))]
  for got, want in checks: assert np.allclose(value(got), want, rtol=2e-5, atol=2e-6)


def test_views_slices_split_merge(rt):
  rng = np.random.default_rng(10)
  a = B.bf16(rng.normal(0, 1, (6, 40, 96)))
  t = Tensor.of(rt, a.tolist())
  assert np.array_equal(value(t[2]), a[2:3])
  assert np.array_equal(value(t[1:5:2, 3:30:3, 7:90]), a[1:5:2, 3:30:3, 7:90])
  m = Tensor.of(rt, a[0].tolist())
  parts = m.split(3)
  assert np.array_equal(value(parts), a[0].reshape(40, 3, 32).transpose(1, 0, 2))
  assert np.array_equal(value(parts.merge()), a[:1])
  assert np.array_equal(value((parts * 2).merge()), a[:1] * 2)
  assert np.array_equal(value(t.T), a.transpose(0, 2, 1))
  assert np.array_equal(value(t.reshape(3, 2, 40, 96)), a.reshape(3, 2, 40, 96))
  r = Tensor.of(rt, a[:2].tolist()).repeat_interleave(3)
  assert np.array_equal(value(r + 0), np.repeat(a[:2], 3, 0))


def test_leading_broadcast(rt):
  rng = np.random.default_rng(11)
  a, b = rng.normal(0, 1, (2, 1, 5, 7)), rng.normal(0, 1, (1, 3, 5, 7))
  got = value(Tensor.of(rt, a.tolist(), "fp32") + Tensor.of(rt, b.tolist(), "fp32"))
  assert np.allclose(got, (a.astype(np.float32) + b.astype(np.float32)))


def test_gather_put_attend(rt):
  rng = np.random.default_rng(12)
  table = B.bf16(rng.normal(0, 1, (300, 64)))
  t = Tensor.of(rt, table.tolist())
  assert np.array_equal(value(t.gather([5, 299, 0, 5])), table[None, [5, 299, 0, 5]])
  with pytest.raises(IndexError): t.gather([300])
  cache = Tensor.zeros(rt, 96, 64, batch=4)
  x = B.bf16(rng.normal(0, 1, (4, 3, 64)))
  cache.put(Tensor.of(rt, [[10, 20, 10]], "int32"), Tensor.of(rt, x.tolist()))
  want = np.zeros((4, 96, 64))
  want[:, 20], want[:, 10] = x[:, 1], x[:, 2]
  assert np.array_equal(value(cache), want)
  q = B.bf16(rng.normal(0, 1, (8, 5, 64)) / 8)
  k, v = B.bf16(rng.normal(0, 1, (2, 96, 64))), B.bf16(rng.normal(0, 1, (2, 96, 64)))
  places = rng.integers(40, 96, (1, 5, 1))
  kt, vt = Tensor.of(rt, k.tolist()).repeat_interleave(4), Tensor.of(rt, v.tolist()).repeat_interleave(4)
  got = value(Tensor.of(rt, q.tolist()).attend(kt, vt, Tensor.of(rt, places.tolist(), "int32")))
  assert np.allclose(got, ops.attention(q, k, v, places, 0, 4), rtol=0.011, atol=0.011)


def test_jit_replays_with_new_inputs(rt):
  rng = np.random.default_rng(13)
  w = Tensor.of(rt, rng.normal(0, 0.1, (64, 96)).tolist()).cast("bfp8").columns()
  f = jit(lambda x: (x @ w).relu() * 2)
  xs = [Tensor.of(rt, rng.normal(0, 1, (4, 64)).tolist()) for _ in range(5)]
  want = [((x @ w).relu() * 2).tolist() for x in xs]
  got = [f(x).tolist() for x in xs]
  assert got == want


def test_errors(rt):
  x = Tensor.of(rt, [[1.0, 2.0]])
  with pytest.raises(ValueError): Tensor.of(rt, [])
  with pytest.raises(ValueError): x @ Tensor.of(rt, [[1.0, 2.0]])
  with pytest.raises(ValueError): x.cast("fp8")
  with pytest.raises(ValueError): x + Tensor.of(rt, [[1.0, 2.0, 3.0]])


def test_topk(rt):
  # test_kernels.py:2029-2062: the k largest of each row in the order of numpy's stable argsort of -x (the first of
  # equals first, -0 equal to 0); bf16 rows of several widths and a batch; fp32 rows in parts, then the best of the
  # parts by their labels (k = 1 too: a greedy pick over a 49152-token vocabulary in 192 parts)
  rng = np.random.default_rng(37)
  for batch, rows, cols, k in ((1, 1, 128, 8), (1, 3, 16, 4), (1, 40, 40, 1), (2, 33, 256, 32), (1, 2, 49152, 64)):
    x = rng.normal(0, 2, (batch, rows, cols))
    x[0, -1, :3], x[0, -1, 3:] = [-0.0, 0.0, -0.0], -np.abs(x[0, -1, 3:]) - 1  # -0 and 0, equal and the largest
    x[0, 0, 9] = x[0, 0, 3] = x[0, 0].max()  # a tie
    x = B.bf16(x)
    values, ids = Tensor.of(rt, x).topk(k)
    want = np.argsort(-x, -1, kind="stable")[..., :k]
    got_ids = np.array(ids.tolist()).reshape(batch, rows, k)
    got_values = np.array(values.tolist()).reshape(batch, rows, k)
    assert np.array_equal(got_ids, want), (batch, rows, cols, k)
    assert np.array_equal(got_values, np.take_along_axis(x, want, -1)), (batch, rows, cols, k)
  for rows, cols, parts, k in ((5, 2560, 4, 64), (5, 2560, 4, 1), (1, 49152, 192, 1), (40, 1024, 2, 32)):
    x = rng.normal(0, 3, (rows, cols)).astype(np.float32)
    x[0, 100] = x[0, cols // 2 + 3] = x[0].max() + 1  # a tie across parts
    values, ids = Tensor.of(rt, x, "fp32").topk(k, parts)
    w = cols // parts
    want = np.concatenate([np.argsort(-x[:, p * w:(p + 1) * w], -1, kind="stable")[:, :k] + p * w for p in range(parts)], 1)
    assert np.array_equal(np.array(ids.tolist()), want)
    assert np.array_equal(np.array(values.tolist(), np.float32), np.take_along_axis(x, want, -1))
    values, ids = values.topk(k, labels=ids)
    want = np.argsort(-x, -1, kind="stable")[:, :k]
    assert np.array_equal(np.array(ids.tolist()), want)
    assert np.array_equal(np.array(values.tolist(), np.float32), np.take_along_axis(x, want, -1))
  with pytest.raises(ValueError): Tensor.of(rt, x, "fp32").topk(65)
  with pytest.raises(ValueError): Tensor.of(rt, x, "fp32").topk(4, parts=3)
  # out: the same results written into given tensors, which come back; a wrong shape or dtype is refused
  t = Tensor.of(rt, x, "fp32")
  values, ids = t.topk(3, parts=2)
  out = (Tensor.zeros(rt, x.shape[0], 6, dtype="fp32"), Tensor.zeros(rt, x.shape[0], 6, dtype="int32"))
  got = t.topk(3, parts=2, out=out)
  assert got[0] is out[0] and got[1] is out[1]
  assert out[0].tolist() == values.tolist() and out[1].tolist() == ids.tolist()
  with pytest.raises(ValueError, match="out"): t.topk(3, parts=2, out=(out[1], out[0]))
  with pytest.raises(ValueError, match="out"): t.topk(2, parts=2, out=out)


def _weights(rt, k, n, fmt, seed):
  w = np.random.default_rng(seed).normal(0, 0.05, (k, n)).astype(np.float32)
  t = Tensor.of(rt, w)
  t = (t.cast(fmt) if fmt != "bf16" else t).columns()
  if fmt == "bf16": return t, B.bf16(w).astype(np.float64)
  pad = -n % 16  # the oracle takes whole runs of 16; the padding columns' runs don't touch the real ones
  return t, B.bfp(np.pad(w, ((0, 0), (0, pad))), fmt)[:, :n]


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bfp4"])
@pytest.mark.parametrize("kind,k,n", [("plain", 576, 960), ("rms", 576, 3072), ("rms", 4096, 200),
                                      ("swiglu", 1536, 576), ("swiglu", 64, 40)])
def test_matmul_row(rt, fmt, kind, k, n):
  # One row times w with its prologue and residual in one kernel (bt_matmul_row), against NumPy on the documented
  # formula: the prologue's row a' exactly as bf16 of the fp32 computation (a bf16 rounding may flip where the
  # device's fp32 sum or exp differs in the last bit), the product within the reference's bound of a' @ w.
  rng = np.random.default_rng(k + n)
  wt, wq = _weights(rt, k, n, fmt, k * n)
  res = rng.normal(0, 1, n).astype(np.float32)
  if kind == "rms":
    x = (rng.normal(0, 2, k)).astype(np.float32)
    norm = B.bf16(rng.normal(1, 0.1, k).astype(np.float32)).astype(np.float32)
    xb = packed(x).astype(np.float32)
    r = np.float32(1) / np.sqrt(np.float32(np.mean(xb.astype(np.float64) ** 2)) + np.float32(1e-5))
    a = packed(xb * r * norm)
    got = Tensor.of(rt, x[None], "fp32").matmul_row(wt, "fp32", norm=Tensor.of(rt, norm[None]), eps=1e-5,
                                                     residual=Tensor.of(rt, res[None], "fp32"))
  elif kind == "swiglu":
    gu = B.bf16(rng.normal(0, 2, 2 * k).astype(np.float32)).astype(np.float32)
    g, u = gu[:k], gu[k:]
    a = packed(g / (np.float32(1) + np.exp(-g)) * u)
    got = Tensor.of(rt, gu[None]).matmul_row(wt, "fp32", swiglu=True, residual=Tensor.of(rt, res[None], "fp32"))
  else:
    a = B.bf16(rng.normal(0, 1, k).astype(np.float32)).astype(np.float64)
    got = Tensor.of(rt, a[None].astype(np.float32)).matmul_row(wt, "fp32", residual=Tensor.of(rt, res[None], "fp32"))
  want = a @ wq + res
  bound = ops.matmul_bound(a, wq) * 2 + 1e-6 * np.abs(want)
  assert got.shape[-2:] == (1, n)
  assert np.all(np.abs(value(got).reshape(n) - want) <= bound)
  # bf16 output: the fp32 result rounded half up
  if kind == "plain":
    g16 = Tensor.of(rt, a[None].astype(np.float32)).matmul_row(wt, "bf16")
    assert np.all(np.abs(value(g16).reshape(n) - a @ wq) <= ops.matmul_bound(a, wq) + 2.0 ** -8 * np.abs(a @ wq))


def test_matmul_row_rejects_bad_inputs(rt):
  wt, _ = _weights(rt, 64, 32, "bfp8", 0)
  with pytest.raises(ValueError, match="contiguous bf16 row of 64"):
    Tensor.of(rt, np.ones((1, 32), np.float32)).matmul_row(wt)
  with pytest.raises(ValueError, match="fp32 row"):
    Tensor.of(rt, np.ones((1, 64), np.float32)).matmul_row(wt, norm=Tensor.of(rt, np.ones((1, 64), np.float32)))
  with pytest.raises(ValueError, match="columns"):
    Tensor.of(rt, np.ones((1, 64), np.float32)).matmul_row(Tensor.of(rt, np.ones((64, 32), np.float32)))


@pytest.mark.parametrize("hd", [64, 128])
def test_rope_put(rt, hd):
  # RoPE of every head with the key and value heads put into the cache (bt_rope_put), against x cos + (x @ turn) sin
  # in float64 on the same bf16 inputs, to a bf16 rounding; value heads (cos 1, sin 0) stored exactly.
  from baretile_amd.models import llama
  heads, kv, rows, size = 4, 2, 3, 16
  c = llama.model(dim=heads * hd, heads=heads, kv=kv, layers=1, eps=1e-5, theta=10000.0, head_dim=hd)
  cos, sin, turn = llama.rotary(c, size)
  rng = np.random.default_rng(hd)
  nh = heads + 2 * kv
  x = B.bf16(rng.normal(0, 1, (rows, nh * hd)).astype(np.float32)).astype(np.float64)
  places = [5, 0, 15]
  cache = Tensor.zeros(rt, size, hd, batch=2 * kv)
  q = Tensor.of(rt, x.astype(np.float32)).rope_put(Tensor.of(rt, cos[places]), Tensor.of(rt, sin[places]), cache,
                                                     Tensor.of(rt, [places], "int32"), heads, kv)
  xs = x.reshape(rows, nh, hd)
  want = xs * cos[places].reshape(rows, nh, hd) + (xs @ turn) * sin[places].reshape(rows, nh, hd)
  got_q = value(q).reshape(rows, heads, hd)
  assert np.all(np.abs(got_q - want[:, :heads]) <= 2.0 ** -8 * np.abs(want[:, :heads]) + 1e-30)
  got_c = value(cache).reshape(2 * kv, size, hd)
  for i, p in enumerate(places):
    assert np.all(np.abs(got_c[:kv, p] - want[i, heads:heads + kv]) <= 2.0 ** -8 * np.abs(want[i, heads:heads + kv]) + 1e-30)
    assert np.array_equal(got_c[kv:, p], xs[i, heads + kv:])
  others = [r for r in range(size) if r not in places]
  assert not np.any(got_c[:, others])


def test_rope_put_aligned_and_unaligned_rows_agree(rt):
  # 16-byte aligned rows take the kernel that moves 8 pairs a thread; rows 4 values longer than their heads (a view
  # of a wider tensor: row strides that aren't a multiple of 8) take the one pair a thread kernel. Same bits.
  from baretile_amd.models import llama
  heads, kv, hd, rows, size = 8, 2, 128, 37, 64
  nh = heads + 2 * kv
  c = llama.model(dim=heads * hd, heads=heads, kv=kv, layers=1, eps=1e-5, theta=10000.0, head_dim=hd)
  cos, sin, _ = llama.rotary(c, size)
  rng = np.random.default_rng(9)
  x = rng.normal(0, 1, (rows, nh * hd)).astype(np.float32)
  places = [int(p) for p in rng.permutation(size)[:rows]]
  wide = lambda a: np.concatenate([a, np.zeros((rows, 4), a.dtype)], 1)
  out = []
  for pad in (False, True):
    xs, cs, sn = x, cos[places], sin[places]
    tx = Tensor.of(rt, wide(xs) if pad else xs)
    tc, ts = Tensor.of(rt, wide(cs) if pad else cs), Tensor.of(rt, wide(sn) if pad else sn)
    if pad: tx, tc, ts = tx[:, :nh * hd], tc[:, :nh * hd], ts[:, :nh * hd]
    cache = Tensor.zeros(rt, size, hd, batch=2 * kv)
    q = tx.rope_put(tc, ts, cache, Tensor.of(rt, [places], "int32"), heads, kv)
    out.append((q.tobytes(), cache.tobytes()))
  assert out[0] == out[1]


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bfp4"])
@pytest.mark.parametrize("k,hd,heads,kv", [(576, 64, 9, 3), (2048, 128, 8, 2), (320, 64, 2, 1)])
def test_matmul_row_rope_equals_two_calls(rt, fmt, k, hd, heads, kv):
  # RMSNorm, qkv product, RoPE and cache put in one kernel (bt_matmul_row_rope) write, bit for bit, what
  # bt_matmul_row to bf16 then bt_rope_put write: q, the new key and value rows, and nothing else in the cache. 2048
  # rows of K split each run's sum between two waves.
  from baretile_amd.models import llama
  nh, size, place = heads + 2 * kv, 24, 17
  c = llama.model(dim=heads * hd, heads=heads, kv=kv, layers=1, eps=1e-5, theta=10000.0, head_dim=hd)
  cos, sin, _ = llama.rotary(c, size)
  rng = np.random.default_rng(k + hd)
  wt, _ = _weights(rt, k, nh * hd, fmt, k + nh)
  x = Tensor.of(rt, rng.normal(0, 2, (1, k)).astype(np.float32), "fp32")
  norm = Tensor.of(rt, B.bf16(rng.normal(1, 0.1, (1, k)).astype(np.float32)))
  cs, sn, pl = Tensor.of(rt, cos[[place]]), Tensor.of(rt, sin[[place]]), Tensor.of(rt, [[place]], "int32")
  c1, c2 = Tensor.zeros(rt, size, hd, batch=2 * kv), Tensor.zeros(rt, size, hd, batch=2 * kv)
  q1 = x.matmul_row(wt, norm=norm, eps=1e-5, rope=(cs, sn, c1, pl, heads, kv))
  q2 = x.matmul_row(wt, "bf16", norm=norm, eps=1e-5).rope_put(cs, sn, c2, pl, heads, kv)
  assert q1.tobytes() == q2.tobytes()
  assert c1.tobytes() == c2.tobytes()
  assert np.any(value(c1).reshape(2 * kv, size, hd)[:, place])


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bfp4"])
@pytest.mark.parametrize("rows,k,hd,heads,kv", [(32, 4096, 128, 4, 2), (5, 1024, 64, 3, 1), (17, 2048, 128, 8, 4)])
def test_matmul_rope_put_equals_two_calls(rt, fmt, rows, k, hd, heads, kv):
  # a batched decode step's qkv product with RoPE and the puts into each slot's caches (bt_matmul_rope_put: the
  # product's split-K partial sums summed in the RoPE kernel) writes, bit for bit, what bt_matmul to bf16 then
  # bt_rope_put write: q, each slot's new key and value rows, and nothing else in the caches
  from baretile_amd.models import llama
  nh, size, place = heads + 2 * kv, 40, 37
  c = llama.model(dim=heads * hd, heads=heads, kv=kv, layers=1, eps=1e-5, theta=10000.0, head_dim=hd)
  cos, sin, _ = llama.rotary(c, size)
  rng = np.random.default_rng(rows + k)
  wt, _ = _weights(rt, k, nh * hd, fmt, k + nh)
  h = Tensor.of(rt, B.bf16(rng.normal(0, 1, (rows, k)).astype(np.float32)))
  cs, sn = Tensor.of(rt, np.repeat(cos[[place]], rows, 0)), Tensor.of(rt, np.repeat(sin[[place]], rows, 0))
  pl = Tensor.of(rt, [[place]], "int32")
  caches = [[Tensor.zeros(rt, size, hd, batch=rows * kv) for _ in range(2)] for _ in range(2)]
  q1 = h.matmul_rope_put(wt, cs, sn, caches[0][0], pl, heads, kv, values=caches[0][1])
  q2 = h.matmul(wt).rope_put(cs, sn, caches[1][0], pl, heads, kv, values=caches[1][1])
  assert q1.tobytes() == q2.tobytes()
  assert caches[0][0].tobytes() == caches[1][0].tobytes() and caches[0][1].tobytes() == caches[1][1].tobytes()
  got = value(caches[0][0]).reshape(rows * kv, size, hd)
  assert np.any(got[:, place]) and not np.any(np.delete(got, place, axis=1))


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bfp4"])
@pytest.mark.parametrize("rows,k,n", [(32, 4096, 4096), (5, 1024, 576), (20, 14336, 1024)])
def test_matmul_residual_rms_equals_unfused(rt, fmt, rows, k, n):
  # a batched decode step's o product with the residual add and the MLP's RMSNorm (bt_matmul_residual_rms: the split-K
  # partial sums summed in the norm's kernel) gives, bit for bit, x = residual + product (bt_matmul's residual
  # epilogue) and rms_rows(x); and x within the reference's bound of the oracle's residual + a @ w
  rng = np.random.default_rng(rows + n)
  wt, wv = _weights(rt, k, n, fmt, k + n)
  a = B.bf16(rng.normal(0, 1, (rows, k)).astype(np.float32))
  res = rng.normal(0, 4, (rows, n)).astype(np.float32)
  norm = Tensor.of(rt, B.bf16(rng.normal(1, 0.1, (1, n)).astype(np.float32)))
  ta, tr = Tensor.of(rt, a), Tensor.of(rt, res[None], "fp32")
  x1, h1 = ta.matmul_residual_rms(wt, tr, norm, 1e-5)
  x2 = (tr + ta.matmul(wt, "fp32")).realize()
  h2 = x2.rms_rows(norm, 1e-5)
  assert x1.tobytes() == x2.tobytes() and h1.tobytes() == h2.tobytes()
  got = np.frombuffer(x1.tobytes(), np.float32).reshape(rows, n)
  want = res + a.astype(np.float64) @ wv
  assert np.all(np.abs(got - want) <= 2.0 ** -8 * (np.abs(a) @ np.abs(wv)) + 1e-3 * np.abs(res) + 1e-6)
  assert np.frombuffer(tr.tobytes(), np.float32).reshape(rows, n).tolist() == res.tolist()  # the residual kept


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
def test_block_float_cache(rt, fmt):
  # test_kernels.py:2106-2132: put writes bf16 rows into a block-float cache, each run of 16 rounded as cast rounds it,
  # bit for bit (one row, rows in two places, a run of 32, the edges, a later duplicate winning); attention reads
  # the cache in place, each key and value head serving two query heads, and gives bit for bit what it gives on the
  # same values in bf16, through the decode kernel (5 query rows) and the prefill kernel (40).
  rng = np.random.default_rng(16)
  cache = Tensor.of(rt, np.zeros((4, 96, 64), np.float32)).cast(fmt).realize()
  want = np.zeros((4, 96, 64))
  for places in ([5], [33, 34, 70], list(range(32, 64)), [0, 95], [7, 9, 7]):
    x = B.bf16(rng.normal(0, 2, (4, len(places), 64)) * 10.0 ** rng.integers(-3, 3, (4, len(places), 1)))
    cache.put(Tensor.of(rt, [places], "int32"), Tensor.of(rt, x.astype(np.float32)))
    cast = value(Tensor.of(rt, x.astype(np.float32)).cast(fmt)).reshape(4, len(places), 64)
    for i, p in enumerate(places): want[:, p] = cast[:, i]
    assert np.array_equal(value(cache).reshape(4, 96, 64), want), (fmt, places)
  same = Tensor.of(rt, want.astype(np.float32))  # the same values in bf16
  kb, vb = cache[0:2, :, :].repeat_interleave(2), cache[2:4, :, :].repeat_interleave(2)
  ks, vs = same[0:2, :, :].repeat_interleave(2), same[2:4, :, :].repeat_interleave(2)
  for rows in (5, 40):
    q = Tensor.of(rt, B.bf16(rng.normal(0, 1, (4, rows, 64)) / 8).astype(np.float32))
    pl = Tensor.of(rt, rng.integers(60, 96, (1, rows, 1)).astype(np.int32), "int32")
    assert q.attend(kb, vb, pl).tobytes() == q.attend(ks, vs, pl).tobytes(), (fmt, rows)


def test_block_float_cache_long_decode(rt):
  # a 2000-row bfp8 cache of 128-wide heads, decode split into parts and combined, against the bf16 values
  rng = np.random.default_rng(21)
  x = B.bf16(rng.normal(0, 1, (4, 2000, 128)))
  cache = Tensor.of(rt, np.zeros((4, 2000, 128), np.float32)).cast("bfp8").realize()
  cache.put(Tensor.of(rt, [list(range(2000))], "int32"), Tensor.of(rt, x.astype(np.float32)))
  same = Tensor.of(rt, value(cache).reshape(4, 2000, 128).astype(np.float32))
  q = Tensor.of(rt, B.bf16(rng.normal(0, 1, (8, 1, 128)) / 11).astype(np.float32))
  pl = Tensor.of(rt, [[[1990]]], "int32")
  got = q.attend(cache[0:2, :, :].repeat_interleave(4), cache[2:4, :, :].repeat_interleave(4), pl, parts=8)
  want = q.attend(same[0:2, :, :].repeat_interleave(4), same[2:4, :, :].repeat_interleave(4), pl, parts=8)
  assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("fmt", ["bfp8", "bfp4"])
@pytest.mark.parametrize("parts", [None, 4])
def test_block_float_cache_split_decode(rt, fmt, parts):
  # 480 cached rows (8 blocks of 64 keys: by default a part a block, one-wave parts; with 4 parts, parts of two blocks
  # on 4-wave blocks; then their combine), 128-wide heads, two query rows: the cache read in place gives bit for bit
  # what its values give in bf16
  rng = np.random.default_rng(22)
  x = B.bf16(rng.normal(0, 1, (4, 480, 128)))
  cache = Tensor.of(rt, np.zeros((4, 480, 128), np.float32)).cast(fmt).realize()
  cache.put(Tensor.of(rt, [list(range(480))], "int32"), Tensor.of(rt, x.astype(np.float32)))
  same = Tensor.of(rt, value(cache).reshape(4, 480, 128).astype(np.float32))
  q = Tensor.of(rt, B.bf16(rng.normal(0, 1, (8, 2, 128)) / 11).astype(np.float32))
  pl = Tensor.of(rt, [[[470], [479]]], "int32")
  got = q.attend(cache[0:2, :, :].repeat_interleave(4), cache[2:4, :, :].repeat_interleave(4), pl, parts=parts)
  want = q.attend(same[0:2, :, :].repeat_interleave(4), same[2:4, :, :].repeat_interleave(4), pl, parts=parts)
  assert got.tobytes() == want.tobytes()


def test_rope_put_slots(rt):
  # the slots' layout: separate key and value caches of rows * kv heads, row i's heads at i * kv, one place for all
  # rows (llama.slots_layer); against the same float64 RoPE, and nothing else written
  from baretile_amd.models import llama
  heads, kv, rows, size, hd = 4, 2, 5, 12, 64
  c = llama.model(dim=heads * hd, heads=heads, kv=kv, layers=1, eps=1e-5, theta=10000.0, head_dim=hd)
  cos, sin, turn = llama.rotary(c, size)
  rng = np.random.default_rng(11)
  nh, place = heads + 2 * kv, 7
  x = B.bf16(rng.normal(0, 1, (rows, nh * hd)).astype(np.float32)).astype(np.float64)
  keys, vals = Tensor.zeros(rt, size, hd, batch=rows * kv), Tensor.zeros(rt, size, hd, batch=rows * kv)
  q = Tensor.of(rt, x.astype(np.float32)).rope_put(Tensor.of(rt, cos[[place] * rows]), Tensor.of(rt, sin[[place] * rows]),
                                                     keys, Tensor.of(rt, [[place]], "int32"), heads, kv, values=vals)
  xs = x.reshape(rows, nh, hd)
  cs, sn = cos[[place] * rows].reshape(rows, nh, hd), sin[[place] * rows].reshape(rows, nh, hd)
  want = xs * cs + (xs @ turn) * sn
  assert np.all(np.abs(value(q).reshape(rows, heads, hd) - want[:, :heads]) <= 2.0 ** -8 * np.abs(want[:, :heads]) + 1e-30)
  got_k, got_v = value(keys).reshape(rows * kv, size, hd), value(vals).reshape(rows * kv, size, hd)
  for i in range(rows):
    wk = want[i, heads:heads + kv]
    assert np.all(np.abs(got_k[i * kv:(i + 1) * kv, place] - wk) <= 2.0 ** -8 * np.abs(wk) + 1e-30)
    assert np.array_equal(got_v[i * kv:(i + 1) * kv, place], xs[i, heads + kv:])
  others = [r for r in range(size) if r != place]
  assert not np.any(got_k[:, others]) and not np.any(got_v[:, others])


@pytest.mark.parametrize("rows,k", [(37, 1000), (32, 4096), (5, 8192), (3, 999), (2, 9000), (300, 576)])
def test_rms_rows(rt, rows, k):
  # RMSNorm of rows in one kernel (bt_rms_rows) against NumPy on the documented formula, to a bf16 rounding: rows
  # held in registers (k a multiple of 4 up to 8192) and the two-pass loop (k = 999, 9000)
  rng = np.random.default_rng(7)
  x = rng.normal(0, 3, (rows, k)).astype(np.float32)
  w = B.bf16(rng.normal(1, 0.1, k).astype(np.float32)).astype(np.float32)
  xb = packed(x).astype(np.float32)
  r = np.float32(1) / np.sqrt(np.mean(xb.astype(np.float64) ** 2, 1, keepdims=True).astype(np.float32) + np.float32(1e-5))
  want = xb * r * w
  got = value(Tensor.of(rt, x, "fp32").rms_rows(Tensor.of(rt, w[None]), 1e-5)).reshape(rows, k)
  assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)


@pytest.mark.parametrize("fmt", ["bf16", "bfp8", "bfp4"])
@pytest.mark.parametrize("m,k,f", [(300, 256, 272), (32, 576, 1536), (5, 256, 272), (48, 4096, 352), (32, 4096, 352),
                                   (9, 1024, 1008), (2048, 64, 4224), (32, 4096, 384), (9, 1024, 1024),
                                   (32, 4096, 14336), (7, 512, 8192)])
def test_matmul_swiglu(rt, fmt, m, k, f):
  # silu(x @ gate) * (x @ up) with the SiLU-mul as the product's epilogue (bt_matmul_swiglu): against the unfused
  # product's gate and up values put through the documented formula, to a bf16 rounding. 300 rows run the tiled GEMM
  # (2048 x 4224: 264 blocks of 256 rows, whose last column goes to a second launch of 128-row blocks);
  # fewer, the kernel that takes a gate run and its up run a wave (48 x 4096: K split over two slices); up to 32 rows
  # with K over 12 chunks, the split-K kernels with SiLU x up in the reduction (f a multiple of 64 or not), or, with
  # K a multiple of 512 and at least 8192 columns of gate, the streaming kernel with SiLU x up in its own epilogue
  rng = np.random.default_rng(11)
  x = Tensor.of(rt, rng.normal(0, 1, (m, k)).astype(np.float32))
  wt, _ = _weights(rt, k, 2 * f, fmt, 3)
  gu = value(x.matmul(wt)).reshape(m, 2 * f)  # bf16, rounded as stored
  g, u = gu[:, :f].astype(np.float32), gu[:, f:].astype(np.float32)
  want = g / (np.float32(1) + np.exp(-g)) * u
  out = x.matmul_swiglu(wt)
  assert out.shape[-2:] == (m, f)
  got = value(out).reshape(m, f)
  assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)


def test_attend_merged_equals_merge(rt):
  rng = np.random.default_rng(5)
  q = Tensor.of(rt, rng.normal(0, 1, (4, 3, 64)).astype(np.float32))
  k = Tensor.of(rt, rng.normal(0, 1, (2, 8, 64)).astype(np.float32))
  v = Tensor.of(rt, rng.normal(0, 1, (2, 8, 64)).astype(np.float32))
  places = Tensor.of(rt, [[2], [5], [7]], "int32")
  a = q.attend(k.repeat_interleave(2), v.repeat_interleave(2), places).merge()
  b = q.attend(k.repeat_interleave(2), v.repeat_interleave(2), places, merged=True)
  assert a.shape[-2:] == b.shape[-2:] == (3, 256)
  assert a.tobytes() == b.tobytes()
