// Fused elementwise programs, reductions, and the row gather and put that fill and read caches.
#include "program.h"
#include "rows.h"
#include <algorithm>

namespace bt {

// A thread an element, in row-major order of the result.
// A thread takes V elements of the flattened result, 256 apart, so every load and store of a wavefront is contiguous
// along the columns. Small results take one element a thread, which keeps the evaluator's code small and the grid
// wide; large ones take 8, so each instruction of the program is decoded once for 8 values. The flat index fits 31
// bits (the launcher checks), and the row and batch entry are split off it by multiplication (FastDiv).
template <int DT, int V>
__global__ void __launch_bounds__(256) elementwise_kernel(const bt_program prog, uint32_t total, FastDiv cols,
                                                          FastDiv rows, const bt_operand out) {
  const uint32_t base = blockIdx.x * (256u * V) + threadIdx.x;
  Coords<V> at;
#pragma unroll
  for (int v = 0; v < V; v++) {
    const uint32_t t = base + 256u * v;
    at.ok[v] = t < total;
    const uint32_t u = at.ok[v] ? t : 0u, q = fdiv(u, cols), bb = fdiv(q, rows);
    at.c[v] = u - q * cols.d, at.r[v] = q - bb * rows.d, at.b[v] = bb;
  }
  uint32_t io[V] = {};
  run_program_v<DT, V>(prog, at, io);
#pragma unroll
  for (int v = 0; v < V; v++)
    if (at.ok[v]) store_value<DT>(out, operand_matrix(out, at.b[v]) * out.sb + at.r[v] * out.sr + at.c[v] * out.sc, io[v]);
}

// Large results: a thread evaluates a segment of SEG neighbouring columns of one row (fetch_segment). segs is the
// number of segments in a row.
template <int DT>
__global__ void __launch_bounds__(256) elementwise_seg_kernel(const bt_program prog, uint32_t nseg, FastDiv segs,
                                                              FastDiv rows, int32_t cols, const bt_operand out) {
  const uint32_t s = blockIdx.x * 256u + threadIdx.x;
  if (s >= nseg) return;
  const uint32_t q = fdiv(s, segs), bb = fdiv(q, rows);
  const int64_t c0 = (int64_t)(s - q * segs.d) * SEG, r = q - bb * rows.d;
  const int n = (int)min((int64_t)SEG, cols - c0);
  prefile pre[SEG];
  fetch_segment<DT>(prog, bb, r, c0, n, pre);
  uint32_t io[SEG] = {};
  eval_program<DT, SEG>(prog, pre, io);
  store_segment<DT>(out, bb, r, c0, n, io);
}

// The same for results of 2^31 elements or more: one element per thread, 64-bit index arithmetic.
template <int DT>
__global__ void __launch_bounds__(256) elementwise_wide_kernel(const bt_program prog, int64_t batch, int64_t rows,
                                                               int64_t cols, const bt_operand out) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = batch * rows * cols;
  for (; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c = t % cols, r = t / cols % rows, b = t / cols / rows;
    const uint32_t v = run_program<DT>(prog, b, r, c, 0);
    store_value<DT>(out, operand_matrix(out, b) * out.sb + r * out.sr + c * out.sc, v);
  }
}

__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = nan_max(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int32_t wave_imax(int32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}

constexpr int RED_V = 1;  // values a lane fetches before folding them

// Sums or maxima of a program's values along one axis. WPO wavefronts share each output: a whole block of WPO waves
// for long sweeps with few outputs, else one (four outputs a block). Lanes stride along the reduced axis; the partial
// results are combined across the wave, then across the block's waves through LDS. Sums accumulate in fp32. With DT
// bf16 each program value is rounded first, as the reference's pack of the folded operand is; the reduced value is
// rounded again when it is stored.
template <int DT, int WPO>
__global__ void __launch_bounds__(WPO > 4 ? 64 * WPO : 256) reduce_kernel(const bt_program prog, int kind, int axis, int64_t batch,
                                                     int64_t rows, int64_t cols, int64_t sweep, int64_t step,
                                                     const bt_operand out) {
  __shared__ uint32_t part[WPO];
  const int lane = threadIdx.x & 63;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t w = WPO > 1 ? (int64_t)blockIdx.x : (int64_t)blockIdx.x * 4 + wib;
  const int64_t ob = axis == 0 ? batch / sweep : batch, orows = axis == 1 ? 1 : rows, ocols = axis == 2 ? 1 : cols;
  if (w >= ob * orows * ocols) return;  // uniform across the block when WPO > 1
  const int64_t c = w % ocols, r = w / ocols % orows, b = w / ocols / orows;
  const int64_t n = axis == 0 ? sweep : axis == 1 ? rows : cols;
  const int64_t base = axis == 0 ? (b / step) * step * sweep + b % step : 0;
  const int64_t stride = 64 * WPO;
  float facc = kind == BT_REDUCE_SUM ? 0.0f : -__builtin_inff();
  int32_t iacc = INT32_MIN;
  for (int64_t i0 = (WPO > 1 ? wib * 64 : 0) + lane; i0 < n; i0 += stride * RED_V) {
    Coords<RED_V> at;
#pragma unroll
    for (int v = 0; v < RED_V; v++) {
      const int64_t i = i0 + stride * v;
      at.ok[v] = i < n;
      const int64_t ii = at.ok[v] ? i : 0;
      at.b[v] = axis == 0 ? base + ii * step : b, at.r[v] = axis == 1 ? ii : r, at.c[v] = axis == 2 ? ii : c;
    }
    uint32_t io[RED_V] = {};
    run_program_v<DT, RED_V>(prog, at, io);
#pragma unroll
    for (int v = 0; v < RED_V; v++) {
      if (!at.ok[v]) continue;
      if (DT == BT_INT32) iacc = max(iacc, (int32_t)io[v]);
      else if (kind == BT_REDUCE_SUM) facc += __uint_as_float(io[v]);
      else facc = nan_max(facc, __uint_as_float(io[v]));
    }
  }
  uint32_t res;
  if (DT == BT_INT32) res = (uint32_t)wave_imax(iacc);
  else res = __float_as_uint(kind == BT_REDUCE_SUM ? wave_sum(facc) : wave_max(facc));
  if (WPO > 1) {
    if (lane == 0) part[wib] = res;
    __syncthreads();
    if (wib != 0) return;
    for (int k = 1; k < WPO; k++) {
      const uint32_t o = part[k];
      if (DT == BT_INT32) res = (uint32_t)max((int32_t)res, (int32_t)o);
      else if (kind == BT_REDUCE_SUM) res = __float_as_uint(__uint_as_float(res) + __uint_as_float(o));
      else res = __float_as_uint(nan_max(__uint_as_float(res), __uint_as_float(o)));
    }
  }
  if (lane == 0) {
    if (DT == BT_BF16) res = __float_as_uint(round_packed(__uint_as_float(res)));
    store_value<DT>(out, operand_matrix(out, b) * out.sb + r * out.sr + c * out.sc, res);
  }
}

// Reductions along the last axis of large inputs: lanes take segments of SEG neighbouring columns (fetch_segment),
// otherwise as reduce_kernel.
template <int DT, int WPO>
__global__ void __launch_bounds__(WPO > 4 ? 64 * WPO : 256) reduce_seg_kernel(const bt_program prog, int kind,
                                                                               int64_t batch, int64_t rows,
                                                                               int64_t cols, const bt_operand out) {
  __shared__ uint32_t part[WPO];
  const int lane = threadIdx.x & 63;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t w = WPO > 1 ? (int64_t)blockIdx.x : (int64_t)blockIdx.x * 4 + wib;
  if (w >= batch * rows) return;  // uniform across the block when WPO > 1
  const int64_t r = w % rows, b = w / rows, nseg = (cols + SEG - 1) / SEG;
  float facc = kind == BT_REDUCE_SUM ? 0.0f : -__builtin_inff();
  int32_t iacc = INT32_MIN;
  for (int64_t sg = (WPO > 1 ? wib * 64 : 0) + lane; sg < nseg; sg += 64 * WPO) {
    const int64_t c0 = sg * SEG;
    const int n = (int)min((int64_t)SEG, cols - c0);
    prefile pre[SEG];
    fetch_segment<DT>(prog, b, r, c0, n, pre);
    uint32_t io[SEG] = {};
    eval_program<DT, SEG>(prog, pre, io);
#pragma unroll
    for (int v = 0; v < SEG; v++) {
      if (v >= n) continue;
      if (DT == BT_INT32) iacc = max(iacc, (int32_t)io[v]);
      else if (kind == BT_REDUCE_SUM) facc += __uint_as_float(io[v]);
      else facc = nan_max(facc, __uint_as_float(io[v]));
    }
  }
  uint32_t res;
  if (DT == BT_INT32) res = (uint32_t)wave_imax(iacc);
  else res = __float_as_uint(kind == BT_REDUCE_SUM ? wave_sum(facc) : wave_max(facc));
  if (WPO > 1) {
    if (lane == 0) part[wib] = res;
    __syncthreads();
    if (wib != 0) return;
    for (int k = 1; k < WPO; k++) {
      const uint32_t o = part[k];
      if (DT == BT_INT32) res = (uint32_t)max((int32_t)res, (int32_t)o);
      else if (kind == BT_REDUCE_SUM) res = __float_as_uint(__uint_as_float(res) + __uint_as_float(o));
      else res = __float_as_uint(nan_max(__uint_as_float(res), __uint_as_float(o)));
    }
  }
  if (lane == 0) {
    if (DT == BT_BF16) res = __float_as_uint(round_packed(__uint_as_float(res)));
    store_value<DT>(out, operand_matrix(out, b) * out.sb + r * out.sr, res);
  }
}

// A block a gathered row: 256 threads copy its 32-bit words (a bf16 row of odd width copies its last half word).
__global__ void __launch_bounds__(256) gather_kernel(const uint8_t *table, int64_t rows, int64_t row_bytes,
                                                     int64_t table_rstride_bytes, const int32_t *ids, uint8_t *out,
                                                     int64_t out_rstride_bytes) {
  int64_t i = blockIdx.x;
  int32_t id = ids[i];
  uint8_t *dst = out + i * out_rstride_bytes;
  const uint8_t *src = table + (int64_t)id * table_rstride_bytes;
  bool in = id >= 0 && id < rows;
  for (int64_t at = threadIdx.x * 2; at < row_bytes; at += 2 * blockDim.x)
    *(uint16_t *)(dst + at) = in ? *(const uint16_t *)(src + at) : 0;
}

// One block per (batch entry, column piece). Each block walks the n rows in order, so a later duplicate place
// overwrites an earlier one, and no two blocks write the same element.
__global__ void __launch_bounds__(256) put_kernel(uint8_t *dst, int64_t dst_rows, int64_t row_bytes, int64_t dst_sb,
                                                  int64_t dst_sr, const int32_t *ids, int64_t n, const uint8_t *x,
                                                  int64_t x_sb, int64_t x_sr, int64_t pieces) {
  int64_t b = blockIdx.x / pieces, piece = blockIdx.x % pieces;
  int64_t at = (piece * blockDim.x + threadIdx.x) * 2;
  if (at >= row_bytes) return;
  for (int64_t i = 0; i < n; i++) {
    int32_t p = ids[i];
    if (p < 0 || p >= dst_rows) continue;
    *(uint16_t *)(dst + b * dst_sb + p * dst_sr + at) = *(const uint16_t *)(x + b * x_sb + i * x_sr + at);
  }
}

// Blocks (i, y) for row i of x, for all batch entries at once, the y blocks of a row taking its pieces in turn (as
// many as make 512 pieces a block, so a wide row is not left to one block). A later duplicate place wins
// (tensor.py:223-241): each block first looks for a j > i with the same place, and writes nothing if there is one.
// Rows move in 16-byte pieces when both sides allow it. For n up to PUT_SCAN rows; the scan is O(n) a block.
constexpr int64_t PUT_SCAN = 8192;
__global__ void __launch_bounds__(256) put_rows_kernel(uint8_t *dst, int64_t dst_rows, int64_t row_bytes,
                                                       int64_t dst_sb, int64_t dst_sr, const int32_t *ids, int64_t n,
                                                       const uint8_t *x, int64_t x_sb, int64_t x_sr, int64_t batch,
                                                       int wide) {
  __shared__ int later;
  const int64_t i = blockIdx.x;
  const int32_t p = ids[i];
  if (p < 0 || p >= dst_rows) return;
  if (threadIdx.x == 0) later = 0;
  __syncthreads();
  bool found = false;
  for (int64_t j = i + 1 + threadIdx.x; j < n; j += blockDim.x) found |= ids[j] == p;
  if (found) later = 1;
  __syncthreads();
  if (later) return;
  const int64_t first = (int64_t)blockIdx.y * blockDim.x + threadIdx.x, step = (int64_t)gridDim.y * blockDim.x;
  if (wide) {
    const int64_t pieces = row_bytes / 16;
    for (int64_t e = first; e < batch * pieces; e += step) {
      const int64_t b = e / pieces, at = e % pieces * 16;
      *(uint4 *)(dst + b * dst_sb + p * dst_sr + at) = *(const uint4 *)(x + b * x_sb + i * x_sr + at);
    }
  } else {
    const int64_t halves = row_bytes / 2;
    for (int64_t e = first; e < batch * halves; e += step) {
      const int64_t b = e / halves, at = e % halves * 2;
      *(uint16_t *)(dst + b * dst_sb + p * dst_sr + at) = *(const uint16_t *)(x + b * x_sb + i * x_sr + at);
    }
  }
}

static int check_program(const bt_program *prog) {
  if (!prog) return fail(BT_EINVAL, "no program");
  if (prog->n_inst < 0 || prog->n_inst > BT_MAX_INST)
    return fail(BT_EINVAL, "a program has at most %d instructions, not %d", BT_MAX_INST, prog->n_inst);
  if (prog->n_inputs < 0 || prog->n_inputs > BT_MAX_INPUTS)
    return fail(BT_EINVAL, "a program has at most %d inputs, not %d", BT_MAX_INPUTS, prog->n_inputs);
  if (prog->dtype != BT_BF16 && prog->dtype != BT_FP32 && prog->dtype != BT_INT32)
    return fail(BT_EINVAL, "a program computes in bf16, fp32 or int32, not %d", prog->dtype);
  if (prog->result < 0 || prog->result >= BT_MAX_REGS) return fail(BT_EINVAL, "result register %d", prog->result);
  for (int i = 0; i < prog->n_inst; i++) {
    const bt_inst &in = prog->inst[i];
    if (in.op >= BT_OP_COUNT) return fail(BT_EINVAL, "instruction %d: unknown op %d", i, in.op);
    if (in.dst >= BT_MAX_REGS || in.a >= BT_MAX_REGS || in.b >= BT_MAX_REGS || in.c >= BT_MAX_REGS)
      return fail(BT_EINVAL, "instruction %d: register out of range", i);
    if (in.op == BT_OP_LOAD && in.a >= prog->n_inputs) return fail(BT_EINVAL, "instruction %d loads input %d", i, in.a);
  }
  for (int i = 0; i < prog->n_inputs; i++) {
    const bt_operand &o = prog->in[i];
    if (!o.ptr) return fail(BT_EINVAL, "input %d has no address", i);
    if (o.rep < 1 || o.cyc < 0) return fail(BT_EINVAL, "input %d: rep %d, cyc %d", i, o.rep, o.cyc);
    if (o.dtype != BT_BF16 && o.dtype != BT_FP32 && o.dtype != BT_INT32)
      return fail(BT_EINVAL, "input %d: dtype %d", i, o.dtype);
  }
  return BT_OK;
}

int check_out(const bt_operand *out) {
  if (!out || !out->ptr) return fail(BT_EINVAL, "no output");
  if (out->dtype != BT_BF16 && out->dtype != BT_FP32 && out->dtype != BT_INT32)
    return fail(BT_EINVAL, "output dtype %d", out->dtype);
  if (out->rep < 1 || out->cyc < 0) return fail(BT_EINVAL, "output rep %d, cyc %d", out->rep, out->cyc);
  return BT_OK;
}

int validate_program(const bt_program *prog) { return check_program(prog); }

}  // namespace bt

using namespace bt;

extern "C" {

int bt_elementwise(bt_runtime *rt, const bt_program *prog, int64_t batch, int64_t rows, int64_t cols,
                   const bt_operand *out) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (int s = check_program(prog)) return s;
  if (int s = check_out(out)) return s;
  if (batch <= 0 || rows <= 0 || cols <= 0) return fail(BT_EINVAL, "elementwise shape must be positive");
  const int64_t total = batch * rows * cols;
  if (total < (1ll << 31)) {
    const FastDiv fc = make_fastdiv((uint32_t)cols), fr = make_fastdiv((uint32_t)rows);
#define BT_EW(V)                                                                                                  \
  do {                                                                                                            \
    const unsigned blocks = (unsigned)((total + 256 * V - 1) / (256 * V));                                        \
    if (prog->dtype == BT_BF16)                                                                                   \
      elementwise_kernel<BT_BF16, V><<<blocks, 256, 0, r->stream>>>(*prog, (uint32_t)total, fc, fr, *out);        \
    else if (prog->dtype == BT_FP32)                                                                              \
      elementwise_kernel<BT_FP32, V><<<blocks, 256, 0, r->stream>>>(*prog, (uint32_t)total, fc, fr, *out);        \
    else elementwise_kernel<BT_INT32, V><<<blocks, 256, 0, r->stream>>>(*prog, (uint32_t)total, fc, fr, *out);    \
  } while (0)
    const int64_t segs = (cols + SEG - 1) / SEG, nseg = batch * rows * segs;
    if (total >= (1 << 16) && cols >= SEG && nseg < (1ll << 31)) {
      const FastDiv fs = make_fastdiv((uint32_t)segs);
      const unsigned blocks = (unsigned)((nseg + 255) / 256);
      if (prog->dtype == BT_BF16)
        elementwise_seg_kernel<BT_BF16><<<blocks, 256, 0, r->stream>>>(*prog, (uint32_t)nseg, fs, fr, (int32_t)cols, *out);
      else if (prog->dtype == BT_FP32)
        elementwise_seg_kernel<BT_FP32><<<blocks, 256, 0, r->stream>>>(*prog, (uint32_t)nseg, fs, fr, (int32_t)cols, *out);
      else elementwise_seg_kernel<BT_INT32><<<blocks, 256, 0, r->stream>>>(*prog, (uint32_t)nseg, fs, fr, (int32_t)cols, *out);
    } else {
      BT_EW(1);
    }
#undef BT_EW
  } else {
    const unsigned blocks = 1u << 20;
    if (prog->dtype == BT_BF16)
      elementwise_wide_kernel<BT_BF16><<<blocks, 256, 0, r->stream>>>(*prog, batch, rows, cols, *out);
    else if (prog->dtype == BT_FP32)
      elementwise_wide_kernel<BT_FP32><<<blocks, 256, 0, r->stream>>>(*prog, batch, rows, cols, *out);
    else elementwise_wide_kernel<BT_INT32><<<blocks, 256, 0, r->stream>>>(*prog, batch, rows, cols, *out);
  }
  BT_LAUNCHED("elementwise");
  return BT_OK;
}

int bt_reduce(bt_runtime *rt, const bt_program *prog, int kind, int axis, int64_t batch, int64_t rows, int64_t cols,
              int64_t sweep, int64_t step, const bt_operand *out) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (int s = check_program(prog)) return s;
  if (int s = check_out(out)) return s;
  if (kind != BT_REDUCE_SUM && kind != BT_REDUCE_MAX) return fail(BT_EINVAL, "reduction kind %d", kind);
  if (axis < 0 || axis > 2) return fail(BT_EINVAL, "reduction axis %d", axis);
  if (batch <= 0 || rows <= 0 || cols <= 0) return fail(BT_EINVAL, "reduction shape must be positive");
  if (prog->dtype == BT_INT32 && kind == BT_REDUCE_SUM) return fail(BT_EINVAL, "int32 sums go through fp32");
  if (axis == 0) {
    if (sweep <= 1) { sweep = batch; step = 1; }
    if (step < 1 || batch % (sweep * step)) return fail(BT_EINVAL, "sweep %lld x step %lld doesn't fold batch %lld",
                                                        (long long)sweep, (long long)step, (long long)batch);
  }
  int64_t outs = (axis == 0 ? batch / sweep : batch) * (axis == 1 ? 1 : rows) * (axis == 2 ? 1 : cols);
  const int64_t n = axis == 0 ? sweep : axis == 1 ? rows : cols;
  if (outs >= (1ll << 33)) return fail(BT_EINVAL, "a reduction of %lld outputs is too large", (long long)outs);
#define BT_REDUCE(WPO, blocks)                                                                                    \
  do {                                                                                                          \
    const unsigned threads = WPO > 4 ? 64 * WPO : 256;                                                          \
    if (prog->dtype == BT_BF16)                                                                                 \
      reduce_kernel<BT_BF16, WPO><<<blocks, threads, 0, r->stream>>>(*prog, kind, axis, batch, rows, cols, sweep, step, *out); \
    else if (prog->dtype == BT_FP32)                                                                            \
      reduce_kernel<BT_FP32, WPO><<<blocks, threads, 0, r->stream>>>(*prog, kind, axis, batch, rows, cols, sweep, step, *out); \
    else reduce_kernel<BT_INT32, WPO><<<blocks, threads, 0, r->stream>>>(*prog, kind, axis, batch, rows, cols, sweep, step, *out); \
  } while (0)
  if (axis == 2 && cols >= 64 && outs * cols >= (1 << 16)) {  // large: segments of neighbouring columns
#define BT_RSEG(WPO, blocks)                                                                                      \
  do {                                                                                                          \
    const unsigned threads = WPO > 4 ? 64 * WPO : 256;                                                          \
    if (prog->dtype == BT_BF16)                                                                                 \
      reduce_seg_kernel<BT_BF16, WPO><<<blocks, threads, 0, r->stream>>>(*prog, kind, batch, rows, cols, *out);   \
    else if (prog->dtype == BT_FP32)                                                                            \
      reduce_seg_kernel<BT_FP32, WPO><<<blocks, threads, 0, r->stream>>>(*prog, kind, batch, rows, cols, *out);   \
    else reduce_seg_kernel<BT_INT32, WPO><<<blocks, threads, 0, r->stream>>>(*prog, kind, batch, rows, cols, *out); \
  } while (0)
    if (outs < 2048) BT_RSEG(4, (unsigned)outs);  // (16 waves would leave each lane too few registers)
    else BT_RSEG(1, (unsigned)((outs + 3) / 4));
#undef BT_RSEG
    BT_LAUNCHED("reduce");
    return BT_OK;
  }
  // with too few outputs to fill the chip, a block of waves on each output: about one value a lane
  if (outs < 2048 && n > 512) BT_REDUCE(16, (unsigned)outs);
  else if (outs < 2048 && n > 128) BT_REDUCE(4, (unsigned)outs);
  else BT_REDUCE(1, (unsigned)((outs + 3) / 4));
#undef BT_REDUCE
  BT_LAUNCHED("reduce");
  return BT_OK;
}

int bt_gather(bt_runtime *rt, int dtype, uint64_t table, int64_t rows, int64_t cols, int64_t table_rstride,
              uint64_t ids, int64_t n, uint64_t out, int64_t out_rstride) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (dtype != BT_BF16 && dtype != BT_FP32 && dtype != BT_INT32) return fail(BT_EINVAL, "gather dtype %d", dtype);
  if (rows <= 0 || cols <= 0 || n < 0) return fail(BT_EINVAL, "gather shape");
  if (!n) return BT_OK;
  int size = dtype == BT_BF16 ? 2 : 4;
  gather_kernel<<<(unsigned)n, 256, 0, r->stream>>>((const uint8_t *)table, rows, cols * size, table_rstride * size,
                                                    (const int32_t *)ids, (uint8_t *)out, out_rstride * size);
  BT_LAUNCHED("gather");
  return BT_OK;
}

int bt_put(bt_runtime *rt, int dtype, uint64_t dst, int64_t batch, int64_t dst_rows, int64_t cols, int64_t dst_sb,
           int64_t dst_sr, uint64_t ids, int64_t n, uint64_t x, int64_t x_sb, int64_t x_sr) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (dtype != BT_BF16 && dtype != BT_FP32 && dtype != BT_INT32) return fail(BT_EINVAL, "put dtype %d", dtype);
  if (batch <= 0 || dst_rows <= 0 || cols <= 0 || n < 0) return fail(BT_EINVAL, "put shape");
  if (!n) return BT_OK;
  int size = dtype == BT_BF16 ? 2 : 4;
  int64_t row_bytes = cols * size;
  if (n <= PUT_SCAN) {
    const int wide = row_bytes % 16 == 0 && dst % 16 == 0 && x % 16 == 0 && (dst_sb * size) % 16 == 0 &&
                     (dst_sr * size) % 16 == 0 && (x_sb * size) % 16 == 0 && (x_sr * size) % 16 == 0;
    const int64_t units = batch * (wide ? row_bytes / 16 : row_bytes / 2);
    const dim3 grid((unsigned)n, (unsigned)std::min<int64_t>((units + 511) / 512, 65535));
    put_rows_kernel<<<grid, 256, 0, r->stream>>>((uint8_t *)dst, dst_rows, row_bytes, dst_sb * size, dst_sr * size,
                                                 (const int32_t *)ids, n, (const uint8_t *)x, x_sb * size, x_sr * size,
                                                 batch, wide);
  } else {
    int64_t pieces = (row_bytes / 2 + 255) / 256;
    put_kernel<<<(unsigned)(batch * pieces), 256, 0, r->stream>>>((uint8_t *)dst, dst_rows, row_bytes, dst_sb * size,
                                                                  dst_sr * size, (const int32_t *)ids, n,
                                                                  (const uint8_t *)x, x_sb * size, x_sr * size, pieces);
  }
  BT_LAUNCHED("put");
  return BT_OK;
}

}  // extern "C"

namespace bt {

// RoPE and the cache put of a decode step: a thread per (token, head, pair j, j + d/2), both outputs of the pair from
// the same two inputs.
__global__ void __launch_bounds__(256) rope_put_kernel(const bt_rope_args a) {
  const int half = a.head_dim / 2, nh = a.heads + 2 * a.kv;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)a.rows * nh * half) return;
  const int j = (int)(t % half), hh = (int)(t / half % nh), i = (int)(t / half / nh);
  const uint16_t *x = (const uint16_t *)(uintptr_t)a.qkv + (int64_t)i * a.qkv_sr + (int64_t)hh * a.head_dim;
  const uint16_t *cs = (const uint16_t *)(uintptr_t)a.cos + (int64_t)i * a.cs_sr + (int64_t)hh * a.head_dim;
  const uint16_t *sn = (const uint16_t *)(uintptr_t)a.sin + (int64_t)i * a.cs_sr + (int64_t)hh * a.head_dim;
  const float x1 = bf16_value(x[j]), x2 = bf16_value(x[j + half]);
  // products and sums rounded one by one (no fused multiply-add), as the qkv product's fused RoPE computes them
  const float y1 = __fsub_rn(__fmul_rn(x1, bf16_value(cs[j])), __fmul_rn(x2, bf16_value(sn[j])));
  const float y2 = __fadd_rn(__fmul_rn(x2, bf16_value(cs[j + half])), __fmul_rn(x1, bf16_value(sn[j + half])));
  uint16_t *dst;
  if (hh < a.heads) {
    dst = (uint16_t *)(uintptr_t)a.q + (int64_t)i * a.q_sr + (int64_t)hh * a.head_dim;
  } else {
    const int place = ((const int32_t *)(uintptr_t)a.places)[a.one_place ? 0 : i];
    if (place < 0 || place >= a.cache_rows) return;
    const int hk = hh - a.heads;
    const bool own = a.vcache && hk >= a.kv;  // a value head with a cache of its own
    dst = (uint16_t *)(uintptr_t)(own ? a.vcache : a.cache) + (int64_t)(own ? hk - a.kv : hk) * a.cache_sh +
          (int64_t)i * a.cache_tsh + (int64_t)place * a.cache_sr;
  }
  dst[j] = (uint16_t)bf16_packed(y1);
  dst[j + half] = (uint16_t)bf16_packed(y2);
}

// The same, 8 neighbouring pairs a thread with 16-byte loads and stores and 32-bit index arithmetic: for head widths
// a multiple of 16 with every row and head on a 16-byte boundary. Element by element the arithmetic of
// rope_put_kernel. hq divides by the head's 8-pair groups, nh by the heads.
__global__ void __launch_bounds__(256) rope_put8_kernel(const bt_rope_args a, const FastDiv hq, const FastDiv nh,
                                                        uint32_t threads) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= threads) return;
  const int half = a.head_dim / 2;
  const uint32_t th = fdiv(t, hq), ti = fdiv(th, nh);
  const int j = 8 * (int)(t - th * hq.d), hh = (int)(th - ti * nh.d), i = (int)ti;
  const uint16_t *x = (const uint16_t *)(uintptr_t)a.qkv + (int64_t)i * a.qkv_sr + (int64_t)hh * a.head_dim;
  const uint16_t *cs = (const uint16_t *)(uintptr_t)a.cos + (int64_t)i * a.cs_sr + (int64_t)hh * a.head_dim;
  const uint16_t *sn = (const uint16_t *)(uintptr_t)a.sin + (int64_t)i * a.cs_sr + (int64_t)hh * a.head_dim;
  const uint4 xa = *(const uint4 *)(x + j), xb = *(const uint4 *)(x + j + half);
  const uint4 ca = *(const uint4 *)(cs + j), cb = *(const uint4 *)(cs + j + half);
  const uint4 sa = *(const uint4 *)(sn + j), sb = *(const uint4 *)(sn + j + half);
  uint4 oa, ob;
  rope8(xa, xb, ca, cb, sa, sb, oa, ob);
  uint16_t *dst = rope_dst(a, i, hh);
  if (!dst) return;
  *(uint4 *)(dst + j) = oa;
  *(uint4 *)(dst + j + half) = ob;
}

}  // namespace bt

extern "C" int bt_rope_put(bt_runtime *rt, const bt_rope_args *args) {
  using namespace bt;
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!args) return fail(BT_EINVAL, "rope_put needs its arguments");
  const bt_rope_args &a = *args;
  if (!a.qkv || !a.cos || !a.sin || !a.q || !a.cache || !a.places) return fail(BT_EINVAL, "rope_put needs every buffer");
  if (a.rows < 1 || a.heads < 1 || a.kv < 1 || a.head_dim < 2 || a.head_dim % 2 || a.cache_rows < 1)
    return fail(BT_EINVAL, "rope_put shape: %d rows, %d heads, %d key heads of %d", a.rows, a.heads, a.kv, a.head_dim);
  const int64_t threads = (int64_t)a.rows * (a.heads + 2 * a.kv) * (a.head_dim / 2);
  if (threads >= (1ll << 31)) return fail(BT_EINVAL, "rope_put too large");
  const bool aligned = a.head_dim % 16 == 0 && (a.qkv | a.cos | a.sin | a.q | a.cache | a.vcache) % 16 == 0 &&
                       (a.qkv_sr | a.cs_sr | a.q_sr | a.cache_sh | a.cache_sr | a.cache_tsh) % 8 == 0;
  if (aligned) {
    const uint32_t t8 = (uint32_t)(threads / 8);
    rope_put8_kernel<<<(t8 + 255) / 256, 256, 0, r->stream>>>(a, make_fastdiv((uint32_t)(a.head_dim / 16)),
                                                               make_fastdiv((uint32_t)(a.heads + 2 * a.kv)), t8);
  } else {
    rope_put_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, r->stream>>>(a);
  }
  BT_LAUNCHED("rope_put");
  return BT_OK;
}

namespace bt {

// RMSNorm of one row a block. Rows of up to 8192 columns (k a multiple of 4, 16-byte aligned rows) are fetched whole
// into registers by 16-byte loads, every load issued before the first is used, so a row costs one trip to memory;
// longer or unaligned rows loop over the columns and read them twice.
template <bool REGS>
__global__ void __launch_bounds__(RMS_THREADS) rms_rows_kernel(const float *x, int64_t k, int64_t x_sr,
                                                               const uint16_t *w, float eps, uint16_t *out,
                                                               int64_t out_sr) {
  __shared__ float part[RMS_THREADS / 64];
  const int tid = threadIdx.x;
  const float *xr = x + (int64_t)blockIdx.x * x_sr;
  uint16_t *o = out + (int64_t)blockIdx.x * out_sr;
  if constexpr (REGS) {
    float4 v[RMS_NV];
    uint2 wv[RMS_NV];  // the weights, fetched with the row (one trip for both)
#pragma unroll
    for (int i = 0; i < RMS_NV; i++) {
      const int64_t c = ((int64_t)i * RMS_THREADS + tid) * 4;
      v[i] = c < k ? *(const float4 *)(xr + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      wv[i] = c < k ? *(const uint2 *)(w + c) : make_uint2(0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < RMS_NV; i++) {
      v[i].x = round_packed(v[i].x), v[i].y = round_packed(v[i].y);
      v[i].z = round_packed(v[i].z), v[i].w = round_packed(v[i].w);
    }
    const float r = rms_scale(v, k, eps, part);
#pragma unroll
    for (int i = 0; i < RMS_NV; i++) {
      const int64_t c = ((int64_t)i * RMS_THREADS + tid) * 4;
      if (c < k) *(uint2 *)(o + c) = rms_out(v[i], r, wv[i]);
    }
  } else {
    const int lane = tid & 63, wib = tid >> 6;
    float ss = 0.0f;
    for (int64_t c = tid; c < k; c += RMS_THREADS) {
      const float e = round_packed(xr[c]);
      ss += e * e;
    }
    ss = wave_sum(ss);
    if (lane == 0) part[wib] = ss;
    __syncthreads();
    float total = part[0];
#pragma unroll
    for (int i = 1; i < RMS_THREADS / 64; i++) total += part[i];
    const float r = 1.0f / sqrtf(total / (float)k + eps);
    for (int64_t c = tid; c < k; c += RMS_THREADS)
      o[c] = (uint16_t)bf16_packed(round_packed(xr[c]) * r * bf16_value(w[c]));
  }
}

}  // namespace bt

extern "C" int bt_rms_rows(bt_runtime *rt, uint64_t x, int64_t rows, int64_t k, int64_t x_sr, uint64_t w, float eps,
                           uint64_t out, int64_t out_sr) {
  using namespace bt;
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!x || !w || !out) return fail(BT_EINVAL, "rms_rows needs x, w and out");
  if (rows < 1 || rows >= (1ll << 31) || k < 1) return fail(BT_EINVAL, "rms_rows shape %lld x %lld", (long long)rows, (long long)k);
  const bool regs = k <= 8192 && k % 4 == 0 && x % 16 == 0 && x_sr % 4 == 0 && w % 8 == 0 && out % 8 == 0 && out_sr % 4 == 0;
  (regs ? rms_rows_kernel<true> : rms_rows_kernel<false>)<<<(unsigned)rows, RMS_THREADS, 0, r->stream>>>(
      (const float *)(uintptr_t)x, k, x_sr, (const uint16_t *)(uintptr_t)w, eps, (uint16_t *)(uintptr_t)out, out_sr);
  BT_LAUNCHED("rms_rows");
  return BT_OK;
}
