// Top-k of rows: the k (at most 64) largest values of each row, or of each of `parts` equal parts of a row, in
// descending order with equal values in column order (numpy's stable argsort of -x), and -0 equal to 0. Restated from
// the reference's interface (tensor.py:685-706, test_kernels.py:2029-2062), in code of our own.
//
// One block per (row, part). The k-th largest value is found exactly by a radix select: each value becomes a 32-bit
// key whose unsigned order is the value order, and four passes over the part histogram one byte of the keys each
// (LDS atomics), narrowing to the byte prefix that holds the k-th largest: one wave scans the counts from the top,
// where one thread's walk over the 256 bins had made 49152 columns in 12 parts at k = 64 take 68 us, now 20. Then
// every value above that key is taken, and of the values equal to it the first in column order, as many as are still
// needed: a pass in column order, 256 columns at a time, ranks the equal ones with a block-wide count. One wavefront sorts the k picks (bitonic, 64
// lanes) by value, then column, and writes the values and their columns, or their labels when given. For k = 1 the
// largest is found without the select: each thread's best of its columns, then the wave's by lane swaps, then the
// block's.
#include "common.h"

namespace bt {

// The order key of an fp32 value's bits: larger value, larger key; -0 as 0.
__device__ __forceinline__ uint32_t order_key(uint32_t f) {
  if ((f & 0x7FFFFFFFu) == 0) f = 0;
  return f & 0x80000000u ? ~f : f | 0x80000000u;
}

// a comes before b: larger key, or equal keys and the smaller column
__device__ __forceinline__ bool before(uint32_t ka, int32_t ca, uint32_t kb, int32_t cb) {
  return ka > kb || (ka == kb && ca < cb);
}

template <int DT>
__device__ __forceinline__ uint32_t value_bits(const void *row, int64_t c) {  // as fp32 bits
  if (DT == BT_BF16) return (uint32_t)((const uint16_t *)row)[c] << 16;
  return ((const uint32_t *)row)[c];
}

template <int DT>
__global__ void __launch_bounds__(256) topk_kernel(const uint8_t *x, int64_t sb, int64_t sr, int rows, int width,
                                                   int parts, int k, const int32_t *labels, int64_t lsb, int64_t lsr,
                                                   uint8_t *values, int32_t *ids) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t cand_key[64];
  __shared__ int32_t cand_col[64];
  __shared__ uint32_t shared_u[4];  // [0] prefix, [1] still needed, [2] picks taken, [3] equal ones taken so far
  __shared__ uint32_t wave_eq[4];
  constexpr int SZ = DT == BT_BF16 ? 2 : 4;
  const int tid = threadIdx.x, lane = tid & 63, wib = tid >> 6;
  const int64_t unit = blockIdx.x;
  const int part = (int)(unit % parts);
  const int64_t rr = unit / parts, r = rr % rows, b = rr / rows;
  const uint8_t *row = x + (b * sb + r * sr) * SZ + (int64_t)part * width * SZ;

  if (k == 1) {  // the largest key, the first in column order: each thread's columns, then the wave's, then the block's
    uint32_t bk = 0;
    int32_t bc = 0x7FFFFFFF;
    for (int c = tid; c < width; c += 256) {
      const uint32_t key = order_key(value_bits<DT>(row, c));
      if (before(key, c, bk, bc)) bk = key, bc = c;
    }
    for (int stride = 32; stride > 0; stride >>= 1) {
      const uint32_t ok = __shfl_xor(bk, stride, 64);
      const int32_t oc = __shfl_xor(bc, stride, 64);
      if (before(ok, oc, bk, bc)) bk = ok, bc = oc;
    }
    if (lane == 0) cand_key[wib] = bk, cand_col[wib] = bc;
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < 4; w++)
        if (before(cand_key[w], cand_col[w], bk, bc)) bk = cand_key[w], bc = cand_col[w];
      const int64_t o = rr * (int64_t)parts + part;
      if (DT == BT_BF16) ((uint16_t *)values)[o] = ((const uint16_t *)row)[bc];
      else ((uint32_t *)values)[o] = ((const uint32_t *)row)[bc];
      const int64_t c = (int64_t)part * width + bc;
      ids[o] = labels ? labels[b * lsb + r * lsr + c] : (int32_t)c;
    }
    return;
  }

  // radix select of the k-th largest key
  uint32_t prefix = 0, mask = 0, need = (uint32_t)k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0;
    __syncthreads();
    for (int c = tid; c < width; c += 256) {
      const uint32_t key = order_key(value_bits<DT>(row, c));
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    // the highest bin b whose count with every bin above it, S(b), reaches need (S(0) always does: every value left
    // has the prefix); wave 0, four bins a lane, the sums over higher lanes by lane shifts
    if (wib == 0) {
      uint32_t h[4], t = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) h[j] = hist[4 * lane + j], t += h[j];
      uint32_t u = t;  // the lane's bins and every higher lane's
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_down(u, off, 64);
        if (lane + off < 64) u += o;
      }
      uint32_t s = u - t, at_s = 0, at_h = 0;
      int bin = -1;
#pragma unroll
      for (int j = 3; j >= 0; j--) {
        s += h[j];  // S(4 lane + j)
        if (bin < 0 && s >= need) bin = 4 * lane + j, at_s = s, at_h = h[j];
      }
      const uint64_t has = __ballot(bin >= 0);
      if (lane == 63 - __builtin_clzll(has)) {
        shared_u[0] = prefix | (uint32_t)bin << shift;
        shared_u[1] = need - (at_s - at_h);
      }
    }
    __syncthreads();
    prefix = shared_u[0], need = shared_u[1], mask |= 255u << shift;
    __syncthreads();
  }
  // prefix is now the k-th largest key; `need` of the values equal to it are picked, the first in column order
  if (tid == 0) shared_u[2] = 0, shared_u[3] = 0;
  __syncthreads();
  const uint32_t kth = prefix;
  for (int c0 = 0; c0 < width; c0 += 256) {
    const int c = c0 + tid;
    uint32_t key = 0;
    bool gt = false, eq = false;
    if (c < width) {
      key = order_key(value_bits<DT>(row, c));
      gt = key > kth, eq = key == kth;
    }
    if (gt) {
      const uint32_t at = atomicAdd(&shared_u[2], 1u);
      cand_key[at] = key, cand_col[at] = c;
    }
    // the rank of each equal value in column order: within the wave by ballot, across waves by their counts
    const uint64_t ball = __ballot(eq);
    const uint32_t below = __popcll(ball & ((1ull << lane) - 1ull));
    if (lane == 0) wave_eq[wib] = __popcll(ball);
    __syncthreads();
    uint32_t rank = shared_u[3] + below;
    for (int w = 0; w < wib; w++) rank += wave_eq[w];
    if (eq && rank < need) {
      const uint32_t at = atomicAdd(&shared_u[2], 1u);
      cand_key[at] = key, cand_col[at] = c;
    }
    __syncthreads();
    if (tid == 0) shared_u[3] += wave_eq[0] + wave_eq[1] + wave_eq[2] + wave_eq[3];
    __syncthreads();
  }
  if (wib != 0) return;
  // sort the k picks by key (descending), then column
  uint32_t key = lane < k ? cand_key[lane] : 0u;
  int32_t col = lane < k ? cand_col[lane] : 0x7FFFFFFF;
  for (int size = 2; size <= 64; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t ok = __shfl_xor(key, stride, 64);
      const int32_t oc = __shfl_xor(col, stride, 64);
      const bool up = (lane & size) == 0, lower = (lane & stride) == 0;
      const bool mine_first = before(key, col, ok, oc);
      if ((lower == up) != mine_first) key = ok, col = oc;
    }
  if (lane < k) {
    const int64_t o = rr * (int64_t)parts * k + (int64_t)part * k + lane;
    if (DT == BT_BF16) ((uint16_t *)values)[o] = ((const uint16_t *)row)[col];
    else ((uint32_t *)values)[o] = ((const uint32_t *)row)[col];
    const int64_t c = (int64_t)part * width + col;
    ids[o] = labels ? labels[b * lsb + r * lsr + c] : (int32_t)c;
  }
}

}  // namespace bt

using namespace bt;

extern "C" int bt_topk(bt_runtime *rt, int dtype, uint64_t x, int64_t batch, int64_t rows, int64_t cols, int64_t sb,
                       int64_t sr, int32_t parts, int32_t k, uint64_t labels, int64_t lsb, int64_t lsr,
                       uint64_t values, uint64_t ids) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (dtype != BT_BF16 && dtype != BT_FP32) return fail(BT_EINVAL, "topk takes bf16 or fp32, not dtype %d", dtype);
  if (!x || !values || !ids) return fail(BT_EINVAL, "topk needs x, values and ids");
  if (batch <= 0 || rows <= 0 || cols <= 0 || parts <= 0 || cols % parts)
    return fail(BT_EINVAL, "topk shape: %lld x %lld x %lld in %d parts", (long long)batch, (long long)rows,
                (long long)cols, parts);
  const int64_t width = cols / parts;
  if (k <= 0 || k > 64 || k > width) return fail(BT_EINVAL, "topk needs 1 <= k <= 64 and k up to a part's width");
  if (width >= (1ll << 31) || batch * rows * parts >= (1ll << 31)) return fail(BT_EINVAL, "topk too large");
  const unsigned blocks = (unsigned)(batch * rows * parts);
  if (dtype == BT_BF16)
    topk_kernel<BT_BF16><<<blocks, 256, 0, r->stream>>>((const uint8_t *)x, sb, sr, (int)rows, (int)width, parts, k,
                                                        (const int32_t *)labels, lsb, lsr, (uint8_t *)values,
                                                        (int32_t *)ids);
  else
    topk_kernel<BT_FP32><<<blocks, 256, 0, r->stream>>>((const uint8_t *)x, sb, sr, (int)rows, (int)width, parts, k,
                                                        (const int32_t *)labels, lsb, lsr, (uint8_t *)values,
                                                        (int32_t *)ids);
  BT_LAUNCHED("topk");
  return BT_OK;
}
