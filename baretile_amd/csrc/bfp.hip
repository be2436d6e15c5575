// Block floats on the GPU: the cast into the plain planes, the exact unpacker, and the one-time repack into the
// columns tiles that the matmul kernels read.
//
// Rules (restated from the reference, in code of our own):
//   cast   models/gpt2.py:19-30, kernels.py:1074-1081 (NIBBLE), kernels.py:1108-1114 (put's bfp8 rule): round to bf16
//          (nearest even), take the run's largest exponent field `top`, keep 7 (bfp8) or 3 (bfp4) bits of magnitude
//          below it, rounding half up (bfp8) or to nearest with ties up (bfp4), saturating at 127 / 7. A zero keeps no
//          sign.
//   decode tensor.py:1093-1104 (_bf16s): normalize the magnitude, exponent (e - shift) mod 256.
#include "common.h"

namespace bt {

// A run of 16 bf16 values with its largest exponent field `top` into the plain planes: the exponent byte, then the
// 16 signed magnitudes (bfp8: a byte each; bfp4: two to a byte, the first in the low nibble).
template <int FMT>
__device__ __forceinline__ void store_run(const uint32_t (&bits)[16], uint32_t top, uint8_t *exp, uint8_t *val) {
  *exp = (uint8_t)top;
  if (FMT == BT_BFP8) {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; i++) w[i / 4] |= ((uint32_t)bfp_signed<8>(bits[i], top) & 255u) << (8 * (i % 4));
    *(uint4 *)val = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    uint32_t w[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 16; i++) w[i / 8] |= ((uint32_t)bfp_signed<4>(bits[i], top) & 15u) << (4 * (i % 8));
    *(uint2 *)val = make_uint2(w[0], w[1]);
  }
}

// One thread a run: 16 values of one row sharing an exponent. Runs are numbered along rows, so neighbouring threads
// read neighbouring 32-byte pieces of a bf16 row.
template <int FMT>
__global__ void __launch_bounds__(256) pack_kernel(const void *src, int src_dtype, int64_t batch, int64_t rows,
                                                   int64_t cols, int64_t sb, int64_t sr, int64_t sc, uint8_t *exps,
                                                   uint8_t *vals) {
  int64_t runs = (cols + 15) / 16;
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= batch * rows * runs) return;
  int64_t j = t % runs, r = t / runs % rows, b = t / runs / rows;
  uint32_t bits[16];
  uint32_t top = 0;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    int64_t c = j * 16 + i;
    uint32_t v = 0;
    if (c < cols) {
      int64_t at = b * sb + r * sr + c * sc;
      v = src_dtype == BT_BF16 ? ((const uint16_t *)src)[at] : bf16_rne(((const float *)src)[at]);
    }
    bits[i] = v;
    top = max(top, (v >> 7) & 255u);
  }
  store_run<FMT>(bits, top, exps + t, vals + t * (FMT == BT_BFP8 ? 16 : 8));
}

// One row of x (bf16) put into a plain block-float tensor at each place (Tensor.put into a block-float cache,
// kernels.py:1083-1168): a block a row of x, a thread a run of 16 of it in every batch entry, rounded as the cast
// rounds. A later duplicate place wins: the block first looks for a j > i with the same place. Strides are in
// values (multiples of 16); the planes hold a value's exponent byte at its index / 16 and its q at its index (bfp8)
// or index / 2 (bfp4).
template <int FMT>
__global__ void __launch_bounds__(256) put_bfp_kernel(uint8_t *exps, uint8_t *vals, int64_t dst_rows, int64_t cols,
                                                      int64_t dst_sb, int64_t dst_sr, const int32_t *ids, int64_t n,
                                                      const uint16_t *x, int64_t x_sb, int64_t x_sr, int64_t batch) {
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
  const int64_t runs = cols / 16;
  for (int64_t e = threadIdx.x; e < batch * runs; e += blockDim.x) {
    const int64_t b = e / runs, j = e % runs;
    const uint16_t *src = x + b * x_sb + i * x_sr + j * 16;
    uint32_t bits[16], top = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) bits[k] = src[k], top = max(top, (bits[k] >> 7) & 255u);
    const int64_t at = b * dst_sb + (int64_t)p * dst_sr + j * 16;  // the run's first value
    store_run<FMT>(bits, top, exps + at / 16, vals + (FMT == BT_BFP8 ? at : at / 2));
  }
}

// Counts, into *bad, the runs of the plain planes that hold a nonzero value under an exponent the matmul kernels can't
// read: they take the exponent byte as the signed power (e - 133) (bfp8) or (e - 120) (bfp4), so bfp8 needs e >= 5 and
// bfp4 e <= 247; and a bfp4 B decoded in registers needs e >= 3, where every value is a normal bf16. A run of zeros
// multiplies to zero under any exponent, so it never counts. One thread a run.
template <int FMT>
__global__ void __launch_bounds__(256) range_kernel(const uint8_t *exps, const uint8_t *vals, int64_t runs,
                                                   uint32_t *bad) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= runs) return;
  const uint32_t e = exps[t];
  if (FMT == BT_BFP8 ? e >= 5u : e >= 3u && e <= 247u) return;
  uint32_t any = 0;
  if (FMT == BT_BFP8) {
    const uint4 v = *(const uint4 *)(vals + t * 16);
    any = v.x | v.y | v.z | v.w;
  } else {
    const uint2 v = *(const uint2 *)(vals + t * 8);
    any = v.x | v.y;
  }
  if (any) atomicAdd(bad, 1u);
}

__global__ void zero_word_kernel(uint32_t *word) {
  if (threadIdx.x == 0) word[0] = 0;
}

// Signed q of value c in row r of matrix b of the plain planes.
template <int FMT>
__device__ __forceinline__ int plain_q(const uint8_t *vals, int64_t row_bytes, int64_t b_rows_r, int64_t c) {
  if (FMT == BT_BFP8) return (int)(int8_t)vals[b_rows_r * row_bytes + c];
  uint32_t byte = vals[b_rows_r * row_bytes + c / 2];
  int nib = (int)((byte >> (4 * (c & 1))) & 15u);
  return nib >= 8 ? nib - 16 : nib;
}

// One thread a value: bf16 bits exactly as the unpacker gives them.
template <int FMT>
__global__ void __launch_bounds__(256) unpack_kernel(const uint8_t *exps, const uint8_t *vals, int64_t batch,
                                                     int64_t rows, int64_t cols, uint16_t *dst) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= batch * rows * cols) return;
  int64_t c = t % cols, br = t / cols;  // br = b * rows + r
  int64_t runs = (cols + 15) / 16, cols16 = runs * 16;
  int q = plain_q<FMT>(vals, FMT == BT_BFP8 ? cols16 : cols16 / 2, br, c);
  uint32_t e = exps[br * runs + c / 16];
  dst[t] = (uint16_t)unpacked_bits(FMT == BT_BFP8 ? q : q * 16, e);
}

// Row of exponent byte p of a columns tile, and row of value j (of 8) for lane l, half h.
__device__ __forceinline__ int tile_row_of_exp(int p) { return 32 * ((p >> 3) & 1) + 8 * (p >> 4) + (p & 7); }
__device__ __forceinline__ int tile_row(int l, int h, int j) { return 32 * h + 8 * (l >> 4) + j; }

// A columns tile keeps each run's exponent as d = (e - bias) mod 256, read by the matmul as a signed byte: the
// power of two it applies to the integer magnitude (bfp8: q * 2^d) or to q * 2^-9, what a bfp4 value's fp8 form
// converts to (bfp4: q * 2^-9 * 2^d). The map is a bijection, so readback recovers e exactly.
template <int FMT> __device__ __forceinline__ uint32_t exp_bias() { return FMT == BT_BFP8 ? 133u : 120u; }

// Where value j (0..7) of a lane's half sits in its 4 bytes of a bfp4 columns tile, as sign and magnitude: for j < 4
// byte j's bit 7 and bits 0-2; for j >= 4 bits 4-6 of byte j - 4 and bit 3 of byte (j - 3) % 4. The matmul reads
// these as fp8 bytes with one mask, and with one rotate and a mask.
__device__ __forceinline__ uint32_t nibble_bits(int q, int j) {
  const uint32_t mag = (uint32_t)(q < 0 ? -q : q), sgn = q < 0 ? 1u : 0u;
  return j < 4 ? mag << (8 * j) | sgn << (8 * j + 7) : mag << (8 * (j - 4) + 4) | sgn << (8 * ((j - 3) & 3) + 3);
}
__device__ __forceinline__ int nibble_q(uint32_t w, int j) {  // the inverse: value j's signed q from the 4 bytes
  const uint32_t mag = (w >> (j < 4 ? 8 * j : 8 * (j - 4) + 4)) & 7u;
  const uint32_t sgn = (w >> (j < 4 ? 8 * j + 7 : 8 * ((j - 3) & 3) + 3)) & 1u;
  return sgn ? -(int)mag : (int)mag;
}

// One block a columns tile, one thread a lane. Reads the plain planes, writes the tile.
template <int FMT>
__global__ void __launch_bounds__(64) columns_kernel(const uint8_t *exps, const uint8_t *vals, int64_t rows,
                                                     int64_t cols, int64_t chunks, int64_t nruns, uint8_t *dst) {
  constexpr int TB = FMT == BT_BFP8 ? 1088 : 576;
  int64_t tile = blockIdx.x;  // (b * nruns + run) * chunks + chunk
  int64_t chunk = tile % chunks, run = tile / chunks % nruns, b = tile / chunks / nruns;
  int l = threadIdx.x;
  int64_t runs = (cols + 15) / 16, cols16 = runs * 16;
  uint8_t *out = dst + tile * TB;
  {  // exponent byte l
    int64_t k = chunk * 64 + tile_row_of_exp(l);
    uint32_t e = k < rows ? exps[(b * rows + k) * runs + run] : 0;
    out[l] = (uint8_t)((e - exp_bias<FMT>()) & 255u);
  }
  int64_t n = run * 16 + (l & 15);
  uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
  for (int h = 0; h < 2; h++)
#pragma unroll
    for (int j = 0; j < 8; j++) {
      int64_t k = chunk * 64 + tile_row(l, h, j);
      int q = (k < rows && n < cols16) ? plain_q<FMT>(vals, FMT == BT_BFP8 ? cols16 : cols16 / 2, b * rows + k, n) : 0;
      if (FMT == BT_BFP8) w[(h * 8 + j) / 4] |= ((uint32_t)q & 255u) << (8 * (j % 4));
      else w[h] |= nibble_bits(q, j);
    }
  if (FMT == BT_BFP8) *(uint4 *)(out + 64 + 16 * l) = make_uint4(w[0], w[1], w[2], w[3]);
  else *(uint2 *)(out + 64 + 8 * l) = make_uint2(w[0], w[1]);
}

__global__ void __launch_bounds__(64) bf16_columns_kernel(const uint16_t *src, int64_t rows, int64_t cols, int64_t sb,
                                                          int64_t sr, int64_t sc, int64_t chunks, int64_t nruns,
                                                          uint16_t *dst) {
  int64_t tile = blockIdx.x;
  int64_t chunk = tile % chunks, run = tile / chunks % nruns, b = tile / chunks / nruns;
  int l = threadIdx.x;
  int64_t n = run * 16 + (l & 15);
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    uint32_t pair = 0;
#pragma unroll
    for (int u = 0; u < 2; u++) {
      int h = (i + u) / 8, j = (i + u) % 8;
      int64_t k = chunk * 64 + tile_row(l, h, j);
      uint32_t v = (k < rows && n < cols) ? src[b * sb + k * sr + n * sc] : 0;
      pair |= v << (16 * u);
    }
    w[i / 2] = pair;
  }
  uint4 *out = (uint4 *)(dst + tile * 1024 + 16 * l);
  out[0] = make_uint4(w[0], w[1], w[2], w[3]);
  out[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// One thread a value of the result: finds it in its tile, decodes it exactly.
template <int FMT>
__global__ void __launch_bounds__(256) columns_unpack_kernel(const uint8_t *src, int64_t batch, int64_t rows,
                                                             int64_t cols, int64_t chunks, int64_t nruns,
                                                             uint16_t *dst) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= batch * rows * cols) return;
  int64_t n = t % cols, k = t / cols % rows, b = t / cols / rows;
  int64_t run = n / 16, chunk = k / 64;
  int kk = (int)(k % 64), h = kk / 32, g = (kk % 32) / 8, j = kk % 8, l = g * 16 + (int)(n % 16);
  int64_t tile = (b * nruns + run) * chunks + chunk;
  if (FMT == BT_BF16) {
    dst[t] = ((const uint16_t *)src)[tile * 1024 + 16 * l + 8 * h + j];
    return;
  }
  constexpr int TB = FMT == BT_BFP8 ? 1088 : 576;
  const uint8_t *tp = src + tile * TB;
  uint32_t e = (tp[16 * g + 8 * h + j] + exp_bias<FMT>()) & 255u;
  int q;
  if (FMT == BT_BFP8) q = (int)(int8_t)tp[64 + 16 * l + 8 * h + j];
  else {
    q = nibble_q(*(const uint32_t *)(tp + 64 + 8 * l + 4 * h), j) * 16;
  }
  dst[t] = (uint16_t)unpacked_bits(q, e);
}

static int check_fmt(int fmt) {
  if (fmt != BT_BFP8 && fmt != BT_BFP4) return fail(BT_EINVAL, "block-float format must be bfp8 or bfp4, not %d", fmt);
  return BT_OK;
}

static int check_shape(int64_t batch, int64_t rows, int64_t cols) {
  if (batch <= 0 || rows <= 0 || cols <= 0)
    return fail(BT_EINVAL, "shape %lld x %lld x %lld must be positive", (long long)batch, (long long)rows,
                (long long)cols);
  return BT_OK;
}

static unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace bt

using namespace bt;

extern "C" {

int bt_bfp_pack(bt_runtime *rt, int fmt, uint64_t src, int src_dtype, int64_t batch, int64_t rows, int64_t cols,
                int64_t sb, int64_t sr, int64_t sc, uint64_t exps, uint64_t vals) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (int s = check_fmt(fmt)) return s;
  if (int s = check_shape(batch, rows, cols)) return s;
  if (src_dtype != BT_BF16 && src_dtype != BT_FP32) return fail(BT_EINVAL, "a block float is cast from bf16 or fp32");
  if (vals % 16) return fail(BT_EINVAL, "the value plane must be 16-byte aligned");
  int64_t n = batch * rows * ((cols + 15) / 16);
  if (fmt == BT_BFP8)
    pack_kernel<BT_BFP8><<<blocks_for(n, 256), 256, 0, r->stream>>>((const void *)src, src_dtype, batch, rows, cols,
                                                                     sb, sr, sc, (uint8_t *)exps, (uint8_t *)vals);
  else
    pack_kernel<BT_BFP4><<<blocks_for(n, 256), 256, 0, r->stream>>>((const void *)src, src_dtype, batch, rows, cols,
                                                                     sb, sr, sc, (uint8_t *)exps, (uint8_t *)vals);
  BT_LAUNCHED("bfp_pack");
  return BT_OK;
}

int bt_bfp_unpack(bt_runtime *rt, int fmt, uint64_t exps, uint64_t vals, int64_t batch, int64_t rows, int64_t cols,
                  uint64_t dst) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (int s = check_fmt(fmt)) return s;
  if (int s = check_shape(batch, rows, cols)) return s;
  int64_t n = batch * rows * cols;
  if (fmt == BT_BFP8)
    unpack_kernel<BT_BFP8><<<blocks_for(n, 256), 256, 0, r->stream>>>((const uint8_t *)exps, (const uint8_t *)vals,
                                                                       batch, rows, cols, (uint16_t *)dst);
  else
    unpack_kernel<BT_BFP4><<<blocks_for(n, 256), 256, 0, r->stream>>>((const uint8_t *)exps, (const uint8_t *)vals,
                                                                       batch, rows, cols, (uint16_t *)dst);
  BT_LAUNCHED("bfp_unpack");
  return BT_OK;
}

int bt_bfp_columns(bt_runtime *rt, int fmt, uint64_t exps, uint64_t vals, int64_t batch, int64_t rows, int64_t cols,
                   uint64_t dst) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (int s = check_fmt(fmt)) return s;
  if (int s = check_shape(batch, rows, cols)) return s;
  if (dst % 16) return fail(BT_EINVAL, "columns tiles must be 16-byte aligned");
  int64_t chunks = (rows + 63) / 64, nruns = (cols + 15) / 16, tiles = batch * nruns * chunks;
  if (tiles >= (1ll << 31)) return fail(BT_EINVAL, "too many tiles");
  if (fmt == BT_BFP8)
    columns_kernel<BT_BFP8><<<(unsigned)tiles, 64, 0, r->stream>>>((const uint8_t *)exps, (const uint8_t *)vals, rows,
                                                                    cols, chunks, nruns, (uint8_t *)dst);
  else
    columns_kernel<BT_BFP4><<<(unsigned)tiles, 64, 0, r->stream>>>((const uint8_t *)exps, (const uint8_t *)vals, rows,
                                                                    cols, chunks, nruns, (uint8_t *)dst);
  BT_LAUNCHED("bfp_columns");
  return BT_OK;
}

int bt_bfp_range(bt_runtime *rt, int fmt, uint64_t exps, uint64_t vals, int64_t batch, int64_t rows, int64_t cols,
                 uint64_t bad) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (int s = check_fmt(fmt)) return s;
  if (int s = check_shape(batch, rows, cols)) return s;
  if (vals % 16 || bad % 4) return fail(BT_EINVAL, "the value plane must be 16-byte aligned and the count 4-byte aligned");
  const int64_t runs = batch * rows * ((cols + 15) / 16);
  zero_word_kernel<<<1, 64, 0, r->stream>>>((uint32_t *)(uintptr_t)bad);
  BT_LAUNCHED("bfp_range");
  if (fmt == BT_BFP8)
    range_kernel<BT_BFP8><<<blocks_for(runs, 256), 256, 0, r->stream>>>((const uint8_t *)exps, (const uint8_t *)vals,
                                                                         runs, (uint32_t *)(uintptr_t)bad);
  else
    range_kernel<BT_BFP4><<<blocks_for(runs, 256), 256, 0, r->stream>>>((const uint8_t *)exps, (const uint8_t *)vals,
                                                                         runs, (uint32_t *)(uintptr_t)bad);
  BT_LAUNCHED("bfp_range");
  return BT_OK;
}

int bt_bf16_columns(bt_runtime *rt, uint64_t src, int64_t batch, int64_t rows, int64_t cols, int64_t sb, int64_t sr,
                    int64_t sc, uint64_t dst) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (int s = check_shape(batch, rows, cols)) return s;
  if (dst % 16) return fail(BT_EINVAL, "columns tiles must be 16-byte aligned");
  int64_t chunks = (rows + 63) / 64, nruns = (cols + 15) / 16, tiles = batch * nruns * chunks;
  if (tiles >= (1ll << 31)) return fail(BT_EINVAL, "too many tiles");
  bf16_columns_kernel<<<(unsigned)tiles, 64, 0, r->stream>>>((const uint16_t *)src, rows, cols, sb, sr, sc, chunks,
                                                              nruns, (uint16_t *)dst);
  BT_LAUNCHED("bf16_columns");
  return BT_OK;
}

int bt_columns_unpack(bt_runtime *rt, int fmt, uint64_t src, int64_t batch, int64_t rows, int64_t cols,
                      uint64_t dst) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (fmt != BT_BF16 && fmt != BT_BFP8 && fmt != BT_BFP4) return fail(BT_EINVAL, "columns format %d", fmt);
  if (int s = check_shape(batch, rows, cols)) return s;
  int64_t chunks = (rows + 63) / 64, nruns = (cols + 15) / 16, n = batch * rows * cols;
  if (fmt == BT_BF16)
    columns_unpack_kernel<BT_BF16><<<blocks_for(n, 256), 256, 0, r->stream>>>((const uint8_t *)src, batch, rows, cols,
                                                                               chunks, nruns, (uint16_t *)dst);
  else if (fmt == BT_BFP8)
    columns_unpack_kernel<BT_BFP8><<<blocks_for(n, 256), 256, 0, r->stream>>>((const uint8_t *)src, batch, rows, cols,
                                                                               chunks, nruns, (uint16_t *)dst);
  else
    columns_unpack_kernel<BT_BFP4><<<blocks_for(n, 256), 256, 0, r->stream>>>((const uint8_t *)src, batch, rows, cols,
                                                                               chunks, nruns, (uint16_t *)dst);
  BT_LAUNCHED("columns_unpack");
  return BT_OK;
}

int bt_put_bfp(bt_runtime *rt, int fmt, uint64_t exps, uint64_t vals, int64_t batch, int64_t dst_rows, int64_t cols,
               int64_t dst_sb, int64_t dst_sr, uint64_t ids, int64_t n, uint64_t x, int64_t x_sb, int64_t x_sr) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (fmt != BT_BFP8 && fmt != BT_BFP4) return fail(BT_EINVAL, "put_bfp writes bfp8 or bfp4, not %d", fmt);
  if (!exps || !vals || !ids || !x) return fail(BT_EINVAL, "put_bfp needs its planes, ids and x");
  if (batch < 1 || dst_rows < 1 || cols < 16 || cols % 16 || n < 0 || dst_sb % 16 || dst_sr % 16)
    return fail(BT_EINVAL, "put_bfp shape: batch %lld, %lld rows of %lld (a multiple of 16), strides %lld %lld",
                (long long)batch, (long long)dst_rows, (long long)cols, (long long)dst_sb, (long long)dst_sr);
  if (ids % 4 || x % 2) return fail(BT_EINVAL, "put_bfp needs aligned ids and x");
  if (n == 0) return BT_OK;
  if (n >= (1ll << 31)) return fail(BT_EINVAL, "put_bfp: too many rows");
  if (fmt == BT_BFP8)
    put_bfp_kernel<BT_BFP8><<<(unsigned)n, 256, 0, r->stream>>>((uint8_t *)exps, (uint8_t *)vals, dst_rows, cols, dst_sb,
                                                               dst_sr, (const int32_t *)ids, n, (const uint16_t *)x, x_sb,
                                                               x_sr, batch);
  else
    put_bfp_kernel<BT_BFP4><<<(unsigned)n, 256, 0, r->stream>>>((uint8_t *)exps, (uint8_t *)vals, dst_rows, cols, dst_sb,
                                                               dst_sr, (const int32_t *)ids, n, (const uint16_t *)x, x_sb,
                                                               x_sr, batch);
  BT_LAUNCHED("put_bfp");
  return BT_OK;
}

}  // extern "C"
