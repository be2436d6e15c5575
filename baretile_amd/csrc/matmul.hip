// Matmul on the matrix cores: out = epilogue(A @ B), with A bf16 and B in columns tiles (bf16, bfp8 or bfp4).
//
// Every path multiplies with v_mfma_f32_16x16x32_bf16 in the same order: for each 64-row chunk of K, its lower then
// upper 32 rows. A block-float B is turned into bf16 in registers, value by value, as q * 2^(e - 133) (bfp8) or
// q * 2^(e - 129) (bfp4), which is exact. So a block-float B gives bit for bit the product with the bf16 matrix of its
// values, as the reference promises (docs/api.md:128-129, test_kernels.py:709-724).
//
// The skinny kernel gives each wavefront 16 rows of A and one 16-column run of B, over all of K. It is the decode
// GEMV: the weight streams once from HBM in 64 x 16 tiles that are contiguous along K, each wave reading a run's tiles
// one after another, with 16-byte loads per lane.
#include "program.h"

namespace bt {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MatmulArgs {
  bt_operand a;
  const uint8_t *b;
  int64_t b_matrix_bytes;  // bytes of one matrix of B's tiles, or 0 when every batch entry reads matrix 0
  int64_t batch, m, k, n, chunks, nruns, mtiles;
  bt_program prog;
  bt_operand out;
};

template <int FMT> struct Tile;
template <> struct Tile<BT_BF16> { static constexpr int bytes = 2048; };
template <> struct Tile<BT_BFP8> { static constexpr int bytes = 1088; };
template <> struct Tile<BT_BFP4> { static constexpr int bytes = 576; };

// 8 bf16 of a bfp8 tile: bytes h*8 .. h*8+7 of the lane's 16, exponents likewise from the lane group's 16.
__device__ __forceinline__ bf16x8 dequant8(uint2 q, uint2 e) {
  bf16x8 out;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    uint32_t qw = j < 4 ? q.x : q.y, ew = j < 4 ? e.x : e.y;
    int qi = (int)(int8_t)(qw >> (8 * (j & 3)));
    int ei = (int)((ew >> (8 * (j & 3))) & 255u) - 133;
    out[j] = (short)(__float_as_uint(ldexpf((float)qi, ei)) >> 16);
  }
  return out;
}

__device__ __forceinline__ bf16x8 dequant4(uint32_t q, uint2 e) {
  bf16x8 out;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    int qi = ((int)(q << (28 - 4 * j))) >> 28;  // nibble j, sign-extended
    uint32_t ew = j < 4 ? e.x : e.y;
    int ei = (int)((ew >> (8 * (j & 3))) & 255u) - 129;
    out[j] = (short)(__float_as_uint(ldexpf((float)qi, ei)) >> 16);
  }
  return out;
}

// Lane l's 8 values of A for rows of the 16-row tile starting at m0, columns k0 .. k0+7 (zero outside A).
__device__ __forceinline__ bf16x8 load_a(const bt_operand &a, int64_t b, int64_t m, int64_t mrows, int64_t k0,
                                         int64_t kcols, bool vec) {
  bf16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (m >= mrows) return v;
  const uint16_t *row = (const uint16_t *)a.ptr + operand_matrix(a, b) * a.sb + m * a.sr;
  if (vec && k0 + 8 <= kcols) {
    uint4 w = *(const uint4 *)(row + k0);
    v[0] = (short)(w.x & 0xFFFF); v[1] = (short)(w.x >> 16); v[2] = (short)(w.y & 0xFFFF); v[3] = (short)(w.y >> 16);
    v[4] = (short)(w.z & 0xFFFF); v[5] = (short)(w.z >> 16); v[6] = (short)(w.w & 0xFFFF); v[7] = (short)(w.w >> 16);
    return v;
  }
#pragma unroll
  for (int j = 0; j < 8; j++)
    if (k0 + j < kcols) v[j] = (short)row[(k0 + j) * a.sc];
  return v;
}

template <int FMT, int DT>
__global__ void __launch_bounds__(256) skinny_kernel(const MatmulArgs args) {
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t total = args.batch * args.mtiles * args.nruns;
  if (wave >= total) return;
  // waves of a block take neighbouring runs, which are neighbouring tiles of B
  const int64_t run = wave % args.nruns, mt = wave / args.nruns % args.mtiles, b = wave / args.nruns / args.mtiles;
  const int64_t m = mt * 16 + col;
  const bool vec = args.a.sc == 1 && (args.a.sr % 8) == 0 && (args.a.ptr % 16) == 0 && (args.a.sb % 8) == 0;
  const uint8_t *tiles = args.b + (args.b_matrix_bytes ? b * args.b_matrix_bytes : 0) +
                         run * args.chunks * (int64_t)Tile<FMT>::bytes;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t c = 0; c < args.chunks; c++) {
    const uint8_t *t = tiles + c * Tile<FMT>::bytes;
    bf16x8 bv[2];
    if (FMT == BT_BF16) {
      const uint4 *p = (const uint4 *)(t + 32 * lane);
      uint4 w0 = p[0], w1 = p[1];
      bv[0] = *(const bf16x8 *)&w0;
      bv[1] = *(const bf16x8 *)&w1;
    } else {
      uint4 ex = *(const uint4 *)(t + 16 * g);
      if (FMT == BT_BFP8) {
        uint4 q = *(const uint4 *)(t + 64 + 16 * lane);
        bv[0] = dequant8(make_uint2(q.x, q.y), make_uint2(ex.x, ex.y));
        bv[1] = dequant8(make_uint2(q.z, q.w), make_uint2(ex.z, ex.w));
      } else {
        uint2 q = *(const uint2 *)(t + 64 + 8 * lane);
        bv[0] = dequant4(q.x, make_uint2(ex.x, ex.y));
        bv[1] = dequant4(q.y, make_uint2(ex.z, ex.w));
      }
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      bf16x8 av = load_a(args.a, b, m, args.m, c * 64 + 32 * h + 8 * g, args.k, vec);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv[h], acc, 0, 0, 0);
    }
  }
  // lane holds rows 4g .. 4g+3 of the tile, column `col`
  const int64_t n = run * 16 + col;
  if (n >= args.n) return;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int64_t mm = mt * 16 + 4 * g + i;
    if (mm >= args.m) continue;
    float v = acc[i];
    uint32_t x = __float_as_uint(DT == BT_BF16 ? round_packed(v) : v);
    uint32_t y = run_program<DT>(args.prog, b, mm, n, x);
    store_value<DT>(args.out, operand_matrix(args.out, b) * args.out.sb + mm * args.out.sr + n * args.out.sc, y);
  }
}

int validate_program(const bt_program *prog);
int check_out(const bt_operand *out);

template <int FMT>
static void launch_skinny(const MatmulArgs &args, hipStream_t s) {
  int64_t waves = args.batch * args.mtiles * args.nruns;
  unsigned blocks = (unsigned)((waves + 3) / 4);
  if (args.prog.dtype == BT_FP32) skinny_kernel<FMT, BT_FP32><<<blocks, 256, 0, s>>>(args);
  else skinny_kernel<FMT, BT_BF16><<<blocks, 256, 0, s>>>(args);
}

}  // namespace bt

using namespace bt;

extern "C" int bt_matmul(bt_runtime *rt, const bt_operand *a, int b_fmt, uint64_t b, int64_t b_batch, int64_t batch,
                         int64_t m, int64_t k, int64_t n, const bt_program *epilogue, const bt_operand *out) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!a || !a->ptr || !b) return fail(BT_EINVAL, "matmul needs A and B");
  if (a->dtype != BT_BF16) return fail(BT_EINVAL, "matmul's A is bf16");
  if (a->rep < 1 || a->cyc < 0) return fail(BT_EINVAL, "A's rep %d, cyc %d", a->rep, a->cyc);
  if (b_fmt != BT_BF16 && b_fmt != BT_BFP8 && b_fmt != BT_BFP4) return fail(BT_EINVAL, "B format %d", b_fmt);
  if (batch <= 0 || m <= 0 || k <= 0 || n <= 0) return fail(BT_EINVAL, "matmul shape must be positive");
  if (b_batch != 1 && b_batch != batch) return fail(BT_EINVAL, "B's batch %lld for a batch of %lld",
                                                    (long long)b_batch, (long long)batch);
  if (b % 16) return fail(BT_EINVAL, "B's tiles must be 16-byte aligned");
  if (int s = check_out(out)) return s;
  MatmulArgs args;
  args.a = *a;
  args.b = (const uint8_t *)b;
  args.batch = batch;
  args.m = m;
  args.k = k;
  args.n = n;
  args.chunks = (k + 63) / 64;
  args.nruns = (n + 15) / 16;
  args.mtiles = (m + 15) / 16;
  int tb = b_fmt == BT_BF16 ? 2048 : b_fmt == BT_BFP8 ? 1088 : 576;
  args.b_matrix_bytes = b_batch > 1 ? args.chunks * args.nruns * (int64_t)tb : 0;
  if (epilogue) {
    if (int s = validate_program(epilogue)) return s;
    if (epilogue->dtype == BT_INT32) return fail(BT_EINVAL, "a matmul's epilogue computes in bf16 or fp32");
    args.prog = *epilogue;
  } else {
    args.prog = bt_program{};
    args.prog.dtype = out->dtype == BT_FP32 ? BT_FP32 : BT_BF16;
  }
  args.out = *out;
  if (b_fmt == BT_BF16) launch_skinny<BT_BF16>(args, r->stream);
  else if (b_fmt == BT_BFP8) launch_skinny<BT_BFP8>(args, r->stream);
  else launch_skinny<BT_BFP4>(args, r->stream);
  BT_LAUNCHED("matmul");
  return BT_OK;
}
