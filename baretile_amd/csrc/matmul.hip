// Matmul on the matrix cores: out = epilogue(A @ B), with A bf16 and B in columns tiles (bf16, bfp8 or bfp4).
//
// Every path multiplies with v_mfma_f32_16x16x32_bf16 in the same order: for each 64-row chunk of K, its lower then
// upper 32 rows, the products exact and summed in fp32. A block-float value is q * 2^(e - 133) (bfp8) or
// q * 2^(e - 129) (bfp4). The kernels split that power of two off the integer q and put it on whichever operand is
// cheaper to scale, which keeps every product exactly x * q * 2^(e - bias). So a block-float B gives bit for bit the
// product with the bf16 matrix of its values (docs/api.md:128-129, test_kernels.py:709-724), whichever way it is read.
//
// The skinny kernel is the decode GEMV: each wavefront takes 16 rows of A and one 16-column run of B over all of K,
// and the weight streams once from HBM in 64 x 16 tiles that are contiguous along K. All the tiles of a group of
// chunks are requested before the first is multiplied.
//   A-side scaling (up to 4 rows of A): per chunk, each lane scales one k of x by its run's 2^(e - bias) into LDS, so a
//     bfp8 weight needs only int -> bf16 (1.5 instructions a value) and a bfp4 weight goes through fp8 subnormals
//     with v_cvt_scalef32_pk_bf16_fp8 (1.25 a value).
//   B-side scaling (more rows): each weight gets its power of two with v_ldexp_f32, reading the biased exponent byte
//     straight from the tile.
#include "program.h"

namespace bt {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MatmulArgs {
  bt_operand a;
  const uint8_t *b;
  int64_t b_matrix_bytes;  // bytes of one matrix of B's tiles, or 0 when every batch entry reads matrix 0
  int32_t batch, m, k, n, chunks, nruns, mtiles;
  bt_program prog;
  bt_operand out;
};

template <int FMT> struct Tile;
template <> struct Tile<BT_BF16> { static constexpr int bytes = 2048; };
template <> struct Tile<BT_BFP8> { static constexpr int bytes = 1088; };
template <> struct Tile<BT_BFP4> { static constexpr int bytes = 576; };

// Loads through the global address space, so the compiler emits global_load (vector memory only) rather than flat.
// (The host pass of hipcc also parses device functions, and has no such address space.)
template <class T> __device__ __forceinline__ T gload(const T *p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return *(const __attribute__((address_space(1))) T *)p;
#else
  return *p;
#endif
}

__device__ __forceinline__ uint32_t pack_hi(float lo, float hi) {  // two exact fp32 values -> a bf16 pair
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// bfp8: eight signed bytes (k = 0..7 of the lane) -> bf16, optionally times 2^d per value (d: signed exponent bytes).
template <bool SCALED>
__device__ __forceinline__ bf16x8 q8_to_bf16(uint2 q, uint2 d) {
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; p++) {
    float f[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int j = 2 * p + u;
      const uint32_t qw = j < 4 ? q.x : q.y, dw = j < 4 ? d.x : d.y;
      f[u] = (float)(int)(int8_t)(qw >> (8 * (j & 3)));
      if (SCALED) f[u] = ldexpf(f[u], (int)(int8_t)(dw >> (8 * (j & 3))));
    }
    w[p] = pack_hi(f[0], f[1]);
  }
  uint4 v = make_uint4(w[0], w[1], w[2], w[3]);
  return *(const bf16x8 *)&v;
}

// bfp4: a lane's 4 bytes for one half hold values i and i + 4 in byte i (low, high nibble), each sign << 3 | magnitude.
// As fp8 e4m3 a byte sign << 7 | magnitude is the subnormal magnitude * 2^-9, so spreading the nibbles into bytes and
// converting gives q * 2^-9 exactly.
__device__ __forceinline__ void q4_to_fp8(uint32_t w, uint32_t &lo, uint32_t &hi) {
  lo = (w & 0x07070707u) | ((w << 4) & 0x80808080u);  // values 0..3
  hi = ((w >> 4) & 0x07070707u) | (w & 0x80808080u);  // values 4..7
}

__device__ __forceinline__ bf16x8 q4_to_bf16(uint32_t w) {  // q * 2^-9 as bf16, in k order
  uint32_t lo, hi;
  q4_to_fp8(w, lo, hi);
  uint32_t r[4];
  auto c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  auto c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  auto c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  auto c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  r[0] = __builtin_bit_cast(uint32_t, c0);
  r[1] = __builtin_bit_cast(uint32_t, c1);
  r[2] = __builtin_bit_cast(uint32_t, c2);
  r[3] = __builtin_bit_cast(uint32_t, c3);
  uint4 v = make_uint4(r[0], r[1], r[2], r[3]);
  return *(const bf16x8 *)&v;
}

__device__ __forceinline__ bf16x8 q4_to_bf16_scaled(uint32_t w, uint2 d) {  // q * 2^-9 * 2^d, in k order
  uint32_t lo, hi;
  q4_to_fp8(w, lo, hi);
  float f[8];
  auto a = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
  auto b = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
  auto c = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
  auto e = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
  f[0] = a[0]; f[1] = a[1]; f[2] = b[0]; f[3] = b[1]; f[4] = c[0]; f[5] = c[1]; f[6] = e[0]; f[7] = e[1];
  uint32_t r[4];
#pragma unroll
  for (int p = 0; p < 4; p++) {
    float u0 = ldexpf(f[2 * p], (int)(int8_t)((2 * p < 4 ? d.x : d.y) >> (8 * ((2 * p) & 3))));
    float u1 = ldexpf(f[2 * p + 1], (int)(int8_t)((2 * p + 1 < 4 ? d.x : d.y) >> (8 * ((2 * p + 1) & 3))));
    r[p] = pack_hi(u0, u1);
  }
  uint4 v = make_uint4(r[0], r[1], r[2], r[3]);
  return *(const bf16x8 *)&v;
}

// Lane l's 8 values of A for its row, columns k0 .. k0+7 (zero outside A). row is the lane's row of A (row 0 for a
// lane past the last row, which row_in marks). With VEC (row-major A on 16-byte boundaries, K a multiple of 8) it is
// one 16-byte load from an always valid address, then a select, so no lane branches around a load.
template <bool VEC>
__device__ __forceinline__ uint4 load_a(const uint16_t *row, bool row_in, int64_t sc, int k0, int kcols) {
  const bool in = row_in && k0 < kcols;
  if (VEC) {
    uint4 w = gload((const uint4 *)(row + (in ? k0 : 0)));
    return in ? w : make_uint4(0, 0, 0, 0);
  }
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 8; j++) h[j] = (in && k0 + j < kcols) ? gload(row + (int64_t)(k0 + j) * sc) : 0u;
  return make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
}

// The row within a tile of the exponent byte p (and of lane p's own k when A is scaled per k).
__device__ __forceinline__ int exp_row(int p) { return 32 * ((p >> 3) & 1) + 8 * (p >> 4) + (p & 7); }

// Registers of one chunk in flight.
struct Chunk {
  uint4 b0, b1;  // B's values: bf16 32 bytes; bfp8 16 bytes in b0; bfp4 8 bytes in b0.xy
  uint4 ex;      // B-side: the lane group's 16 exponent bytes. A-side: ex.x = the lane's own exponent byte
  uint4 a0, a1;  // B-side: A's two fragments. A-side: a0 = x at the lane's k for rows 0..3, a half word each
};

template <int FMT>
__device__ __forceinline__ void load_b(Chunk &r, const uint8_t *t, int lane) {
  if (FMT == BT_BF16) {
    r.b0 = gload((const uint4 *)(t + 32 * lane));
    r.b1 = gload((const uint4 *)(t + 32 * lane + 16));
  } else if (FMT == BT_BFP8) {
    r.b0 = gload((const uint4 *)(t + 64 + 16 * lane));
  } else {
    uint2 q = gload((const uint2 *)(t + 64 + 8 * lane));
    r.b0 = make_uint4(q.x, q.y, 0, 0);
  }
}

constexpr int GROUP_A = 12, GROUP_B = 8;  // chunks requested together (A-side, B-side)

// The epilogue of both kernels: lane holds rows 4g .. 4g+3 of the 16 x 16 tile at (mt, run), column col.
template <int DT>
__device__ __forceinline__ void store_tile(const MatmulArgs &args, const f32x4 &acc, int b, int mt, int run, int g,
                                           int col) {
  const int n = run * 16 + col;
  if (n >= args.n) return;
  const int64_t obase = operand_matrix(args.out, b) * args.out.sb + (int64_t)n * args.out.sc;
#pragma unroll 1
  for (int i = 0; i < 4; i++) {
    const int mm = mt * 16 + 4 * g + i;
    if (mm >= args.m) break;
    const uint32_t x = __float_as_uint(DT == BT_BF16 ? round_packed(acc[i]) : acc[i]);
    const uint32_t y = args.prog.n_inst ? run_program<DT>(args.prog, b, mm, n, x) : x;
    store_value<DT>(args.out, obase + (int64_t)mm * args.out.sr, y);
  }
}

// The wave's place in the grid: waves of a block take neighbouring runs, which are neighbouring tiles of B. The wave's
// index within its block is read once into a scalar register, so everything derived from it stays uniform.
struct WavePos {
  int lane, g, col, wib, run, mt, b;
  bool valid;
};
__device__ __forceinline__ WavePos wave_pos(const MatmulArgs &args) {
  WavePos p;
  p.lane = threadIdx.x & 63;
  p.g = p.lane >> 4;
  p.col = p.lane & 15;
  p.wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wave = blockIdx.x * 4 + p.wib;
  p.valid = wave < args.batch * args.mtiles * args.nruns;
  p.run = wave % args.nruns;
  p.mt = wave / args.nruns % args.mtiles;
  p.b = wave / args.nruns / args.mtiles;
  return p;
}

// A buffer resource over [base, base + bytes): loads through it take a scalar base and a 32-bit offset, and a load at
// or past `bytes` reads 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// A-side scaling, for up to 4 rows of A (ROWS = 1, or 4 with absent rows read as zeros) in row-major rows. Per chunk,
// lane l owns one k of the tile (the row of exponent byte l): it scales x at that k by the run's 2^d for each row into
// the wave's LDS slot for the chunk. Then each lane reads its A fragments from the slot, turns its B values into bf16
// integers (bfp8) or q * 2^-9 (bfp4), and multiplies. Lanes of rows past the last read row 0 of the slot: the matrix
// instruction keeps output rows independent, and those rows are never stored.
template <int FMT, int DT, int ROWS>
__global__ void __launch_bounds__(256) gemv_kernel(const MatmulArgs args) {
  constexpr int G = GROUP_A, SLOT = ROWS * 64, TB = Tile<FMT>::bytes;  // SLOT: halfwords of one chunk's scaled x
  __shared__ __attribute__((aligned(16))) uint16_t lds[4][G * SLOT];
  const WavePos p = wave_pos(args);
  if (!p.valid) return;
  const int lane = p.lane, g = p.g, col = p.col;
  const int rows = min(ROWS, args.m);
  uint16_t *slots = lds[p.wib];
  const uint8_t *tiles = args.b + (args.b_matrix_bytes ? p.b * args.b_matrix_bytes : 0) +
                         (int64_t)p.run * args.chunks * TB;
  const __amdgpu_buffer_rsrc_t tr = buffer(tiles, (uint32_t)args.chunks * TB);
  const uint16_t *abase = (const uint16_t *)args.a.ptr + operand_matrix(args.a, p.b) * args.a.sb;
  __amdgpu_buffer_rsrc_t xr[ROWS];
#pragma unroll
  for (int m = 0; m < ROWS; m++)
    xr[m] = buffer(abase + (int64_t)min(m, rows - 1) * args.a.sr, m < rows ? (uint32_t)args.k * 2 : 0u);
  const int kl = exp_row(lane);
  const int frag = min(col, rows - 1) * 64 + 8 * g;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < args.chunks; c0 += G) {
    uint32_t bq[G][4], ex[G], x[G][ROWS];  // B's value bytes (bfp8: 16, bfp4: 8), exponent byte, x at the lane's k
#pragma unroll
    for (int i = 0; i < G; i++) {
      const int c = c0 + i;
      if (c < args.chunks) {
        if (FMT == BT_BFP8 || FMT == BT_BF16) {  // block-float values start after the 64 exponent bytes
          const int at = FMT == BT_BFP8 ? 64 + 16 * lane : 32 * lane;
          const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at, c * TB, 0);
          bq[i][0] = q[0]; bq[i][1] = q[1]; bq[i][2] = q[2]; bq[i][3] = q[3];
        } else {
          const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr, 64 + 8 * lane, c * TB, 0);
          bq[i][0] = q[0]; bq[i][1] = q[1];
        }
        if (FMT != BT_BF16) ex[i] = __builtin_amdgcn_raw_buffer_load_b8(tr, lane, c * TB, 0);
#pragma unroll
        for (int m = 0; m < ROWS; m++) x[i][m] = __builtin_amdgcn_raw_buffer_load_b16(xr[m], 2 * (c * 64 + kl), 0, 0);
      }
    }
    uint4 bhi[G];  // bf16 B: the second 16 bytes of the lane's 32
    if (FMT == BT_BF16) {
#pragma unroll
      for (int i = 0; i < G; i++)
        if (c0 + i < args.chunks) {
          const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, 32 * lane + 16, (c0 + i) * TB, 0);
          bhi[i] = make_uint4(q[0], q[1], q[2], q[3]);
        }
    }
    // chunk by chunk, in load order, so each starts as soon as its own loads have landed: the scaled x into the
    // chunk's slot, then the fragments out of it
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (c0 + i >= args.chunks) continue;
      const int d = FMT == BT_BF16 ? 0 : (int)(int8_t)(ex[i] & 255u);
#pragma unroll
      for (int m = 0; m < ROWS; m++) {
        uint32_t v = x[i][m] & 0xFFFFu;
        if (FMT != BT_BF16) v = __float_as_uint(ldexpf(__uint_as_float(v << 16), d)) >> 16;
        slots[i * SLOT + m * 64 + kl] = (uint16_t)v;
      }
      __builtin_amdgcn_wave_barrier();
      bf16x8 av[2], bv[2];
#pragma unroll
      for (int h = 0; h < 2; h++) av[h] = *(const bf16x8 *)(slots + i * SLOT + frag + 32 * h);
      if (FMT == BT_BF16) {
        const uint4 lo = make_uint4(bq[i][0], bq[i][1], bq[i][2], bq[i][3]);
        bv[0] = *(const bf16x8 *)&lo;
        bv[1] = *(const bf16x8 *)&bhi[i];
      } else if (FMT == BT_BFP8) {
        bv[0] = q8_to_bf16<false>(make_uint2(bq[i][0], bq[i][1]), make_uint2(0, 0));
        bv[1] = q8_to_bf16<false>(make_uint2(bq[i][2], bq[i][3]), make_uint2(0, 0));
      } else {
        bv[0] = q4_to_bf16(bq[i][0]);
        bv[1] = q4_to_bf16(bq[i][1]);
      }
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bv[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[1], bv[1], acc, 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  }
  store_tile<DT>(args, acc, p.b, p.mt, p.run, g, col);
}

// B-side scaling, for any number of rows: each lane turns its 16 B values into bf16 q * 2^d with v_ldexp_f32 and
// reads its A fragments straight from memory.
template <int FMT, int DT, bool VEC>
__global__ void __launch_bounds__(256) skinny_kernel(const MatmulArgs args) {
  constexpr int G = GROUP_B;
  const WavePos p = wave_pos(args);
  if (!p.valid) return;
  const int lane = p.lane, g = p.g, col = p.col;
  const int rows = min(16, args.m - p.mt * 16);
  const uint8_t *tiles = args.b + (args.b_matrix_bytes ? p.b * args.b_matrix_bytes : 0) +
                         (int64_t)p.run * args.chunks * Tile<FMT>::bytes;
  const bool row_in = col < rows;
  const uint16_t *arow = (const uint16_t *)args.a.ptr + operand_matrix(args.a, p.b) * args.a.sb +
                         (int64_t)(p.mt * 16 + (row_in ? col : 0)) * args.a.sr;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < args.chunks; c0 += G) {
    Chunk r[G];
#pragma unroll
    for (int i = 0; i < G; i++) {
      const int c = c0 + i;
      if (c < args.chunks) {
        const uint8_t *t = tiles + (int64_t)c * Tile<FMT>::bytes;
        load_b<FMT>(r[i], t, lane);
        if (FMT != BT_BF16) r[i].ex = gload((const uint4 *)(t + 16 * g));
        r[i].a0 = load_a<VEC>(arow, row_in, args.a.sc, c * 64 + 8 * g, args.k);
        r[i].a1 = load_a<VEC>(arow, row_in, args.a.sc, c * 64 + 32 + 8 * g, args.k);
      }
    }
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (c0 + i >= args.chunks) continue;
      bf16x8 av[2], bv[2];
      av[0] = *(const bf16x8 *)&r[i].a0;
      av[1] = *(const bf16x8 *)&r[i].a1;
      if (FMT == BT_BF16) {
        bv[0] = *(const bf16x8 *)&r[i].b0;
        bv[1] = *(const bf16x8 *)&r[i].b1;
      } else if (FMT == BT_BFP8) {
        bv[0] = q8_to_bf16<true>(make_uint2(r[i].b0.x, r[i].b0.y), make_uint2(r[i].ex.x, r[i].ex.y));
        bv[1] = q8_to_bf16<true>(make_uint2(r[i].b0.z, r[i].b0.w), make_uint2(r[i].ex.z, r[i].ex.w));
      } else {
        bv[0] = q4_to_bf16_scaled(r[i].b0.x, make_uint2(r[i].ex.x, r[i].ex.y));
        bv[1] = q4_to_bf16_scaled(r[i].b0.y, make_uint2(r[i].ex.z, r[i].ex.w));
      }
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bv[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[1], bv[1], acc, 0, 0, 0);
    }
  }
  store_tile<DT>(args, acc, p.b, p.mt, p.run, g, col);
}

int validate_program(const bt_program *prog);
int check_out(const bt_operand *out);

template <int FMT, int DT>
static void launch_dt(const MatmulArgs &args, unsigned blocks, hipStream_t s, bool vec) {
  const bool rows_contiguous = args.a.sc == 1 && (int64_t)args.k * 2 < (1ll << 31);
  if (args.m == 1 && rows_contiguous) gemv_kernel<FMT, DT, 1><<<blocks, 256, 0, s>>>(args);
  else if (args.m <= 4 && rows_contiguous) gemv_kernel<FMT, DT, 4><<<blocks, 256, 0, s>>>(args);
  else if (vec) skinny_kernel<FMT, DT, true><<<blocks, 256, 0, s>>>(args);
  else skinny_kernel<FMT, DT, false><<<blocks, 256, 0, s>>>(args);
}

template <int FMT>
static void launch_skinny(const MatmulArgs &args, hipStream_t s) {
  const int64_t waves = (int64_t)args.batch * args.mtiles * args.nruns;
  const unsigned blocks = (unsigned)((waves + 3) / 4);
  const bt_operand &a = args.a;
  const bool vec = a.sc == 1 && a.sr % 8 == 0 && a.ptr % 16 == 0 && a.sb % 8 == 0 && args.k % 8 == 0;
  if (args.prog.dtype == BT_FP32) launch_dt<FMT, BT_FP32>(args, blocks, s, vec);
  else launch_dt<FMT, BT_BF16>(args, blocks, s, vec);
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
  if (batch > (1 << 30) || m > (1 << 30) || k > (1 << 30) || n > (1 << 30))
    return fail(BT_EINVAL, "matmul dimensions must stay below 2^30");
  if (b_batch != 1 && b_batch != batch) return fail(BT_EINVAL, "B's batch %lld for a batch of %lld",
                                                    (long long)b_batch, (long long)batch);
  if (b % 16) return fail(BT_EINVAL, "B's tiles must be 16-byte aligned");
  if (int s = check_out(out)) return s;
  MatmulArgs args;
  args.a = *a;
  args.b = (const uint8_t *)b;
  args.batch = (int32_t)batch;
  args.m = (int32_t)m;
  args.k = (int32_t)k;
  args.n = (int32_t)n;
  args.chunks = (int32_t)((k + 63) / 64);
  args.nruns = (int32_t)((n + 15) / 16);
  args.mtiles = (int32_t)((m + 15) / 16);
  if ((int64_t)args.batch * args.mtiles * args.nruns >= (1ll << 31) - 4) return fail(BT_EINVAL, "matmul too large");
  const int tb = b_fmt == BT_BF16 ? 2048 : b_fmt == BT_BFP8 ? 1088 : 576;
  args.b_matrix_bytes = b_batch > 1 ? (int64_t)args.chunks * args.nruns * tb : 0;
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
