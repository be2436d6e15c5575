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
//     with v_cvt_scalef32_pk_bf16_fp8 (7 instructions for 8 values: a mask, a rotate and a mask, 4 conversions).
//   B-side scaling (more rows): each weight gets its power of two with v_ldexp_f32, reading the biased exponent byte
//     straight from the tile.
#include "rows.h"
#include "lds_load.h"
#include <cstdlib>

namespace bt {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The kernel arguments. What a wave reads comes first: the shape, A and the output operand sit in the first 144
// bytes, so they arrive in the first scalar loads; the program, which only an epilogue reads, comes last.
struct MatmulArgs {
  const uint8_t *b;
  int64_t b_matrix_bytes;  // bytes of one matrix of B's tiles, or 0 when every batch entry reads matrix 0
  int32_t batch, m, k, n, chunks, nruns, mtiles;
  int32_t n_inst;  // prog.n_inst
  bt_operand a;
  bt_operand out;
  bt_program prog;
};

// Every argument but the program, read at the start of a kernel. One statement takes them all, so their scalar loads
// are issued together and waited for once, rather than each sunk to its first use (a kernel argument first read near
// the end is one more trip to memory there).
struct Head {
  const uint8_t *b;
  int64_t b_matrix_bytes;
  int32_t batch, m, k, n, chunks, nruns, mtiles, n_inst;
  bt_operand a, out;
};
__device__ __forceinline__ Head early_head(const MatmulArgs &args) {
  Head h;
  h.b = args.b, h.b_matrix_bytes = args.b_matrix_bytes;
  h.batch = args.batch, h.m = args.m, h.k = args.k, h.n = args.n;
  h.chunks = args.chunks, h.nruns = args.nruns, h.mtiles = args.mtiles, h.n_inst = args.n_inst;
  h.a = args.a, h.out = args.out;
  asm volatile("" ::"s"(h.b), "s"(h.b_matrix_bytes), "s"(h.batch), "s"(h.m), "s"(h.k), "s"(h.n), "s"(h.chunks),
               "s"(h.nruns), "s"(h.mtiles), "s"(h.n_inst), "s"(h.a.ptr), "s"(h.a.sb), "s"(h.a.sr), "s"(h.a.sc),
               "s"(h.a.dtype), "s"(h.a.rep), "s"(h.a.cyc), "s"(h.out.ptr), "s"(h.out.sb), "s"(h.out.sr),
               "s"(h.out.sc), "s"(h.out.dtype), "s"(h.out.rep), "s"(h.out.cyc));
  return h;
}

template <int FMT> struct Tile;
template <> struct Tile<BT_BF16> { static constexpr int bytes = 2048; };
template <> struct Tile<BT_BFP8> { static constexpr int bytes = 1088; };
template <> struct Tile<BT_BFP4> { static constexpr int bytes = 576; };


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

// bfp4: a lane's 4 bytes for one half hold its 8 values as sign and magnitude. Byte i has value i's sign in bit 7 and
// magnitude in bits 0-2, value i + 4's magnitude in bits 4-6, and in bit 3 the sign of value 4 + (i + 3) % 4. So
// w & 0x87 in every byte is value i as an fp8 e4m3 byte sign << 7 | magnitude, and the same mask over w rotated right
// by 4 bits is value i + 4 (its magnitude comes down from bits 4-6, its sign from bit 3 of the next byte up). As fp8
// e4m3 such a byte is the subnormal magnitude * 2^-9, so converting gives q * 2^-9 exactly: 3 instructions spread 8
// values into bytes.
__device__ __forceinline__ void q4_to_fp8(uint32_t w, uint32_t &lo, uint32_t &hi) {
  lo = w & 0x87878787u;                                           // values 0..3
  hi = __builtin_amdgcn_alignbit(w, w, 4u) & 0x87878787u;         // values 4..7
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

// bfp4, B side, without a per-value ldexp: the lane's 8 values of one half (w, laid out as q4_to_fp8 reads it) times
// their own powers of two. Each pair converts through fp8 with the scale 2^127, which puts a nonzero q at the bf16
// exponent field lg|q| + 245, normal whatever q is; then a saturating 16-bit subtraction takes each value's gap
// x = 247 - e off its exponent field (the sign bit is above it, the mantissa below), giving q * 2^(e - 129) exactly,
// and leaves a zero at zero (0 - anything saturates to 0). x0 and x1 hold the gaps of values 0..3 and 4..7 as bytes;
// a columns tile stores d = e - 120 as a byte, and 247 - e = 127 - d = d ^ 0x7F bytewise. Exact for run exponents e in
// 3..247, where every result is a normal bf16.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t sub_placed(uint32_t bits, uint32_t placed) {  // placed: two gaps << 7
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, bits),
                                                                    __builtin_bit_cast(u16x2, placed)));
}
__device__ __forceinline__ uint32_t gap_sub(uint32_t bits, uint32_t x, uint32_t sel) {
  return sub_placed(bits, __builtin_amdgcn_perm(0u, x, sel) << 7);  // two gaps, one in each half's exponent field
}
// A columns tile's exponent bytes d (4 a word) as the gaps 127 - d of values (0, 1) and (2, 3), each pair two 16-bit
// halves already shifted into the bf16 exponent field: what q4_to_bf16_placed takes.
__device__ __forceinline__ uint2 place_gaps(uint32_t d) {
  const uint32_t x = d ^ 0x7F7F7F7Fu;
  return make_uint2(__builtin_amdgcn_perm(0u, x, 0x0C010C00u) << 7, __builtin_amdgcn_perm(0u, x, 0x0C030C02u) << 7);
}
__device__ __forceinline__ bf16x8 q4_to_bf16_gaps(uint32_t w, uint32_t x0, uint32_t x1) {
  uint32_t lo, hi;
  q4_to_fp8(w, lo, hi);
  const uint32_t c0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 0x1p127f, false));
  const uint32_t c1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 0x1p127f, true));
  const uint32_t c2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 0x1p127f, false));
  const uint32_t c3 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 0x1p127f, true));
  uint4 v = make_uint4(gap_sub(c0, x0, 0x0C010C00u), gap_sub(c1, x0, 0x0C030C02u), gap_sub(c2, x1, 0x0C010C00u),
                       gap_sub(c3, x1, 0x0C030C02u));
  return *(const bf16x8 *)&v;
}
// The same with the gaps of values (0, 1), (2, 3), (4, 5), (6, 7) placed beforehand (place_gaps), in p.x .. p.w.
__device__ __forceinline__ bf16x8 q4_to_bf16_placed(uint32_t w, uint4 p) {
  uint32_t lo, hi;
  q4_to_fp8(w, lo, hi);
  const uint32_t c0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 0x1p127f, false));
  const uint32_t c1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 0x1p127f, true));
  const uint32_t c2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 0x1p127f, false));
  const uint32_t c3 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 0x1p127f, true));
  uint4 v = make_uint4(sub_placed(c0, p.x), sub_placed(c1, p.y), sub_placed(c2, p.z), sub_placed(c3, p.w));
  return *(const bf16x8 *)&v;
}

// q * 2^-9 * 2^d for a lane's 8 bfp4 values, d the signed exponent bytes of values 0..3 (d.x) and 4..7 (d.y) as a
// columns tile stores them: the same exact values as q4_to_bf16_gaps, which computes them.
__device__ __forceinline__ bf16x8 q4_to_bf16_scaled(uint32_t w, uint2 d) {
  return q4_to_bf16_gaps(w, d.x ^ 0x7F7F7F7Fu, d.y ^ 0x7F7F7F7Fu);
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

constexpr int GROUP_B = 8;  // chunks requested together by the B-side kernel

// The epilogue of both kernels: lane holds rows 4g .. 4g+3 of the 16 x 16 tile at (mt, run), column col.
// ONE: a batch of one, so the output's matrix is matrix 0. PROG: 1 runs the epilogue program, 0 stores plainly, -1
// reads which from the arguments.
template <int DT, bool INL = false, bool ONE = false, int PROG = -1>
__device__ __forceinline__ void store_tile(const MatmulArgs &args, const Head &h, const f32x4 &acc, int b, int mt,
                                           int run, int g, int col) {
  const int n = run * 16 + col;
  if (n >= h.n) return;
  const bt_operand &out = h.out;
  const int m = h.m;
  const int64_t obase = (ONE ? 0 : operand_matrix(out, b) * out.sb) + (int64_t)n * out.sc;
  // two loops, so the program's setup (its operands' fields, loop invariant) is hoisted only into the loop that needs
  // it, never onto the path of a plain store
  if (PROG == 0 || (PROG < 0 && h.n_inst == 0)) {
#pragma unroll 1
    for (int i = 0; i < 4; i++) {
      const int mm = mt * 16 + 4 * g + i;
      if (mm >= m) break;
      store_value<DT>(out, obase + (int64_t)mm * out.sr, __float_as_uint(DT == BT_BF16 ? round_packed(acc[i]) : acc[i]));
    }
    return;
  }
  if constexpr (PROG != 0) {
  // a program of one operation on the product and no inputs (relu(x), silu(x), x * x, ...): the operation straight on
  // the lane's 4 values, without the evaluator's register file (its other registers read as 0 until written); the
  // same arithmetic, so the same bits
  const bt_inst in0 = args.prog.inst[0];
  if (h.n_inst == 1 && args.prog.n_inputs == 0 && args.prog.result == in0.dst && in0.op != BT_OP_LOAD &&
      in0.op != BT_OP_CONST && in0.op != BT_OP_MOV && in0.op != BT_OP_WHERE) {
    Vals<4> va, vb;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t x = __float_as_uint(DT == BT_BF16 ? round_packed(acc[i]) : acc[i]);
      va.x[i] = in0.a == 0 ? x : 0u;
      vb.x[i] = in0.b == 0 ? x : 0u;
    }
    const Vals<4> o = apply_op<DT, 4, INL>(in0.op, va, vb);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int mm = mt * 16 + 4 * g + i;
      if (mm < m) store_value<DT>(out, obase + (int64_t)mm * out.sr, o.x[i]);
    }
    return;
  }
#pragma unroll 1
  for (int i = 0; i < 4; i++) {
    const int mm = mt * 16 + 4 * g + i;
    if (mm >= m) break;
    const uint32_t x = __float_as_uint(DT == BT_BF16 ? round_packed(acc[i]) : acc[i]);
    store_value<DT>(out, obase + (int64_t)mm * out.sr, run_program<DT, INL>(args.prog, b, mm, n, x));
  }
  }
}

// The wave's place in the grid: waves of a block take neighbouring runs, which are neighbouring tiles of B. The wave's
// index within its block is read once into a scalar register, so everything derived from it stays uniform.
struct WavePos {
  int lane, g, col, wib, run, mt, b;
  bool valid;
};
template <bool ONE = false> __device__ __forceinline__ WavePos wave_pos(const Head &h) {
  WavePos p;
  p.lane = threadIdx.x & 63;
  p.g = p.lane >> 4;
  p.col = p.lane & 15;
  p.wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wave = blockIdx.x * 4 + p.wib;
  const int batch = h.batch, mtiles = h.mtiles, nruns = h.nruns;
  if (ONE) {  // one matrix (a batch of one): waves are runs of each 16-row tile in turn
    p.valid = wave < mtiles * nruns;
    p.b = 0;
    if (mtiles == 1) p.run = wave, p.mt = 0;
    else p.run = wave % nruns, p.mt = wave / nruns;
    return p;
  }
  p.valid = wave < batch * mtiles * nruns;
  if (batch == 1 && mtiles == 1) {  // a single GEMV: no division
    p.run = wave, p.mt = 0, p.b = 0;
  } else {
    p.run = wave % nruns;
    p.mt = wave / nruns % mtiles;
    p.b = wave / nruns / mtiles;
  }
  return p;
}

// A buffer resource over [base, base + bytes): loads through it take a scalar base and a 32-bit offset, and a load at
// or past `bytes` reads 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// The place of a wave in the decode kernels' grid. There are `units` output tiles (a 16-column run of one batch entry,
// with one group of 16-row tiles for the skinny kernel); each is split along K into `slices` (1, 2, 4 or 8) whose
// waves sit side by side in one block, so a deep K still gives enough waves to keep every CU's loads in flight. A
// slice is a whole number of `step` chunks; the last slices may be short or empty.
struct SlicePos {
  int lane, g, col, wib, unit, s, c_begin, c_end;
  bool valid;
};
__device__ __forceinline__ SlicePos slice_pos(int units, int chunks, int slices, int step) {
  SlicePos p;
  p.lane = threadIdx.x & 63;
  p.g = p.lane >> 4;
  p.col = p.lane & 15;
  p.wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wpb = slices == 8 ? 8 : 4;  // the launch's waves a block (blockDim would be a load from the packet)
  p.unit = blockIdx.x * (wpb / slices) + p.wib / slices;
  p.s = p.wib % slices;
  p.valid = p.unit < units;
  const int per = ((chunks + slices - 1) / slices + step - 1) / step * step;
  p.c_begin = min(chunks, p.s * per);
  p.c_end = min(chunks, p.c_begin + per);
  return p;
}

// Adds the partial tiles of a unit's slices into its first wave, in slice order: ((slice 0 + slice 1) + slice 2) ...
// Every wave of the block must call it: it holds a block barrier.
template <int MT>
__device__ __forceinline__ void sum_slices(f32x4 (&acc)[MT], const SlicePos &p, int slices, f32x4 *red) {
  if (p.s != 0)
#pragma unroll
    for (int t = 0; t < MT; t++) red[(p.wib * MT + t) * 64 + p.lane] = acc[t];
  __syncthreads();
  if (p.s == 0)
    for (int j = 1; j < slices; j++)
#pragma unroll
      for (int t = 0; t < MT; t++) acc[t] += red[((p.wib + j) * MT + t) * 64 + p.lane];
}

// A-side scaling, for up to 4 rows of A (ROWS = 1, or 4 with absent rows read as zeros) in row-major rows. Per chunk,
// lane l owns one k of the tile (the row of exponent byte l): it scales x at that k by the run's 2^d for each row into
// the wave's LDS slot for the chunk. Then each lane reads its A fragments from the slot, turns its B values into bf16
// integers (bfp8) or q * 2^-9 (bfp4), and multiplies. Lanes of rows past the last read row 0 of the slot: the matrix
// instruction keeps output rows independent, and those rows are never stored.
//
// The loads of a group of G chunks are issued together and unconditionally: a chunk past the last falls outside the
// tile buffer and reads zeros without touching memory, so the compiler can count the loads and let each chunk start
// as soon as its own have landed. Weight bytes are read once, so they are loaded non-temporal (sc1 nt), which keeps
// them from displacing cached lines on their way. ONE: a single matrix (batch of one), without broadcast arithmetic.
// PROG: whether the epilogue runs a program; the plain kernels carry no interpreter, so their code stays small.
constexpr int STREAM = 18;  // cache-policy bits of a buffer load: sc1 | nt

template <int FMT, int DT, int ROWS, int G, bool ONE, bool PROG, bool SL>
__global__ void __launch_bounds__(SL ? 512 : 256) gemv_kernel(const MatmulArgs args, int slices_arg) {
  constexpr int SLOT = ROWS * 64, TB = Tile<FMT>::bytes;  // SLOT: halfwords of one chunk's scaled x
  // LDS, sized at launch: each wave's slots, then (with slices) each wave's partial tile
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  const int slices = SL ? slices_arg : 1;
  const Head h = early_head(args);
  const SlicePos p = slice_pos(h.batch * h.nruns, h.chunks, slices, G);
  f32x4 *red = (f32x4 *)(dyn + (slices == 8 ? 8 : 4) * G * SLOT * 2);
  if (slices == 1 && !p.valid) return;
  const int lane = p.lane, g = p.g, col = p.col;
  const int b = ONE ? 0 : p.unit / h.nruns, run = ONE ? p.unit : p.unit % h.nruns;
  const int chunks = p.valid ? p.c_end - p.c_begin : 0;  // this wave's slice
  const int rows = min(ROWS, h.m);
  uint16_t *slots = (uint16_t *)dyn + p.wib * G * SLOT;
  const uint8_t *tiles = h.b + (!ONE && h.b_matrix_bytes ? b * h.b_matrix_bytes : 0) +
                         ((int64_t)run * h.chunks + p.c_begin) * TB;
  const __amdgpu_buffer_rsrc_t tr = buffer(tiles, (uint32_t)chunks * TB);
  const uint16_t *abase = (const uint16_t *)h.a.ptr + (ONE ? 0 : operand_matrix(h.a, b) * h.a.sb) + p.c_begin * 64;
  const uint32_t xbytes = (uint32_t)max(0, h.k - p.c_begin * 64) * 2;
  __amdgpu_buffer_rsrc_t xr[ROWS];
#pragma unroll
  for (int m = 0; m < ROWS; m++) xr[m] = buffer(abase + (int64_t)min(m, rows - 1) * h.a.sr, m < rows ? xbytes : 0u);
  const int kl = exp_row(lane);
  const int frag = min(col, rows - 1) * 64 + 8 * g;
  f32x4 acc[1] = {{0.0f, 0.0f, 0.0f, 0.0f}};
  for (int c0 = 0; c0 < chunks; c0 += G) {
    uint32_t bq[G][4], ex[G], x[G][ROWS];  // B's value bytes (bfp8: 16, bfp4: 8), exponent byte, x at the lane's k
    uint4 bhi[G];                          // bf16 B: the second 16 bytes of the lane's 32
#pragma unroll
    for (int i = 0; i < G; i++) {
      const uint32_t at = (uint32_t)(c0 + i) * TB;
      if (FMT == BT_BFP8 || FMT == BT_BF16) {  // block-float values start after the 64 exponent bytes
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + (FMT == BT_BFP8 ? 64 + 16 * lane : 32 * lane),
                                                             0, STREAM);
        bq[i][0] = q[0]; bq[i][1] = q[1]; bq[i][2] = q[2]; bq[i][3] = q[3];
      } else {
        const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr, at + 64 + 8 * lane, 0, STREAM);
        bq[i][0] = q[0]; bq[i][1] = q[1];
      }
      if (FMT == BT_BF16) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 32 * lane + 16, 0, STREAM);
        bhi[i] = make_uint4(q[0], q[1], q[2], q[3]);
      } else {
        ex[i] = __builtin_amdgcn_raw_buffer_load_b8(tr, at + lane, 0, STREAM);
      }
#pragma unroll
      for (int m = 0; m < ROWS; m++)
        x[i][m] = __builtin_amdgcn_raw_buffer_load_b16(xr[m], 2 * ((c0 + i) * 64 + kl), 0, 0);
    }
    // chunk by chunk, in load order, so each starts as soon as its own loads have landed: the scaled x into the
    // chunk's slot, then the fragments out of it
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (c0 + i >= chunks) continue;
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
      for (int hh = 0; hh < 2; hh++) av[hh] = *(const bf16x8 *)(slots + i * SLOT + frag + 32 * hh);
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
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bv[0], acc[0], 0, 0, 0);
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[1], bv[1], acc[0], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (SL && slices > 1) sum_slices<1>(acc, p, slices, red);
  if (p.s != 0 || !p.valid) return;
  if constexpr (ONE && !PROG) {
    // the lean kernels' output is one bf16 or fp32 matrix with contiguous rows whose byte offsets fit 32 bits (the
    // host checks): one buffer store a row, without store_tile's 64-bit address arithmetic and dtype dispatch, whose
    // dependent instructions sit on the path between a wave's last product and the end of the launch
    const bool bf = h.out.dtype == BT_BF16;
    const int n = run * 16 + col;
    const __amdgpu_buffer_rsrc_t orr =
        buffer((const void *)(uintptr_t)h.out.ptr, (uint32_t)(((int64_t)(h.m - 1) * h.out.sr + h.n) * (bf ? 2 : 4)));
#pragma unroll
    for (int i = 0; i < (ROWS == 1 ? 1 : 4); i++) {
      const int mm = 4 * g + i;
      if (mm >= rows || n >= h.n) continue;
      const uint32_t at = (uint32_t)(mm * (int)h.out.sr + n);
      if (bf) __builtin_amdgcn_raw_buffer_store_b16((uint16_t)bf16_packed(acc[0][i]), orr, at * 2, 0, 0);
      else __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(DT == BT_BF16 ? round_packed(acc[0][i]) : acc[0][i]),
                                                 orr, at * 4, 0, 0);
    }
  } else {
    store_tile<DT, false, ONE, PROG ? 1 : 0>(args, h, acc[0], b, 0, run, g, col);
  }
}

// The plain decode GEMV of 1 to 4 rows of one matrix against block-float B with at most 12 chunks of K (the lm head's
// 576 rows: 9), A-side scaled as gemv_kernel and summing in its order, with fewer and wider loads: the block's waves
// stage the rows of A once in LDS (16-byte words), and a run's exponent bytes come 4 chunks to a dword load (lanes
// 16c .. 16c + 15 the 64 bytes of chunk 4 t + c, the loads past the last chunk reading zeros through the buffer's
// range). The lane whose dword holds exponent bytes 4q .. 4q + 3 (K-rows exp_row(4q) + 0 .. 3, consecutive) scales
// those 4 rows of A for every row of the matrix and writes them to the chunk's slot; then each chunk's fragments, B's
// decode and 2 matrix instructions as in gemv_kernel. Per wave 9 loads of B's values and 3 of its exponents at
// K = 576, against gemv_kernel's 9 + 9 + 9 x ROWS. The order of the loads is the order the data is needed: A's rows
// (into registers), the exponent dwords, B's values; then A goes to LDS and is scaled for all rounds while the values
// are still in flight, so after the last value arrives only its decode and products remain (scheduling barriers keep
// the compiler from sinking the exponent loads among the value loads, or the reads of A behind the writes of slots).
// For the lm head in bfp4: 4.62 us a launch at 1 row and 5.44 at 4, against 4.81 and 6.00 with A staged before B's
// loads were issued and each round scaled after its values. G: chunks the kernel holds (4, 8, 9 or 12), at least the
// product's. Each buffer resource is uniform across the wave (one made per lane would have the compiler loop over the
// lanes' resources).
struct XArgs {  // what the kernel reads of a MatmulArgs: 56 bytes instead of the kilobyte that carries a program
  const uint8_t *b;
  uint64_t a, out;
  int64_t a_sr, out_sr;
  int32_t m, k, n, chunks, nruns, out_bf16;
};
template <int FMT, int DT, int ROWS, int G>
__global__ void __launch_bounds__(256) gemv_x_kernel(const XArgs h) {
  constexpr int TB = Tile<FMT>::bytes, R = (G + 3) / 4, GC = 4 * R;  // rounds of 4 chunks, and their chunks
  __shared__ __attribute__((aligned(16))) uint16_t slots_all[4 * GC * ROWS * 64];
  __shared__ __attribute__((aligned(16))) uint16_t xs[ROWS * GC * 64];
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rows = min(ROWS, h.m);
  uint16_t *slots = slots_all + wib * GC * ROWS * 64;
  static_assert(GC * 8 <= 256, "a thread stages at most one 16-byte piece of each row of A");
  uint4 xv[ROWS];
#pragma unroll
  for (int m = 0; m < ROWS; m++) {  // A's rows, zeros past K and past the last row
    const __amdgpu_buffer_rsrc_t xr = buffer((const uint16_t *)(uintptr_t)h.a + (int64_t)min(m, rows - 1) * h.a_sr,
                                             m < rows ? (uint32_t)h.k * 2 : 0u);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(xr, 16 * threadIdx.x, 0, 0);
    xv[m] = make_uint4(v[0], v[1], v[2], v[3]);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t bq[G][4], ew[R];
  const int run = blockIdx.x * 4 + wib;
  const bool in = run < h.nruns;
  const __amdgpu_buffer_rsrc_t tr = buffer(h.b + (int64_t)(in ? run : 0) * h.chunks * TB, in ? (uint32_t)h.chunks * TB : 0u);
#pragma unroll
  for (int rd = 0; rd < R; rd++)  // exponents first: A is scaled while the values are in flight
    ew[rd] = __builtin_amdgcn_raw_buffer_load_b32(tr, (4 * rd + g) * TB + 4 * col, 0, STREAM);
  __builtin_amdgcn_sched_barrier(0);  // (the scheduler would otherwise sink them among the value loads)
#pragma unroll
  for (int i = 0; i < G; i++) {
    if (FMT == BT_BFP8) {
      const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, i * TB + 64 + 16 * lane, 0, STREAM);
      bq[i][0] = q[0], bq[i][1] = q[1], bq[i][2] = q[2], bq[i][3] = q[3];
    } else {
      const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr, i * TB + 64 + 8 * lane, 0, STREAM);
      bq[i][0] = q[0], bq[i][1] = q[1];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if (threadIdx.x < GC * 8)
#pragma unroll
    for (int m = 0; m < ROWS; m++) *(uint4 *)(xs + m * GC * 64 + 8 * threadIdx.x) = xv[m];
  __syncthreads();
  const int r0 = exp_row(4 * col);  // the 4 consecutive K-rows of the lane's exponent dword
  const int frag = (ROWS == 1 ? 0 : min(col, rows - 1) * 64) + 8 * g;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  uint2 xw[R][ROWS];  // every piece of A the lane scales, read before the first is used
#pragma unroll
  for (int rd = 0; rd < R; rd++)
#pragma unroll
    for (int m = 0; m < ROWS; m++) xw[rd][m] = *(const uint2 *)(xs + m * GC * 64 + (4 * rd + g) * 64 + r0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int rd = 0; rd < R; rd++) {
    const int c = 4 * rd + g;  // the lane's chunk in the round
    const uint32_t e = ew[rd];
#pragma unroll
    for (int m = 0; m < ROWS; m++) {
      if (ROWS > 1 && m >= rows) break;
      uint32_t sv[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t xb = (j < 2 ? xw[rd][m].x : xw[rd][m].y) >> (16 * (j & 1)) & 0xFFFFu;
        sv[j] = __float_as_uint(ldexpf(__uint_as_float(xb << 16), (int)(int8_t)(e >> (8 * j))));
      }
      *(uint2 *)(slots + (c * ROWS + m) * 64 + r0) = make_uint2(__builtin_amdgcn_perm(sv[1], sv[0], 0x07060302u),
                                                                 __builtin_amdgcn_perm(sv[3], sv[2], 0x07060302u));
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // all of A scaled before the first product waits for its values
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < G; i++) {
    bf16x8 av[2], bv[2];
    av[0] = *(const bf16x8 *)(slots + i * ROWS * 64 + frag);
    av[1] = *(const bf16x8 *)(slots + i * ROWS * 64 + frag + 32);
    if (FMT == BT_BFP8) {
      bv[0] = q8_to_bf16<false>(make_uint2(bq[i][0], bq[i][1]), make_uint2(0, 0));
      bv[1] = q8_to_bf16<false>(make_uint2(bq[i][2], bq[i][3]), make_uint2(0, 0));
    } else {
      bv[0] = q4_to_bf16(bq[i][0]);
      bv[1] = q4_to_bf16(bq[i][1]);
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[0], bv[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[1], bv[1], acc, 0, 0, 0);
  }
  // lanes of rows 4g + i < rows store them, one buffer store a value
  const int n = run * 16 + col;
  if (!in || n >= h.n) return;
  const __amdgpu_buffer_rsrc_t orr =
      buffer((const void *)(uintptr_t)h.out, (uint32_t)(((int64_t)(rows - 1) * h.out_sr + h.n) * (h.out_bf16 ? 2 : 4)));
#pragma unroll
  for (int i = 0; i < (ROWS == 1 ? 1 : 4); i++) {
    const int mm = 4 * g + i;
    if (mm >= rows) continue;
    const uint32_t at = (uint32_t)(mm * (int)h.out_sr + n);
    if (h.out_bf16) __builtin_amdgcn_raw_buffer_store_b16((uint16_t)bf16_packed(acc[i]), orr, at * 2, 0, 0);
    else __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(DT == BT_BF16 ? round_packed(acc[i]) : acc[i]), orr,
                                               at * 4, 0, 0);
  }
}

// B-side scaling with row-major, 16-byte aligned A: each lane turns its 16 B values into bf16 q * 2^d with
// v_ldexp_f32 and reads its A fragments straight from memory. A wave takes MT 16-row tiles of A against one run, so
// each B value is loaded and converted once for MT tiles; the waves that share a run (more tiles than MT) are
// neighbours in the grid, so they read it at the same time. Loads go out as in gemv_kernel: a group of G chunks
// together and unconditionally, past the last chunk (and for rows past the last) reading zeros through the buffers'
// ranges; the weights non-temporal when a run has a single reader.
// Two 16-row tiles of A against two neighbouring runs a wave (17 to 64 rows): each A fragment loaded feeds both
// runs, halving the loads of A per run, which is what limits the one-run kernel here (its texture units stay busy
// with A's 16-byte reads while HBM idles). A run's 64 exponent bytes come in one 4-byte load a lane and are handed
// to the lanes that use them with ds_bpermute. Otherwise as skinny_vec_kernel: groups of G chunks issued together
// and unconditionally, B scaled by its exponents into bf16, K split into slices summed in order in LDS.
// Up to 256 rows of A (one matrix) with a short K (at most G chunks, G <= 12), 16 MT of them a block (blockIdx.y):
// the block stages its rows of A (at most 48 KB) in LDS once while its waves' weights are in flight, and each of its 4
// waves multiplies NRW runs of B from there. A is read from memory once a block instead of once a run, which is what limits the one-run kernels at 16
// rows (their A and exponent loads keep the texture units busy while HBM idles). Exponents as in skinny2_kernel,
// loaded ahead of the values and made ready (bfp4's gaps placed, bfp8's handed out) while the values are in flight:
// 6.25 us for the lm head at 16 rows in bfp4 and 8.83 in bfp8, against 6.72 and 9.87 with each round's exponents
// waited for behind the values. The weights are read with the streaming cache policy (read once): 6.18 and 8.61.
// A's rows in LDS are G chunks long, so mapping a thread's pieces of A to rows divides by a constant (about 75
// fewer VALU instructions a wave than a division by the product's K): 5.92 and 8.35.
template <int FMT, int DT, int MT, int NRW, int G, bool PROG>
__global__ void __launch_bounds__(256) skinny_lds_kernel(const MatmulArgs args) {
  constexpr int TB = Tile<FMT>::bytes, R = (G + 3) / 4;  // R: rounds of 4 chunks (bfp4)
  extern __shared__ __attribute__((aligned(16))) uint16_t la[];  // A: 16 MT rows, kp halfwords apart
  // bfp4: each chunk's exponents as gaps placed in the bf16 exponent field (place_gaps), 128 bytes a chunk a run
  __shared__ __attribute__((aligned(16))) uint8_t gaps_all[FMT == BT_BFP4 ? 4 * NRW * 4 * R * 128 : 16];
  const Head h = early_head(args);
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // A's rows in LDS are G chunks long whatever the product's K (padded: a fragment read's 16 rows hit distinct
  // banks), so that a piece's row and place are a division by a constant
  const int chunks = h.chunks;
  constexpr int kp = G * 64 + 8;
  const int run0 = ((int)blockIdx.x * 4 + wib) * NRW;
  const int row0 = 16 * MT * (int)blockIdx.y;  // the block's rows of A (and of the output): row0 .. row0 + 16 MT - 1
  // 1. A's pieces for this thread (16 bytes each; rows past the last and columns past K are zeros), loaded before
  // the weights so that staging them waits for these alone
  // (buffer loads: the wait for them then counts them alone, where a flat load's wait would be for every load issued)
  const int kw = h.k / 8;
  constexpr int pieces = G * 8, total = 16 * MT * pieces;
  constexpr int AP = (total + 255) / 256;
  const __amdgpu_buffer_rsrc_t ar = buffer((const void *)(uintptr_t)h.a.ptr,
                                           (uint32_t)(((int64_t)(h.m - 1) * h.a.sr + h.k) * 2));
  uint4 av[AP];
#pragma unroll
  for (int j = 0; j < AP; j++) {
    const int q = (int)threadIdx.x + 256 * j, row = q / pieces, c8 = q % pieces;
    const uint32_t off =
        q < total && row0 + row < h.m && c8 < kw ? (uint32_t)((row0 + row) * (int)h.a.sr + c8 * 8) * 2 : 0x80000000u;
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(ar, off, 0, 0);
    av[j] = make_uint4(v[0], v[1], v[2], v[3]);
  }
  // 2. the wave's exponents, then its weights: in flight while A is staged, the exponents first so that they are
  // ready to use (placed as gaps, or handed to the lanes that use them) while the values are still on their way
  uint4 bq[NRW][G];
  uint32_t ew[NRW][FMT == BT_BFP4 ? R : G];  // bfp8: dword col of each chunk's exponents; bfp4: of chunk 4 t + g
#pragma unroll
  for (int r = 0; r < NRW; r++) {
    const bool in = run0 + r < h.nruns;
    const __amdgpu_buffer_rsrc_t tr = buffer(h.b + (int64_t)(in ? run0 + r : 0) * chunks * TB, in ? (uint32_t)chunks * TB : 0u);
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (FMT == BT_BFP8) ew[r][i] = __builtin_amdgcn_raw_buffer_load_b32(tr, i * TB + 4 * col, 0, STREAM);
      else if (i % 4 == 0) ew[r][i / 4] = __builtin_amdgcn_raw_buffer_load_b32(tr, (i + g) * TB + 4 * col, 0, STREAM);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // (the scheduler would otherwise sink them among the value loads)
#pragma unroll
  for (int r = 0; r < NRW; r++) {
    const bool in = run0 + r < h.nruns;
    const __amdgpu_buffer_rsrc_t tr = buffer(h.b + (int64_t)(in ? run0 + r : 0) * chunks * TB, in ? (uint32_t)chunks * TB : 0u);
#pragma unroll
    for (int i = 0; i < G; i++) {
      const uint32_t at = (uint32_t)i * TB;
      if (FMT == BT_BFP8) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 64 + 16 * lane, 0, STREAM);
        bq[r][i] = make_uint4(q[0], q[1], q[2], q[3]);
      } else {
        const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr, at + 64 + 8 * lane, 0, STREAM);
        bq[r][i] = make_uint4(q[0], q[1], 0, 0);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // 3. A into LDS
#pragma unroll
  for (int j = 0; j < AP; j++) {
    const int q = (int)threadIdx.x + 256 * j, row = q / pieces, c8 = q % pieces;
    if (q < total) *(uint4 *)(la + row * kp + c8 * 8) = av[j];
  }
  // 4. the exponents made ready for every chunk of every run before the first value is waited for: bfp4's placed
  // in LDS as gaps (lane (g, col) places dword col of chunk 4 t + g, once for the wave), bfp8's handed to the lanes
  // whose values they scale
  uint32_t ex[FMT == BT_BFP8 ? NRW : 1][FMT == BT_BFP8 ? G : 1][4];
#pragma unroll
  for (int r = 0; r < NRW; r++) {
    if (FMT == BT_BFP8) {
#pragma unroll
      for (int i = 0; i < G; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) ex[FMT == BT_BFP8 ? r : 0][FMT == BT_BFP8 ? i : 0][k] =
            (uint32_t)__shfl((int)ew[r][i], 4 * g + k, 64);
    } else {
      uint8_t *gp = gaps_all + (wib * NRW + r) * 4 * R * 128;
#pragma unroll
      for (int t = 0; t < R; t++) *(uint2 *)(gp + (4 * t + g) * 128 + 8 * col) = place_gaps(ew[r][FMT == BT_BFP4 ? t : 0]);
    }
  }
  __syncthreads();  // A and the gaps in LDS
  // 5. each run: the chunks' products from A in LDS and the run's B, scaled by its exponents into bf16
#pragma unroll
  for (int r = 0; r < NRW; r++) {
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint8_t *gp = gaps_all + (wib * NRW + r) * 4 * R * 128;
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (i >= chunks) continue;
      bf16x8 bv[2];
      if (FMT == BT_BFP8) {
        const uint32_t *e4 = ex[FMT == BT_BFP8 ? r : 0][FMT == BT_BFP8 ? i : 0];
        bv[0] = q8_to_bf16<true>(make_uint2(bq[r][i].x, bq[r][i].y), make_uint2(e4[0], e4[1]));
        bv[1] = q8_to_bf16<true>(make_uint2(bq[r][i].z, bq[r][i].w), make_uint2(e4[2], e4[3]));
      } else {
        bv[0] = q4_to_bf16_placed(bq[r][i].x, *(const uint4 *)(gp + i * 128 + 32 * g));
        bv[1] = q4_to_bf16_placed(bq[r][i].y, *(const uint4 *)(gp + i * 128 + 32 * g + 16));
      }
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const uint16_t *ar = la + (16 * t + col) * kp + 64 * i + 8 * g;
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)ar, bv[0], acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)(ar + 32), bv[1], acc[t], 0, 0, 0);
      }
    }
    if (run0 + r >= h.nruns) continue;
    if constexpr (PROG) {
#pragma unroll
      for (int t = 0; t < MT; t++)
        store_tile<DT, false, true, 1>(args, h, acc[t], 0, (int)blockIdx.y * MT + t, run0 + r, g, col);
    } else {
      // without a program the output is plain (bf16 or fp32, contiguous rows, byte offsets within 32 bits: the host
      // checks): a buffer store a value, as the lean GEMV stores
      const bool bf = h.out.dtype == BT_BF16;
      const int n = (run0 + r) * 16 + col;
      const __amdgpu_buffer_rsrc_t orr =
          buffer((const void *)(uintptr_t)h.out.ptr, (uint32_t)(((int64_t)(h.m - 1) * h.out.sr + h.n) * (bf ? 2 : 4)));
#pragma unroll
      for (int t = 0; t < MT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int mm = row0 + 16 * t + 4 * g + i;
          if (mm >= h.m || n >= h.n) continue;
          const uint32_t at = (uint32_t)(mm * (int)h.out.sr + n);
          if (bf) __builtin_amdgcn_raw_buffer_store_b16((uint16_t)bf16_packed(acc[t][i]), orr, at * 2, 0, 0);
          else __builtin_amdgcn_raw_buffer_store_b32(
              __float_as_uint(DT == BT_BF16 ? round_packed(acc[t][i]) : acc[t][i]), orr, at * 4, 0, 0);
        }
    }
  }
}

// RES: fp32 out plus an fp32 residual (the epilogue program `x + r`), added straight from the accumulators.
// SWI: B holds gate columns then up columns (n = 2f); a wave's two runs are gate run u and up run u + n / 32, and it
// writes silu(g) * u for its 16 columns of the bf16 out (f wide), g and u rounded to bf16 first, as the tiled GEMM's
// SiLU-mul epilogue does.
template <int FMT, int DT, int G, bool PROG, bool SL, bool RES = false, bool SWI = false>
__global__ void __launch_bounds__(SL ? 512 : 256) skinny2_kernel(const MatmulArgs args, int slices_arg,
                                                                 const bt_operand res) {
  constexpr int TB = Tile<FMT>::bytes, MT = 2, NR = 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];  // with slices: each wave's partial tiles
  f32x4 *red = (f32x4 *)dyn;
  const int slices = SL ? slices_arg : 1;
  const Head h = early_head(args);
  const int groups = (h.mtiles + MT - 1) / MT, pairs = (h.nruns + NR - 1) / NR, per = pairs * groups;
  const SlicePos p = slice_pos(h.batch * per, h.chunks, slices, G);
  if (slices == 1 && !p.valid) return;
  const int lane = p.lane, g = p.g, col = p.col;
  const int b = p.unit / per, rem = p.unit % per;
  const int pu = groups == 1 ? rem : rem / groups, mg = groups == 1 ? 0 : rem % groups;
  const int run0 = pu * NR, half = h.nruns / 2;
  const int chunks = p.valid ? p.c_end - p.c_begin : 0;  // this wave's slice
  const int row0 = mg * MT * 16, rows = min(MT * 16, h.m - row0);
  __amdgpu_buffer_rsrc_t tr[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) {
    const int run = SWI ? pu + r * half : run0 + r;
    const bool in = run < h.nruns;
    const uint8_t *tiles = h.b + (h.b_matrix_bytes ? b * h.b_matrix_bytes : 0) +
                           ((int64_t)(in ? run : 0) * h.chunks + p.c_begin) * TB;
    tr[r] = buffer(tiles, in ? (uint32_t)chunks * TB : 0u);
  }
  const uint16_t *abase = (const uint16_t *)h.a.ptr + operand_matrix(h.a, b) * h.a.sb + (int64_t)row0 * h.a.sr;
  const uint32_t abytes = (uint32_t)(((int64_t)(rows - 1) * h.a.sr + h.k) * 2);
  const __amdgpu_buffer_rsrc_t ar = buffer(abase, abytes);
  uint32_t arow[MT];
#pragma unroll
  for (int t = 0; t < MT; t++)
    arow[t] = t * 16 + col < rows ? (uint32_t)((t * 16 + col) * h.a.sr * 2 + p.c_begin * 128) : abytes;
  f32x4 acc[NR * MT];
#pragma unroll
  for (int i = 0; i < NR * MT; i++) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < chunks; c0 += G) {
    uint4 bq[G][NR], bh[G][NR], a0[G][MT], a1[G][MT];
    uint32_t ew[G][NR];
#pragma unroll
    for (int i = 0; i < G; i++) {
      const uint32_t at = (uint32_t)(c0 + i) * TB, ak = (uint32_t)(c0 + i) * 128 + 16 * g;
#pragma unroll
      for (int r = 0; r < NR; r++) {
        if (FMT == BT_BF16) {
          const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr[r], at + 32 * lane, 0, 0);
          const auto u = __builtin_amdgcn_raw_buffer_load_b128(tr[r], at + 32 * lane + 16, 0, 0);
          bq[i][r] = make_uint4(q[0], q[1], q[2], q[3]);
          bh[i][r] = make_uint4(u[0], u[1], u[2], u[3]);
        } else {
          if (FMT == BT_BFP8) {
            const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr[r], at + 64 + 16 * lane, 0, 0);
            bq[i][r] = make_uint4(q[0], q[1], q[2], q[3]);
          } else {
            const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr[r], at + 64 + 8 * lane, 0, 0);
            bq[i][r] = make_uint4(q[0], q[1], 0, 0);
          }
          ew[i][r] = __builtin_amdgcn_raw_buffer_load_b32(tr[r], at + 4 * col, 0, 0);  // exponent word col of 16
        }
      }
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const auto x0 = __builtin_amdgcn_raw_buffer_load_b128(ar, arow[t] + ak, 0, 0);
        const auto x1 = __builtin_amdgcn_raw_buffer_load_b128(ar, arow[t] + ak + 64, 0, 0);
        a0[i][t] = make_uint4(x0[0], x0[1], x0[2], x0[3]);
        a1[i][t] = make_uint4(x1[0], x1[1], x1[2], x1[3]);
      }
    }
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (c0 + i >= chunks) continue;
#pragma unroll
      for (int r = 0; r < NR; r++) {
        bf16x8 bv[2];
        if (FMT == BT_BF16) {
          bv[0] = *(const bf16x8 *)&bq[i][r];
          bv[1] = *(const bf16x8 *)&bh[i][r];
        } else {
          // the lane's 16 exponent bytes (rows 8g + j, then 32 + 8g + j): words 4g .. 4g + 3, held by lanes 4g ..
          uint32_t ex[4];
#pragma unroll
          for (int k = 0; k < 4; k++) ex[k] = (uint32_t)__shfl((int)ew[i][r], 4 * g + k, 64);
          if (FMT == BT_BFP8) {
            bv[0] = q8_to_bf16<true>(make_uint2(bq[i][r].x, bq[i][r].y), make_uint2(ex[0], ex[1]));
            bv[1] = q8_to_bf16<true>(make_uint2(bq[i][r].z, bq[i][r].w), make_uint2(ex[2], ex[3]));
          } else {
            bv[0] = q4_to_bf16_scaled(bq[i][r].x, make_uint2(ex[0], ex[1]));
            bv[1] = q4_to_bf16_scaled(bq[i][r].y, make_uint2(ex[2], ex[3]));
          }
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
          acc[r * MT + t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)&a0[i][t], bv[0], acc[r * MT + t], 0, 0, 0);
          acc[r * MT + t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)&a1[i][t], bv[1], acc[r * MT + t], 0, 0, 0);
        }
      }
    }
  }
  if (SL && slices > 1) sum_slices<NR * MT>(acc, p, slices, red);
  if (p.s != 0 || !p.valid) return;
  if constexpr (SWI) {
    const bt_operand &out = h.out;
    const int n = pu * 16 + col;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = (mg * MT + t) * 16 + 4 * g + i;
        if (m >= h.m) continue;
        const float gv = bf16_value(bf16_packed(acc[t][i])), uv = bf16_value(bf16_packed(acc[MT + t][i]));
        ((uint16_t *)out.ptr)[(int64_t)m * out.sr + n] = (uint16_t)bf16_packed(gv / (1.0f + expf(-gv)) * uv);
      }
    return;
  }
  if constexpr (RES) {
    const bt_operand &out = h.out;
    const int64_t ob = operand_matrix(out, b) * out.sb, rb = res.ptr ? operand_matrix(res, b) * res.sb : 0;
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const int n = (run0 + r) * 16 + col;
      if (n >= h.n) continue;
#pragma unroll
      for (int t = 0; t < MT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int m = (mg * MT + t) * 16 + 4 * g + i;
          if (m >= h.m) continue;
          float v = acc[r * MT + t][i];
          if (res.ptr) v += ((const float *)res.ptr)[rb + (int64_t)m * res.sr + (int64_t)n * res.sc];
          ((float *)out.ptr)[ob + (int64_t)m * out.sr + (int64_t)n * out.sc] = v;
        }
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < NR; r++) {
    if (run0 + r >= h.nruns) continue;
#pragma unroll
    for (int t = 0; t < MT; t++)
      store_tile<DT, false, false, PROG ? 1 : 0>(args, h, acc[r * MT + t], b, mg * MT + t, run0 + r, g, col);
  }
}

template <int FMT, int DT, int G, bool ONE, bool PROG, int MT, bool SL>
__global__ void __launch_bounds__(SL ? 512 : 256) skinny_vec_kernel(const MatmulArgs args, int slices_arg) {
  constexpr int TB = Tile<FMT>::bytes;
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];  // with slices: each wave's partial tiles
  f32x4 *red = (f32x4 *)dyn;
  const int slices = SL ? slices_arg : 1;
  const Head h = early_head(args);
  const int groups = (h.mtiles + MT - 1) / MT, per = h.nruns * groups;
  const SlicePos p = slice_pos(h.batch * per, h.chunks, slices, G);
  if (slices == 1 && !p.valid) return;
  const int lane = p.lane, g = p.g, col = p.col;
  const int b = ONE ? 0 : p.unit / per, rem = ONE ? p.unit : p.unit % per;
  const int run = groups == 1 ? rem : rem / groups, mg = groups == 1 ? 0 : rem % groups;
  const int chunks = p.valid ? p.c_end - p.c_begin : 0;  // this wave's slice
  const int row0 = mg * MT * 16, rows = min(MT * 16, h.m - row0);  // this wave's rows of A
  const uint8_t *tiles = h.b + (!ONE && h.b_matrix_bytes ? b * h.b_matrix_bytes : 0) +
                         ((int64_t)run * h.chunks + p.c_begin) * TB;
  const __amdgpu_buffer_rsrc_t tr = buffer(tiles, (uint32_t)chunks * TB);
  // A's rows through one (uniform) buffer: each lane's row at its byte offset, a row past the last at the end of the
  // range, so it reads zeros
  const uint16_t *abase = (const uint16_t *)h.a.ptr + (ONE ? 0 : operand_matrix(h.a, b) * h.a.sb) +
                          (int64_t)row0 * h.a.sr;
  const uint32_t abytes = (uint32_t)(((int64_t)(rows - 1) * h.a.sr + h.k) * 2);
  const __amdgpu_buffer_rsrc_t ar = buffer(abase, abytes);
  uint32_t arow[MT];
#pragma unroll
  for (int t = 0; t < MT; t++)
    arow[t] = t * 16 + col < rows ? (uint32_t)((t * 16 + col) * h.a.sr * 2 + p.c_begin * 128) : abytes;
  const bool alone = groups == 1;
  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < chunks; c0 += G) {
    uint4 b0[G], b1[G], ex[G], a0[G][MT], a1[G][MT];
#pragma unroll
    for (int i = 0; i < G; i++) {
      const uint32_t at = (uint32_t)(c0 + i) * TB, ak = (uint32_t)(c0 + i) * 128 + 16 * g;
      // the cache policy is an immediate: two copies of the loads, one chosen per wave
      if (alone) {
        if (FMT == BT_BF16) {
          const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 32 * lane, 0, STREAM);
          const auto u = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 32 * lane + 16, 0, STREAM);
          b0[i] = make_uint4(q[0], q[1], q[2], q[3]);
          b1[i] = make_uint4(u[0], u[1], u[2], u[3]);
        } else if (FMT == BT_BFP8) {
          const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 64 + 16 * lane, 0, STREAM);
          b0[i] = make_uint4(q[0], q[1], q[2], q[3]);
        } else {
          const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr, at + 64 + 8 * lane, 0, STREAM);
          b0[i] = make_uint4(q[0], q[1], 0, 0);
        }
        if (FMT != BT_BF16) {
          const auto e = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 16 * g, 0, STREAM);
          ex[i] = make_uint4(e[0], e[1], e[2], e[3]);
        }
      } else {
        if (FMT == BT_BF16) {
          const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 32 * lane, 0, 0);
          const auto u = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 32 * lane + 16, 0, 0);
          b0[i] = make_uint4(q[0], q[1], q[2], q[3]);
          b1[i] = make_uint4(u[0], u[1], u[2], u[3]);
        } else if (FMT == BT_BFP8) {
          const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 64 + 16 * lane, 0, 0);
          b0[i] = make_uint4(q[0], q[1], q[2], q[3]);
        } else {
          const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr, at + 64 + 8 * lane, 0, 0);
          b0[i] = make_uint4(q[0], q[1], 0, 0);
        }
        if (FMT != BT_BF16) {
          const auto e = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 16 * g, 0, 0);
          ex[i] = make_uint4(e[0], e[1], e[2], e[3]);
        }
      }
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const auto x0 = __builtin_amdgcn_raw_buffer_load_b128(ar, arow[t] + ak, 0, 0);
        const auto x1 = __builtin_amdgcn_raw_buffer_load_b128(ar, arow[t] + ak + 64, 0, 0);
        a0[i][t] = make_uint4(x0[0], x0[1], x0[2], x0[3]);
        a1[i][t] = make_uint4(x1[0], x1[1], x1[2], x1[3]);
      }
    }
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (c0 + i >= chunks) continue;
      bf16x8 bv[2];
      if (FMT == BT_BF16) {
        bv[0] = *(const bf16x8 *)&b0[i];
        bv[1] = *(const bf16x8 *)&b1[i];
      } else if (FMT == BT_BFP8) {
        bv[0] = q8_to_bf16<true>(make_uint2(b0[i].x, b0[i].y), make_uint2(ex[i].x, ex[i].y));
        bv[1] = q8_to_bf16<true>(make_uint2(b0[i].z, b0[i].w), make_uint2(ex[i].z, ex[i].w));
      } else {
        bv[0] = q4_to_bf16_scaled(b0[i].x, make_uint2(ex[i].x, ex[i].y));
        bv[1] = q4_to_bf16_scaled(b0[i].y, make_uint2(ex[i].z, ex[i].w));
      }
#pragma unroll
      for (int t = 0; t < MT; t++) {
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)&a0[i][t], bv[0], acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)&a1[i][t], bv[1], acc[t], 0, 0, 0);
      }
    }
  }
  if (SL && slices > 1) sum_slices<MT>(acc, p, slices, red);
  if (p.s == 0 && p.valid)
#pragma unroll
    for (int t = 0; t < MT; t++)
      store_tile<DT, false, ONE, PROG ? 1 : 0>(args, h, acc[t], b, mg * MT + t, run, g, col);
}

// B-side scaling, for A of any strides: each lane turns its 16 B values into bf16 q * 2^d with v_ldexp_f32 and
// reads its A fragments straight from memory.
template <int FMT, int DT, bool VEC>
__global__ void __launch_bounds__(256) skinny_kernel(const MatmulArgs args) {
  constexpr int G = GROUP_B;
  const Head h = early_head(args);
  const WavePos p = wave_pos(h);
  if (!p.valid) return;
  const int lane = p.lane, g = p.g, col = p.col, chunks = h.chunks;
  const int rows = min(16, h.m - p.mt * 16);
  const uint8_t *tiles = h.b + (h.b_matrix_bytes ? p.b * h.b_matrix_bytes : 0) +
                         (int64_t)p.run * chunks * Tile<FMT>::bytes;
  const bool row_in = col < rows;
  const uint16_t *arow = (const uint16_t *)h.a.ptr + operand_matrix(h.a, p.b) * h.a.sb +
                         (int64_t)(p.mt * 16 + (row_in ? col : 0)) * h.a.sr;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < chunks; c0 += G) {
    Chunk r[G];
#pragma unroll
    for (int i = 0; i < G; i++) {
      const int c = c0 + i;
      if (c < chunks) {
        const uint8_t *t = tiles + (int64_t)c * Tile<FMT>::bytes;
        load_b<FMT>(r[i], t, lane);
        if (FMT != BT_BF16) r[i].ex = gload((const uint4 *)(t + 16 * g));
        r[i].a0 = load_a<VEC>(arow, row_in, h.a.sc, c * 64 + 8 * g, h.k);
        r[i].a1 = load_a<VEC>(arow, row_in, h.a.sc, c * 64 + 32 + 8 * g, h.k);
      }
    }
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (c0 + i >= chunks) continue;
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
  store_tile<DT>(args, h, acc, p.b, p.mt, p.run, g, col);
}

// The end of both GEMM kernels: the block's BM x BN starting values are in LDS (row stride ES bytes, ESZ bytes each:
// bf16-rounded for a bf16 epilogue, fp32 otherwise). Without a program, and with rows of the output contiguous and
// 16-byte aligned, each lane copies 16 bytes at a time; otherwise each value goes through the program and is stored.
template <int DT, int BM, int BN, int ES, int ESZ, int NT = 256>
__device__ __forceinline__ void gemm_epilogue(const MatmulArgs &args, const uint8_t *lds, int b, int m0, int n0,
                                              int tid) {
  const int rows = min(BM, args.m - m0), cols = min(BN, args.n - n0);
  const int64_t obase = operand_matrix(args.out, b) * args.out.sb;
  const int osz = args.out.dtype == BT_BF16 ? 2 : 4;
  const bool same = (DT == BT_FP32 && args.out.dtype == BT_FP32) || (DT == BT_BF16 && args.out.dtype == BT_BF16);
  const bool direct = args.n_inst == 0 && same && args.out.sc == 1 && cols == BN &&
                      (args.out.ptr + (uint64_t)(obase + (int64_t)m0 * args.out.sr + n0) * osz) % 16 == 0 &&
                      (args.out.sr * osz) % 16 == 0;
  if (direct) {
    constexpr int PER_ROW = BN * ESZ / 16;  // 16-byte pieces of a row
    uint8_t *out = (uint8_t *)args.out.ptr + (obase + (int64_t)m0 * args.out.sr + n0) * osz;
#pragma unroll 1
    for (int e = tid; e < rows * PER_ROW; e += NT) {
      const int r = e / PER_ROW, piece = e % PER_ROW;
      *(uint4 *)(out + (int64_t)r * args.out.sr * osz + piece * 16) = *(const uint4 *)(lds + r * ES + piece * 16);
    }
    return;
  }
  // through the program, a segment of SEG neighbouring columns a thread (fetch_segment), so the program is decoded
  // once for SEG values and contiguous inputs and outputs move 16 bytes at a time
  (void)obase;
  constexpr int GS = BN / SEG;
#pragma unroll 1
  for (int e = tid; e < rows * GS; e += NT) {
    const int r = e / GS, c0 = e % GS * SEG;
    if (c0 >= cols) continue;
    const int n = min(SEG, cols - c0);
    uint32_t io[SEG];
#pragma unroll
    for (int v = 0; v < SEG; v++) {
      const uint8_t *src = lds + r * ES + (c0 + v) * ESZ;
      io[v] = DT == BT_FP32 ? *(const uint32_t *)src : (uint32_t)*(const uint16_t *)src << 16;
    }
    if (args.n_inst) {
      prefile pre[SEG];
      fetch_segment<DT>(args.prog, b, m0 + r, n0 + c0, n, pre);
      eval_program<DT, SEG>(args.prog, pre, io);
    }
    store_segment<DT>(args.out, b, m0 + r, n0 + c0, n, io);
  }
}

// ---- the prefill GEMM ----------------------------------------------------------------------------------------------
// Blocks of BM x BN outputs with 4 waves in 2 x 2, each wave WM x WN tiles of 16 x 16, stepping K by one 64-row chunk.
// Per chunk the block stages A's BM x 64 rows (bf16, row-major, rows padded to 72 halfwords so the fragment reads hit
// distinct banks) and B's BN / 16 tiles in LDS. B is turned into bf16 once, by the block, as it is staged: q * 2^d per
// value, exact, laid out per tile as [k half][lane][8 values], the matrix instruction's operand order, so each wave
// reads its fragments with one 16-byte load per lane. Two stages: the global loads of the next chunk are in flight in
// registers while the current one is multiplied, and one barrier a chunk keeps the stages apart.
// At the end the accumulators go through LDS once more, as the values the epilogue starts from (bf16-rounded for a
// bf16 epilogue, fp32 otherwise), so that the epilogue runs as one loop over the block in row order: its program is
// evaluated by code that appears once, and its stores are whole rows.
template <int WM, int WN, int DT> struct Gemm {
  static constexpr int BM = 32 * WM, BN = 32 * WN, AS = 72;
  static constexpr int A_BYTES = BM * AS * 2, B_BYTES = BN / 16 * 2048, STAGE = A_BYTES + B_BYTES;
  static constexpr int APT = BM * 8 / 256;       // 16-byte pieces of A a thread stages per chunk
  static constexpr int BPT = BN / 16 * 64 / 256;  // tile lanes of B a thread stages per chunk
  static constexpr int ESZ = DT == BT_FP32 ? 4 : 2, ES = BN * ESZ + 16;  // epilogue value size, row stride (bytes)
  static constexpr int LDS = 2 * STAGE > BM * ES ? 2 * STAGE : BM * ES;
};

template <int FMT, int DT, int WM, int WN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_kernel(const MatmulArgs args, int mblocks, int nblocks) {
  using G = Gemm<WM, WN, DT>;
  constexpr int TB = Tile<FMT>::bytes;
  __shared__ __attribute__((aligned(16))) uint8_t lds[G::LDS];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, col = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wib >> 1, wn = wib & 1;
  // Blocks are dealt to the 8 XCDs in turn: renumber them so each XCD's blocks are consecutive, then walk those in
  // groups of 8 block rows, so the blocks sharing an L2 also share rows of A and columns of B.
  const int per = mblocks * nblocks, total = per * args.batch, full = total / 8 * 8;
  int pid = blockIdx.x;
  if (pid < full) pid = (pid % 8) * (full / 8) + pid / 8;
  const int b = pid / per;
  pid %= per;
  constexpr int GROUP = 8;
  const int width = GROUP * nblocks, first = pid / width * GROUP, gsz = min(mblocks - first, GROUP);
  const int bm = first + pid % width % gsz, bn = pid % width / gsz;
  const int m0 = bm * G::BM, n0 = bn * G::BN;

  const uint16_t *abase = (const uint16_t *)args.a.ptr + operand_matrix(args.a, b) * args.a.sb;
  const __amdgpu_buffer_rsrc_t ar = buffer(abase, (uint32_t)(((int64_t)(args.m - 1) * args.a.sr + args.k) * 2));
  const uint8_t *bbase = args.b + (args.b_matrix_bytes ? b * args.b_matrix_bytes : 0);

  uint4 areg[G::APT], bq0[G::BPT], bq1[G::BPT], bex[G::BPT];
  auto fetch = [&](int c) {
    const int k0 = c * 64;
#pragma unroll
    for (int i = 0; i < G::APT; i++) {
      const int piece = tid + 256 * i, row = piece >> 3, kc = (piece & 7) * 8;
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(
          ar, (uint32_t)(((int64_t)(m0 + row) * args.a.sr + k0 + kc) * 2), 0, 0);
      areg[i] = k0 + kc < args.k ? make_uint4(v[0], v[1], v[2], v[3]) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < G::BPT; i++) {
      const int slot = tid + 256 * i, tile = slot >> 6, tl = slot & 63, run = n0 / 16 + tile;
      bq0[i] = bq1[i] = bex[i] = make_uint4(0, 0, 0, 0);
      if (run < args.nruns) {
        const uint8_t *t = bbase + ((int64_t)run * args.chunks + c) * TB;
        if (FMT == BT_BF16) {
          bq0[i] = gload((const uint4 *)(t + 32 * tl));
          bq1[i] = gload((const uint4 *)(t + 32 * tl + 16));
        } else {
          if (FMT == BT_BFP8) bq0[i] = gload((const uint4 *)(t + 64 + 16 * tl));
          else {
            const uint2 q = gload((const uint2 *)(t + 64 + 8 * tl));
            bq0[i] = make_uint4(q.x, q.y, 0, 0);
          }
          bex[i] = gload((const uint4 *)(t + 16 * (tl >> 4)));
        }
      }
    }
  };
  auto stage_in = [&](uint8_t *st) {
#pragma unroll
    for (int i = 0; i < G::APT; i++) {
      const int piece = tid + 256 * i, row = piece >> 3, kc = (piece & 7) * 8;
      *(uint4 *)(st + (row * G::AS + kc) * 2) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < G::BPT; i++) {
      const int slot = tid + 256 * i, tile = slot >> 6, tl = slot & 63;
      bf16x8 h0, h1;
      if (FMT == BT_BF16) {
        h0 = *(const bf16x8 *)&bq0[i];
        h1 = *(const bf16x8 *)&bq1[i];
      } else if (FMT == BT_BFP8) {
        h0 = q8_to_bf16<true>(make_uint2(bq0[i].x, bq0[i].y), make_uint2(bex[i].x, bex[i].y));
        h1 = q8_to_bf16<true>(make_uint2(bq0[i].z, bq0[i].w), make_uint2(bex[i].z, bex[i].w));
      } else {
        h0 = q4_to_bf16_scaled(bq0[i].x, make_uint2(bex[i].x, bex[i].y));
        h1 = q4_to_bf16_scaled(bq0[i].y, make_uint2(bex[i].z, bex[i].w));
      }
      uint8_t *bl = st + G::A_BYTES + tile * 2048 + tl * 16;
      *(bf16x8 *)bl = h0;
      *(bf16x8 *)(bl + 1024) = h1;
    }
  };

  f32x4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  fetch(0);
  stage_in(lds);
  __syncthreads();
  for (int c = 0; c < args.chunks; c++) {
    uint8_t *st = lds + (c & 1) * G::STAGE;
    // the next chunk's loads go out first; its staging comes after this chunk's matrix instructions are issued, so
    // the conversions run while the matrix cores work
    const bool more = c + 1 < args.chunks;
    if (more) fetch(c + 1);
    const uint16_t *al = (const uint16_t *)st + (wm * WM * 16 + col) * G::AS + 8 * g;
    const uint8_t *bl = st + G::A_BYTES + wn * WN * 2048 + lane * 16;
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      bf16x8 af[WM], bv[WN];
#pragma unroll
      for (int i = 0; i < WM; i++) af[i] = *(const bf16x8 *)(al + 16 * i * G::AS + 32 * kk);
#pragma unroll
      for (int j = 0; j < WN; j++) bv[j] = *(const bf16x8 *)(bl + j * 2048 + kk * 1024);
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (more) stage_in(lds + ((c + 1) & 1) * G::STAGE);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        uint8_t *at = lds + (wm * WM * 16 + 16 * i + 4 * g + r) * G::ES + (wn * WN * 16 + 16 * j + col) * G::ESZ;
        if (DT == BT_FP32) *(float *)at = acc[i][j][r];
        else *(uint16_t *)at = (uint16_t)bf16_packed(acc[i][j][r]);
      }
  __syncthreads();
  gemm_epilogue<DT, G::BM, G::BN, G::ES, G::ESZ>(args, lds, b, m0, n0, tid);
}

// ---- the prefill GEMM with loads straight into LDS ------------------------------------------------------------------
// As gemm_kernel, but the global loads of A and of B's raw tiles go straight into LDS (buffer_load ... lds), S chunks
// deep, so the loads of the next S - 1 chunks are in flight while one is multiplied, without holding registers.
// A wave's such load writes 1 KB of LDS in lane order; which 16 bytes of the matrix each lane fetches sets the layout:
//   A: row r of the block (64 halfwords, 128 bytes) holds its 16-byte column c at position c ^ ((r >> 1) & 7), so the
//      16 lanes that read one column of 16 rows for a fragment hit 16 different groups of 4 banks;
//   B bf16: the tile in the operand order, [k half][lane][8 values];
//   B block float: the raw tiles, which the block then turns into bf16 operand order once per chunk.
// Needs K a multiple of 64: a chunk's loads cannot zero the columns of A past K.
template <int FMT, int DT, int WM, int WN, int S> struct Gemm2 {
  static constexpr int BM = 32 * WM, BN = 32 * WN, TB = Tile<FMT>::bytes;
  static constexpr bool CONVERT = FMT != BT_BF16;
  static constexpr int A_LOADS = BM / 8;                        // wave loads of 1 KB
  static constexpr int B_REAL = (BN / 16 * TB + 1023) / 1024;   // B's, and rounded up to whole rounds of 4 waves:
  static constexpr int B_LOADS = (B_REAL + 3) / 4 * 4;          // the extra ones read nothing into a junk KB
  static constexpr int PER_WAVE = (A_LOADS + B_LOADS) / 4;
  static constexpr int A_BYTES = BM * 128, STAGE = A_BYTES + B_REAL * 1024;
  static constexpr int BBF = CONVERT ? BN / 16 * 2048 : 0;
  static constexpr int BPT = BN / 16 * 64 / 256;
  static constexpr int ESZ = DT == BT_FP32 ? 4 : 2, ES = BN * ESZ + 16;
  static constexpr int JUNK = S * STAGE + BBF, MAIN = JUNK + 1024;
  static constexpr int LDS = MAIN > BM * ES ? MAIN : BM * ES;
};

// Up to 32 rows of A (one matrix, K a multiple of 64) against a long K, in two launches. skinny_part_kernel cuts K
// into splits of G chunks: block (group, split) stages its split of A's rows in LDS with direct loads, each of one
// row's 1 KB (whole cache lines, where the fragment-shaped reads of the other skinny kernels take 16 rows' 64 bytes
// at once, 8 KB or more apart), while its 4 waves' weights are in flight; each wave then multiplies NRW runs of B
// from there and writes its fp32 partial tiles. A is read once a block instead of once a wave. parts_reduce_kernel
// sums each output's splits in split order and runs the epilogue (rounding, program, or SiLU x up).
template <int FMT, int MT, int NRW, int G, bool FULL = false>
__global__ void __launch_bounds__(256) skinny_part_kernel(const MatmulArgs args, int groups, float *part) {
  constexpr int TB = Tile<FMT>::bytes, KP = G * 64 + 8;  // padded rows: a fragment read's 16 rows hit distinct banks
  __shared__ __attribute__((aligned(16))) uint16_t la[16 * MT * KP];
  const Head h = early_head(args);
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = (int)blockIdx.x % groups, sp = (int)blockIdx.x / groups;
  const int c0 = sp * G, cnt = min(G, h.chunks - c0);
  const int run0 = (grp * 4 + wib) * NRW;
  // 1. the split of A's rows into LDS: row r's G * 128 bytes in G / 8 loads of 1 KB, the block's waves taking them in
  // turn (rows past the last read zeros: their offset lies past the buffer's range)
  const uint32_t abytes = (uint32_t)(((int64_t)(h.m - 1) * h.a.sr + h.k) * 2);
  const i32x4 ar = buffer_words((const void *)h.a.ptr, abytes);
  constexpr int LOADS = 16 * MT * G / 8, PER = LOADS / 4;
  static_assert(LOADS % 4 == 0, "each wave issues the same number of A loads");
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int q = wib + 4 * j, r = q / (G / 8), piece = q % (G / 8);
    const uint32_t voff =
        r < h.m ? (uint32_t)(((int64_t)r * h.a.sr + (int64_t)c0 * 64 + piece * 512) * 2) + 16u * lane : abytes;
    lds_load16(ar, voff, la + r * KP + piece * 512);
  }
  // 2. the wave's weights: G chunks of each of its runs from chunk c0 (past the split's last: zeros). A bfp4 lane takes
  // its group's 16 exponent bytes (rows 16g .. 16g + 15 of the tile: both halves' 8) with one load; the other formats
  // take one exponent word a lane and share them by shuffles.
  uint32_t bq[NRW][G][FMT == BT_BF16 ? 8 : FMT == BT_BFP8 ? 4 : 2], ew[NRW][G][FMT == BT_BFP4 ? 4 : 1];
#pragma unroll
  for (int r = 0; r < NRW; r++) {
    const bool in = run0 + r < h.nruns;
    const __amdgpu_buffer_rsrc_t tr =
        buffer(h.b + ((int64_t)(in ? run0 + r : 0) * h.chunks + c0) * TB, in ? (uint32_t)cnt * TB : 0u);
#pragma unroll
    for (int i = 0; i < G; i++) {
      const uint32_t at = (uint32_t)i * TB;
      if (FMT == BT_BF16) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 32 * lane, 0, 0);
        const auto u = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 32 * lane + 16, 0, 0);
#pragma unroll
        for (int w = 0; w < 4; w++) bq[r][i][w] = q[w], bq[r][i][4 + w] = u[w];
        continue;
      }
      if (FMT == BT_BFP8) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 64 + 16 * lane, 0, 0);
#pragma unroll
        for (int w = 0; w < 4; w++) bq[r][i][w] = q[w];
      } else {
        const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr, at + 64 + 8 * lane, 0, 0);
        bq[r][i][0] = q[0], bq[r][i][1] = q[1];
        const auto e = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 16 * g, 0, 0);
#pragma unroll
        for (int w = 0; w < 4; w++) ew[r][i][w] = e[w];
        continue;
      }
      ew[r][i][0] = __builtin_amdgcn_raw_buffer_load_b32(tr, at + 4 * col, 0, 0);  // exponent word col of 16
    }
  }
  // A's loads, issued first, have landed (loads complete in order; at most 63 can be counted, and with more B loads
  // than that, 63 outstanding still leaves every A load done)
  wait_vm<(2 * NRW * G < 63 ? 2 * NRW * G : 63)>();
  __syncthreads();
  // 3. each run's products over the split
#pragma unroll
  for (int r = 0; r < NRW; r++) {
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (!FULL && i >= cnt) continue;
      bf16x8 bv[2];
      uint32_t ex[4];
      if (FMT == BT_BFP8)
#pragma unroll
        for (int k = 0; k < 4; k++) ex[k] = (uint32_t)__shfl((int)ew[r][i][0], 4 * g + k, 64);
      if (FMT == BT_BF16) {
        const uint4 lo = make_uint4(bq[r][i][0], bq[r][i][1], bq[r][i][2], bq[r][i][3]);
        const uint4 hi = make_uint4(bq[r][i][4], bq[r][i][5], bq[r][i][6], bq[r][i][7]);
        bv[0] = *(const bf16x8 *)&lo;
        bv[1] = *(const bf16x8 *)&hi;
      } else if (FMT == BT_BFP8) {
        bv[0] = q8_to_bf16<true>(make_uint2(bq[r][i][0], bq[r][i][1]), make_uint2(ex[0], ex[1]));
        bv[1] = q8_to_bf16<true>(make_uint2(bq[r][i][2], bq[r][i][3]), make_uint2(ex[2], ex[3]));
      } else {
        bv[0] = q4_to_bf16_gaps(bq[r][i][0], ew[r][i][0] ^ 0x7F7F7F7Fu, ew[r][i][1] ^ 0x7F7F7F7Fu);
        bv[1] = q4_to_bf16_gaps(bq[r][i][1], ew[r][i][2] ^ 0x7F7F7F7Fu, ew[r][i][3] ^ 0x7F7F7F7Fu);
      }
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const uint16_t *at = la + (16 * t + col) * KP + 64 * i + 8 * g;
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)at, bv[0], acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)(at + 32), bv[1], acc[t], 0, 0, 0);
      }
    }
    const int n = (run0 + r) * 16 + col;
    if (n >= h.n) continue;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = 16 * t + 4 * g + i;
        if (m < h.m) part[((int64_t)sp * 16 * MT + m) * h.n + n] = acc[t][i];
      }
  }
}

// The sum of an output's splits, in split order, through the matmul's epilogue: one output a thread. SWI: the
// product's columns are gate then up (n = 2f); the output is silu(g) * u for f columns, g and u rounded to bf16 first.
// p[0] + p[stride] + ... + p[(splits - 1) * stride], added in that order; the loads of 8 splits at a time are all
// issued before the first is added (a split past the last reloads the last one's value and isn't added)
__device__ __forceinline__ float sum_splits(const float *p, int splits, int64_t stride) {
  float v = 0.0f;
  for (int s0 = 0; s0 < splits; s0 += 8) {
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; i++) t[i] = p[(int64_t)min(s0 + i, splits - 1) * stride];
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (s0 + i < splits) v = s0 + i == 0 ? t[i] : v + t[i];
  }
  return v;
}

template <int DT, bool SWI>
__global__ void __launch_bounds__(256) parts_reduce_kernel(const MatmulArgs args, int splits, int rows, const float *part) {
  const int nout = SWI ? args.n / 2 : args.n;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)args.m * nout) return;
  const int m = (int)(e / nout), n = (int)(e % nout);
  const int64_t stride = (int64_t)rows * args.n;
  const float *p = part + (int64_t)m * args.n + n;
  const bt_operand &out = args.out;
  if constexpr (SWI) {
    const float v = sum_splits(p, splits, stride), u = sum_splits(p + nout, splits, stride);
    const float gv = bf16_value(bf16_packed(v)), uv = bf16_value(bf16_packed(u));
    ((uint16_t *)out.ptr)[(int64_t)m * out.sr + n] = (uint16_t)bf16_packed(gv / (1.0f + expf(-gv)) * uv);
  } else {
    // the epilogue's inputs (a residual) are fetched first, so their loads are in flight with the partials'
    Coords<1> at;
    at.b[0] = 0, at.r[0] = m, at.c[0] = n, at.ok[0] = true;
    prefile pre[1];
    const bool prog = args.n_inst != 0;
    if (prog) fetch_inputs<DT, 1>(args.prog, at, pre);
    const float v = sum_splits(p, splits, stride);
    uint32_t x[1] = {__float_as_uint(DT == BT_BF16 ? round_packed(v) : v)};
    if (prog) eval_program<DT, 1, false>(args.prog, pre, x);
    store_value<DT>(out, (int64_t)m * out.sr + (int64_t)n * out.sc, x[0]);
  }
}

// 5 to 32 rows of one A (K a multiple of 256) against B streamed once. Block (group, split) takes W runs of B, a wave
// each, over its split's stages of 4 chunks (256 rows of K). Every load goes straight into LDS, whole and aligned: a
// stage of a run's tiles is one contiguous stretch (4 x 576 bytes for bfp4), loaded 1 KB a wave instruction, and each
// 512-byte row of A for the stage half an instruction, each 16-byte unit of row r placed at unit u ^ (r % 16) so that
// the fragment reads of 16 rows fall in distinct banks. A ring of D stages keeps the next D - 1 in flight while one is
// multiplied; the loads are issued as assembly, which the compiler doesn't count, and waited for here, once a stage
// (loads complete in order). A wave decodes its B values and exponents out of LDS. Every run sums its chunks in the
// same order as the other kernels (a chunk's lower 32 rows, then its upper 32), in one accumulator over the split.
// EPI 0 writes fp32 partial tiles for parts_reduce_kernel (more than one split); 1 stores through the matmul's
// epilogue (one split); 2 is SiLU x up (one split): the first W / 2 waves take gate runs, the others the up runs at
// the same columns of the other half, and the up tiles reach the gate waves through LDS.
template <int FMT> struct Stream {
  static constexpr int C = 4, TB = Tile<FMT>::bytes, BW = C * TB;  // a wave's B bytes a stage
  static constexpr int BL = (BW + 1023) / 1024, BLAST = (BW - (BL - 1) * 1024) / 16;  // its loads; the last one's lanes
  static constexpr int D = FMT == BT_BFP4 ? 3 : 2;  // ring stages (4 for bfp4 measured no faster)
  // waves (runs) a block: bfp4 8, so that each stage of A, whose bytes outweigh a run's tiles', serves twice the runs
  // (one 107 KB block a CU); 4 otherwise (at most 80 KB, two blocks a CU)
  static constexpr int W = FMT == BT_BFP4 ? 8 : 4;
};
template <int FMT, int MT, int EPI, int DT>
__global__ void __launch_bounds__(64 * Stream<FMT>::W) skinny_stream_kernel(const MatmulArgs args, int groups, int stages,
                                                                            float *part) {
  using S = Stream<FMT>;
  constexpr int W = S::W, C = S::C, TB = S::TB, ROWS = 16 * MT, ABYTES = ROWS * 512, STAGE = ABYTES + W * S::BW;
  constexpr int D = S::D;
  constexpr int AL = ROWS / (2 * W);  // a wave's A loads a stage (two rows each)
  constexpr int L = AL + S::BL;       // a wave's loads a stage
  constexpr int GAPS = FMT == BT_BFP4 ? C * 128 : 0;  // bfp4: a wave's tiles' exponents as placed gaps
  __shared__ __attribute__((aligned(1024))) uint8_t lds[D * STAGE + W * GAPS];
  const Head h = early_head(args);
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = (int)blockIdx.x % groups, sp = (int)blockIdx.x / groups;
  const int pos = W / 2 * grp + wib % (W / 2);  // SiLU x up: the gate run (the first W / 2 waves) whose up run the
  const int run = EPI == 2 ? pos + (wib < W / 2 ? 0 : h.nruns / 2) : grp * W + wib;  // other waves take
  const bool in = EPI == 2 ? pos < h.nruns / 2 : run < h.nruns;
  const int first = sp * stages * C;  // the split's first chunk
  const uint32_t abytes = (uint32_t)(((int64_t)(h.m - 1) * h.a.sr + h.k) * 2);
  const i32x4 ar = buffer_words((const void *)h.a.ptr, abytes);
  const i32x4 br = buffer_words(h.b + (int64_t)(in ? run : 0) * h.chunks * TB, in ? (uint32_t)h.chunks * TB : 0u);
  // stage st into ring slot st % D: this wave's A rows (load j: rows 2q, 2q + 1 with q = wib + W j; lane l takes
  // row 2q + l / 32, unit (l % 32) ^ (row % 16) of its 32) and its run's C tiles
  auto issue = [&](int st, int k) {  // k = st % D, a constant where the loop below is unrolled
    uint8_t *slot = lds + k * STAGE;
    const int c0 = first + st * C;
#pragma unroll
    for (int j = 0; j < AL; j++) {
      const int r = 2 * (wib + W * j) + (lane >> 5);
      const uint32_t unit = (uint32_t)((lane & 31) ^ (r & 15));
      const uint32_t voff = r < h.m ? (uint32_t)(((int64_t)r * h.a.sr + (int64_t)c0 * 64) * 2) + 16u * unit : abytes;
      lds_load16(ar, voff, slot + 2 * (wib + W * j) * 512);
    }
    uint8_t *bs = slot + ABYTES + wib * S::BW;
#pragma unroll
    for (int j = 0; j < S::BL; j++) {
      const uint32_t voff = (uint32_t)c0 * TB + 1024u * j + 16u * lane;
      if (j < S::BL - 1 || S::BLAST == 64 || lane < S::BLAST) lds_load16(br, voff, bs + 1024 * j);
    }
  };
  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  uint8_t *gp = lds + D * STAGE + wib * GAPS;
  auto multiply = [&](int k) {
    const uint8_t *slot = lds + k * STAGE;
    const uint8_t *bs = slot + ABYTES + wib * S::BW;
    if (FMT == BT_BFP4) {  // once for the wave's 64 lanes, not by each lane for its own 8 values (C = 4: lane l
      static_assert(FMT != BT_BFP4 || C == 4, "one exponent word a lane");  // places tile l / 16's word l % 16)
      *(uint2 *)(gp + (lane >> 4) * 128 + 8 * (lane & 15)) =
          place_gaps(*(const uint32_t *)(bs + (lane >> 4) * TB + 4 * (lane & 15)));
    }
#pragma unroll
    for (int i = 0; i < C; i++) {
      const uint8_t *tile = bs + i * TB;
      bf16x8 bv[2];
      if (FMT == BT_BF16) {
        bv[0] = *(const bf16x8 *)(tile + 32 * lane);
        bv[1] = *(const bf16x8 *)(tile + 32 * lane + 16);
      } else if (FMT == BT_BFP8) {
        const uint4 q = *(const uint4 *)(tile + 64 + 16 * lane);
        const uint4 e = *(const uint4 *)(tile + 16 * g);
        bv[0] = q8_to_bf16<true>(make_uint2(q.x, q.y), make_uint2(e.x, e.y));
        bv[1] = q8_to_bf16<true>(make_uint2(q.z, q.w), make_uint2(e.z, e.w));
      } else {
        const uint2 q = *(const uint2 *)(tile + 64 + 8 * lane);
        bv[0] = q4_to_bf16_placed(q.x, *(const uint4 *)(gp + i * 128 + 32 * g));
        bv[1] = q4_to_bf16_placed(q.y, *(const uint4 *)(gp + i * 128 + 32 * g + 16));
      }
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const int r = 16 * t + col;
        const uint8_t *row = slot + r * 512;
        const uint32_t u0 = (uint32_t)((8 * i + g) ^ (r & 15)), u1 = (uint32_t)((8 * i + g + 4) ^ (r & 15));
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)(row + 16 * u0), bv[0], acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)(row + 16 * u1), bv[1], acc[t], 0, 0, 0);
      }
    }
  };
  // the first D - 1 stages; then for each stage: wait for its loads (those of the later stages already issued may
  // stay out), a barrier (every wave's loads have landed, and every wave is done with the previous stage), the stage
  // D - 1 ahead into the slot the previous stage freed, and the multiply
#pragma unroll
  for (int st = 0; st < D - 1; st++)
    if (st < stages) issue(st, st);
  // the stages D at a time, unrolled, so that each one's ring slot is a constant and the LDS addresses of its loads
  // and fragment reads are fixed offsets from a few registers
  for (int s0 = 0; s0 < stages; s0 += D) {
#pragma unroll
    for (int k = 0; k < D; k++) {
      const int st = s0 + k;
      if (st >= stages) break;
      const int later = min(D - 2, stages - 1 - st);
      if (D == 4 && later == 2) wait_vm<2 * L>();
      else if (D >= 3 && later == 1) wait_vm<L>();
      else wait_vm<0>();
      __syncthreads();
      if (st + D - 1 < stages) issue(st + D - 1, (k + D - 1) % D);
      multiply(k);
    }
  }
  if constexpr (EPI == 0) {
    const int n = run * 16 + col;
    if (n >= h.n) return;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = 16 * t + 4 * g + i;
        if (m < h.m) part[((int64_t)sp * ROWS + m) * h.n + n] = acc[t][i];
      }
  } else if constexpr (EPI == 1) {
    if (!in) return;
#pragma unroll
    for (int t = 0; t < MT; t++) store_tile<DT>(args, h, acc[t], 0, t, run, g, col);
  } else {
    __syncthreads();  // every wave is done with the ring
    float *up = (float *)lds;  // the up waves' tiles, for the gate waves
    if (wib >= W / 2)
#pragma unroll
      for (int t = 0; t < MT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) up[(((wib - W / 2) * MT + t) * 4 + i) * 64 + lane] = acc[t][i];
    __syncthreads();
    if (wib >= W / 2 || !in) return;
    const int n = pos * 16 + col;  // the gate column, and the output's
    const bt_operand &out = h.out;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = 16 * t + 4 * g + i;
        if (m >= h.m) continue;
        const float gv = bf16_value(bf16_packed(acc[t][i]));
        const float uv = bf16_value(bf16_packed(up[((wib * MT + t) * 4 + i) * 64 + lane]));
        ((uint16_t *)out.ptr)[(int64_t)m * out.sr + n] = (uint16_t)bf16_packed(gv / (1.0f + expf(-gv)) * uv);
      }
  }
}

template <int FMT, int DT, int WM, int WN, int S>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm2_kernel(const MatmulArgs args, int mblocks, int nblocks) {
  using G = Gemm2<FMT, DT, WM, WN, S>;
  constexpr int TB = G::TB;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[G::LDS];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, col = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wib >> 1, wn = wib & 1;
  const int per = mblocks * nblocks, total = per * args.batch, full = total / 8 * 8;
  int pid = blockIdx.x;
  if (pid < full) pid = (pid % 8) * (full / 8) + pid / 8;
  const int b = pid / per;
  pid %= per;
  constexpr int GROUP = 8;
  const int width = GROUP * nblocks, first = pid / width * GROUP, gsz = min(mblocks - first, GROUP);
  const int bm = first + pid % width % gsz, bn = pid % width / gsz;
  const int m0 = bm * G::BM, n0 = bn * G::BN;

  const uint16_t *abase = (const uint16_t *)args.a.ptr + operand_matrix(args.a, b) * args.a.sb;
  const i32x4 ar = buffer_words(abase, (uint32_t)(((int64_t)(args.m - 1) * args.a.sr + args.k) * 2));
  const uint8_t *bbase = args.b + (args.b_matrix_bytes ? b * args.b_matrix_bytes : 0);
  const i32x4 br = buffer_words(bbase, (uint32_t)((int64_t)args.nruns * args.chunks * TB));
  constexpr uint32_t NOWHERE = 0xFFFFFFF0u;  // an offset past every buffer: the load writes zeros

  // the 16-byte source of each lane for each of the wave's loads of one chunk (the chunk adds 128 bytes to A's and
  // one tile to B's offsets)
  uint32_t src[G::PER_WAVE];
#pragma unroll
  for (int j = 0; j < G::PER_WAVE; j++) {
    const int li = wib + 4 * j;  // the block's load index
    if (li < G::A_LOADS) {
      const int slot = li * 64 + lane, r = slot >> 3, c = (slot & 7) ^ ((r >> 1) & 7);
      src[j] = (uint32_t)(((int64_t)(m0 + r) * args.a.sr + 8 * c) * 2);
    } else {
      const int slot = (li - G::A_LOADS) * 64 + lane;
      int tile, off;
      if (FMT == BT_BF16) {
        tile = slot >> 7;
        const int q = slot & 127;
        off = 32 * (q & 63) + 16 * (q >> 6);
      } else {
        tile = slot * 16 / TB;
        off = slot * 16 % TB;
      }
      const int run = n0 / 16 + tile;
      src[j] = li - G::A_LOADS < G::B_REAL && tile < G::BN / 16 && run < args.nruns
                   ? (uint32_t)((int64_t)run * args.chunks * TB + off) : NOWHERE;
    }
  }
  auto issue = [&](int c) {  // chunk c's loads into stage c % S
    uint8_t *st = lds + (c % S) * G::STAGE;
#pragma unroll
    for (int j = 0; j < G::PER_WAVE; j++) {
      const int li = wib + 4 * j;
      const bool isa = li < G::A_LOADS;
      const uint32_t off = src[j] == NOWHERE ? NOWHERE : src[j] + (isa ? c * 128u : (uint32_t)c * TB);
      uint8_t *dst = isa ? st + li * 1024
                     : li - G::A_LOADS < G::B_REAL ? st + G::A_BYTES + (li - G::A_LOADS) * 1024 : lds + G::JUNK;
      lds_load16(isa ? ar : br, off, dst);
    }
  };

  f32x4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < S - 1; c++)
    if (c < args.chunks) issue(c);
  uint8_t *bbf = lds + S * G::STAGE;
  for (int c = 0; c < args.chunks; c++) {
    // chunk c has landed once at most the later chunks' loads are outstanding (fewer near the end)
    if (c + S - 2 < args.chunks) wait_vm<G::PER_WAVE * (S - 2)>();
    else wait_vm<0>();
    __syncthreads();
    uint8_t *st = lds + (c % S) * G::STAGE;
    if (G::CONVERT) {
      const uint8_t *raw = st + G::A_BYTES;
#pragma unroll
      for (int i = 0; i < G::BPT; i++) {
        const int slot = tid + 256 * i, tile = slot >> 6, tl = slot & 63;
        const uint8_t *t = raw + tile * TB;
        const uint4 ex = *(const uint4 *)(t + 16 * (tl >> 4));
        bf16x8 h0, h1;
        if (FMT == BT_BFP8) {
          const uint4 q = *(const uint4 *)(t + 64 + 16 * tl);
          h0 = q8_to_bf16<true>(make_uint2(q.x, q.y), make_uint2(ex.x, ex.y));
          h1 = q8_to_bf16<true>(make_uint2(q.z, q.w), make_uint2(ex.z, ex.w));
        } else {
          const uint2 q = *(const uint2 *)(t + 64 + 8 * tl);
          h0 = q4_to_bf16_scaled(q.x, make_uint2(ex.x, ex.y));
          h1 = q4_to_bf16_scaled(q.y, make_uint2(ex.z, ex.w));
        }
        uint8_t *bl = bbf + tile * 2048 + tl * 16;
        *(bf16x8 *)bl = h0;
        *(bf16x8 *)(bl + 1024) = h1;
      }
      __syncthreads();
    }
    if (c + S - 1 < args.chunks) issue(c + S - 1);  // into the stage chunk c - 1 used
    const uint8_t *bsrc = G::CONVERT ? bbf : st + G::A_BYTES;
    const uint8_t *bl = bsrc + wn * WN * 2048 + lane * 16;
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      bf16x8 af[WM], bv[WN];
#pragma unroll
      for (int i = 0; i < WM; i++) {
        const int r = wm * WM * 16 + 16 * i + col, cc = (g + 4 * kk) ^ ((r >> 1) & 7);
        af[i] = *(const bf16x8 *)(st + r * 128 + 16 * cc);
      }
#pragma unroll
      for (int j = 0; j < WN; j++) bv[j] = *(const bf16x8 *)(bl + j * 2048 + kk * 1024);
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bv[j], acc[i][j], 0, 0, 0);
    }
  }
  __syncthreads();  // every wave is done with the stages
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        uint8_t *at = lds + (wm * WM * 16 + 16 * i + 4 * g + r) * G::ES + (wn * WN * 16 + 16 * j + col) * G::ESZ;
        if (DT == BT_FP32) *(float *)at = acc[i][j][r];
        else *(uint16_t *)at = (uint16_t)bf16_packed(acc[i][j][r]);
      }
  __syncthreads();
  gemm_epilogue<DT, G::BM, G::BN, G::ES, G::ESZ>(args, lds, b, m0, n0, tid);
}

// ---- the prefill GEMM for bf16 B, K in steps of 32 ----------------------------------------------------------------
// 256 x 256 blocks of 8 waves (2 x 4, 128 x 64 each), two waves a SIMD, so one wave's LDS reads run under the other's
// matrix instructions. A step of 32 along K stages A (256 rows of 64 bytes, each row's four 16-byte columns at
// c ^ ((r >> 1) & 3), so a fragment's 16 rows meet different banks) and B (16 tiles' half, 1 KB each in operand order)
// in LDS through direct loads, S steps deep. One barrier a step: after it a wave issues its loads of step t + S - 1
// into the stage that step t - 1 used, reads its fragments of step t and multiplies. The sums run in the order of the
// other kernels (chunk by chunk, its lower 32 rows then its upper), so the result is the same bits. Needs K a multiple
// of 32.
// MODE 1 (RES): fp32 out written straight from the accumulators, plus (if res.ptr) the fp32 operand res at the same
// element: the residual add that a program `out = value + x` asks for, without staging the tile.
// MODE 2 (SWIGLU): B holds gate then up side by side (n = 2 f columns); a block takes 128 columns of each, at the
// same place in both halves, and writes silu(gate) * up for those 128 columns (out: m x f, bf16): the gate and up
// values rounded to bf16 as stored, silu(g) = g / (1 + exp(-g)) and the product in fp32, rounded once.
constexpr int GEMM_PLAIN = 0, GEMM_RES = 1, GEMM_SWIGLU = 2;
// BM: the block's rows, 256 or 128 (a wave BM / 2 of them by 64 columns), for products whose 256-row blocks would
// leave CUs idle.
// FMT 4 (bfp4 B) stages a chunk (64 rows of K) at a time, CS = 3 deep (4 for 128-row blocks): A as BM rows of 128
// bytes (unit u of row r at u ^ (r % 8), so the fragment reads of 8 neighbouring rows meet different banks) and the
// block's 16 tiles as they are stored, 576 bytes each (36 lanes of a direct load). The wave that loaded a tile places
// its exponent bytes in LDS as 16-bit gaps before the chunk's barrier; each wave then reads its 4 tiles' value bytes
// and gaps and decodes them into bf16 fragments in registers (q * 2^(e - 129) by subtracting the gaps, the values the
// unpacker gives), the second half's decode between the first half's matrix instructions. So B crosses HBM and LDS
// at 0.28 of its bf16 size and needs no unpacking pass. The sums run in the same order, so the result is the same
// bits as the bf16 GEMM on B's unpacked tiles.
// BN: the block's columns, 256 or 192 (the stages keep room for 16 tiles either way, and the slots of missing tiles
// take loads that read nothing, so every wave issues the same loads), for products whose 256-column blocks would leave
// a round of the CUs part empty; or, on bfp4 B, 128 x 384 (24 tiles a stage, three a wave): 6144 columns make 256
// such blocks, one round, each tile decoded once and each A byte staged for 384 columns.
template <int FMT, int DT, int S, int MODE = GEMM_PLAIN, int BM = 256, int BN = 256>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm3_kernel(const MatmulArgs args, int mblocks, int nblocks, const bt_operand res, int nb_off = 0) {
  static_assert(FMT == BT_BF16 || FMT == BT_BFP4, "gemm3 takes bf16 or bfp4 B");
  static_assert(BN == 256 || (BN == 192 && MODE != GEMM_SWIGLU) ||
                    (BN == 384 && FMT == BT_BFP4 && BM == 128 && MODE != GEMM_SWIGLU),
                "gemm3 blocks are 256 or 192 columns, or 128 x 384 on bfp4 B");
  constexpr bool RES = MODE == GEMM_RES;
  // the 8 waves as 2 x 4 (each BM / 2 rows by BN / 4 columns); bfp4 B, where the columns allow, as 1 x 8 (each all BM
  // rows by BN / 8 columns), so that each tile is decoded by one wave, not two, for as many matrix instructions
  constexpr int WAVES_M = FMT == BT_BFP4 && BN % 128 == 0 ? 1 : 2, WAVES_N = 8 / WAVES_M;
  constexpr int A_BYTES = BM * 64, STAGE = A_BYTES + 16384, WM = BM / (16 * WAVES_M), WN = BN / (16 * WAVES_N),
                WR = BM / WAVES_M, T = BN / 16;
  static_assert(WN * 16 * WAVES_N == BN, "the waves' columns cover the block");
  constexpr int AL = BM / 128;  // A loads a wave issues a step
  // bfp4: chunk stages of A's rows, the 16 tiles as stored, then the tiles' exponents as placed gaps (128 B a tile)
  // TT: tile slots a stage (16, or 24 for 384 columns), NB of them loaded by each wave
  constexpr int TT = BN / 16 > 16 ? BN / 16 : 16, NB = TT / 8;
  constexpr int CS = BM == 128 ? 4 : 3, QTB = 576, QA = BM * 128, QG = QA + TT * QTB, QSTAGE = QG + TT * 128, QAL = BM / 64;
  constexpr int RING = FMT == BT_BF16 ? S * STAGE : CS * QSTAGE;
  constexpr int ESZ = DT == BT_FP32 ? 4 : 2, ES = BN * ESZ + 16;
  constexpr int HALF = (DT == BT_FP32 ? 128 : 256) < BM ? (DT == BT_FP32 ? 128 : 256) : BM;
  constexpr int LDS = RES ? RING : RING > HALF * ES ? RING : HALF * ES;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS];
  const Head h = early_head(args);
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, col = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wib / WAVES_N, wn = wib % WAVES_N;
  const int per = mblocks * nblocks, total = per * h.batch, full = total / 8 * 8;
  int pid = blockIdx.x;
  if (pid < full) pid = (pid % 8) * (full / 8) + pid / 8;  // neighbouring blocks on one XCD
  const int b = pid / per;
  pid %= per;
  // blocks of a column of GROUP block rows run together, sharing B's tiles in L2: 8 rows with bf16 B; 2 with bfp4 B,
  // whose tiles are 0.28 of A's bytes, so that each XCD's blocks hold fewer rows of A at once (1-2% faster there)
  constexpr int GROUP = FMT == BT_BFP4 ? 2 : 8;
  const int width = GROUP * nblocks, first = pid / width * GROUP, gsz = min(mblocks - first, GROUP);
  const int bm = first + pid % width % gsz, bn = nb_off + pid % width / gsz;  // nb_off: the launch's first block column
  const int m0 = bm * BM, n0 = bn * BN;

  const uint16_t *abase = (const uint16_t *)h.a.ptr + operand_matrix(h.a, b) * h.a.sb;
  const i32x4 ar = buffer_words(abase, (uint32_t)(((int64_t)(h.m - 1) * h.a.sr + h.k) * 2));
  const uint8_t *bbase = h.b + (h.b_matrix_bytes ? b * h.b_matrix_bytes : 0);
  constexpr uint32_t NOWHERE = 0xFFFFFFF0u;  // an offset past every buffer: the load writes zeros
  // the run of B whose tile the block's tile li (0..15) is, and whether it exists
  auto b_run = [&](int li, bool &in) {
    int run = n0 / 16 + li;
    in = li < T && run < h.nruns;
    if (MODE == GEMM_SWIGLU) {  // tiles 0..7: gate columns from 128 bn, 8..15: the same up columns
      const int f = h.n / 2, c0 = bn * 128 + 16 * (li & 7);
      run = ((li < 8 ? 0 : f) + c0) / 16;
      in = c0 < f;
    }
    return run;
  };
  f32x4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (FMT == BT_BF16) {
  const i32x4 br = buffer_words(bbase, (uint32_t)((int64_t)h.nruns * h.chunks * 2048));

  // each lane's source for the wave's 2 A and 2 B loads of step 0 (a step adds 64 bytes to A's; B's move by half a
  // tile, then to the next chunk)
  uint32_t asrc[2], bsrc[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int li = wib + 8 * j;  // rows 16 li .. 16 li + 15 of A (li < BM / 16), tile li of B
    const int r = 16 * li + lane / 4, c = (lane & 3) ^ ((r >> 1) & 3);
    asrc[j] = j < AL && m0 + r < h.m ? (uint32_t)(((int64_t)(m0 + r) * h.a.sr + 8 * c) * 2) : NOWHERE;
    bool in;
    const int run = b_run(li, in);
    bsrc[j] = in ? (uint32_t)((int64_t)run * h.chunks * 2048 + 32 * lane) : NOWHERE;
  }
  auto issue = [&](int t) {  // step t's loads into stage t % S
    uint8_t *st = lds + (t % S) * STAGE;
    const uint32_t ao = (uint32_t)t * 64, bo = (uint32_t)(t >> 1) * 2048 + (t & 1) * 16;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int li = wib + 8 * j;
      if (j < AL) lds_load16(ar, asrc[j] == NOWHERE ? NOWHERE : asrc[j] + ao, st + li * 1024);
      lds_load16(br, bsrc[j] == NOWHERE ? NOWHERE : bsrc[j] + bo, st + A_BYTES + li * 1024);
    }
  };
  const int steps = h.k / 32;
#pragma unroll
  for (int t = 0; t < S - 1; t++)
    if (t < steps) issue(t);
  for (int t = 0; t < steps; t++) {
    // step t landed once at most the later steps' loads are outstanding (fewer near the end)
    if (t + S - 2 < steps) wait_vm<(AL + 2) * (S - 2)>();
    else wait_vm<0>();
    __syncthreads();
    if (t + S - 1 < steps) issue(t + S - 1);  // into the stage step t - 1 used
    const uint8_t *st = lds + (t % S) * STAGE;
    bf16x8 fa[WM], fb[WN];
#pragma unroll
    for (int i = 0; i < WM; i++) {
      const int r = wm * WR + 16 * i + col;
      fa[i] = *(const bf16x8 *)(st + r * 64 + 16 * (g ^ ((r >> 1) & 3)));
    }
#pragma unroll
    for (int j = 0; j < WN; j++) fb[j] = *(const bf16x8 *)(st + A_BYTES + (wn * WN + j) * 1024 + lane * 16);
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
      for (int j = 0; j < WN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
  }
  } else {
    const i32x4 br = buffer_words(bbase, (uint32_t)((int64_t)h.nruns * h.chunks * QTB));
    // each lane's source for the wave's QAL A loads (8 rows of 128 bytes each; lane l takes row l / 8, unit
    // (l % 8) ^ (row % 8)) and 2 B tiles (tiles wib and wib + 8, lanes 0..35) of chunk 0; a chunk adds 128 bytes to
    // A's, one tile to B's
    uint32_t aq[QAL], bq[NB];
#pragma unroll
    for (int j = 0; j < QAL; j++) {
      const int r = 8 * (wib + 8 * j) + (lane >> 3), u = (lane & 7) ^ (r & 7);
      aq[j] = m0 + r < h.m ? (uint32_t)(((int64_t)(m0 + r) * h.a.sr + 8 * u) * 2) : NOWHERE;
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
      bool in;
      const int run = b_run(wib + 8 * j, in);
      bq[j] = in ? (uint32_t)((int64_t)run * h.chunks * QTB + 16 * lane) : NOWHERE;
    }
    auto issue = [&](int c) {  // chunk c's loads into stage c % CS
      uint8_t *st = lds + (c % CS) * QSTAGE;
      const uint32_t ao = (uint32_t)c * 128, bo = (uint32_t)c * QTB;
#pragma unroll
      for (int j = 0; j < QAL; j++) lds_load16(ar, aq[j] == NOWHERE ? NOWHERE : aq[j] + ao, st + (wib + 8 * j) * 1024);
#pragma unroll
      for (int j = 0; j < NB; j++)
        if (lane < QTB / 16) lds_load16(br, bq[j] == NOWHERE ? NOWHERE : bq[j] + bo, st + QA + (wib + 8 * j) * QTB);
    };
    const int chunks = h.k / 64;
#pragma unroll
    for (int c = 0; c < CS - 1; c++)
      if (c < chunks) issue(c);
    for (int c = 0; c < chunks; c++) {
      if (c + CS - 2 < chunks) wait_vm<(QAL + NB) * (CS - 2)>();
      else wait_vm<0>();
      uint8_t *st = lds + (c % CS) * QSTAGE;
      // the exponent bytes of the wave's own two tiles have landed (its loads wrote them): placed as gaps once here,
      // for every wave that reads the tiles, instead of by each of them (lanes 16 s .. 16 s + 15: tile wib + 8 s)
      if (lane < 16 * NB) {
        const int s = wib + 8 * (lane >> 4), w = lane & 15;
        *(uint2 *)(st + QG + s * 128 + 8 * w) = place_gaps(*(const uint32_t *)(st + QA + s * QTB + 4 * w));
      }
      __syncthreads();
      if (c + CS - 1 < chunks) issue(c + CS - 1);  // into the stage chunk c - 1 used
      uint2 q[WN];
#pragma unroll
      for (int j = 0; j < WN; j++) q[j] = *(const uint2 *)(st + QA + (wn * WN + j) * QTB + 64 + 8 * lane);
      // lane group g's 8 values of half hh: A's 16-byte unit g + 4 hh of each row, B's gaps 16 g + 8 hh ..
      auto a_frag = [&](int i, int hh) {
        const int r = wm * WR + 16 * i + col;
        return *(const bf16x8 *)(st + r * 128 + 16 * ((g + 4 * hh) ^ (r & 7)));
      };
      auto gaps = [&](int j, int hh) { return *(const uint4 *)(st + QG + (wn * WN + j) * 128 + 32 * g + 16 * hh); };
      bf16x8 fa[WM], fb[WN], fb1[WN];
      uint4 gp[WN];
#pragma unroll
      for (int i = 0; i < WM; i++) fa[i] = a_frag(i, 0);
#pragma unroll
      for (int j = 0; j < WN; j++) fb[j] = q4_to_bf16_placed(q[j].x, gaps(j, 0));
      __builtin_amdgcn_sched_barrier(0);
      // the first half's matrix instructions a row of tiles at a time, the second half's reads and decode between
      // them, so that their VALU work issues while the matrix core is busy: after row i, A's fragment i of the second
      // half (into the registers row i is done with), the gaps after row 0, and one tile's decode after each of the
      // last WN rows; the order is held by scheduling barriers
#pragma unroll
      for (int i = 0; i < WM; i++) {
#pragma unroll
        for (int j = 0; j < WN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        fa[i] = a_frag(i, 1);
        if (i == 0)
#pragma unroll
          for (int j = 0; j < WN; j++) gp[j] = gaps(j, 1);
        if (i >= WM - WN) fb1[i - (WM - WN)] = q4_to_bf16_placed(q[i - (WM - WN)].y, gp[i - (WM - WN)]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb1[j], acc[i][j], 0, 0, 0);
    }
  }
  if constexpr (RES) {
    // lanes 0..15 of a row group write 16 neighbouring columns: 64 bytes
    // The residual may be the output itself (x += o), so a residual can't be loaded after a store the compiler can't
    // tell apart from it: the residuals of GI row tiles are all loaded before any of their sums is stored, one trip
    // to memory for the group instead of one for each value.
    const int64_t ob = operand_matrix(h.out, b) * h.out.sb, rb = res.ptr ? operand_matrix(res, b) * res.sb : 0;
    constexpr int GI = WM < 4 ? WM : 4;
#pragma unroll
    for (int i0 = 0; i0 < WM; i0 += GI) {
      float rv[GI][4][WN];
#pragma unroll
      for (int ii = 0; ii < GI; ii++)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
          for (int j = 0; j < WN; j++) {
            const int m = m0 + wm * WR + 16 * (i0 + ii) + 4 * g + r, n = n0 + wn * 16 * WN + 16 * j + col;
            rv[ii][r][j] = res.ptr && m < h.m && n < h.n
                               ? ((const float *)res.ptr)[rb + (int64_t)m * res.sr + (int64_t)n * res.sc] : 0.0f;
          }
#pragma unroll
      for (int ii = 0; ii < GI; ii++)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
          for (int j = 0; j < WN; j++) {
            const int m = m0 + wm * WR + 16 * (i0 + ii) + 4 * g + r, n = n0 + wn * 16 * WN + 16 * j + col;
            if (m < h.m && n < h.n)
              ((float *)h.out.ptr)[ob + (int64_t)m * h.out.sr + (int64_t)n * h.out.sc] =
                  res.ptr ? acc[i0 + ii][j][r] + rv[ii][r][j] : acc[i0 + ii][j][r];
          }
    }
    return;
  }
  __syncthreads();  // every wave is done with the stages
  // the tile through LDS to the epilogue: 256 rows (bf16) or 128 at a time (fp32)
#pragma unroll
  for (int half = 0; half < BM / HALF; half++) {
#pragma unroll
    for (int i = 0; i < WM; i++) {
      const int row0 = wm * WR + 16 * i;  // the row tile's first row in the block: written in its own half
      if (row0 / HALF != half) continue;
#pragma unroll
      for (int j = 0; j < WN; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          uint8_t *at = lds + (row0 % HALF + 4 * g + r) * ES + (wn * 16 * WN + 16 * j + col) * ESZ;
          if (DT == BT_FP32) *(float *)at = acc[i][j][r];
          else *(uint16_t *)at = (uint16_t)bf16_packed(acc[i][j][r]);
        }
    }
    __syncthreads();
    if constexpr (MODE == GEMM_SWIGLU) {
      // a thread 8 neighbouring columns of a row at a time: gate at column c of the tile, up at c + 128
      const int f = h.n / 2, rows = min(BM, h.m - m0), c0 = bn * 128;
      const int64_t ob = operand_matrix(h.out, b) * h.out.sb;
#pragma unroll 1
      for (int e = tid; e < rows * 16; e += 512) {
        const int r = e >> 4, c = (e & 15) * 8;
        if (c0 + c >= f) continue;
        const uint4 gw = *(const uint4 *)(lds + r * ES + c * 2), uw = *(const uint4 *)(lds + r * ES + (128 + c) * 2);
        const uint32_t gs[4] = {gw.x, gw.y, gw.z, gw.w}, us[4] = {uw.x, uw.y, uw.z, uw.w};
        uint32_t o[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
          uint32_t w = 0;
#pragma unroll
          for (int hf = 0; hf < 2; hf++) {
            const float gv = bf16_value(gs[v] >> (16 * hf) & 0xFFFFu), uv = bf16_value(us[v] >> (16 * hf) & 0xFFFFu);
            w |= bf16_packed(gv / (1.0f + expf(-gv)) * uv) << (16 * hf);
          }
          o[v] = w;
        }
        *(uint4 *)((uint16_t *)h.out.ptr + ob + (int64_t)(m0 + r) * h.out.sr + c0 + c) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    } else {
      gemm_epilogue<DT, HALF, BN, ES, ESZ, 512>(args, lds, b, m0 + half * HALF, n0, tid);
    }
    if (BM != HALF) __syncthreads();
  }
}

// Block-float columns tiles -> bf16 columns tiles of the same values (the conversion gemm2 does in LDS), a thread a
// lane of a tile: for the prefill GEMM, which takes bf16 B.
template <int FMT>
__global__ void __launch_bounds__(256) tiles_bf16_kernel(const uint8_t *src, uint8_t *dst, int64_t tiles) {
  constexpr int TB = Tile<FMT>::bytes;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= tiles) return;
  const uint8_t *s = src + t * TB;
  const uint4 ex = *(const uint4 *)(s + 16 * (lane >> 4));
  bf16x8 h0, h1;
  if (FMT == BT_BFP8) {
    const uint4 q = *(const uint4 *)(s + 64 + 16 * lane);
    h0 = q8_to_bf16<true>(make_uint2(q.x, q.y), make_uint2(ex.x, ex.y));
    h1 = q8_to_bf16<true>(make_uint2(q.z, q.w), make_uint2(ex.z, ex.w));
  } else {
    const uint2 q = *(const uint2 *)(s + 64 + 8 * lane);
    h0 = q4_to_bf16_scaled(q.x, make_uint2(ex.x, ex.y));
    h1 = q4_to_bf16_scaled(q.y, make_uint2(ex.z, ex.w));
  }
  uint8_t *d = dst + t * 2048 + 32 * lane;
  *(bf16x8 *)d = h0;
  *(bf16x8 *)(d + 16) = h1;
}

// ---- one row with its prologue and residual (bt_matmul_row) ------------------------------------------------------
// The decode GEMV of gemv_kernel for a single row whose A is made in the kernel: the block reads the prologue's inputs
// straight into LDS (1 KB a load) before its first group of weight loads, works out a' (the norm, or silu(g) * u)
// into an LDS row while those loads are in flight, and each wave then takes its A values from that row. The residual
// is added to the fp32 sum before the store.
struct RowArgs {  // 72 bytes: brought by the kernel's first round of scalar loads
  const uint8_t *b;
  const uint8_t *a;
  const uint8_t *norm;
  const float *res;
  uint8_t *out;
  int32_t chunks, nruns, k, n, out_dtype;
  float eps;
  int32_t slices;     // waves a run (1, 2 or 4), each a slice of K, summed in slice order
  int32_t half_runs;  // with RoPE: 16-column runs in half a head
};

// RoPE of the product and the cache put (bt_rope_put's fields, read in the epilogue only).
struct RopeTail {
  const uint16_t *cos, *sin;
  const int32_t *places;
  uint16_t *q, *cache, *vcache;
  int64_t cache_sh, cache_sr, cache_tsh, cache_rows;
  int32_t heads, kv, head_dim;
};


// The block's inputs a 1 KB load: lane l's 16 bytes of piece p at p * 1024 + 16 l, into LDS at lds + p * 1024; the
// buffer's range gives zeros past its end. Each wave takes every fourth piece.
__device__ __forceinline__ int row_pieces(const i32x4 &rsrc, int pieces, uint8_t *lds, int wib, int lane) {
  int issued = 0;
  for (int p = wib; p < pieces; p += 4, issued++) lds_load16(rsrc, p * 1024 + 16 * lane, lds + p * 1024);
  return issued;
}

//
// With ROPE the product is rounded to bf16 (as bt_matmul_row stores it) and goes through RoPE and the cache put as
// bt_rope_put does, in one kernel: a block's waves take the runs of RoPE's partner columns (j and j + d/2 of a head)
// side by side and swap their values through LDS.
template <int FMT, int G, int KIND, bool ROPE>
__global__ void __launch_bounds__(256) gemv_row_kernel(const RowArgs args, const RopeTail rp) {
  constexpr int TB = Tile<FMT>::bytes;
  // weights loaded with the default cache policy: a decode step reads the same matrices every token, and a small
  // model's stay in the 256 MB Infinity Cache between steps
  constexpr int KEEP = 0;
  extern __shared__ __attribute__((aligned(1024))) uint8_t dyn[];
  const RowArgs h = args;
  asm volatile("" ::"s"(h.b), "s"(h.a), "s"(h.norm), "s"(h.res), "s"(h.out), "s"(h.chunks), "s"(h.nruns), "s"(h.k),
               "s"(h.n), "s"(h.out_dtype), "s"(h.eps), "s"(h.slices), "s"(h.half_runs));
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = h.slices, sl = wib % S, lr = wib / S;  // lr: the wave's run among the block's 4 / S
  // with RoPE, runs u and u + half_runs of a head side by side: block run i is of pair blockIdx.x * (2 / S) + i / 2
  auto run_of = [&](int i) -> int {
    if (!ROPE) return (int)blockIdx.x * (4 / S) + i;
    const int pair = blockIdx.x * (2 / S) + i / 2, hr = h.half_runs;
    return pair / hr * 2 * hr + pair % hr + (i & 1) * hr;
  };
  const int run = run_of(lr);
  const int chunks = h.chunks, K = h.k, kpad = chunks * 64;
  const bool valid = run < h.nruns;
  const int per = (chunks + S - 1) / S, c_begin = min(chunks, sl * per), mine = min(chunks, c_begin + per) - c_begin;
  // LDS: the inputs' pieces (raw0, raw1), the row a' (bf16, kpad values), each wave's slots, the norm's partial sums
  const int p0 = KIND == BT_ROW_RMS ? (K * 4 + 1023) / 1024 : KIND == BT_ROW_SWIGLU ? (K * 2 + 1023) / 1024 : 0;
  const int p1 = KIND == BT_ROW_PLAIN ? 0 : (K * 2 + 1023) / 1024;
  const int prow = (kpad * 2 + 1023) / 1024;
  uint8_t *raw0 = dyn, *raw1 = dyn + p0 * 1024;
  uint16_t *arow = (uint16_t *)(raw1 + p1 * 1024);
  uint16_t *slots = arow + prow * 512 + wib * G * 64;
  float *red = (float *)(arow + prow * 512 + 4 * G * 64);
  f32x4 *part = (f32x4 *)(red + 4);  // the slices' partial tiles
  float *xch = (float *)(part + 256);  // with RoPE: each run's 16 values, as stored (bf16)
  uint8_t *rtab = (uint8_t *)(xch + 64);  // with RoPE: cos and sin of the block's runs (1 KB each), the place
  // 0. RoPE's tables for the block's runs and the token's place: lane i of wave 0 (cos) or 1 (sin) brings columns
  // 8 (i % 2) .. + 7 of block run i / 2; lane 0 of wave 2 the place
  if (ROPE && wib < 2) {
    const int i = lane / 2, rn = run_of(i);
    const uint32_t off = lane < 2 * (4 / S) && rn < h.nruns ? (uint32_t)(rn * 16 + (lane & 1) * 8) * 2 : 0xFFFFFFF0u;
    lds_load16(buffer_words(wib == 0 ? rp.cos : rp.sin, (uint32_t)h.n * 2), off, rtab + wib * 1024);
  } else if (ROPE && wib == 2) {
    lds_load4(buffer_words(rp.places, 4), lane == 0 ? 0u : 0xFFFFFFF0u, rtab + 2048);
  }
  // 1. the prologue's inputs into LDS
  if (KIND == BT_ROW_PLAIN) {
    row_pieces(buffer_words(h.a, (uint32_t)K * 2), prow, (uint8_t *)arow, wib, lane);
  } else if (KIND == BT_ROW_RMS) {
    row_pieces(buffer_words(h.a, (uint32_t)K * 4), p0, raw0, wib, lane);
    row_pieces(buffer_words(h.norm, (uint32_t)K * 2), p1, raw1, wib, lane);
  } else {
    row_pieces(buffer_words(h.a, (uint32_t)K * 2), p0, raw0, wib, lane);
    row_pieces(buffer_words(h.a + (int64_t)K * 2, (uint32_t)K * 2), p1, raw1, wib, lane);
  }
  // the residual at the lane's column (row 0: lanes 0..15 of the run's first slice), requested with the inputs so it
  // has landed by step 3's wait; read at the end, it would add a trip to memory after the last product
  float resv = 0.0f;
  if (!ROPE && h.res) {
    const int n = run * 16 + col;
    const bool mine_col = valid && sl == 0 && g == 0 && n < h.n;
    resv = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(buffer(h.res, (uint32_t)h.n * 4),
                                                                mine_col ? (uint32_t)n * 4 : 0xFFFFFFF0u, 0, 0));
  }
  // 2. the first group's weights (every wave issues 2 G loads; a wave past the last run reads nothing)
  const uint8_t *tiles = h.b + ((int64_t)(valid ? run : 0) * chunks + c_begin) * TB;
  const __amdgpu_buffer_rsrc_t tr = buffer(tiles, valid ? (uint32_t)mine * TB : 0u);
  const int kl = exp_row(lane), frag = 8 * g;
  uint32_t bq[G][4], ex[G];
  uint4 bhi[G];
  auto load_group = [&](int c0) {
#pragma unroll
    for (int i = 0; i < G; i++) {
      const uint32_t at = (uint32_t)(c0 + i) * TB;
      if (FMT == BT_BFP8 || FMT == BT_BF16) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + (FMT == BT_BFP8 ? 64 + 16 * lane : 32 * lane),
                                                             0, KEEP);
        bq[i][0] = q[0]; bq[i][1] = q[1]; bq[i][2] = q[2]; bq[i][3] = q[3];
      } else {
        const auto q = __builtin_amdgcn_raw_buffer_load_b64(tr, at + 64 + 8 * lane, 0, KEEP);
        bq[i][0] = q[0]; bq[i][1] = q[1];
      }
      if (FMT == BT_BF16) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(tr, at + 32 * lane + 16, 0, KEEP);
        bhi[i] = make_uint4(q[0], q[1], q[2], q[3]);
      } else {
        ex[i] = __builtin_amdgcn_raw_buffer_load_b8(tr, at + lane, 0, KEEP);
      }
    }
  };
  load_group(0);
  // 3. the inputs have landed once at most the 2 G weight loads are outstanding; then the block's
  wait_vm<2 * G>();
  __syncthreads();
  // 4. the row a', each wave a quarter of it
  if (KIND == BT_ROW_RMS) {
    const float *x = (const float *)raw0;
    const uint16_t *w = (const uint16_t *)raw1;
    float ss = 0.0f;
    for (int k = wib * 64 + lane; k < K; k += 256) {
      const float v = round_packed(x[k]);
      ss += v * v;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wib] = ss;
    __syncthreads();
    const float total = ((red[0] + red[1]) + red[2]) + red[3];
    const float r = 1.0f / sqrtf(total / (float)K + h.eps);
    for (int k = wib * 64 + lane; k < kpad; k += 256)
      arow[k] = k < K ? (uint16_t)bf16_packed(round_packed(x[k]) * r * bf16_value(w[k])) : (uint16_t)0;
    __syncthreads();
  } else if (KIND == BT_ROW_SWIGLU) {
    const uint16_t *gate = (const uint16_t *)raw0, *up = (const uint16_t *)raw1;
    for (int k = wib * 64 + lane; k < kpad; k += 256) {
      uint16_t v = 0;
      if (k < K) {
        const float gv = bf16_value(gate[k]);
        v = (uint16_t)bf16_packed(gv / (1.0f + expf(-gv)) * bf16_value(up[k]));
      }
      arow[k] = v;
    }
    __syncthreads();
  }
  if (!ROPE && !valid && S == 1) return;  // with RoPE every wave reaches the swap's barrier (an invalid one sums zeros)
  // 5. the product over this wave's slice, chunk by chunk as gemv_kernel's
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < mine; c0 += G) {
    if (c0 > 0) load_group(c0);
#pragma unroll
    for (int i = 0; i < G; i++) {
      if (c0 + i >= mine) continue;
      const int d = FMT == BT_BF16 ? 0 : (int)(int8_t)(ex[i] & 255u);
      uint32_t v = arow[(c_begin + c0 + i) * 64 + kl];
      if (FMT != BT_BF16) v = __float_as_uint(ldexpf(__uint_as_float(v << 16), d)) >> 16;
      slots[i * 64 + kl] = (uint16_t)v;
      __builtin_amdgcn_wave_barrier();
      bf16x8 av[2], bv[2];
#pragma unroll
      for (int hh = 0; hh < 2; hh++) av[hh] = *(const bf16x8 *)(slots + i * 64 + frag + 32 * hh);
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
  // 6. the slices added in order into the first; row 0 of the tile: lanes 0..15, one column each
  if (S > 1) {
    if (sl != 0) part[wib * 64 + lane] = acc;
    __syncthreads();
    if (!ROPE && (sl != 0 || !valid)) return;
    if (sl == 0)
      for (int j = 1; j < S; j++) acc += part[(wib + j) * 64 + lane];
  }
  if (ROPE) {
    if (sl == 0 && g == 0) xch[lr * 16 + col] = round_packed(acc[0]);
    __syncthreads();
    const int n = run * 16 + col;
    if (sl != 0 || g != 0 || !valid) return;
    const float x = xch[lr * 16 + col], xp = xch[(lr ^ 1) * 16 + col];
    const float cs = bf16_value(((const uint16_t *)rtab)[lr * 16 + col]);
    const float sn = bf16_value(((const uint16_t *)rtab)[512 + lr * 16 + col]);
    const float y = lr & 1 ? __fadd_rn(__fmul_rn(x, cs), __fmul_rn(xp, sn)) : __fsub_rn(__fmul_rn(x, cs), __fmul_rn(xp, sn));
    const int head = n / rp.head_dim, j = n % rp.head_dim;
    if (head < rp.heads) {
      rp.q[n] = (uint16_t)bf16_packed(y);
    } else {
      const int place = *(const int32_t *)(rtab + 2048), hk = head - rp.heads;
      if (place < 0 || place >= rp.cache_rows) return;
      const bool own = rp.vcache && hk >= rp.kv;
      uint16_t *dst = (own ? rp.vcache : rp.cache) + (int64_t)(own ? hk - rp.kv : hk) * rp.cache_sh +
                      (int64_t)place * rp.cache_sr;
      dst[j] = (uint16_t)bf16_packed(y);
    }
    return;
  }
  const int n = run * 16 + col;
  if (g != 0 || n >= h.n) return;
  float v = acc[0];
  if (h.res) v += resv;
  if (h.out_dtype == BT_BF16) ((uint16_t *)h.out)[n] = (uint16_t)bf16_packed(v);
  else ((float *)h.out)[n] = v;
}

int validate_program(const bt_program *prog);
int check_out(const bt_operand *out);

// Slices along K for `units` output tiles: enough that the launch has about 4096 waves, when K is deep enough to give
// each slice at least 16 chunks (a single wave would walk a deep K one group of loads after another). K of fewer than
// 32 chunks is never sliced: such a product sums in the same order as the GEMM.
static int choose_slices(int64_t units, int chunks) {
  int sl = 1;
  while (sl < 8 && units * sl < 4096 && chunks >= 32 * sl) sl *= 2;
  return sl;
}

static bool residual_program(const MatmulArgs &args, bt_operand *res);

// Slices of the two-runs-a-wave skinny kernel: from K = 2048 up (below it, sums in the GEMM's order), up to 8 while
// the launch stays under 2048 waves and each slice keeps 32 chunks or more.
static int pair_slices(const MatmulArgs &args) {
  const int64_t units2 = (int64_t)args.batch * ((args.nruns + 1) / 2) * ((args.mtiles + 1) / 2);
  int sl = 1;
  while (sl < 8 && units2 * sl < 2048 && args.chunks >= 32 * 2 * sl) sl *= 2;
  return sl;
}
// Whether it launches 1024 waves or more; with fewer, one run a wave keeps more of them in flight.
static bool pairs_fill(const MatmulArgs &args) {
  const int64_t units2 = (int64_t)args.batch * ((args.nruns + 1) / 2) * ((args.mtiles + 1) / 2);
  return units2 * pair_slices(args) >= 1024;
}

template <class Kernel>
static void launch_sliced(Kernel kernel, const MatmulArgs &args, int64_t units, int slices, int slot_bytes,
                          int tile_bytes, hipStream_t s) {
  const int wpb = slices == 8 ? 8 : 4;
  const unsigned blocks = (unsigned)((units * slices + wpb - 1) / wpb);
  const size_t lds = (size_t)wpb * slot_bytes + (slices > 1 ? (size_t)wpb * tile_bytes : 0);
  kernel<<<blocks, wpb * 64, lds, s>>>(args, slices);
}

// Whether the output is one bf16 or fp32 matrix with contiguous rows whose byte offsets fit 32 bits: what the kernels
// that store without a program (the lean GEMV, skinny_lds_kernel) assume.
static bool plain_out(const MatmulArgs &args) {
  return (args.out.dtype == BT_BF16 || args.out.dtype == BT_FP32) && args.out.sc == 1 && args.out.sr >= 0 &&
         ((int64_t)(args.m - 1) * args.out.sr + args.n) * 4 < (1ll << 31);
}

template <int FMT, int DT, int MT, int NRW, int G>
static void launch_lds_g(const MatmulArgs &args, unsigned blocks, hipStream_t s) {
  const size_t lds = (size_t)16 * MT * (G * 64 + 8) * 2;  // A, G chunks a row
  const dim3 grid(blocks, (unsigned)((args.m + 16 * MT - 1) / (16 * MT)));  // y: blocks of 16 MT rows
  if (args.n_inst) skinny_lds_kernel<FMT, DT, MT, NRW, G, true><<<grid, 256, lds, s>>>(args);
  else skinny_lds_kernel<FMT, DT, MT, NRW, G, false><<<grid, 256, lds, s>>>(args);
}
template <int FMT, int DT, int MT, int NRW>
static void launch_lds_n(const MatmulArgs &args, unsigned blocks, hipStream_t s) {
  if (args.chunks <= 6) launch_lds_g<FMT, DT, MT, NRW, 6>(args, blocks, s);
  else if (args.chunks <= 9) launch_lds_g<FMT, DT, MT, NRW, 9>(args, blocks, s);
  else launch_lds_g<FMT, DT, MT, NRW, 12>(args, blocks, s);
}
template <int FMT, int DT>
static void launch_lds(const MatmulArgs &args, unsigned blocks, hipStream_t s) {
  launch_lds_n<FMT, DT, 1, 1>(args, blocks, s);
}

template <int FMT, int DT, int ROWS>
static void launch_x_rows(const MatmulArgs &args, hipStream_t s) {
  const unsigned blocks = (unsigned)((args.nruns + 3) / 4);
  XArgs x;
  x.b = args.b;
  x.a = args.a.ptr, x.a_sr = args.a.sr, x.out = args.out.ptr, x.out_sr = args.out.sr;
  x.m = args.m, x.k = args.k, x.n = args.n, x.chunks = args.chunks, x.nruns = args.nruns;
  x.out_bf16 = args.out.dtype == BT_BF16;
  if (args.chunks <= 4) gemv_x_kernel<FMT, DT, ROWS, 4><<<blocks, 256, 0, s>>>(x);
  else if (args.chunks <= 8) gemv_x_kernel<FMT, DT, ROWS, 8><<<blocks, 256, 0, s>>>(x);
  else if (args.chunks <= 9) gemv_x_kernel<FMT, DT, ROWS, 9><<<blocks, 256, 0, s>>>(x);
  else gemv_x_kernel<FMT, DT, ROWS, 12><<<blocks, 256, 0, s>>>(x);
}
template <int FMT, int DT>
static void launch_x(const MatmulArgs &args, hipStream_t s) {
  if constexpr (FMT != BT_BF16) {
    if (args.m == 1) launch_x_rows<FMT, DT, 1>(args, s);
    else launch_x_rows<FMT, DT, 4>(args, s);
  }
}

template <int FMT, int DT>
static void launch_dt(const MatmulArgs &args, unsigned blocks, hipStream_t s, bool vec) {
  const bool rows_contiguous = args.a.sc == 1 && (int64_t)args.k * 2 < (1ll << 31);
  const bool fits = (int64_t)(args.chunks + 12) * Tile<FMT>::bytes < (1ll << 32);  // voffsets of the last group
  // chunks in a group: the size that leaves the fewest unused slots in the last group, the larger on a tie
  const int group = args.chunks % 12 == 0 ? 12 : args.chunks % 9 == 0 ? 9 : args.chunks % 8 == 0 ? 8 : 12;
  if (args.m <= 4 && rows_contiguous && fits) {
    const int64_t units = (int64_t)args.batch * args.nruns;
    const int sl = choose_slices(units, args.chunks);
    // a plain product of one matrix, K unsliced: the lean kernels, group size fitted to K; anything else (a batch,
    // an epilogue program, slices): one kernel with all of them, groups of 8
    // (and a plain output)
    const bool lean = args.batch == 1 && !args.n_inst && sl == 1 && plain_out(args);
    if (FMT != BT_BF16 && lean && args.chunks <= 12 && args.k % 8 == 0 && args.a.ptr % 16 == 0 && args.a.sr % 8 == 0) {
      launch_x<FMT, DT>(args, s);
      return;
    }
    if (args.m == 1) {
      constexpr int SB = 64 * 2;  // slot bytes a chunk
      if (!lean && sl > 1) {
        if (args.n_inst) launch_sliced(gemv_kernel<FMT, DT, 1, 8, false, true, true>, args, units, sl, 8 * SB, 1024, s);
        else launch_sliced(gemv_kernel<FMT, DT, 1, 8, false, false, true>, args, units, sl, 8 * SB, 1024, s);
      } else if (!lean) {
        if (args.n_inst) launch_sliced(gemv_kernel<FMT, DT, 1, 12, false, true, false>, args, units, 1, 12 * SB, 0, s);
        else launch_sliced(gemv_kernel<FMT, DT, 1, 12, false, false, false>, args, units, 1, 12 * SB, 0, s);
      } else if (group == 9) launch_sliced(gemv_kernel<FMT, DT, 1, 9, true, false, false>, args, units, 1, 9 * SB, 0, s);
      else if (group == 8) launch_sliced(gemv_kernel<FMT, DT, 1, 8, true, false, false>, args, units, 1, 8 * SB, 0, s);
      else launch_sliced(gemv_kernel<FMT, DT, 1, 12, true, false, false>, args, units, 1, 12 * SB, 0, s);
    } else {
      constexpr int SB = 4 * 64 * 2;
      if (!lean && sl > 1) {
        if (args.n_inst) launch_sliced(gemv_kernel<FMT, DT, 4, 8, false, true, true>, args, units, sl, 8 * SB, 1024, s);
        else launch_sliced(gemv_kernel<FMT, DT, 4, 8, false, false, true>, args, units, sl, 8 * SB, 1024, s);
      } else if (!lean) {
        if (args.n_inst) launch_sliced(gemv_kernel<FMT, DT, 4, 12, false, true, false>, args, units, 1, 12 * SB, 0, s);
        else launch_sliced(gemv_kernel<FMT, DT, 4, 12, false, false, false>, args, units, 1, 12 * SB, 0, s);
      } else if (group == 9) launch_sliced(gemv_kernel<FMT, DT, 4, 9, true, false, false>, args, units, 1, 9 * SB, 0, s);
      else if (group == 8) launch_sliced(gemv_kernel<FMT, DT, 4, 8, true, false, false>, args, units, 1, 8 * SB, 0, s);
      else launch_sliced(gemv_kernel<FMT, DT, 4, 12, true, false, false>, args, units, 1, 12 * SB, 0, s);
    }
  } else if (FMT != BT_BF16 && vec && fits && args.batch == 1 && args.m <= 256 && args.chunks <= 12 &&
             ((int64_t)(args.m - 1) * args.a.sr + args.k) * 2 < (1ll << 31) && (args.n_inst || plain_out(args))) {
    // A staged in LDS once a block (16 rows a block, the blocks of a run side by side in y), a run a wave (more runs
    // a wave measured slower: fewer waves in flight). Two row tiles a wave, each run's weights decoded once for both,
    // measured 9.85 us for C1's 128 rows against 10.1 for the one-tile skinny kernel while the epilogue ran through the
    // program evaluator; with one-operation epilogues run straight, one tile a wave (twice the waves, half the chain
    // after the last byte) is 4.75 us against 6.41.
    const unsigned blocks = (unsigned)((args.nruns + 3) / 4);
    launch_lds<FMT, DT>(args, blocks, s);
  } else if (vec && fits && ((int64_t)31 * args.a.sr + 2 * (int64_t)args.k + 1024) * 2 < (1ll << 32)) {
    // two 16-row tiles a wave from 17 rows up; the waves of a run side by side. A short K (3-12 chunks) with many
    // rows: one tile a wave and all of K in one group of loads, so each wave makes one trip to memory.
    const bool one_trip = args.m > 16 && args.chunks > 2 && args.chunks <= 12;
    const bool two = args.m > 16 && !one_trip;
    const int64_t units = (int64_t)args.batch * args.nruns * (two ? (args.mtiles + 1) / 2 : args.mtiles);
    const int sl = one_trip ? 1 : choose_slices(units, args.chunks);
    const bool lean = args.batch == 1 && !args.n_inst && sl == 1 && !two && !one_trip;
    if (one_trip && args.chunks % 9 == 0) {
      if (args.n_inst) launch_sliced(skinny_vec_kernel<FMT, DT, 9, false, true, 1, false>, args, units, 1, 0, 0, s);
      else launch_sliced(skinny_vec_kernel<FMT, DT, 9, false, false, 1, false>, args, units, 1, 0, 0, s);
    } else if (one_trip) {
      if (args.n_inst) launch_sliced(skinny_vec_kernel<FMT, DT, 12, false, true, 1, false>, args, units, 1, 0, 0, s);
      else launch_sliced(skinny_vec_kernel<FMT, DT, 12, false, false, 1, false>, args, units, 1, 0, 0, s);
    } else if (two && args.chunks <= 2) {  // short K (a head's width): groups of 2
      if (args.n_inst) launch_sliced(skinny_vec_kernel<FMT, DT, 2, false, true, 2, true>, args, units, sl, 0, 2048, s);
      else launch_sliced(skinny_vec_kernel<FMT, DT, 2, false, false, 2, true>, args, units, sl, 0, 2048, s);
    } else if (two && pairs_fill(args)) {  // two runs a wave: half the units, each slice's partial 4 tiles
      const int64_t units2 = (int64_t)args.batch * ((args.nruns + 1) / 2) * ((args.mtiles + 1) / 2);
      const int sl2 = pair_slices(args);
      const int wpb = sl2 == 8 ? 8 : 4;
      const unsigned blocks = (unsigned)((units2 * sl2 + wpb - 1) / wpb);
      const size_t lds = sl2 > 1 ? (size_t)wpb * 4096 : 0;
      bt_operand res{};
      if (DT == BT_FP32 && residual_program(args, &res))
        skinny2_kernel<FMT, DT, 4, false, true, true><<<blocks, wpb * 64, lds, s>>>(args, sl2, res);
      else if (args.n_inst) skinny2_kernel<FMT, DT, 4, true, true><<<blocks, wpb * 64, lds, s>>>(args, sl2, res);
      else skinny2_kernel<FMT, DT, 4, false, true><<<blocks, wpb * 64, lds, s>>>(args, sl2, res);
    } else if (two) {
      if (args.n_inst) launch_sliced(skinny_vec_kernel<FMT, DT, 8, false, true, 2, true>, args, units, sl, 0, 2048, s);
      else launch_sliced(skinny_vec_kernel<FMT, DT, 8, false, false, 2, true>, args, units, sl, 0, 2048, s);
    } else if (!lean) {
      if (args.n_inst) launch_sliced(skinny_vec_kernel<FMT, DT, 8, false, true, 1, true>, args, units, sl, 0, 1024, s);
      else launch_sliced(skinny_vec_kernel<FMT, DT, 8, false, false, 1, true>, args, units, sl, 0, 1024, s);
    } else if (group == 9) {
      launch_sliced(skinny_vec_kernel<FMT, DT, 9, true, false, 1, false>, args, units, 1, 0, 0, s);
    } else {
      launch_sliced(skinny_vec_kernel<FMT, DT, 8, true, false, 1, false>, args, units, 1, 0, 0, s);
    }
  } else if (vec) skinny_kernel<FMT, DT, true><<<blocks, 256, 0, s>>>(args);
  else skinny_kernel<FMT, DT, false><<<blocks, 256, 0, s>>>(args);
}

// The split-K kernels for 5 to 32 rows of one A against a long K (more than 12 chunks, a multiple of 64): false
// when the product doesn't fit them or the runtime has no scratch for the partials (then the one-launch kernels run
// it). Splits of 16 chunks, or of 8 when 16 would leave 1024 blocks or more (measured the faster at those sizes).
template <int FMT, int MT>
static void launch_part_m(const MatmulArgs &args, int g, int groups, int splits, float *part, hipStream_t s) {
  const unsigned blocks = (unsigned)(groups * splits);
  const bool full = args.chunks % g == 0;  // every split whole: no chunk tests
  if (g == 16 && full) skinny_part_kernel<FMT, MT, 1, 16, true><<<blocks, 256, 0, s>>>(args, groups, part);
  else if (g == 16) skinny_part_kernel<FMT, MT, 1, 16><<<blocks, 256, 0, s>>>(args, groups, part);
  else if (full) skinny_part_kernel<FMT, MT, 1, 8, true><<<blocks, 256, 0, s>>>(args, groups, part);
  else skinny_part_kernel<FMT, MT, 1, 8><<<blocks, 256, 0, s>>>(args, groups, part);
}
static bool launch_parts(Runtime *r, const MatmulArgs &args, int fmt, bool swi) {
  const bt_operand &a = args.a;
  if (args.batch != 1 || args.m < 5 || args.m > 32 || args.k % 64 || args.chunks <= 12 ||
      a.sc != 1 || a.ptr % 16 || a.sr % 8 || ((int64_t)(args.m - 1) * a.sr + args.k) * 2 >= (1ll << 32) ||
      (int64_t)args.chunks * Tile<BT_BF16>::bytes >= (1ll << 32))
    return false;
  const int mt = args.m > 16 ? 2 : 1;
  // the splits depend on the shape alone, so every format of B sums in the same order: a block-float product stays
  // bit for bit the bf16 product of its values. One run a wave (two measured slower: fewer waves in flight).
  const int64_t groups16 = (args.nruns + 3) / 4;
  const int g = groups16 * ((args.chunks + 15) / 16) < 1024 ? 16 : 8, nrw = 1;
  const int groups = (args.nruns + 4 * nrw - 1) / (4 * nrw), splits = (args.chunks + g - 1) / g;
  float *part = (float *)runtime_scratch(r, (size_t)splits * 16 * mt * args.n * 4);
  if (!part) return false;
  if (fmt == BT_BF16 && mt == 2) launch_part_m<BT_BF16, 2>(args, g, groups, splits, part, r->stream);
  else if (fmt == BT_BF16) launch_part_m<BT_BF16, 1>(args, g, groups, splits, part, r->stream);
  else if (fmt == BT_BFP8 && mt == 2) launch_part_m<BT_BFP8, 2>(args, g, groups, splits, part, r->stream);
  else if (fmt == BT_BFP8) launch_part_m<BT_BFP8, 1>(args, g, groups, splits, part, r->stream);
  else if (mt == 2) launch_part_m<BT_BFP4, 2>(args, g, groups, splits, part, r->stream);
  else launch_part_m<BT_BFP4, 1>(args, g, groups, splits, part, r->stream);
  const int64_t outs = (int64_t)args.m * (swi ? args.n / 2 : args.n);
  const unsigned rb = (unsigned)((outs + 255) / 256);
  if (swi) parts_reduce_kernel<BT_BF16, true><<<rb, 256, 0, r->stream>>>(args, splits, 16 * mt, part);
  else if (args.prog.dtype == BT_FP32) parts_reduce_kernel<BT_FP32, false><<<rb, 256, 0, r->stream>>>(args, splits, 16 * mt, part);
  else parts_reduce_kernel<BT_BF16, false><<<rb, 256, 0, r->stream>>>(args, splits, 16 * mt, part);
  return true;
}

// The streaming kernels for 5 to 32 rows of one A with K a multiple of 256 and over 12 chunks (shorter K stages A
// whole in LDS, skinny_lds_kernel): false when the product doesn't fit them (then the split-K or one-launch kernels
// run it). Splits of whole stages, as many as bring a grid of 4-run blocks nearest 512 (two a CU, by LDS; bfp4's
// blocks of 8 runs then number about 256, one a CU), summed by parts_reduce_kernel in split order; one split stores
// the result through the epilogue itself.
template <int FMT, int MT>
static void launch_stream_m(const MatmulArgs &args, int epi, int dt, int splits, int stages, float *part,
                            hipStream_t s) {
  // groups of W runs (SiLU x up: W / 2 gate runs and their up runs), each over every split
  constexpr int W = Stream<FMT>::W;
  const int groups = (args.nruns + W - 1) / W;
  const unsigned blocks = (unsigned)(groups * splits), threads = 64 * W;
  if (epi == 0) skinny_stream_kernel<FMT, MT, 0, BT_FP32><<<blocks, threads, 0, s>>>(args, groups, stages, part);
  else if (epi == 2) skinny_stream_kernel<FMT, MT, 2, BT_BF16><<<blocks, threads, 0, s>>>(args, groups, stages, part);
  else if (dt == BT_FP32) skinny_stream_kernel<FMT, MT, 1, BT_FP32><<<blocks, threads, 0, s>>>(args, groups, stages, part);
  else skinny_stream_kernel<FMT, MT, 1, BT_BF16><<<blocks, threads, 0, s>>>(args, groups, stages, part);
}
// The streaming kernels' plan for a product: whether they take it, and its split of K.
struct StreamPlan {
  int mt, splits, stages;
};
static bool stream_plan(const MatmulArgs &args, StreamPlan *p) {
  const bt_operand &a = args.a;
  if (args.batch != 1 || args.m < 5 || args.m > 32 || args.k % 256 || args.chunks <= 12 || a.sc != 1 || a.ptr % 16 ||
      a.sr % 8 ||
      ((int64_t)(args.m - 1) * a.sr + args.k) * 2 >= (1ll << 32) ||
      (int64_t)args.chunks * Tile<BT_BF16>::bytes >= (1ll << 32))
    return false;
  const int total = args.chunks / 4;
  // the splits follow from groups of 4 runs whatever the kernel's block, so every format of B sums K alike; SiLU x up
  // takes those of the plain product of its shape (one split: each gate run beside its up run in a block; more:
  // partial sums per run)
  const int groups = (args.nruns + 3) / 4;
  int splits = 1;  // the divisor of the stages that brings the grid nearest 512 blocks
  for (int d = 1; d <= total; d++)
    if (total % d == 0 && std::abs(groups * d - 512) < std::abs(groups * splits - 512)) splits = d;
  p->mt = args.m > 16 ? 2 : 1;
  p->splits = splits;
  p->stages = total / splits;
  return true;
}
static void launch_stream_plan(const MatmulArgs &args, int fmt, int epi, int dt, const StreamPlan &p, float *part,
                               hipStream_t s) {
  if (fmt == BT_BF16 && p.mt == 2) launch_stream_m<BT_BF16, 2>(args, epi, dt, p.splits, p.stages, part, s);
  else if (fmt == BT_BF16) launch_stream_m<BT_BF16, 1>(args, epi, dt, p.splits, p.stages, part, s);
  else if (fmt == BT_BFP8 && p.mt == 2) launch_stream_m<BT_BFP8, 2>(args, epi, dt, p.splits, p.stages, part, s);
  else if (fmt == BT_BFP8) launch_stream_m<BT_BFP8, 1>(args, epi, dt, p.splits, p.stages, part, s);
  else if (p.mt == 2) launch_stream_m<BT_BFP4, 2>(args, epi, dt, p.splits, p.stages, part, s);
  else launch_stream_m<BT_BFP4, 1>(args, epi, dt, p.splits, p.stages, part, s);
}
static bool launch_stream(Runtime *r, const MatmulArgs &args, int fmt, bool swi) {
  StreamPlan p;
  if (!stream_plan(args, &p)) return false;
  float *part = nullptr;
  if (p.splits > 1) {
    part = (float *)runtime_scratch(r, (size_t)p.splits * 16 * p.mt * args.n * 4);
    if (!part) return false;
  }
  const int epi = p.splits > 1 ? 0 : swi ? 2 : 1, dt = args.prog.dtype == BT_FP32 ? BT_FP32 : BT_BF16;
  launch_stream_plan(args, fmt, epi, dt, p, part, r->stream);
  if (p.splits > 1) {
    const int64_t outs = (int64_t)args.m * (swi ? args.n / 2 : args.n);
    const unsigned rb = (unsigned)((outs + 255) / 256);
    const int splits = p.splits, rows = 16 * p.mt;
    if (swi) parts_reduce_kernel<BT_BF16, true><<<rb, 256, 0, r->stream>>>(args, splits, rows, part);
    else if (dt == BT_FP32) parts_reduce_kernel<BT_FP32, false><<<rb, 256, 0, r->stream>>>(args, splits, rows, part);
    else parts_reduce_kernel<BT_BF16, false><<<rb, 256, 0, r->stream>>>(args, splits, rows, part);
  }
  return true;
}

// The deepest pipeline (3 or 2 chunks) whose LDS fits the 160 KB of a CU.
template <int FMT, int DT, int WM, int WN> constexpr int gemm2_stages() {
  return Gemm2<FMT, DT, WM, WN, 3>::LDS <= 160 * 1024 ? 3 : 2;
}

template <int FMT, int DT, int WM, int WN>
static void launch_gemm(const MatmulArgs &args, hipStream_t s) {
  const int bm = 32 * WM, bn = 32 * WN;
  const int mb = (args.m + bm - 1) / bm, nb = (args.n + bn - 1) / bn;
  const unsigned blocks = (unsigned)((int64_t)mb * nb * args.batch);
  if (args.k % 64 == 0) {
    constexpr int S = gemm2_stages<FMT, DT, WM, WN>();
    static_assert(Gemm2<FMT, DT, WM, WN, S>::LDS <= 160 * 1024, "GEMM LDS");
    gemm2_kernel<FMT, DT, WM, WN, S><<<blocks, 256, 0, s>>>(args, mb, nb);
  } else if constexpr (WM == 4 && WN == 4) {
    gemm_kernel<FMT, DT, WM, WN><<<blocks, 256, 0, s>>>(args, mb, nb);
  }
}

// Whether the product's epilogue is nothing or a residual add, out = value + x with x an fp32 operand, as gemm3's
// direct fp32 store does it (the same fp32 add, so the same bits); res gets x (ptr 0 for none).
static bool residual_program(const MatmulArgs &args, bt_operand *res) {
  const bt_program &p = args.prog;
  if (args.out.dtype != BT_FP32 || p.dtype != BT_FP32) return false;
  if (p.n_inst == 0) {
    if (res) *res = bt_operand{};
    return true;
  }
  if (p.n_inst != 2 || p.n_inputs != 1 || p.in[0].dtype != BT_FP32) return false;
  const bt_inst &ld = p.inst[0], &add = p.inst[1];
  if (ld.op != BT_OP_LOAD || ld.a != 0 || ld.dst == 0 || add.op != BT_OP_ADD || p.result != add.dst) return false;
  if (!((add.a == 0 && add.b == ld.dst) || (add.a == ld.dst && add.b == 0))) return false;
  if (res) *res = p.in[0];
  return true;
}

// gemm3's block shape: 256 x 256, 256 x 192 or 128 x 256 (and 128 x 384 on bfp4 B), whichever fills the CUs' rounds
// best, a full round of the smaller blocks counted at 0.9, 0.85 and 0.95 of the speed of one of 256 x 256.
struct Gemm3Shape { int bm, bn; };
static Gemm3Shape gemm3_shape(const MatmulArgs &args, bool bfp4) {
  const Gemm3Shape opts[4] = {{256, 256}, {256, 192}, {128, 256}, {128, 384}};
  const double eff[4] = {1.0, 0.9, 0.85, 0.95};
  int best = 0;
  double score = -1.0;
  for (int o = 0; o < (bfp4 ? 4 : 3); o++) {
    const int64_t blocks = (int64_t)args.batch * ((args.m + opts[o].bm - 1) / opts[o].bm) * ((args.n + opts[o].bn - 1) / opts[o].bn);
    const double sc = eff[o] * (double)blocks / (double)((blocks + 255) / 256 * 256);
    if (sc > score + 1e-9) score = sc, best = o;
  }
  return opts[best];
}

// The block shape for a GEMM: the largest tile whose grid still keeps the chip's 256 CUs busy through its last round.
template <int FMT, int DT>
static void launch_gemm_dt(const MatmulArgs &args, hipStream_t s) {
  struct Option { int bm, bn; double eff; };  // eff: throughput of a full round relative to 256 x 256
  const Option opts[3] = {{256, 256, 1.0}, {256, 128, 0.85}, {128, 128, 0.7}};
  int best = 0;
  double score = -1.0;
  for (int o = 0; o < 3; o++) {
    // gemm3: bf16 B, K in 32s, bf16 out or fp32 out with at most a residual add
    const bool steps = FMT == BT_BF16 && args.k % 32 == 0 && (DT == BT_BF16 || residual_program(args, nullptr));
    if (o < 2 && (args.m <= 128 || (args.k % 64 && !(o == 0 && steps)))) continue;  // else the register-staged kernel
    if (o == 0 && DT == BT_FP32 && !steps) continue;  // gemm2's fp32 epilogue values would not fit in LDS
    const int64_t blocks = (int64_t)args.batch * ((args.m + opts[o].bm - 1) / opts[o].bm) * ((args.n + opts[o].bn - 1) / opts[o].bn);
    const int64_t rounds = (blocks + 255) / 256;
    const double sc = opts[o].eff * (double)blocks / (double)(rounds * 256);
    if (sc > score + 1e-9) score = sc, best = o;
  }
  if constexpr (FMT == BT_BF16 || FMT == BT_BFP4) {
    bt_operand res{};
    const bool fits = FMT == BT_BF16 ? args.m > 128 && args.k % 32 == 0
                                     : args.m >= 512 && args.k % 64 == 0 && (int64_t)args.chunks * args.nruns * 576 < (1ll << 32);
    if (fits && (DT == BT_BF16 || residual_program(args, &res))) {
      const Gemm3Shape sh = gemm3_shape(args, FMT == BT_BFP4);
      const int mb = (args.m + sh.bm - 1) / sh.bm, nb = (args.n + sh.bn - 1) / sh.bn;
      const unsigned blocks = (unsigned)((int64_t)mb * nb * args.batch);
      if constexpr (DT == BT_BF16) {
        if constexpr (FMT == BT_BFP4) {
          if (sh.bn == 384) {
            gemm3_kernel<FMT, DT, 4, GEMM_PLAIN, 128, 384><<<blocks, 512, 0, s>>>(args, mb, nb, bt_operand{});
            return;
          }
        }
        if (sh.bm == 128) gemm3_kernel<FMT, DT, 4, GEMM_PLAIN, 128><<<blocks, 512, 0, s>>>(args, mb, nb, bt_operand{});
        else if (sh.bn == 192) gemm3_kernel<FMT, DT, 4, GEMM_PLAIN, 256, 192><<<blocks, 512, 0, s>>>(args, mb, nb, bt_operand{});
        else gemm3_kernel<FMT, DT, 4><<<blocks, 512, 0, s>>>(args, mb, nb, bt_operand{});
      } else {
        if constexpr (FMT == BT_BFP4) {
          if (sh.bn == 384) {
            gemm3_kernel<FMT, DT, 4, GEMM_RES, 128, 384><<<blocks, 512, 0, s>>>(args, mb, nb, res);
            return;
          }
        }
        if (sh.bm == 128) gemm3_kernel<FMT, DT, 4, GEMM_RES, 128><<<blocks, 512, 0, s>>>(args, mb, nb, res);
        else if (sh.bn == 192) gemm3_kernel<FMT, DT, 4, GEMM_RES, 256, 192><<<blocks, 512, 0, s>>>(args, mb, nb, res);
        else gemm3_kernel<FMT, DT, 4, GEMM_RES><<<blocks, 512, 0, s>>>(args, mb, nb, res);
      }
      return;
    }
  }
  if constexpr (DT != BT_FP32) {
    if (best == 0) return launch_gemm<FMT, DT, 8, 8>(args, s);
  }
  if (best == 1) launch_gemm<FMT, DT, 8, 4>(args, s);
  else launch_gemm<FMT, DT, 4, 4>(args, s);
}

template <int FMT>
static void launch_skinny(const MatmulArgs &args, hipStream_t s) {
  const int64_t waves = (int64_t)args.batch * args.mtiles * args.nruns;
  const unsigned blocks = (unsigned)((waves + 3) / 4);
  const bt_operand &a = args.a;
  const bool vec = a.sc == 1 && a.sr % 8 == 0 && a.ptr % 16 == 0 && a.sb % 8 == 0 && args.k % 8 == 0;
  // many rows: the tiled GEMM, when A's rows are contiguous, aligned and within reach of one buffer resource. Up to
  // 256 rows, a product whose 128 x 128 blocks would fill fewer than half the CUs stays on the skinny kernel: its
  // waves (32 rows by one 16-column run each) spread the work over many more CUs, and the extra reads of B (one per
  // 32 rows) come from L2.
  const int64_t gemm_blocks = (int64_t)args.batch * ((args.m + 127) / 128) * ((args.n + 127) / 128);
  const bool gemm = vec && args.m > 64 && !(args.m <= 256 && gemm_blocks < 128) &&
                    ((int64_t)(args.m - 1) * a.sr + args.k) * 2 < (1ll << 32);
  if (gemm) {
    if (args.prog.dtype == BT_FP32) launch_gemm_dt<FMT, BT_FP32>(args, s);
    else launch_gemm_dt<FMT, BT_BF16>(args, s);
    return;
  }
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
  args.n_inst = args.prog.n_inst;
  args.out = *out;
  // A prefill-sized product with bfp8 B (or bfp4 with K not in whole chunks) and bf16 out: B unpacked once into bf16
  // tiles in the runtime's scratch (the same values bit for bit), then the bf16 GEMM. bfp4 B in whole chunks goes to
  // the same GEMM reading it as it is stored, decoded in registers.
  const bool bf16_out = out->dtype == BT_BF16 && (!epilogue || epilogue->dtype != BT_FP32);
  if (b_fmt != BT_BF16 && !(b_fmt == BT_BFP4 && k % 64 == 0) &&
      (bf16_out || residual_program(args, nullptr)) &&
      m >= 512 && k % 32 == 0 && a->sc == 1 && (int64_t)args.chunks * args.nruns * 2048 < (1ll << 32)) {
    const int64_t tiles = (int64_t)args.chunks * args.nruns * (b_batch > 1 ? b_batch : 1);
    void *bt16 = runtime_scratch(r, (size_t)tiles * 2048);
    if (bt16) {
      const unsigned blocks = (unsigned)((tiles + 3) / 4);
      if (b_fmt == BT_BFP8) tiles_bf16_kernel<BT_BFP8><<<blocks, 256, 0, r->stream>>>(args.b, (uint8_t *)bt16, tiles);
      else tiles_bf16_kernel<BT_BFP4><<<blocks, 256, 0, r->stream>>>(args.b, (uint8_t *)bt16, tiles);
      BT_LAUNCHED("matmul");
      args.b = (const uint8_t *)bt16;
      args.b_matrix_bytes = b_batch > 1 ? (int64_t)args.chunks * args.nruns * 2048 : 0;
      b_fmt = BT_BF16;
    }
  }
  if (launch_stream(r, args, b_fmt, false) || launch_parts(r, args, b_fmt, false)) {
    BT_LAUNCHED("matmul");
    return BT_OK;
  }
  if (b_fmt == BT_BF16) launch_skinny<BT_BF16>(args, r->stream);
  else if (b_fmt == BT_BFP8) launch_skinny<BT_BFP8>(args, r->stream);
  else launch_skinny<BT_BFP4>(args, r->stream);
  BT_LAUNCHED("matmul");
  return BT_OK;
}

template <int FMT, int G>
static void launch_row_g(const RowArgs &ra, const RopeTail *rope, int kind, size_t lds, unsigned blocks, hipStream_t s) {
  if (rope) gemv_row_kernel<FMT, G, BT_ROW_RMS, true><<<blocks, 256, lds, s>>>(ra, *rope);
  else if (kind == BT_ROW_RMS) gemv_row_kernel<FMT, G, BT_ROW_RMS, false><<<blocks, 256, lds, s>>>(ra, RopeTail{});
  else if (kind == BT_ROW_SWIGLU) gemv_row_kernel<FMT, G, BT_ROW_SWIGLU, false><<<blocks, 256, lds, s>>>(ra, RopeTail{});
  else gemv_row_kernel<FMT, G, BT_ROW_PLAIN, false><<<blocks, 256, lds, s>>>(ra, RopeTail{});
}

// rope: RoPE and the cache put fused (a kind of BT_ROW_RMS, at most 2 slices so that a block holds a pair of runs)
template <int FMT>
static void launch_row(RowArgs ra, int kind, hipStream_t s, const RopeTail *rope = nullptr) {
  // slices: up to 4 a run while each keeps 2 chunks or more and the launch stays under 1024 waves (a small model's
  // products, 36 to 192 runs, are chains of dependent steps whose waves fill few CUs: shorter slices on more waves
  // measured 4% faster a decode step than 9-chunk ones at K = 576)
  int sl = 1;
  while (sl < (rope ? 2 : 4) && ra.chunks / (2 * sl) >= 2 && (int64_t)ra.nruns * sl < 1024) sl *= 2;
  ra.slices = sl;
  const int c = (ra.chunks + sl - 1) / sl;  // chunks a slice
  const int g = c <= 6 ? 6 : c % 12 == 0 ? 12 : c % 9 == 0 ? 9 : c % 8 == 0 ? 8 : 12;
  const int k = ra.k, p0 = kind == BT_ROW_RMS ? (k * 4 + 1023) / 1024 : kind == BT_ROW_SWIGLU ? (k * 2 + 1023) / 1024 : 0;
  const int p1 = kind == BT_ROW_PLAIN ? 0 : (k * 2 + 1023) / 1024, prow = (ra.chunks * 128 + 1023) / 1024;
  const size_t lds = (size_t)(p0 + p1 + prow) * 1024 + 4 * g * 128 + 16 + 4 * 1024 + (rope ? 256 + 3 * 1024 : 0);
  const unsigned blocks = (unsigned)(((int64_t)ra.nruns * sl + 3) / 4);  // with RoPE nruns is even: whole pairs
  if (g == 9) launch_row_g<FMT, 9>(ra, rope, kind, lds, blocks, s);
  else if (g == 8) launch_row_g<FMT, 8>(ra, rope, kind, lds, blocks, s);
  else if (g == 6) launch_row_g<FMT, 6>(ra, rope, kind, lds, blocks, s);
  else launch_row_g<FMT, 12>(ra, rope, kind, lds, blocks, s);
}

static int row_args(const bt_row_args *args, RowArgs *ra) {
  if (!args) return fail(BT_EINVAL, "matmul_row needs its arguments");
  const bt_row_args &x = *args;
  if (x.kind != BT_ROW_PLAIN && x.kind != BT_ROW_RMS && x.kind != BT_ROW_SWIGLU)
    return fail(BT_EINVAL, "matmul_row prologue %d", x.kind);
  if (x.b_fmt != BT_BF16 && x.b_fmt != BT_BFP8 && x.b_fmt != BT_BFP4) return fail(BT_EINVAL, "B format %d", x.b_fmt);
  if (x.out_dtype != BT_BF16 && x.out_dtype != BT_FP32) return fail(BT_EINVAL, "matmul_row writes bf16 or fp32");
  if (x.k < 1 || x.k > 4096 || x.n < 1 || x.n >= (1 << 30))
    return fail(BT_EINVAL, "matmul_row shape k=%lld (1..4096), n=%lld", (long long)x.k, (long long)x.n);
  if (!x.a || !x.b || (x.kind == BT_ROW_RMS && !x.norm))
    return fail(BT_EINVAL, "matmul_row needs a, B and (for the norm) its weights");
  if (x.a % 16 || x.norm % 16 || x.b % 16 || (x.kind == BT_ROW_SWIGLU && x.k % 8))
    return fail(BT_EINVAL, "matmul_row reads its inputs 16 bytes at a time: a, norm and B 16-byte aligned%s",
                x.kind == BT_ROW_SWIGLU ? ", k a multiple of 8" : "");
  ra->b = (const uint8_t *)(uintptr_t)x.b;
  ra->a = (const uint8_t *)(uintptr_t)x.a;
  ra->norm = (const uint8_t *)(uintptr_t)x.norm;
  ra->res = (const float *)(uintptr_t)x.residual;
  ra->out = (uint8_t *)(uintptr_t)x.out;
  ra->chunks = (int32_t)((x.k + 63) / 64);
  ra->nruns = (int32_t)((x.n + 15) / 16);
  ra->k = (int32_t)x.k;
  ra->n = (int32_t)x.n;
  ra->out_dtype = x.out_dtype;
  ra->eps = x.eps;
  ra->slices = 1;
  ra->half_runs = 0;
  return BT_OK;
}

extern "C" int bt_matmul_row(bt_runtime *rt, const bt_row_args *args) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  RowArgs ra;
  if (int s = row_args(args, &ra)) return s;
  if (!args->out) return fail(BT_EINVAL, "matmul_row needs out");
  if (args->b_fmt == BT_BF16) launch_row<BT_BF16>(ra, args->kind, r->stream);
  else if (args->b_fmt == BT_BFP8) launch_row<BT_BFP8>(ra, args->kind, r->stream);
  else launch_row<BT_BFP4>(ra, args->kind, r->stream);
  BT_LAUNCHED("matmul_row");
  return BT_OK;
}

extern "C" int bt_matmul_row_rope(bt_runtime *rt, const bt_row_args *args, const bt_rope_args *rope) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  RowArgs ra;
  if (int s = row_args(args, &ra)) return s;
  if (!rope) return fail(BT_EINVAL, "matmul_row_rope needs RoPE's arguments");
  const bt_rope_args &p = *rope;
  if (args->kind != BT_ROW_RMS || args->out_dtype != BT_BF16 || args->residual)
    return fail(BT_EINVAL, "matmul_row_rope takes the RMSNorm prologue, a bf16 product and no residual");
  if (p.rows != 1 || p.heads < 1 || p.kv < 1 || p.head_dim < 32 || p.head_dim % 32 || p.cache_rows < 1 ||
      args->n != (int64_t)(p.heads + 2 * p.kv) * p.head_dim)
    return fail(BT_EINVAL, "matmul_row_rope: one row of %d + 2 x %d heads of %d (a multiple of 32) for n=%lld",
                p.heads, p.kv, p.head_dim, (long long)args->n);
  if (!p.cos || !p.sin || !p.q || !p.cache || !p.places) return fail(BT_EINVAL, "matmul_row_rope needs every buffer");
  RopeTail tail;
  tail.cos = (const uint16_t *)(uintptr_t)p.cos;
  tail.sin = (const uint16_t *)(uintptr_t)p.sin;
  tail.places = (const int32_t *)(uintptr_t)p.places;
  tail.q = (uint16_t *)(uintptr_t)p.q;
  tail.cache = (uint16_t *)(uintptr_t)p.cache;
  tail.vcache = (uint16_t *)(uintptr_t)p.vcache;
  tail.cache_sh = p.cache_sh, tail.cache_sr = p.cache_sr, tail.cache_tsh = p.cache_tsh, tail.cache_rows = p.cache_rows;
  tail.heads = p.heads, tail.kv = p.kv, tail.head_dim = p.head_dim;
  ra.half_runs = p.head_dim / 32;
  if (args->b_fmt == BT_BF16) launch_row<BT_BF16>(ra, args->kind, r->stream, &tail);
  else if (args->b_fmt == BT_BFP8) launch_row<BT_BFP8>(ra, args->kind, r->stream, &tail);
  else launch_row<BT_BFP4>(ra, args->kind, r->stream, &tail);
  BT_LAUNCHED("matmul_row_rope");
  return BT_OK;
}

extern "C" int bt_matmul_swiglu(bt_runtime *rt, const bt_operand *a, int b_fmt, uint64_t b, int64_t m, int64_t k,
                                int64_t n, const bt_operand *out) {
  Runtime *r;
  if (int st = enter(rt, &r)) return st;
  if (!a || !a->ptr || !b || !out || !out->ptr) return fail(BT_EINVAL, "matmul_swiglu needs A, B and out");
  if (b_fmt != BT_BF16 && b_fmt != BT_BFP8 && b_fmt != BT_BFP4) return fail(BT_EINVAL, "B format %d", b_fmt);
  if (m < 1 || k < 32 || k % 32 || n < 32 || n % 32 || m >= (1 << 30) || k >= (1 << 30) || n >= (1 << 30))
    return fail(BT_EINVAL, "matmul_swiglu shape %lld x %lld x %lld: k a multiple of 32, n of 32", (long long)m,
                (long long)k, (long long)n);
  if (a->dtype != BT_BF16 || a->sc != 1 || a->rep != 1 || a->cyc != 0 || a->ptr % 2)
    return fail(BT_EINVAL, "matmul_swiglu's A is bf16 with contiguous rows");
  if (out->dtype != BT_BF16 || out->sc != 1 || out->ptr % 16 || out->sr % 8 || out->rep != 1 || out->cyc != 0)
    return fail(BT_EINVAL, "matmul_swiglu's out is bf16, 16-byte aligned contiguous rows");
  if (b % 16) return fail(BT_EINVAL, "B's tiles must be 16-byte aligned");
  if (((m - 1) * a->sr + k) * 2 >= (1ll << 32)) return fail(BT_EINVAL, "matmul_swiglu's A must lie within 4 GB");
  MatmulArgs args;
  args.a = *a;
  args.b = (const uint8_t *)b;
  args.b_matrix_bytes = 0;
  args.batch = 1;
  args.m = (int32_t)m, args.k = (int32_t)k, args.n = (int32_t)n;
  args.chunks = (int32_t)((k + 63) / 64), args.nruns = (int32_t)(n / 16), args.mtiles = (int32_t)((m + 15) / 16);
  args.prog = bt_program{};
  args.prog.dtype = BT_BF16;
  args.n_inst = 0;
  args.out = *out;
  if ((int64_t)args.chunks * args.nruns * 2048 >= (1ll << 32)) return fail(BT_EINVAL, "matmul_swiglu's B is too large");
  const int mb = (int)((m + 255) / 256), nb = (int)((n / 2 + 127) / 128);
  const int64_t gemm_blocks = ((m + 127) / 128) * ((n + 127) / 128);
  if ((m <= 64 || (m <= 256 && gemm_blocks < 128)) && a->sr % 8 == 0 && a->ptr % 16 == 0 && ((31 * a->sr + 2 * k + 1024) * 2 < (1ll << 32))) {
    if (launch_stream(r, args, b_fmt, true) || launch_parts(r, args, b_fmt, true)) {
      BT_LAUNCHED("matmul_swiglu");
      return BT_OK;
    }
    // few rows: two 16-row tiles by a gate run and its up run a wave, reading B as it is stored (block floats
    // included), so no scratch is needed
    const int64_t units2 = (int64_t)(args.nruns / 2) * ((args.mtiles + 1) / 2);
    const int sl = pair_slices(args);
    const int wpb = sl == 8 ? 8 : 4;
    const unsigned blocks = (unsigned)((units2 * sl + wpb - 1) / wpb);
    const size_t lds = sl > 1 ? (size_t)wpb * 4096 : 0;
    if (b_fmt == BT_BF16)
      skinny2_kernel<BT_BF16, BT_BF16, 4, false, true, false, true><<<blocks, wpb * 64, lds, r->stream>>>(args, sl, bt_operand{});
    else if (b_fmt == BT_BFP8)
      skinny2_kernel<BT_BFP8, BT_BF16, 4, false, true, false, true><<<blocks, wpb * 64, lds, r->stream>>>(args, sl, bt_operand{});
    else skinny2_kernel<BT_BFP4, BT_BF16, 4, false, true, false, true><<<blocks, wpb * 64, lds, r->stream>>>(args, sl, bt_operand{});
    BT_LAUNCHED("matmul_swiglu");
    return BT_OK;
  }
  // bfp4 B with K in whole chunks: read as it is stored by the GEMM itself; other block floats unpacked once into bf16
  // tiles in the runtime's scratch
  const bool q4 = b_fmt == BT_BFP4 && k % 64 == 0;
  if (b_fmt != BT_BF16 && !q4) {
    const int64_t tiles = (int64_t)args.chunks * args.nruns;
    void *bt16 = runtime_scratch(r, (size_t)tiles * 2048);
    if (!bt16) return fail(BT_ESTATE, "matmul_swiglu: no scratch for B's bf16 tiles (inside a capture, or out of memory)");
    const unsigned blocks = (unsigned)((tiles + 3) / 4);
    if (b_fmt == BT_BFP8) tiles_bf16_kernel<BT_BFP8><<<blocks, 256, 0, r->stream>>>(args.b, (uint8_t *)bt16, tiles);
    else tiles_bf16_kernel<BT_BFP4><<<blocks, 256, 0, r->stream>>>(args.b, (uint8_t *)bt16, tiles);
    BT_LAUNCHED("matmul_swiglu");
    args.b = (const uint8_t *)bt16;
  }
  // One block a CU (the stages fill its LDS), so the blocks run in rounds of 256. When the last round would be at most
  // half full, the trailing block columns go to a second launch of 128-row blocks: twice the blocks at half the work
  // each, which fill one round that takes half the time (gate_up of 2048 Llama-3-8B tokens: 896 blocks, 3.5 rounds,
  // become 768 + 256 blocks of 128 rows, 3 rounds and a half-length one).
  int tail = 0;
  if (mb * nb > 256 && (mb * nb) % 256 != 0 && (mb * nb) % 256 <= 128) {
    const int mb128 = (int)((m + 127) / 128);
    for (int t = 1; t < nb && mb128 * t <= 256; t++)
      if ((mb * (nb - t)) % 256 == 0) { tail = t; break; }
  }
  const unsigned blocks = (unsigned)((int64_t)mb * (nb - tail));
  if (q4) gemm3_kernel<BT_BFP4, BT_BF16, 4, GEMM_SWIGLU><<<blocks, 512, 0, r->stream>>>(args, mb, nb - tail, bt_operand{}, 0);
  else gemm3_kernel<BT_BF16, BT_BF16, 4, GEMM_SWIGLU><<<blocks, 512, 0, r->stream>>>(args, mb, nb - tail, bt_operand{}, 0);
  BT_LAUNCHED("matmul_swiglu");
  if (tail) {
    const int mb128 = (int)((m + 127) / 128);
    const unsigned tb = (unsigned)((int64_t)mb128 * tail);
    if (q4)
      gemm3_kernel<BT_BFP4, BT_BF16, 4, GEMM_SWIGLU, 128><<<tb, 512, 0, r->stream>>>(args, mb128, tail, bt_operand{}, nb - tail);
    else
      gemm3_kernel<BT_BF16, BT_BF16, 4, GEMM_SWIGLU, 128><<<tb, 512, 0, r->stream>>>(args, mb128, tail, bt_operand{}, nb - tail);
    BT_LAUNCHED("matmul_swiglu");
  }
  return BT_OK;
}

// ---- the batched decode step's products with their neighbours fused: their split-K partial sums are summed by the
// kernel that consumes the product, so neither the product nor its reduction is stored or launched on its own ----

namespace bt {

// 8 neighbouring values of a product row as bf16 bits, two to a word: each the sum of its split-K partials in split
// order (p, p + stride, ...), rounded half up, as parts_reduce_kernel's bf16 store gives them.
__device__ __forceinline__ uint4 sum8_bf16(const float *p, int splits, int64_t stride) {
  float4 lo = *(const float4 *)p, hi = *(const float4 *)(p + 4);
#pragma unroll 4
  for (int s = 1; s < splits; s++) {
    const float4 a = *(const float4 *)(p + s * stride), b = *(const float4 *)(p + s * stride + 4);
    lo.x += a.x, lo.y += a.y, lo.z += a.z, lo.w += a.w;
    hi.x += b.x, hi.y += b.y, hi.z += b.z, hi.w += b.w;
  }
  return make_uint4(bf16_packed(lo.x) | bf16_packed(lo.y) << 16, bf16_packed(lo.z) | bf16_packed(lo.w) << 16,
                    bf16_packed(hi.x) | bf16_packed(hi.y) << 16, bf16_packed(hi.z) | bf16_packed(hi.w) << 16);
}

// bt_rope_put's 8-pair kernel on a product held as split-K partials (row i at part + i * n, split s stride apart).
__global__ void __launch_bounds__(256) rope_parts_kernel(const bt_rope_args a, const FastDiv hq, const FastDiv nh,
                                                         uint32_t threads, const float *part, int splits,
                                                         int64_t stride, int n) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= threads) return;
  const int half = a.head_dim / 2;
  const uint32_t th = fdiv(t, hq), ti = fdiv(th, nh);
  const int j = 8 * (int)(t - th * hq.d), hh = (int)(th - ti * nh.d), i = (int)ti;
  const float *x = part + (int64_t)i * n + (int64_t)hh * a.head_dim;
  const uint16_t *cs = (const uint16_t *)(uintptr_t)a.cos + (int64_t)i * a.cs_sr + (int64_t)hh * a.head_dim;
  const uint16_t *sn = (const uint16_t *)(uintptr_t)a.sin + (int64_t)i * a.cs_sr + (int64_t)hh * a.head_dim;
  const uint4 ca = *(const uint4 *)(cs + j), cb = *(const uint4 *)(cs + j + half);
  const uint4 sa = *(const uint4 *)(sn + j), sb = *(const uint4 *)(sn + j + half);
  const uint4 xa = sum8_bf16(x + j, splits, stride), xb = sum8_bf16(x + j + half, splits, stride);
  uint4 oa, ob;
  rope8(xa, xb, ca, cb, sa, sb, oa, ob);
  uint16_t *dst = rope_dst(a, i, hh);
  if (!dst) return;
  *(uint4 *)(dst + j) = oa;
  *(uint4 *)(dst + j + half) = ob;
}

// One row a block: x = residual + the product (its split-K partials summed in split order, then the residual added in
// fp32, as bt_matmul's residual epilogue does), written out, then bt_rms_rows' RMSNorm of x into h. Every load (the
// residual, each split's partials, the norm's weights) is issued before the first sum.
__global__ void __launch_bounds__(RMS_THREADS) residual_rms_kernel(const float *part, int splits, int64_t stride,
                                                                   int n, const float *res, int64_t res_sr, float *x,
                                                                   int64_t x_sr, const uint16_t *w, float eps,
                                                                   uint16_t *h, int64_t h_sr) {
  __shared__ float lds[RMS_THREADS / 64];
  constexpr int MAXS = 8;  // splits summed from registers; more are added in a second pass
  const int tid = threadIdx.x, m = blockIdx.x;
  const float *p = part + (int64_t)m * n;
  const float *rr = res + (int64_t)m * res_sr;
  float *xr = x + (int64_t)m * x_sr;
  float4 v[RMS_NV], s[RMS_NV];
  uint2 wv[RMS_NV];
#pragma unroll
  for (int i = 0; i < RMS_NV; i++) {
    const int c = (i * RMS_THREADS + tid) * 4;
    const bool in = c < n;
    v[i] = in ? *(const float4 *)(rr + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    wv[i] = in ? *(const uint2 *)(w + c) : make_uint2(0u, 0u);
    float4 q[MAXS];
#pragma unroll
    for (int k = 0; k < MAXS; k++)
      q[k] = in && k < splits ? *(const float4 *)(p + k * stride + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    s[i] = q[0];
#pragma unroll
    for (int k = 1; k < MAXS; k++)
      if (k < splits) s[i].x += q[k].x, s[i].y += q[k].y, s[i].z += q[k].z, s[i].w += q[k].w;
    for (int k = MAXS; k < splits; k++) {
      const float4 t = in ? *(const float4 *)(p + k * stride + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      s[i].x += t.x, s[i].y += t.y, s[i].z += t.z, s[i].w += t.w;
    }
  }
#pragma unroll
  for (int i = 0; i < RMS_NV; i++) {
    const int c = (i * RMS_THREADS + tid) * 4;
    v[i] = make_float4(v[i].x + s[i].x, v[i].y + s[i].y, v[i].z + s[i].z, v[i].w + s[i].w);
    if (c < n) *(float4 *)(xr + c) = v[i];
  }
#pragma unroll
  for (int i = 0; i < RMS_NV; i++) {
    v[i].x = round_packed(v[i].x), v[i].y = round_packed(v[i].y);
    v[i].z = round_packed(v[i].z), v[i].w = round_packed(v[i].w);
  }
  const float r = rms_scale(v, n, eps, lds);
  uint16_t *hr = h + (int64_t)m * h_sr;
#pragma unroll
  for (int i = 0; i < RMS_NV; i++) {
    const int c = (i * RMS_THREADS + tid) * 4;
    if (c < n) *(uint2 *)(hr + c) = rms_out(v[i], r, wv[i]);
  }
}

// The product's split-K partial sums in the runtime's scratch, by the streaming kernels (partials written even for
// one split), for a kernel that consumes them. Fails for a product those kernels don't take.
static int stream_partials(Runtime *r, const bt_operand *a, int b_fmt, uint64_t b, int64_t m, int64_t k, int64_t n,
                           const char *what, StreamPlan *p, float **part) {
  if (!a || !a->ptr || !b) return fail(BT_EINVAL, "%s needs A and B", what);
  if (a->dtype != BT_BF16 || a->rep != 1 || a->cyc != 0) return fail(BT_EINVAL, "%s: A is plain bf16 rows", what);
  if (b_fmt != BT_BF16 && b_fmt != BT_BFP8 && b_fmt != BT_BFP4) return fail(BT_EINVAL, "B format %d", b_fmt);
  if (b % 16) return fail(BT_EINVAL, "B's tiles must be 16-byte aligned");
  if (m < 1 || k < 1 || n < 1 || k > (1 << 30) || n > (1 << 30)) return fail(BT_EINVAL, "%s: shape", what);
  MatmulArgs args{};
  args.a = *a;
  args.b = (const uint8_t *)(uintptr_t)b;
  args.batch = 1, args.m = (int32_t)m, args.k = (int32_t)k, args.n = (int32_t)n;
  args.chunks = (int32_t)((k + 63) / 64);
  args.nruns = (int32_t)((n + 15) / 16);
  args.mtiles = (int32_t)((m + 15) / 16);
  args.b_matrix_bytes = 0;
  args.prog = bt_program{};
  args.prog.dtype = BT_FP32;
  args.n_inst = 0;
  args.out = bt_operand{};
  if (!stream_plan(args, p))
    return fail(BT_EINVAL, "%s takes 5 to 32 rows of A (contiguous, 16-byte aligned rows) and K a multiple of 256 "
                "over 768, not %lld x %lld", what, (long long)m, (long long)k);
  *part = (float *)runtime_scratch(r, (size_t)p->splits * 16 * p->mt * n * 4);
  if (!*part)
    return fail(BT_ESTATE, "%s: no room for the partial sums (inside a graph capture, make the call once before "
                "capturing so the runtime's scratch has grown)", what);
  launch_stream_plan(args, b_fmt, 0, BT_FP32, *p, *part, r->stream);
  BT_LAUNCHED(what);
  return BT_OK;
}

}  // namespace bt

extern "C" int bt_matmul_rope_put(bt_runtime *rt, const bt_operand *a, int b_fmt, uint64_t b, int64_t m, int64_t k,
                                  int64_t n, const bt_rope_args *rope) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!rope) return fail(BT_EINVAL, "matmul_rope_put needs the RoPE arguments");
  const bt_rope_args &ra = *rope;
  if (!ra.cos || !ra.sin || !ra.q || !ra.cache || !ra.places) return fail(BT_EINVAL, "matmul_rope_put needs every buffer");
  if (ra.rows != m || ra.heads < 1 || ra.kv < 1 || ra.head_dim < 16 || ra.head_dim % 16 || ra.cache_rows < 1 ||
      (int64_t)(ra.heads + 2 * ra.kv) * ra.head_dim != n)
    return fail(BT_EINVAL, "matmul_rope_put: %lld rows of %lld columns for %d rows of %d heads and %d key heads of %d "
                "(a multiple of 16)", (long long)m, (long long)n, ra.rows, ra.heads, ra.kv, ra.head_dim);
  if ((ra.cos | ra.sin | ra.q | ra.cache | ra.vcache) % 16 || (ra.cs_sr | ra.q_sr | ra.cache_sh | ra.cache_sr |
                                                               ra.cache_tsh) % 8)
    return fail(BT_EINVAL, "matmul_rope_put writes 16 bytes at a time: tables, q and caches 16-byte aligned, their "
                "strides multiples of 8");
  StreamPlan p;
  float *part;
  if (int s = stream_partials(r, a, b_fmt, b, m, k, n, "matmul_rope_put", &p, &part)) return s;
  const uint32_t t8 = (uint32_t)(m * (n / 2) / 8);
  rope_parts_kernel<<<(t8 + 255) / 256, 256, 0, r->stream>>>(ra, make_fastdiv((uint32_t)(ra.head_dim / 16)),
                                                             make_fastdiv((uint32_t)(ra.heads + 2 * ra.kv)), t8, part,
                                                             p.splits, (int64_t)16 * p.mt * n, (int)n);
  BT_LAUNCHED("matmul_rope_put");
  return BT_OK;
}

extern "C" int bt_matmul_residual_rms(bt_runtime *rt, const bt_operand *a, int b_fmt, uint64_t b, int64_t m,
                                      int64_t k, int64_t n, uint64_t residual, int64_t res_sr, uint64_t x, int64_t x_sr,
                                      uint64_t norm, float eps, uint64_t h, int64_t h_sr) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!residual || !x || !norm || !h) return fail(BT_EINVAL, "matmul_residual_rms needs the residual, x, norm and h");
  if (n > 4 * RMS_THREADS * RMS_NV || n % 4)
    return fail(BT_EINVAL, "matmul_residual_rms: rows of at most %d columns, a multiple of 4, not %lld",
                4 * RMS_THREADS * RMS_NV, (long long)n);
  if ((residual | x) % 16 || (res_sr | x_sr) % 4 || (norm | h) % 8 || h_sr % 4)
    return fail(BT_EINVAL, "matmul_residual_rms: fp32 rows 16-byte aligned, bf16 rows 8-byte aligned");
  StreamPlan p;
  float *part;
  if (int s = stream_partials(r, a, b_fmt, b, m, k, n, "matmul_residual_rms", &p, &part)) return s;
  residual_rms_kernel<<<(unsigned)m, RMS_THREADS, 0, r->stream>>>(part, p.splits, (int64_t)16 * p.mt * n, (int)n,
                                                          (const float *)(uintptr_t)residual, res_sr,
                                                          (float *)(uintptr_t)x, x_sr, (const uint16_t *)(uintptr_t)norm,
                                                          eps, (uint16_t *)(uintptr_t)h, h_sr);
  BT_LAUNCHED("matmul_residual_rms");
  return BT_OK;
}
