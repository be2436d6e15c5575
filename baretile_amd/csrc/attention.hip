// KV-cache attention on the matrix cores: out = softmax(q k^T + mask) v for every query row, the mask taken from each
// row's place (and a sliding window), maxima and sums in fp32, p packed to bf16 before it meets v, the output rounded
// to bf16 once.
//
// Semantics restated from the reference (in code of our own): tensor.py:797-841 (attend), kernels.py:794-1005
// (attention_kernel: fp32 row maxima, p = exp(s - max) packed to bf16, sum(p v) and sum(p) from that packed p in
// fp32, keys past a row's place never count), tensor.py:837-841 (parts combined by rescaling with e^(m_p - M)). Here
// the softmax is online: one sweep over the keys keeps each row's running maximum and rescales what has been summed,
// so K and V are each read once.
//
// The unit of work is a tile of 16 query "pairs" of one key head g: pair p = r * rep + h is query row r of head
// g * rep + h, so the rep heads that share g's keys share one pass over them (grouped-query attention). Scores are
// made transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_bf16: K rows and q rows are both contiguous along the head
// dimension, which is what the two operands want. In the result lane l holds keys 4(l/16)+i of a 16-key tile against
// pair l%16. P V then takes P as the first operand without moving it between lanes: for a 32-key step the lane's 8
// values are keys {4g..4g+3} of the step's first tile and {16+4g..16+4g+3} of its second (g = l/16), and the value
// operand is read from LDS in that same key order.
//
// Decode (at most 4 tiles, 64 pairs, per key head): the block's 4 waves split the keys of one tile, 64 at a time, and
// combine their running sums in LDS at the end. Long caches are split further into parts, each a run of the tile's
// visible keys, written as fp32 partial sums to scratch and combined by a second kernel; from 5 to 16 blocks of keys a
// part is one block, folded by a block of one wave whose state is the part's partial sum. Prefill: the block's waves take 4 consecutive tiles and share each block
// of 64 keys and values through LDS, double-buffered.
#include "common.h"
#include "lds_load.h"
#include <mutex>
#include <algorithm>
#include <type_traits>

namespace bt {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int KB = 64;  // keys per block
// Cache policy of the decode kernels' K and V loads: sc1 | nt, streamed (each byte is read once a step, and a
// cache-allocating read of hundreds of MB only evicts): 537 MB of bf16 K and V in 84 us against 97 with the default
// policy. Prefill keeps the default: its blocks read each key block once per query tile.
constexpr int DEC_POL = 18;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t attn_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Orders a wave's LDS writes before its later reads by other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const uint4 v = make_uint4(a, b, c, d);
  return *(const bf16x8 *)&v;
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4 &v) { return as_bf16x8(v.x, v.y, v.z, v.w); }

// Where a key head's K (or V) rows come from: bf16 (one buffer), or a block-float cache's value and exponent planes.
// Offsets are in values; rows past `span` values read as zeros.
struct KvSrc {
  __amdgpu_buffer_rsrc_t val, exp;
};
template <int KF>
__device__ __forceinline__ KvSrc kv_src(uint64_t vals, uint64_t exps, int64_t head, int64_t span) {
  KvSrc s;
  if (KF == BT_BF16) {
    s.val = attn_rsrc((const uint16_t *)(uintptr_t)vals + head, (uint32_t)(span * 2));
    s.exp = s.val;
  } else {
    const int shift = KF == BT_BFP8 ? 0 : 1;  // value index -> byte of its q
    s.val = attn_rsrc((const uint8_t *)(uintptr_t)vals + (head >> shift), (uint32_t)(span >> shift));
    s.exp = attn_rsrc((const uint8_t *)(uintptr_t)exps + head / 16, (uint32_t)(span / 16));
  }
  return s;
}
// 8 block-float values sharing exponent byte x, as bf16 pairs, exactly as the unpacker decodes them: q (bfp8: 8
// signed bytes in lo, hi; bfp4: 8 signed nibbles in lo) times 2^(x - 133) (bfp8) or 2^(x - 129) (bfp4). For x in
// 7..254 that product is a normal float whose top half is the exact bf16 (a 7-bit magnitude times a power of two);
// other x go through the unpacker's modular exponent rule value by value.
template <int KF>
__device__ __forceinline__ uint4 kv_decode8(uint32_t lo, uint32_t hi, uint32_t x) {
  int q[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    if (KF == BT_BFP8) q[i] = (int)(int8_t)(((i < 4 ? lo : hi) >> (8 * (i % 4))) & 255u);
    else q[i] = ((int)(lo << (28 - 4 * i))) >> 28;
  }
  uint32_t w[4];
  if (x >= 7 && x <= 254) {
    const float sc = __uint_as_float((x - (KF == BT_BFP8 ? 133u : 129u) + 127u) << 23);
#pragma unroll
    for (int p = 0; p < 4; p++)
      w[p] = (__float_as_uint((float)q[2 * p] * sc) >> 16) | (__float_as_uint((float)q[2 * p + 1] * sc) & 0xFFFF0000u);
  } else {
#pragma unroll
    for (int p = 0; p < 4; p++)
      w[p] = unpacked_bits(KF == BT_BFP8 ? q[2 * p] : q[2 * p] * 16, x) |
             unpacked_bits(KF == BT_BFP8 ? q[2 * p + 1] : q[2 * p + 1] * 16, x) << 16;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}
// The value bytes of 8 values from value e on (e a multiple of 8): bfp8 two words, bfp4 one.
template <int KF, int POL = 0>
__device__ __forceinline__ uint2 kv_raw8(const KvSrc &s, uint32_t e) {
  if (KF == BT_BFP8) {
    const auto q = __builtin_amdgcn_raw_buffer_load_b64(s.val, e, 0, POL);
    return make_uint2(q[0], q[1]);
  }
  return make_uint2(__builtin_amdgcn_raw_buffer_load_b32(s.val, e / 2, 0, POL), 0u);
}
// 8 values from value e on (e a multiple of 8), as bf16 pairs; a block float's exponent byte read at e / 16.
template <int KF>
__device__ __forceinline__ uint4 kv_load8(const KvSrc &s, uint32_t e) {
  if (KF == BT_BF16) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(s.val, e * 2, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
  }
  const uint32_t x = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(s.exp, e / 16, 0, 0);
  const uint2 q = kv_raw8<KF>(s, e);
  return kv_decode8<KF>(q.x, q.y, x);
}
// A row's HD / 16 exponent bytes (row start e, a multiple of 16), for decoding its pieces one by one.
template <int KF, int HD, int POL = 0>
__device__ __forceinline__ uint2 kv_row_exps(const KvSrc &s, uint32_t e) {
  if (KF == BT_BF16) return make_uint2(0, 0);
  if (HD == 64) return make_uint2(__builtin_amdgcn_raw_buffer_load_b32(s.exp, e / 16, 0, POL), 0u);
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(s.exp, e / 16, 0, POL);
  return make_uint2(v[0], v[1]);
}

// 8 values' bytes as loaded, decoded later (kv_value8): bf16 four words, bfp8 two, bfp4 one.
template <int KF> struct Raw8 {
  uint32_t w[KF == BT_BF16 ? 4 : KF == BT_BFP8 ? 2 : 1];
};
template <int KF, int POL = 0>
__device__ __forceinline__ Raw8<KF> kv_fetch8(const KvSrc &s, uint32_t e) {
  Raw8<KF> r;
  if constexpr (KF == BT_BF16) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(s.val, e * 2, 0, POL);
#pragma unroll
    for (int i = 0; i < 4; i++) r.w[i] = v[i];
  } else {
    const uint2 q = kv_raw8<KF, POL>(s, e);
    r.w[0] = q.x;
    if constexpr (KF == BT_BFP8) r.w[1] = q.y;
  }
  return r;
}
template <int KF>
__device__ __forceinline__ uint4 kv_value8(const Raw8<KF> &r, uint32_t x) {
  if constexpr (KF == BT_BF16) return make_uint4(r.w[0], r.w[1], r.w[2], r.w[3]);
  else if constexpr (KF == BT_BFP8) return kv_decode8<KF>(r.w[0], r.w[1], x);
  else return kv_decode8<KF>(r.w[0], 0u, x);
}
// A block-float value's exponent byte (value e); 0 for bf16, which has none.
template <int KF, int POL = 0>
__device__ __forceinline__ uint32_t kv_exp8(const KvSrc &s, uint32_t e) {
  if constexpr (KF == BT_BF16) return 0u;
  else return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(s.exp, e / 16, 0, POL);
}

// x of lane l combined with lanes l ^ 16 and l ^ 32 (hence l ^ 48): the matrix-core layout's 4 lane groups that hold
// one column. VALU lane swaps (v_permlane16_swap / v_permlane32_swap with both operands x: the pair comes back as
// x[l] and x[l ^ 16], in one order or the other), where a shuffle would take a trip through LDS; max and the sum are
// commutative, so the result is the shuffles' to the bit.
__device__ __forceinline__ float max_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// A lane's pair: which query row it is, which keys it sees, where its q and output rows are.
struct Pair {
  int lo, hi;  // visible keys lo..hi (empty when lo > hi)
  int64_t q, o;  // element offsets of the pair's q and output rows
  bool valid;
};

__device__ __forceinline__ Pair pair_of(const bt_attention_args &a, int kvh, int p) {
  Pair x;
  const int np = a.rep * a.rows;
  x.valid = p < np;
  const int pp = x.valid ? p : 0, h = pp % a.rep, r = pp / a.rep, e = kvh * a.rep + h;
  const int place = ((const int32_t *)a.places)[(int64_t)e * a.places_sh + r];
  x.lo = a.window > 0 ? max(0, place - a.window + 1) : 0;
  if (a.firsts) x.lo = max(x.lo, ((const int32_t *)a.firsts)[(int64_t)e * a.firsts_sh + r]);
  x.hi = min(place, a.keys - 1);
  if (!x.valid) x.lo = 1, x.hi = 0;
  x.q = (int64_t)e * a.q_sh + (int64_t)r * a.q_sr;
  x.o = (int64_t)e * a.o_sh + (int64_t)r * a.o_sr;
  return x;
}

// The running state of one wave's tile: maximum and sum of packed p per pair (every lane holds its pair l%16's), and
// the unnormalized output O in the matrix-core layout (lane l: pairs 4(l/16)+i, column 16c + l%16).
template <int HD> struct State {
  float m, l;
  f32x4 o[HD / 16];
};

// One block of 64 keys starting at kb. kf: the K operand fragments (lane l: key kb + 16kt + l%16,
// dims 32kk + 8(l/16) .. +8). vl: the block's values in LDS, row-major with a row stride of VS halfwords.
// block_scores makes the block's scores S^T = K Q^T; fold_scores folds them and the values into st.
template <int HD>
__device__ __forceinline__ void block_scores(f32x4 (&s)[4], const bf16x8 (&kf)[4][HD / 32], const bf16x8 (&qf)[HD / 32]) {
#pragma unroll
  for (int kt = 0; kt < 4; kt++) {
    s[kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk++) s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kt][kk], qf[kk], s[kt], 0, 0, 0);
  }
}
// fresh (wave-uniform): st is still the initial state, whose zero O needs no rescale (skipping it gives the same bits)
template <int HD, int VS>
__device__ __forceinline__ void fold_scores(State<HD> &st, f32x4 (&s)[4], const uint16_t *vl, int kb, const Pair &pr,
                                            int lane, bool fresh) {
  const int g = lane >> 4, n = lane & 15;
  float mx = -__builtin_inff();
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int j = kb + 16 * kt + 4 * g + i;
      if (j < pr.lo || j > pr.hi) s[kt][i] = -__builtin_inff();
      mx = fmaxf(mx, s[kt][i]);
    }
  mx = max_groups(mx);
  const float mn = fmaxf(st.m, mx);
  const bool none = mn == -__builtin_inff();  // no key of the pair seen yet
  const float scale = none ? 1.0f : __expf(st.m - mn);
  uint32_t pb[4][4];
  float sum = 0.0f;
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float p = none ? 0.0f : __expf(s[kt][i] - mn);
      pb[kt][i] = bf16_packed(p);
      sum += bf16_value(pb[kt][i]);
    }
  sum = sum_groups(sum);
  st.l = st.l * scale + sum;
  st.m = mn;
  if (!fresh) {
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sc[i] = __shfl(scale, 4 * g + i, 64);
#pragma unroll
    for (int c = 0; c < HD / 16; c++)
#pragma unroll
      for (int i = 0; i < 4; i++) st.o[c][i] *= sc[i];
  }
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    const bf16x8 pa = as_bf16x8(pb[2 * ks][0] | pb[2 * ks][1] << 16, pb[2 * ks][2] | pb[2 * ks][3] << 16,
                                pb[2 * ks + 1][0] | pb[2 * ks + 1][1] << 16, pb[2 * ks + 1][2] | pb[2 * ks + 1][3] << 16);
    // transposing reads (ds_read_b64_tr_b16) of the row-major values: lane n of a 16-lane group addresses key
    // 32ks + 4g + n / 4 (and 16 further), dims 16c + 4 (n % 4) .. + 3, and is handed the group's 4 keys of dim
    // 16c + n, the operand's keys 4g .. 4g + 3 (then 16 + 4g ..) in order: two reads where 16-bit gathers took eight
    const uint16_t *rows = vl + (32 * ks + 4 * g + n / 4) * VS + 4 * (n & 3);
#pragma unroll
    for (int c = 0; c < HD / 16; c++) {
      typedef short s16x4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
      const s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(rows + 16 * c));
      const s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(rows + 16 * VS + 16 * c));
      const uint2 a0 = __builtin_bit_cast(uint2, r0), a1 = __builtin_bit_cast(uint2, r1);
      st.o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, as_bf16x8(a0.x, a0.y, a1.x, a1.y), st.o[c], 0, 0, 0);
    }
  }
}

// pair_of with the Q^T operand fragments of the lane's pair (dims 32kk + 8(l/16) .. +8, zeros for a pair past the
// last), every load issued before any is used: the place, the first key, the q row, as global loads from addresses
// that are always valid (a pair past the last reads pair 0's and is then marked empty, a call without firsts reads the
// place twice). So a kernel's prologue is one trip to memory rather than a chain of three.
template <int HD>
__device__ __forceinline__ Pair pair_q(const bt_attention_args &a, int kvh, int p, int lane, bf16x8 (&qf)[HD / 32]) {
  Pair x;
  const int np = a.rep * a.rows;
  x.valid = p < np;
  const int pp = x.valid ? p : 0, h = pp % a.rep, r = pp / a.rep, e = kvh * a.rep + h;
  x.q = (int64_t)e * a.q_sh + (int64_t)r * a.q_sr;
  x.o = (int64_t)e * a.o_sh + (int64_t)r * a.o_sr;
  const int32_t *pl = (const int32_t *)a.places + (int64_t)e * a.places_sh + r;
  const int32_t *fp = a.firsts ? (const int32_t *)a.firsts + (int64_t)e * a.firsts_sh + r : pl;
  const uint16_t *q = (const uint16_t *)a.q + x.q + 8 * (lane >> 4);
  const int place = gload(pl), first = gload(fp);
  uint4 v[HD / 32];
#pragma unroll
  for (int kk = 0; kk < HD / 32; kk++) v[kk] = gload((const uint4 *)(q + 32 * kk));
  x.lo = a.window > 0 ? max(0, place - a.window + 1) : 0;
  x.lo = max(x.lo, a.firsts ? first : 0);
  x.hi = min(place, a.keys - 1);
  if (!x.valid) x.lo = 1, x.hi = 0;
#pragma unroll
  for (int kk = 0; kk < HD / 32; kk++) {
    const uint4 w = x.valid ? v[kk] : make_uint4(0, 0, 0, 0);
    qf[kk] = *(const bf16x8 *)&w;
  }
  return x;
}

// The smallest first key and largest last key over the 16 pairs of the wave's tile (each 16-lane row holds them
// all): min and max over a row by DPP lane moves (swaps within quads, then the half-row and row mirrors), which take
// no trip through LDS; min and max are exact, so the order doesn't matter.
__device__ __forceinline__ int row_min(int x) {
  x = min(x, __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false));   // quad_perm [1, 0, 3, 2]
  x = min(x, __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false));   // quad_perm [2, 3, 0, 1]
  x = min(x, __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false));  // row_half_mirror
  return min(x, __builtin_amdgcn_update_dpp(x, x, 0x140, 0xF, 0xF, false));  // row_mirror
}
__device__ __forceinline__ int row_max(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false));
  return max(x, __builtin_amdgcn_update_dpp(x, x, 0x140, 0xF, 0xF, false));
}
__device__ __forceinline__ void tile_range(const Pair &pr, int &lo, int &hi) {
  lo = __builtin_amdgcn_readfirstlane(row_min(pr.lo <= pr.hi ? pr.lo : 0x7FFFFFFF));
  hi = __builtin_amdgcn_readfirstlane(row_max(pr.lo <= pr.hi ? pr.hi : -1));
}

// Floats of one tile's partial result: m[16], l[16], then O[16][HD].
template <int HD> constexpr int partial_floats() { return 32 + 16 * HD; }

// Writes the block's combined result for its tile: the bf16 output of each valid pair (parts == 1), or the partial
// result into scratch. parts: the wave states in LDS `ws` (4 waves, partial_floats each).
template <int HD>
__device__ __forceinline__ void finish_tile(const bt_attention_args &a, const float *ws, int nwaves, int kvh, int t,
                                            int part, int parts, int tiles, float *scratch) {
  constexpr int PF = partial_floats<HD>();
  const int tid = threadIdx.x;
  // each thread: one pair and HD / 16 columns
  const int pr_i = tid / 16, c0 = tid % 16;
  float M = -__builtin_inff();
  for (int w = 0; w < nwaves; w++) M = fmaxf(M, ws[w * PF + pr_i]);
  float wgt[4], L = 0.0f;
  for (int w = 0; w < nwaves; w++) {
    wgt[w] = M == -__builtin_inff() ? 0.0f : __expf(ws[w * PF + pr_i] - M);
    L += wgt[w] * ws[w * PF + 16 + pr_i];
  }
  float o[HD / 16];
#pragma unroll
  for (int c = 0; c < HD / 16; c++) {
    float v = 0.0f;
    for (int w = 0; w < nwaves; w++) v += wgt[w] * ws[w * PF + 32 + pr_i * HD + c0 + 16 * c];
    o[c] = v;
  }
  if (parts == 1) {
    const Pair pr = pair_of(a, kvh, 16 * t + pr_i);
    if (!pr.valid) return;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    uint16_t *out = (uint16_t *)a.out + pr.o;
#pragma unroll
    for (int c = 0; c < HD / 16; c++) out[c0 + 16 * c] = (uint16_t)bf16_packed(o[c] * inv);
  } else {
    float *dst = scratch + ((int64_t)(kvh * tiles + t) * parts + part) * PF;
    if (c0 == 0) dst[pr_i] = M, dst[16 + pr_i] = L;
#pragma unroll
    for (int c = 0; c < HD / 16; c++) dst[32 + pr_i * HD + c0 + 16 * c] = o[c];
  }
}

// Writes a wave's state into its LDS partial: m and l by lanes 0..15, O from the matrix-core layout.
template <int HD>
__device__ __forceinline__ void store_state(float *ws, const State<HD> &st, int lane) {
  const int g = lane >> 4, n = lane & 15;
  if (lane < 16) ws[n] = st.m, ws[16 + n] = st.l;
#pragma unroll
  for (int c = 0; c < HD / 16; c++)
#pragma unroll
    for (int i = 0; i < 4; i++) ws[32 + (4 * g + i) * HD + 16 * c + n] = st.o[c][i];
}

// Decode: block (kvh, t, part). The tile's visible keys, from its smallest first to its largest last, are cut into
// `parts` runs of whole 64-key blocks; the 4 waves take the part's blocks in turn. A wave's loads run a block ahead:
// the next block's keys and values are fetched once the current scores are made (the current values are in LDS by
// then), so they arrive while the current block is folded. Block-float bytes are held as loaded and decoded where they are
// used. WIDE (block floats): every key row's exponents sit at a multiple of their HD / 16 bytes, one load a row.
// Two waves a SIMD at least: the block-float caches' decoding would otherwise take enough registers to leave one.
template <int HD, int KF, bool WIDE> struct KeyBytes {
  static constexpr int XW = KF == BT_BF16 ? 1 : WIDE ? (HD == 64 ? 1 : 2) : HD / 32;
  Raw8<KF> q[4][HD / 32];
  uint32_t x[4][XW];
};
template <int HD, int KF, bool WIDE>
__device__ __forceinline__ void fetch_keys(KeyBytes<HD, KF, WIDE> &kb_, const KvSrc &kr, int kb, int64_t k_sr, int lane) {
  const int g = lane >> 4, n = lane & 15;
#pragma unroll
  for (int kt = 0; kt < 4; kt++) {
    const uint32_t row = (uint32_t)((int64_t)(kb + 16 * kt + n) * k_sr);
    if constexpr (KF != BT_BF16 && WIDE) {
      const uint2 xs = kv_row_exps<KF, HD, DEC_POL>(kr, row);
      kb_.x[kt][0] = xs.x;
      if constexpr (HD != 64) kb_.x[kt][1] = xs.y;
    }
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk++) {
      kb_.q[kt][kk] = kv_fetch8<KF, DEC_POL>(kr, row + 32 * kk + 8 * g);
      if constexpr (KF != BT_BF16 && !WIDE) kb_.x[kt][kk] = kv_exp8<KF, DEC_POL>(kr, row + 32 * kk + 8 * g);
    }
  }
}
template <int HD, int KF, bool WIDE>
__device__ __forceinline__ void decode_keys(bf16x8 (&kf)[4][HD / 32], const KeyBytes<HD, KF, WIDE> &kb_, int lane) {
  const int g = lane >> 4;
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk++) {
      uint32_t x = 0;
      if constexpr (KF != BT_BF16 && WIDE) {
        const int run = 2 * kk + g / 2;  // the piece's run of 16 in its row
        x = ((run < 4 ? kb_.x[kt][0] : kb_.x[kt][KeyBytes<HD, KF, WIDE>::XW - 1]) >> (8 * (run % 4))) & 255u;
      } else if constexpr (KF != BT_BF16) {
        x = kb_.x[kt][kk];
      }
      kf[kt][kk] = as_bf16x8(kv_value8<KF>(kb_.q[kt][kk], x));
    }
}

template <int HD, int KF, bool WIDE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
attention_decode_kernel(const bt_attention_args a, int tiles, int parts, float *scratch) {
  // halfwords of one wave's value block: rows of HD + 16, so that the 8 rows a transposing read's pass of 32 lanes
  // addresses (8 dwords each) start 8 banks apart
  constexpr int VS = HD + 16, VR = KB * VS;
  constexpr int PF = partial_floats<HD>();
  static_assert(4 * PF * 4 <= 4 * VR * 2, "the wave partials fit in the value blocks' LDS");
  __shared__ __attribute__((aligned(16))) uint16_t lds[4 * VR];
  const int lane = threadIdx.x & 63, n = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int bid = blockIdx.x;
  const int part = bid % parts;
  bid /= parts;
  const int t = bid % tiles, kvh = bid / tiles;
  bf16x8 qf[HD / 32];
  const Pair pr = pair_q<HD>(a, kvh, 16 * t + n, lane, qf);
  int lo, hi;
  tile_range(pr, lo, hi);
  const int start = lo & ~(KB - 1), nblk = hi >= lo ? (hi - start) / KB + 1 : 0, per = (nblk + parts - 1) / parts;
  const int first = start + part * per * KB, last = min(first + per * KB - 1, hi);
  State<HD> st;
  st.m = -__builtin_inff(), st.l = 0.0f;
#pragma unroll
  for (int c = 0; c < HD / 16; c++) st.o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const KvSrc kr = kv_src<KF>(a.k, a.k_exps, (int64_t)kvh * a.k_sh, (int64_t)(a.keys - 1) * a.k_sr + HD);
  const KvSrc vr = kv_src<KF>(a.v, a.v_exps, (int64_t)kvh * a.v_sh, (int64_t)(a.keys - 1) * a.v_sr + HD);
  uint16_t *vl = lds + wib * VR;
  constexpr int RPI = 64 * 8 / HD, VI = KB / RPI;  // value rows one load instruction covers; loads a block
  const int vrow = lane / (HD / 8), vcol = lane % (HD / 8) * 8;
  KeyBytes<HD, KF, WIDE> kbytes;
  Raw8<KF> vq[VI];
  uint32_t vx[VI];
  auto fetch_values = [&](int kb) {
#pragma unroll
    for (int i = 0; i < VI; i++) {
      const uint32_t e = (uint32_t)((int64_t)(kb + vrow + RPI * i) * a.v_sr + vcol);
      vq[i] = kv_fetch8<KF, DEC_POL>(vr, e);
      vx[i] = kv_exp8<KF, DEC_POL>(vr, e);
    }
  };
  int kb = first + KB * wib;
  if (kb <= last) {
    fetch_values(kb);  // values first, as in the loop: a block's values are waited for before its keys
    fetch_keys<HD, KF, WIDE>(kbytes, kr, kb, a.k_sr, lane);
  }
  // a block's values go out as soon as the previous block's are in LDS (B = 8 at 1024 keys 13.1 -> 10.9 us, B = 32 at
  // 4096 keys 95.5 -> 90-93 us), its keys once the previous scores are made; the last block's step is its own copy,
  // so the loop's fetches carry no condition.
  bool fresh = true;  // the wave's first block
  auto step = [&](int kb, auto more) {
    constexpr bool MORE = decltype(more)::value;
    wave_lds_sync();  // the previous block's reads of vl are done
#pragma unroll
    for (int i = 0; i < VI; i++) *(uint4 *)(vl + (vrow + RPI * i) * VS + vcol) = kv_value8<KF>(vq[i], vx[i]);
    if constexpr (MORE) fetch_values(kb + 4 * KB);
    wave_lds_sync();
    f32x4 s[4];
    {
      bf16x8 kf[4][HD / 32];
      decode_keys<HD, KF, WIDE>(kf, kbytes, lane);
      block_scores<HD>(s, kf, qf);
    }
    if constexpr (MORE) fetch_keys<HD, KF, WIDE>(kbytes, kr, kb + 4 * KB, a.k_sr, lane);
    fold_scores<HD, VS>(st, s, vl, kb, pr, lane, fresh);
    fresh = false;
  };
  for (; kb + 4 * KB <= last; kb += 4 * KB) step(kb, std::true_type{});
  if (kb <= last) step(kb, std::false_type{});
  __syncthreads();
  float *ws = (float *)lds;
  store_state<HD>(ws + wib * PF, st, lane);
  __syncthreads();
  finish_tile<HD>(a, ws, 4, kvh, t, part, parts, tiles, scratch);
}

// Decode in parts of one 64-key block each, a block of one wave: the wave folds its block and writes its state as the
// part's partial result, from its registers, with no join through LDS (which a 4-wave block of one or two blocks of
// keys spends most of its time on). The combine kernel joins the parts.
template <int HD, int KF, bool WIDE>
__global__ void __launch_bounds__(64) attention_decode1_kernel(const bt_attention_args a, int tiles, int parts,
                                                               float *scratch) {
  constexpr int VS = HD + 16, VR = KB * VS, PF = partial_floats<HD>();
  __shared__ __attribute__((aligned(16))) uint16_t vl[VR];
  const int lane = threadIdx.x, g = lane >> 4, n = lane & 15;
  int bid = blockIdx.x;
  const int part = bid % parts;
  bid /= parts;
  const int t = bid % tiles, kvh = bid / tiles;
  bf16x8 qf[HD / 32];
  const Pair pr = pair_q<HD>(a, kvh, 16 * t + n, lane, qf);
  int lo, hi;
  tile_range(pr, lo, hi);
  const int start = lo & ~(KB - 1), nblk = hi >= lo ? (hi - start) / KB + 1 : 0, per = (nblk + parts - 1) / parts;
  const int first = start + part * per * KB, last = min(first + per * KB - 1, hi);
  State<HD> st;
  st.m = -__builtin_inff(), st.l = 0.0f;
#pragma unroll
  for (int c = 0; c < HD / 16; c++) st.o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const KvSrc kr = kv_src<KF>(a.k, a.k_exps, (int64_t)kvh * a.k_sh, (int64_t)(a.keys - 1) * a.k_sr + HD);
  const KvSrc vr = kv_src<KF>(a.v, a.v_exps, (int64_t)kvh * a.v_sh, (int64_t)(a.keys - 1) * a.v_sr + HD);
  constexpr int RPI = 64 * 8 / HD, VI = KB / RPI;
  const int vrow = lane / (HD / 8), vcol = lane % (HD / 8) * 8;
  bool fresh = true;
  for (int kb = first; kb <= last; kb += KB) {
    Raw8<KF> vq[VI];
    uint32_t vx[VI];
#pragma unroll
    for (int i = 0; i < VI; i++) {
      const uint32_t e = (uint32_t)((int64_t)(kb + vrow + RPI * i) * a.v_sr + vcol);
      vq[i] = kv_fetch8<KF, DEC_POL>(vr, e);
      vx[i] = kv_exp8<KF, DEC_POL>(vr, e);
    }
    KeyBytes<HD, KF, WIDE> kbytes;
    fetch_keys<HD, KF, WIDE>(kbytes, kr, kb, a.k_sr, lane);
    wave_lds_sync();  // the previous block's reads of vl are done
#pragma unroll
    for (int i = 0; i < VI; i++) *(uint4 *)(vl + (vrow + RPI * i) * VS + vcol) = kv_value8<KF>(vq[i], vx[i]);
    wave_lds_sync();
    f32x4 sc[4];
    {
      bf16x8 kf[4][HD / 32];
      decode_keys<HD, KF, WIDE>(kf, kbytes, lane);
      block_scores<HD>(sc, kf, qf);
    }
    fold_scores<HD, VS>(st, sc, vl, kb, pr, lane, fresh);
    fresh = false;
  }
  float *dst = scratch + ((int64_t)(kvh * tiles + t) * parts + part) * PF;
  if (lane < 16) dst[n] = st.m, dst[16 + n] = st.l;
#pragma unroll
  for (int c = 0; c < HD / 16; c++)
#pragma unroll
    for (int i = 0; i < 4; i++) dst[32 + (4 * g + i) * HD + 16 * c + n] = st.o[c][i];
}

// Joins the parts of each tile: M = max m_p, L = sum e^(m_p - M) l_p, out = sum e^(m_p - M) O_p / L. The block
// first finds every pair's M, weights and L with its 16 groups of 16 threads splitting the parts (weights kept in
// LDS), then each thread sums its output columns over the parts, loads independent of one another.
constexpr int MAX_PARTS = 256;
template <int HD>
__global__ void __launch_bounds__(256) attention_combine_kernel(const bt_attention_args a, int tiles, int parts,
                                                                const float *scratch) {
  constexpr int PF = partial_floats<HD>();
  __shared__ float wgt[MAX_PARTS * 16];  // [part][pair]
  __shared__ float red[16][16], mx[16], ls[16];
  const int t = blockIdx.x % tiles, kvh = blockIdx.x / tiles;
  const float *src = scratch + (int64_t)(kvh * tiles + t) * parts * PF;
  const int pr = threadIdx.x & 15, grp = threadIdx.x >> 4;
  float M = -__builtin_inff();
  for (int p = grp; p < parts; p += 16) M = fmaxf(M, src[p * PF + pr]);
  red[grp][pr] = M;
  __syncthreads();
  if (grp == 0) {
    for (int g = 1; g < 16; g++) M = fmaxf(M, red[g][pr]);
    mx[pr] = M;
  }
  __syncthreads();
  M = mx[pr];
  float L = 0.0f;
  for (int p = grp; p < parts; p += 16) {
    const float w = M == -__builtin_inff() ? 0.0f : __expf(src[p * PF + pr] - M);
    wgt[p * 16 + pr] = w;
    L += w * src[p * PF + 16 + pr];
  }
  red[grp][pr] = L;
  __syncthreads();
  if (grp == 0) {
    for (int g = 1; g < 16; g++) L += red[g][pr];
    ls[pr] = L;
  }
  __syncthreads();
  const int pi = threadIdx.x / 16, c0 = threadIdx.x % 16;
  const Pair pair = pair_of(a, kvh, 16 * t + pi);
  if (!pair.valid) return;
  float o[HD / 16];
#pragma unroll
  for (int c = 0; c < HD / 16; c++) o[c] = 0.0f;
  const float *col = src + 32 + pi * HD + c0;
#pragma unroll 4
  for (int p = 0; p < parts; p++) {
    const float w = wgt[p * 16 + pi];
#pragma unroll
    for (int c = 0; c < HD / 16; c++) o[c] += w * col[p * PF + 16 * c];
  }
  const float inv = ls[pi] > 0.0f ? 1.0f / ls[pi] : 0.0f;
  uint16_t *out = (uint16_t *)a.out + pair.o;
#pragma unroll
  for (int c = 0; c < HD / 16; c++) out[c0 + 16 * c] = (uint16_t)bf16_packed(o[c] * inv);
}

// Prefill. A block is 4 waves and 128 consecutive pairs of one key head; wave w takes pairs 32w .. 32w + 31 of them as
// two groups of 16 (the 16-pair tile of the scheme above), so every K and V fragment it reads from LDS feeds two
// matrix instructions. The block's keys come through LDS 64 at a time, double-buffered, one barrier a step: K and V
// as they are stored (row-major); P V's value operand, 8 keys of one column, is two transposing 8-byte reads
// (ds_read_b64_tr_b16), so V is never transposed by VALU work. The row sums come from the matrix cores too: P times a column of ones, accumulated and rescaled like O.
// Masks are applied only on blocks of keys that some pair of the wave sees in part, and the running output is
// rescaled only when some pair's maximum moved. p is rounded to bf16 to nearest even (v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_rne(float lo, float hi) {
  const bf16x2 r = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
  return *(const uint32_t *)&r;
}

template <int HD> struct Group {
  f32x4 o[HD / 16];  // lane (g, n): pairs 4g + i, columns 16c + n
  f32x4 l;           // row sums of the same pairs (every column holds them)
  float m;           // pair n's reference maximum, in log2 units: p = 2^(s log2(e) - m)
};

// The reference maximum moves only when a block's maximum passes it by more than 2^8 (then O and l are rescaled), so
// p stays below 256 and most blocks need no rescale; O / l is the same for any reference.
constexpr float LAZY = 8.0f;

// The prefill stages K and V row-major, HD halfwords a row, the 16-byte units of row r permuted: logical unit u sits
// at u ^ swz<HD>(r). LDS has 64 banks of 4 bytes, 256 bytes a bank line. A K fragment read takes 16 rows a pass, one
// unit each; a transposed V read 8 rows a pass (4 keys of two lane groups), two neighbouring units each. At HD 128 (a
// row a bank line, 16 units) swz is a permutation of 0..15 whose halves (rows 0-7, 8-15) differ in their top three
// bits; at HD 64 (two rows a line, 8 units each) rows of one parity get distinct permutations of 0..7. Either way both
// reads fall in distinct banks with no padding between rows, so rows can be loaded straight into LDS, 1 KB a wave
// instruction.
template <int HD> __device__ __forceinline__ int swz(int r) {
  if constexpr (HD == 128) return 2 * (r & 7) + ((r >> 3) & 1);
  else return 2 * ((r >> 1) & 3) + ((r >> 3) & 1);
}

// mask: some pair of the wave sees only part of the block (wave-uniform). A block no pair sees leaves the state as
// it was (every p is 0). mid() runs once the scores are made: the caller's loads of a later block, issued where fewer
// registers are live.
template <int HD, typename Mid>
__device__ __forceinline__ void fold_pairs(Group<HD> (&gr)[2], const bf16x8 (&qf)[2][HD / 32], const uint16_t *kl,
                                           const uint16_t *vt, int kb, const int (&lo)[2], const int (&hi)[2],
                                           int lane, bool mask, Mid mid) {
  constexpr float L2E = 1.4426950408889634f;
  const int g = lane >> 4, n = lane & 15;
  int kcol[HD / 32];  // the lane's K fragment units (rows 16 kt + n: the same swizzle for every kt)
#pragma unroll
  for (int kk = 0; kk < HD / 32; kk++) kcol[kk] = ((4 * kk + g) ^ swz<HD>(n)) * 8;
  f32x4 s[2][4];
  uint32_t pb[2][4][2];  // [group][key tile][pair of keys]: packed p
  // p = 2^(s log2(e) - m) against the reference m before this block; if the block moves some pair's reference, those
  // of key tiles 0 and 1 are made again below, so they can be made while the scores of tiles 2 and 3 are
  float nb[2];
#pragma unroll
  for (int q = 0; q < 2; q++) nb[q] = gr[q].m == -__builtin_inff() ? 0.0f : -gr[q].m;  // no key seen yet: p 0
  auto exps = [&](int q, int kt) {
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[q][kt][i], L2E, nb[q]));
    pb[q][kt][0] = pack_rne(p[0], p[1]);
    pb[q][kt][1] = pack_rne(p[2], p[3]);
  };
  auto mask_tile = [&](int q, int kt) {
    if (!mask) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int j = kb + 16 * kt + 4 * g + i;
      if (j < lo[q] || j > hi[q]) s[q][kt][i] = -__builtin_inff();
    }
  };
  bf16x8 kf[2][HD / 32];  // two key tiles' K fragments, the next read while the current one is multiplied
#pragma unroll
  for (int kk = 0; kk < HD / 32; kk++) kf[0][kk] = *(const bf16x8 *)(kl + n * HD + kcol[kk]);
#pragma unroll
  for (int kt = 0; kt < 4; kt++) {
    if (kt < 3) {
#pragma unroll
      for (int kk = 0; kk < HD / 32; kk++)
        kf[(kt + 1) & 1][kk] = *(const bf16x8 *)(kl + (16 * (kt + 1) + n) * HD + kcol[kk]);
    }
    s[0][kt] = s[1][kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk++) {
      s[0][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kt & 1][kk], qf[0][kk], s[0][kt], 0, 0, 0);
      s[1][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kt & 1][kk], qf[1][kk], s[1][kt], 0, 0, 0);
    }
    if (kt >= 1) {  // the previous tile's scores: masked, and tiles 0 and 1 turned into p, while this tile's run
#pragma unroll
      for (int q = 0; q < 2; q++) {
        mask_tile(q, kt - 1);
        if (kt - 1 < 2) exps(q, kt - 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int q = 0; q < 2; q++) mask_tile(q, 3);
  __builtin_amdgcn_sched_barrier(0);
  mid();
  __builtin_amdgcn_sched_barrier(0);
  bool need = false;
  float mnew[2];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    float mx = s[q][0][0];
#pragma unroll
    for (int e = 1; e < 16; e += 2) mx = fmaxf(fmaxf(mx, s[q][e / 4][e % 4]), s[q][(e + 1) / 4 % 4][(e + 1) % 4]);
    mx = max_groups(mx);
    const float m2 = mx * L2E;
    const bool up = m2 > gr[q].m + LAZY;  // false for a pair with no visible key in the block
    need |= up;
    mnew[q] = up ? m2 : gr[q].m;
  }
  if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
    for (int q = 0; q < 2; q++) {
      // 1 where the reference stays (also -inf to -inf), 0 from no reference to the first
      const float scale = mnew[q] == gr[q].m ? 1.0f : __builtin_amdgcn_exp2f(gr[q].m - mnew[q]);
      gr[q].m = mnew[q];
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; i++) sc[i] = __shfl(scale, 4 * g + i, 64);
#pragma unroll
      for (int c = 0; c < HD / 16; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) gr[q].o[c][i] *= sc[i];
#pragma unroll
      for (int i = 0; i < 4; i++) gr[q].l[i] *= sc[i];
      nb[q] = gr[q].m == -__builtin_inff() ? 0.0f : -gr[q].m;
      exps(q, 0);
      exps(q, 1);
    }
  }
  // key tiles 2 and 3 are made between the first P V step's matrix instructions (one group and tile after each of its
  // first 4 column tiles: 68.6-69.6 -> 66.0-67.5 us at 2048 rows; spread over all 8 at HD 128, 67.7-68.8), so their
  // VALU work issues while the matrix core is busy; the order is held by scheduling barriers
  __builtin_amdgcn_sched_barrier(0);
  const bf16x8 ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    bf16x8 pa[2];
#pragma unroll
    for (int q = 0; q < 2; q++)
      pa[q] = as_bf16x8(pb[q][2 * ks][0], pb[q][2 * ks][1], pb[q][2 * ks + 1][0], pb[q][2 * ks + 1][1]);
    // transposed reads of row-major V: lane n of a 16-lane group addresses key 4g + n / 4 of the step (and 16
    // further), dims 16c + 4 (n % 4) .. + 3 (logical unit 2c + (n % 4) / 2); the read hands lane n the group's 4 keys
    // of dim 16c + n
    const uint16_t *row = vt + (32 * ks + 4 * g + n / 4) * HD + 4 * (n & 1);
    const int fv = swz<HD>(4 * g + n / 4), nu = (n & 3) >> 1;  // rows 32ks + 4g + n/4 (+ 16) swizzle as row 4g + n/4
#pragma unroll
    for (int c = 0; c < HD / 16; c++) {
      typedef short s16x4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
      const int at = ((2 * c + nu) ^ fv) * 8;
      const s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(row + at));
      const s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(row + 16 * HD + at));
      const uint2 a0 = __builtin_bit_cast(uint2, r0), a1 = __builtin_bit_cast(uint2, r1);
      const bf16x8 vf = as_bf16x8(a0.x, a0.y, a1.x, a1.y);
      gr[0].o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[0], vf, gr[0].o[c], 0, 0, 0);
      gr[1].o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[1], vf, gr[1].o[c], 0, 0, 0);
      if (ks == 0 && c < 4) {
        exps(c / 2, 2 + c % 2);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    gr[0].l = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[0], ones, gr[0].l, 0, 0, 0);
    gr[1].l = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[1], ones, gr[1].l, 0, 0, 0);
  }
}

// Prefill. A block is 8 waves and 128 consecutive pairs of one key head. Waves w and w + 4 take the same 32 pairs,
// as two groups of 16 (the tile of the scheme above), so every K and V fragment a wave reads from LDS feeds two matrix
// instructions; the two halves of the block (waves 0-3, 4-7) split the keys, half h folding blocks 2t + h of 64 keys,
// each half with its own double-buffered LDS stage, one barrier a step. K and V are staged as stored (row-major); P V's
// value operand, 8 keys of one column, is two transposing 8-byte reads of V (ds_read_b64_tr_b16: within each 16 lanes,
// slot k of lane i is halfword i % 4 of what lane 4k + i / 4 addressed), which replaced staging V transposed by VALU
// permutes (2048-row prefill 65.2-67.6 -> 61.4-63.2 us). The row sums come from the
// matrix cores too: P times a column of ones, accumulated and rescaled like O. At the end half 1 hands its state to
// half 0 through LDS, which joins the two (rescaling both to the larger maximum) and stores the output.
//
// Blocks go heaviest first (the last rows of the causal triangle see the most keys): block u takes key head u % kvhs
// and row block rblocks - 1 - u / kvhs.
template <int HD, int KF>
__global__ void __launch_bounds__(512, 1) attention_prefill_kernel(const bt_attention_args a, int rblocks, int kvhs) {
  constexpr int KBUF = KB * HD, STG = 2 * KBUF;  // halfwords of one stage: K, then V, row-major, units swizzled (swz)
  constexpr int KW = KB * HD / 8 / 256;  // 16-byte words of K (and of V) each thread of a half moves per block
  constexpr int XF = 2 * (HD / 4 + 8);   // floats per lane a wave hands over: O, l and the maxima of both groups
  static_assert(4 * XF * 64 * 4 <= 4 * STG * 2, "the hand-over fits in the stages");
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][STG];  // [half][stage]
  __shared__ int range[4][2];
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), wq = wib & 3, hf = wib >> 2;
  const int th = threadIdx.x & 255;
  const int u = blockIdx.x, kvh = u % kvhs, rb = rblocks - 1 - u / kvhs;
  const int base = 128 * rb + 32 * wq;
  Pair pr[2];
  bf16x8 qf[2][HD / 32];
  int lo[2], hi[2];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    pr[q] = pair_q<HD>(a, kvh, base + 16 * q + n, lane, qf[q]);
    lo[q] = pr[q].lo, hi[q] = pr[q].hi;
  }
  // the wave's range (union over its pairs) and the keys every valid pair sees (intersection)
  int wlo = 0x7FFFFFFF, whi = -1, alo = -1, ahi = 0x7FFFFFFF;
#pragma unroll
  for (int q = 0; q < 2; q++) {
    if (pr[q].lo <= pr[q].hi) wlo = min(wlo, pr[q].lo), whi = max(whi, pr[q].hi);
    if (pr[q].valid) alo = max(alo, pr[q].lo), ahi = min(ahi, pr[q].hi);
  }
  wlo = row_min(wlo), whi = row_max(whi), alo = row_max(alo), ahi = row_min(ahi);
  wlo = __builtin_amdgcn_readfirstlane(wlo), whi = __builtin_amdgcn_readfirstlane(whi);
  alo = __builtin_amdgcn_readfirstlane(alo), ahi = __builtin_amdgcn_readfirstlane(ahi);
  if (lane == 0 && hf == 0) range[wq][0] = wlo, range[wq][1] = whi;
  __syncthreads();
  int blo = 0x7FFFFFFF, bhi = -1;
#pragma unroll
  for (int w = 0; w < 4; w++) blo = min(blo, range[w][0]), bhi = max(bhi, range[w][1]);
  blo = __builtin_amdgcn_readfirstlane(blo), bhi = __builtin_amdgcn_readfirstlane(bhi);
  Group<HD> gr[2];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    gr[q].m = -__builtin_inff();
    gr[q].l = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < HD / 16; c++) gr[q].o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // rows past the block's last visible key read as zeros (they are masked, and may never have been written): the
  // buffers end there
  const KvSrc kr = kv_src<KF>(a.k, a.k_exps, (int64_t)kvh * a.k_sh, bhi < 0 ? 0 : (int64_t)bhi * a.k_sr + HD);
  const KvSrc vr = kv_src<KF>(a.v, a.v_exps, (int64_t)kvh * a.v_sh, bhi < 0 ? 0 : (int64_t)bhi * a.v_sr + HD);
  // half hf folds blocks first + 64 (2t + hf), t < steps, the same count for both halves (a block past the last
  // visible key reads as zeros and is masked whole)
  const int first = blo & ~(KB - 1);
  const int nblk = bhi >= first ? (bhi - first) / KB + 1 : 0, steps = (nblk + 1) / 2;
  uint16_t *const st0 = lds[hf][0], *const st1 = lds[hf][1];
  if constexpr (KF == BT_BF16) {
    // bf16: each stage straight from memory into LDS, 1 KB a wave instruction, a block's stage requested at the start
    // of the step before it (into the buffer that step's barrier freed), so it has a whole step to land and holds no
    // registers. Wave wq's instruction i fills rows (wq + 4 i) RPI .. + RPI - 1: lane l row (l / UPR), unit l % UPR,
    // which holds logical unit (l % UPR) ^ swz<HD>(row). (2048-row prefill 61.0-62.1 -> 60.4-60.8 us against loads into
    // registers issued after the scores and stashed at the end of the step.)
    constexpr int UPR = HD / 8, RPI = 64 / UPR, NI = KB / RPI / 4;
    const i32x4 kw4 = buffer_words((const uint16_t *)(uintptr_t)a.k + (int64_t)kvh * a.k_sh,
                                   bhi < 0 ? 0u : (uint32_t)(((int64_t)bhi * a.k_sr + HD) * 2));
    const i32x4 vw4 = buffer_words((const uint16_t *)(uintptr_t)a.v + (int64_t)kvh * a.v_sh,
                                   bhi < 0 ? 0u : (uint32_t)(((int64_t)bhi * a.v_sr + HD) * 2));
    uint32_t kof[NI], vof[NI];  // byte offsets from a block's first row
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int r = (wq + 4 * i) * RPI + lane / UPR, uu = (lane % UPR) ^ swz<HD>(r);
      kof[i] = (uint32_t)(((int64_t)r * a.k_sr + 8 * uu) * 2);
      vof[i] = (uint32_t)(((int64_t)r * a.v_sr + 8 * uu) * 2);
    }
    auto load_stage = [&](int kb, uint16_t *stage) {
      const uint32_t kbo = (uint32_t)((int64_t)kb * a.k_sr * 2), vbo = (uint32_t)((int64_t)kb * a.v_sr * 2);
#pragma unroll
      for (int i = 0; i < NI; i++) lds_load16(kw4, kbo + kof[i], stage + (wq + 4 * i) * RPI * HD);
#pragma unroll
      for (int i = 0; i < NI; i++) lds_load16(vw4, vbo + vof[i], stage + KBUF + (wq + 4 * i) * RPI * HD);
    };
    if (steps > 0) load_stage(first + KB * hf, st0);
    wait_vm<0>();
    __syncthreads();
    auto step = [&](int t, uint16_t *cur, uint16_t *nxt) {
      const int kb = first + KB * (2 * t + hf);
      const bool more = t + 1 < steps, mask = kb < alo || kb + KB - 1 > ahi;
      if (more) load_stage(kb + 2 * KB, nxt);
      fold_pairs<HD>(gr, qf, cur, cur + KBUF, kb, lo, hi, lane, mask, [] {});
      wait_vm<0>();
      __syncthreads();
    };
    for (int t = 0; t < steps; t++) step(t, t & 1 ? st1 : st0, t & 1 ? st0 : st1);
  } else {
    // block floats: loaded into registers, decoded there, and written to LDS in the same layout. The thread's words
    // at row kr0 + (256 / (HD / 8)) i, logical unit kc / 8.
    const KvSrc kr = kv_src<KF>(a.k, a.k_exps, (int64_t)kvh * a.k_sh, bhi < 0 ? 0 : (int64_t)bhi * a.k_sr + HD);
    const KvSrc vr = kv_src<KF>(a.v, a.v_exps, (int64_t)kvh * a.v_sh, bhi < 0 ? 0 : (int64_t)bhi * a.v_sr + HD);
    const int kr0 = th / (HD / 8), kc = th % (HD / 8) * 8;
    constexpr int KSTEP = 256 / (HD / 8);
    // value offsets from a block's first row: the thread's first word, then uniform steps
    const uint32_t koff = (uint32_t)((int64_t)kr0 * a.k_sr + kc), voff = (uint32_t)((int64_t)kr0 * a.v_sr + kc);
    const uint32_t kstep = (uint32_t)(KSTEP * a.k_sr), vstep = (uint32_t)(KSTEP * a.v_sr);
    uint4 kreg[KW], vreg[KW];
    auto fetch = [&](int kb) {
      const uint32_t kbo = (uint32_t)((int64_t)kb * a.k_sr), vbo = (uint32_t)((int64_t)kb * a.v_sr);
#pragma unroll
      for (int i = 0; i < KW; i++) kreg[i] = kv_load8<KF>(kr, koff + (kbo + i * kstep));
#pragma unroll
      for (int i = 0; i < KW; i++) vreg[i] = kv_load8<KF>(vr, voff + (vbo + i * vstep));
    };
    auto stash = [&](uint16_t *stage) {
#pragma unroll
      for (int i = 0; i < KW; i++) {
        const int r = kr0 + KSTEP * i, at = r * HD + (((kc >> 3) ^ swz<HD>(r)) << 3);
        *(uint4 *)(stage + at) = kreg[i];
        *(uint4 *)(stage + KBUF + at) = vreg[i];
      }
    };
    if (steps > 0) {
      fetch(first + KB * hf);
      stash(st0);
    }
    __syncthreads();
    auto step = [&](int t, uint16_t *cur, uint16_t *nxt) {
      const int kb = first + KB * (2 * t + hf);
      const bool more = t + 1 < steps, mask = kb < alo || kb + KB - 1 > ahi;
      fold_pairs<HD>(gr, qf, cur, cur + KBUF, kb, lo, hi, lane, mask, [&] {
        if (more) fetch(kb + 2 * KB);
      });
      if (more) stash(nxt);
      __syncthreads();
    };
    for (int t = 0; t < steps; t++) step(t, t & 1 ? st1 : st0, t & 1 ? st0 : st1);
  }
  // half 1 hands over O, l and its maxima (row i's, for the rows this lane holds); half 0 joins and stores
  float *xs = (float *)&lds[0][0][0] + wq * XF * 64 + lane;
  float md[2][4];
#pragma unroll
  for (int q = 0; q < 2; q++)
#pragma unroll
    for (int i = 0; i < 4; i++) md[q][i] = __shfl(gr[q].m, 4 * g + i, 64);
  if (hf == 1) {
#pragma unroll
    for (int q = 0; q < 2; q++) {
      float *x = xs + q * (HD / 4 + 8) * 64;
#pragma unroll
      for (int c = 0; c < HD / 16; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) x[(4 * c + i) * 64] = gr[q].o[c][i];
#pragma unroll
      for (int i = 0; i < 4; i++) x[(HD / 4 + i) * 64] = gr[q].l[i], x[(HD / 4 + 4 + i) * 64] = md[q][i];
    }
  }
  __syncthreads();
  if (hf == 1) return;
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const float *x = xs + q * (HD / 4 + 8) * 64;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int p = base + 16 * q + 4 * g + i;
      if (p >= a.rep * a.rows) continue;
      const float m1 = x[(HD / 4 + 4 + i) * 64], m0 = md[q][i], M = fmaxf(m0, m1);
      const float w0 = m0 == M ? 1.0f : __builtin_amdgcn_exp2f(m0 - M);
      const float w1 = m1 == M ? 1.0f : __builtin_amdgcn_exp2f(m1 - M);
      const float l = gr[q].l[i] * w0 + x[(HD / 4 + i) * 64] * w1;
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
      const int h = p % a.rep, r = p / a.rep, e = kvh * a.rep + h;
      uint16_t *out = (uint16_t *)a.out + (int64_t)e * a.o_sh + (int64_t)r * a.o_sr;
#pragma unroll
      for (int c = 0; c < HD / 16; c++)
        out[16 * c + n] = (uint16_t)bf16_packed((gr[q].o[c][i] * w0 + x[(4 * c + i) * 64] * w1) * inv);
    }
  }
}

template <int HD>
static void launch_decode_hd(const bt_attention_args &a, unsigned blocks, int tiles, int parts, float *scratch,
                             hipStream_t s) {
  // a key row's exponents in one load when every row's start in the plane is aligned to their HD / 16 bytes
  const bool wide = a.k_sr % HD == 0 && a.k_sh % HD == 0 && a.k_exps % (HD / 16) == 0;
  if (a.kv_fmt == BT_BFP8 && wide) attention_decode_kernel<HD, BT_BFP8, true><<<blocks, 256, 0, s>>>(a, tiles, parts, scratch);
  else if (a.kv_fmt == BT_BFP8) attention_decode_kernel<HD, BT_BFP8, false><<<blocks, 256, 0, s>>>(a, tiles, parts, scratch);
  else if (a.kv_fmt == BT_BFP4 && wide) attention_decode_kernel<HD, BT_BFP4, true><<<blocks, 256, 0, s>>>(a, tiles, parts, scratch);
  else if (a.kv_fmt == BT_BFP4) attention_decode_kernel<HD, BT_BFP4, false><<<blocks, 256, 0, s>>>(a, tiles, parts, scratch);
  else attention_decode_kernel<HD, BT_BF16, false><<<blocks, 256, 0, s>>>(a, tiles, parts, scratch);
}
static void launch_decode(const bt_attention_args &a, unsigned blocks, int tiles, int parts, float *scratch,
                          hipStream_t s) {
  if (a.head_dim == 64) launch_decode_hd<64>(a, blocks, tiles, parts, scratch, s);
  else launch_decode_hd<128>(a, blocks, tiles, parts, scratch, s);
}
template <int HD>
static void launch_decode1_hd(const bt_attention_args &a, unsigned blocks, int tiles, int parts, float *scratch,
                              hipStream_t s) {
  const bool wide = a.k_sr % HD == 0 && a.k_sh % HD == 0 && a.k_exps % (HD / 16) == 0;
  if (a.kv_fmt == BT_BFP8 && wide) attention_decode1_kernel<HD, BT_BFP8, true><<<blocks, 64, 0, s>>>(a, tiles, parts, scratch);
  else if (a.kv_fmt == BT_BFP8) attention_decode1_kernel<HD, BT_BFP8, false><<<blocks, 64, 0, s>>>(a, tiles, parts, scratch);
  else if (a.kv_fmt == BT_BFP4 && wide) attention_decode1_kernel<HD, BT_BFP4, true><<<blocks, 64, 0, s>>>(a, tiles, parts, scratch);
  else if (a.kv_fmt == BT_BFP4) attention_decode1_kernel<HD, BT_BFP4, false><<<blocks, 64, 0, s>>>(a, tiles, parts, scratch);
  else attention_decode1_kernel<HD, BT_BF16, false><<<blocks, 64, 0, s>>>(a, tiles, parts, scratch);
}
template <int HD>
static void launch_prefill_hd(const bt_attention_args &a, unsigned blocks, int rblocks, int kvh, hipStream_t s) {
  if (a.kv_fmt == BT_BFP8) attention_prefill_kernel<HD, BT_BFP8><<<blocks, 512, 0, s>>>(a, rblocks, kvh);
  else if (a.kv_fmt == BT_BFP4) attention_prefill_kernel<HD, BT_BFP4><<<blocks, 512, 0, s>>>(a, rblocks, kvh);
  else attention_prefill_kernel<HD, BT_BF16><<<blocks, 512, 0, s>>>(a, rblocks, kvh);
}
static void launch_prefill(const bt_attention_args &a, unsigned blocks, int rblocks, int kvh, hipStream_t s) {
  if (a.head_dim == 64) launch_prefill_hd<64>(a, blocks, rblocks, kvh, s);
  else launch_prefill_hd<128>(a, blocks, rblocks, kvh, s);
}

struct AttnPlan {
  bool decode;
  bool one;  // decode parts of one block of keys each, a wave a part (attention_decode1_kernel)
  int tiles, parts, kpp;
  uint64_t scratch_bytes;
};

static int plan_attention(const bt_attention_args *a, AttnPlan *p) {
  if (!a || !a->q || !a->k || !a->v || !a->out || !a->places) return fail(BT_EINVAL, "attention needs q, k, v, out, places");
  if (a->heads <= 0 || a->rep <= 0 || a->heads % a->rep || a->rows <= 0 || a->keys <= 0 || a->window < 0 || a->parts < 0)
    return fail(BT_EINVAL, "attention shape: %d heads, rep %d, %d rows, %d keys, window %d, parts %d", a->heads, a->rep,
                a->rows, a->keys, a->window, a->parts);
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(BT_EINVAL, "attention takes heads 64 or 128 wide, not %d", a->head_dim);
  if (a->q % 16 || (a->kv_fmt == BT_BF16 && (a->k | a->v) % 16) || a->q_sr % 8 || a->k_sr % 8 || a->v_sr % 8 ||
      a->q_sh % 8 || a->k_sh % 8 || a->v_sh % 8)
    return fail(BT_EINVAL, "attention needs q, k and v rows on 16-byte boundaries");
  if (a->places_sh != 0 && a->places_sh != a->rows) return fail(BT_EINVAL, "places' head stride is 0 or rows");
  if (((int64_t)(a->keys + KB) * std::max(a->k_sr, a->v_sr) + a->head_dim) * 2 >= (1ll << 32))
    return fail(BT_EINVAL, "a key head's rows (and 64 more) must span less than 4 GiB");
  if (a->kv_fmt != BT_BF16 && a->kv_fmt != BT_BFP8 && a->kv_fmt != BT_BFP4)
    return fail(BT_EINVAL, "attention's cache is bf16, bfp8 or bfp4, not %d", a->kv_fmt);
  if (a->kv_fmt != BT_BF16 && (!a->k_exps || !a->v_exps || a->k % 8 || a->v % 8 || a->k_sr % 16 || a->v_sr % 16 ||
                               a->k_sh % 16 || a->v_sh % 16))
    return fail(BT_EINVAL, "a block-float cache needs its exponent planes, 8-byte aligned value planes and strides "
                           "that are multiples of 16");
  if (a->firsts && a->firsts % 4) return fail(BT_EINVAL, "attention's firsts must be int32-aligned");
  if (a->firsts && a->firsts_sh != 0 && a->firsts_sh != a->rows) return fail(BT_EINVAL, "firsts' head stride is 0 or rows");
  const int kvh = a->heads / a->rep, np = a->rep * a->rows;
  p->tiles = (np + 15) / 16;
  p->decode = p->tiles <= 4;  // few query rows for each key head: split the keys instead
  p->parts = 1, p->kpp = 0, p->scratch_bytes = 0, p->one = false;
  if (p->decode) {
    const int nblk = (a->keys + KB - 1) / KB;
    int parts = a->parts;
    // bf16: one block a CU (MI355X's 256), each wave's loads a block ahead through all of its share of the keys;
    // block floats: two a CU, so one block's decoding overlaps the other's loads. Measured faster than more,
    // shorter-lived blocks at 1-32 batch entries and 4096-16384 keys. A part's keys are a chain of dependent loads,
    // so up to 32 blocks of 64 keys, parts of two blocks (and the combine's launch) beat longer ones; beyond, four;
    // up to 4 blocks, one part (no combine) is the fastest.
    // 5 to 16 blocks of keys over at most 512 blocks of the grid: a part a block of keys, a wave a part, joined by the
    // combine alone (B=1 at 512 keys 7.55 -> 6.79 us, at 1024 7.99 -> 7.70; B=8 at 512 the same, at 1024 slower)
    const int target = a->kv_fmt == BT_BF16 ? 256 : 512, units = kvh * p->tiles;
    const int per_part = nblk <= 4 ? nblk : nblk <= 32 ? 2 : 4;
    if (parts == 0) {
      if (nblk > 4 && nblk <= 16 && units * nblk <= 512) parts = nblk;
      else parts = std::min((target + units / 2) / units, std::max(1, nblk / per_part));
    }
    p->parts = std::max(1, std::min(std::min(parts, nblk), MAX_PARTS));
    p->one = p->parts > 1 && p->parts >= nblk;
    const int pf = 32 + 16 * a->head_dim;
    if (p->parts > 1) p->scratch_bytes = (uint64_t)kvh * p->tiles * p->parts * pf * 4;
  }
  return BT_OK;
}

// The working memory of bt_attention_noalloc: one array a GPU, the split decode's partial sums. Host code never passes
// the array's name to a kernel (on the host it stands for no device address): at bt_open, with the device current,
// hipGetSymbolAddress gives each device's own copy's address, kept here per device.
static __device__ __align__(256) uint8_t scratch[BT_ATTENTION_NOALLOC_BYTES];
static std::mutex noalloc_lock;
static void *noalloc_ptr[BT_MAX_DEVICES];
static hipError_t noalloc_error[BT_MAX_DEVICES];

void attention_noalloc_init(int device) {
  if (device < 0 || device >= BT_MAX_DEVICES) return;
  std::lock_guard<std::mutex> hold(noalloc_lock);
  if (noalloc_ptr[device]) return;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) (void)hipGetLastError();
  noalloc_error[device] = e;
  if (e == hipSuccess) noalloc_ptr[device] = p;
}

static int run_attention(Runtime *r, const bt_attention_args *a, const AttnPlan &p, float *scratch) {
  const int kvh = a->heads / a->rep;
  if (p.decode) {
    const unsigned blocks = (unsigned)(kvh * p.tiles * p.parts);
    if (p.one) {
      if (a->head_dim == 64) launch_decode1_hd<64>(*a, blocks, p.tiles, p.parts, scratch, r->stream);
      else launch_decode1_hd<128>(*a, blocks, p.tiles, p.parts, scratch, r->stream);
    } else {
      launch_decode(*a, blocks, p.tiles, p.parts, scratch, r->stream);
    }
    BT_LAUNCHED("attention");
    if (p.parts > 1) {
      const unsigned cb = (unsigned)(kvh * p.tiles);
      if (a->head_dim == 64) attention_combine_kernel<64><<<cb, 256, 0, r->stream>>>(*a, p.tiles, p.parts, scratch);
      else attention_combine_kernel<128><<<cb, 256, 0, r->stream>>>(*a, p.tiles, p.parts, scratch);
      BT_LAUNCHED("attention combine");
    }
  } else {
    const int rblocks = (a->rep * a->rows + 127) / 128;
    const unsigned blocks = (unsigned)(kvh * rblocks);
    launch_prefill(*a, blocks, rblocks, kvh, r->stream);
    BT_LAUNCHED("attention");
  }
  return BT_OK;
}

}  // namespace bt

using namespace bt;

extern "C" {

int bt_attention_scratch(const bt_attention_args *a, uint64_t *bytes) {
  if (!bytes) return fail(BT_EINVAL, "no result pointer");
  AttnPlan p;
  if (int s = plan_attention(a, &p)) return s;
  *bytes = p.scratch_bytes;
  return BT_OK;
}

int bt_attention(bt_runtime *rt, const bt_attention_args *a) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  AttnPlan p;
  if (int s = plan_attention(a, &p)) return s;
  if (p.scratch_bytes && (!a->scratch || a->scratch_bytes < p.scratch_bytes || a->scratch % 16))
    return fail(BT_EINVAL, "attention in %d parts needs %llu bytes of 16-byte aligned scratch", p.parts,
                (unsigned long long)p.scratch_bytes);
  return run_attention(r, a, p, (float *)(uintptr_t)a->scratch);
}

int bt_attention_noalloc(bt_runtime *rt, const bt_attention_args *a) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  AttnPlan p;
  if (int s = plan_attention(a, &p)) return s;
  if (p.scratch_bytes > BT_ATTENTION_NOALLOC_BYTES)
    return fail(BT_EINVAL, "attention in %d parts needs %llu bytes of working memory, and bt_attention_noalloc has %u: "
                "take fewer parts, or bt_attention with a workspace", p.parts, (unsigned long long)p.scratch_bytes,
                (unsigned)BT_ATTENTION_NOALLOC_BYTES);
  void *ptr = nullptr;
  {
    std::lock_guard<std::mutex> hold(noalloc_lock);
    if (r->device < BT_MAX_DEVICES) ptr = noalloc_ptr[r->device];
  }
  if (!ptr)
    return fail(BT_ESTATE, "bt_attention_noalloc's working memory on device %d has no address: %s", r->device,
                r->device < BT_MAX_DEVICES ? hipGetErrorString(noalloc_error[r->device]) : "device index too large");
  return run_attention(r, a, p, (float *)ptr);
}

}  // extern "C"
