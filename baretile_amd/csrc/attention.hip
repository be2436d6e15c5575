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
// visible keys, written as fp32 partial sums to scratch and combined by a second kernel. Prefill: the block's waves take 4 consecutive tiles and share each block
// of 64 keys and values through LDS, double-buffered.
#include "common.h"
#include <algorithm>

namespace bt {

typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int KB = 64;  // keys per block

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

// Folds one block of 64 keys starting at kb into st. kf: the K operand fragments (lane l: key kb + 16kt + l%16,
// dims 32kk + 8(l/16) .. +8). vl: the block's values in LDS, row-major with a row stride of VS halfwords.
template <int HD, int VS>
__device__ __forceinline__ void fold_block(State<HD> &st, const bf16x8 (&kf)[4][HD / 32], const bf16x8 (&qf)[HD / 32],
                                           const uint16_t *vl, int kb, const Pair &pr, int lane) {
  const int g = lane >> 4, n = lane & 15;
  f32x4 s[4];
#pragma unroll
  for (int kt = 0; kt < 4; kt++) {
    s[kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < HD / 32; kk++) s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kt][kk], qf[kk], s[kt], 0, 0, 0);
  }
  float mx = -__builtin_inff();
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int j = kb + 16 * kt + 4 * g + i;
      if (j < pr.lo || j > pr.hi) s[kt][i] = -__builtin_inff();
      mx = fmaxf(mx, s[kt][i]);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
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
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  st.l = st.l * scale + sum;
  st.m = mn;
  float sc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) sc[i] = __shfl(scale, 4 * g + i, 64);
#pragma unroll
  for (int c = 0; c < HD / 16; c++)
#pragma unroll
    for (int i = 0; i < 4; i++) st.o[c][i] *= sc[i];
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    const bf16x8 pa = as_bf16x8(pb[2 * ks][0] | pb[2 * ks][1] << 16, pb[2 * ks][2] | pb[2 * ks][3] << 16,
                                pb[2 * ks + 1][0] | pb[2 * ks + 1][1] << 16, pb[2 * ks + 1][2] | pb[2 * ks + 1][3] << 16);
    const uint16_t *rows = vl + (32 * ks + 4 * g) * VS + n;
#pragma unroll
    for (int c = 0; c < HD / 16; c++) {
      const uint16_t *at = rows + 16 * c;
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        w[j / 2] = (uint32_t)at[j * VS] | (uint32_t)at[(j + 1) * VS] << 16;            // keys 4g + j, 4g + j + 1
        w[2 + j / 2] = (uint32_t)at[(16 + j) * VS] | (uint32_t)at[(17 + j) * VS] << 16;  // keys 16 + 4g + j, +1
      }
      st.o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, as_bf16x8(w[0], w[1], w[2], w[3]), st.o[c], 0, 0, 0);
    }
  }
}

// The Q^T operand fragments of the lane's pair: dims 32kk + 8(l/16) .. +8, zeros for a pair past the last.
template <int HD>
__device__ __forceinline__ void load_q(const bt_attention_args &a, const Pair &pr, int lane, bf16x8 (&qf)[HD / 32]) {
  const uint16_t *q = (const uint16_t *)a.q + pr.q;
#pragma unroll
  for (int kk = 0; kk < HD / 32; kk++) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (pr.valid) v = *(const uint4 *)(q + 32 * kk + 8 * (lane >> 4));
    qf[kk] = *(const bf16x8 *)&v;
  }
}

// The smallest first key and largest last key over the 16 pairs of the wave's tile (lanes 0..15 hold them all).
__device__ __forceinline__ void tile_range(const Pair &pr, int &lo, int &hi) {
  lo = pr.lo <= pr.hi ? pr.lo : 0x7FFFFFFF;
  hi = pr.lo <= pr.hi ? pr.hi : -1;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    lo = min(lo, __shfl_xor(lo, o, 64));
    hi = max(hi, __shfl_xor(hi, o, 64));
  }
  lo = __builtin_amdgcn_readfirstlane(lo);
  hi = __builtin_amdgcn_readfirstlane(hi);
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
// `parts` runs of whole 64-key blocks; the 4 waves take the part's blocks in turn.
template <int HD>
__global__ void __launch_bounds__(256) attention_decode_kernel(const bt_attention_args a, int tiles, int parts,
                                                               float *scratch) {
  constexpr int VS = HD + 8, VR = KB * VS;  // halfwords of one wave's value block
  constexpr int PF = partial_floats<HD>();
  static_assert(4 * PF * 4 <= 4 * VR * 2, "the wave partials fit in the value blocks' LDS");
  __shared__ __attribute__((aligned(16))) uint16_t lds[4 * VR];
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int bid = blockIdx.x;
  const int part = bid % parts;
  bid /= parts;
  const int t = bid % tiles, kvh = bid / tiles;
  const Pair pr = pair_of(a, kvh, 16 * t + n);
  bf16x8 qf[HD / 32];
  load_q<HD>(a, pr, lane, qf);
  int lo, hi;
  tile_range(pr, lo, hi);
  const int start = lo & ~(KB - 1), nblk = hi >= lo ? (hi - start) / KB + 1 : 0, per = (nblk + parts - 1) / parts;
  const int first = start + part * per * KB, last = min(first + per * KB - 1, hi);
  State<HD> st;
  st.m = -__builtin_inff(), st.l = 0.0f;
#pragma unroll
  for (int c = 0; c < HD / 16; c++) st.o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t kbytes = (uint32_t)(((int64_t)(a.keys - 1) * a.k_sr + HD) * 2);
  const uint32_t vbytes = (uint32_t)(((int64_t)(a.keys - 1) * a.v_sr + HD) * 2);
  const __amdgpu_buffer_rsrc_t kr = attn_rsrc((const uint16_t *)a.k + (int64_t)kvh * a.k_sh, kbytes);
  const __amdgpu_buffer_rsrc_t vr = attn_rsrc((const uint16_t *)a.v + (int64_t)kvh * a.v_sh, vbytes);
  uint16_t *vl = lds + wib * VR;
  constexpr int RPI = 64 * 8 / HD;  // value rows one load instruction covers
  const int vrow = lane / (HD / 8), vcol = lane % (HD / 8) * 8;
  for (int kb = first + KB * wib; kb <= last; kb += 4 * KB) {
    bf16x8 kf[4][HD / 32];
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
      for (int kk = 0; kk < HD / 32; kk++) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(
            kr, (uint32_t)(((int64_t)(kb + 16 * kt + n) * a.k_sr + 32 * kk + 8 * g) * 2), 0, 0);
        kf[kt][kk] = as_bf16x8(v[0], v[1], v[2], v[3]);
      }
    uint4 vv[KB / RPI];
#pragma unroll
    for (int i = 0; i < KB / RPI; i++) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(
          vr, (uint32_t)(((int64_t)(kb + vrow + RPI * i) * a.v_sr + vcol) * 2), 0, 0);
      vv[i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    wave_lds_sync();  // the previous block's reads of vl are done
#pragma unroll
    for (int i = 0; i < KB / RPI; i++) *(uint4 *)(vl + (vrow + RPI * i) * VS + vcol) = vv[i];
    wave_lds_sync();
    fold_block<HD, VS>(st, kf, qf, vl, kb, pr, lane);
  }
  __syncthreads();
  float *ws = (float *)lds;
  store_state<HD>(ws + wib * PF, st, lane);
  __syncthreads();
  finish_tile<HD>(a, ws, 4, kvh, t, part, parts, tiles, scratch);
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

// Prefill: block (kvh, 4 consecutive tiles); wave w takes tile 4 * blockIdx + w. Each block of 64 keys and values is
// loaded once by the whole block into LDS (two buffers), then every wave whose tile sees part of it folds it in.
template <int HD>
__global__ void __launch_bounds__(256) attention_prefill_kernel(const bt_attention_args a, int tiles) {
  constexpr int VS = HD + 8, BUF = KB * VS;  // halfwords of one 64-row block
  constexpr int PER = KB * HD / 8 / 256;      // 16-byte words of K (and of V) each thread moves per block
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][BUF];  // [buffer][K, V]
  __shared__ int range[4][2];
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blocks4 = (tiles + 3) / 4;
  const int kvh = blockIdx.x / blocks4, t = (blockIdx.x % blocks4) * 4 + wib;
  const Pair pr = pair_of(a, kvh, 16 * t + n);
  bf16x8 qf[HD / 32];
  load_q<HD>(a, pr, lane, qf);
  int lo, hi;
  tile_range(pr, lo, hi);
  if (lane == 0) range[wib][0] = lo, range[wib][1] = hi;
  __syncthreads();
  int blo = 0x7FFFFFFF, bhi = -1;
#pragma unroll
  for (int w = 0; w < 4; w++) blo = min(blo, range[w][0]), bhi = max(bhi, range[w][1]);
  State<HD> st;
  st.m = -__builtin_inff(), st.l = 0.0f;
#pragma unroll
  for (int c = 0; c < HD / 16; c++) st.o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t kbytes = (uint32_t)(((int64_t)(a.keys - 1) * a.k_sr + HD) * 2);
  const uint32_t vbytes = (uint32_t)(((int64_t)(a.keys - 1) * a.v_sr + HD) * 2);
  const __amdgpu_buffer_rsrc_t kr = attn_rsrc((const uint16_t *)a.k + (int64_t)kvh * a.k_sh, kbytes);
  const __amdgpu_buffer_rsrc_t vr = attn_rsrc((const uint16_t *)a.v + (int64_t)kvh * a.v_sh, vbytes);
  // thread's words: row (tid / (HD / 8)) + (256 * 8 / HD) * i, column (tid % (HD / 8)) * 8
  const int tr = threadIdx.x / (HD / 8), tc = threadIdx.x % (HD / 8) * 8;
  constexpr int RSTEP = 256 * 8 / HD;
  uint4 kreg[PER], vreg[PER];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const auto k = __builtin_amdgcn_raw_buffer_load_b128(kr, (uint32_t)(((int64_t)(kb + tr + RSTEP * i) * a.k_sr + tc) * 2), 0, 0);
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(vr, (uint32_t)(((int64_t)(kb + tr + RSTEP * i) * a.v_sr + tc) * 2), 0, 0);
      kreg[i] = make_uint4(k[0], k[1], k[2], k[3]);
      vreg[i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
  const int first = blo & ~(KB - 1);
  if (first <= bhi) fetch(first);
  int buf = 0;
  for (int kb = first; kb <= bhi; kb += KB, buf ^= 1) {
    uint16_t *kl = lds[buf][0], *vl = lds[buf][1];
#pragma unroll
    for (int i = 0; i < PER; i++) {
      *(uint4 *)(kl + (tr + RSTEP * i) * VS + tc) = kreg[i];
      *(uint4 *)(vl + (tr + RSTEP * i) * VS + tc) = vreg[i];
    }
    __syncthreads();
    if (kb + KB <= bhi) fetch(kb + KB);
    if (kb <= hi && kb + KB - 1 >= lo) {
      bf16x8 kf[4][HD / 32];
#pragma unroll
      for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int kk = 0; kk < HD / 32; kk++) kf[kt][kk] = *(const bf16x8 *)(kl + (16 * kt + n) * VS + 32 * kk + 8 * g);
      fold_block<HD, VS>(st, kf, qf, vl, kb, pr, lane);
    }
  }
  // the wave's own tile is complete: normalize and store its valid pairs (lane l: pairs 4g + i, column 16c + n)
  const float inv_n = st.l > 0.0f ? 1.0f / st.l : 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float inv = __shfl(inv_n, 4 * g + i, 64);
    const Pair pi = pair_of(a, kvh, 16 * t + 4 * g + i);
    if (!pi.valid) continue;
    uint16_t *out = (uint16_t *)a.out + pi.o;
#pragma unroll
    for (int c = 0; c < HD / 16; c++) out[16 * c + n] = (uint16_t)bf16_packed(st.o[c][i] * inv);
  }
}

struct AttnPlan {
  bool decode;
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
  if ((a->q | a->k | a->v) % 16 || a->q_sr % 8 || a->k_sr % 8 || a->v_sr % 8 || a->q_sh % 8 || a->k_sh % 8 ||
      a->v_sh % 8)
    return fail(BT_EINVAL, "attention needs q, k and v rows on 16-byte boundaries");
  if (a->places_sh != 0 && a->places_sh != a->rows) return fail(BT_EINVAL, "places' head stride is 0 or rows");
  if (((int64_t)(a->keys - 1) * std::max(a->k_sr, a->v_sr) + a->head_dim) * 2 >= (1ll << 32))
    return fail(BT_EINVAL, "a key head's rows must span less than 4 GiB");
  if (a->firsts && a->firsts % 4) return fail(BT_EINVAL, "attention's firsts must be int32-aligned");
  if (a->firsts && a->firsts_sh != 0 && a->firsts_sh != a->rows) return fail(BT_EINVAL, "firsts' head stride is 0 or rows");
  const int kvh = a->heads / a->rep, np = a->rep * a->rows;
  p->tiles = (np + 15) / 16;
  p->decode = p->tiles <= 4;  // few query rows for each key head: split the keys instead
  p->parts = 1, p->kpp = 0, p->scratch_bytes = 0;
  if (p->decode) {
    const int nblk = (a->keys + KB - 1) / KB;
    int parts = a->parts;
    if (parts == 0) parts = std::min((2048 + kvh * p->tiles - 1) / (kvh * p->tiles), (nblk + 3) / 4);
    p->parts = std::max(1, std::min(std::min(parts, nblk), MAX_PARTS));
    const int pf = 32 + 16 * a->head_dim;
    if (p->parts > 1) p->scratch_bytes = (uint64_t)kvh * p->tiles * p->parts * pf * 4;
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
  const int kvh = a->heads / a->rep;
  float *scratch = (float *)(uintptr_t)a->scratch;
  if (p.decode) {
    const unsigned blocks = (unsigned)(kvh * p.tiles * p.parts);
    if (a->head_dim == 64) attention_decode_kernel<64><<<blocks, 256, 0, r->stream>>>(*a, p.tiles, p.parts, scratch);
    else attention_decode_kernel<128><<<blocks, 256, 0, r->stream>>>(*a, p.tiles, p.parts, scratch);
    BT_LAUNCHED("attention");
    if (p.parts > 1) {
      const unsigned cb = (unsigned)(kvh * p.tiles);
      if (a->head_dim == 64) attention_combine_kernel<64><<<cb, 256, 0, r->stream>>>(*a, p.tiles, p.parts, scratch);
      else attention_combine_kernel<128><<<cb, 256, 0, r->stream>>>(*a, p.tiles, p.parts, scratch);
      BT_LAUNCHED("attention combine");
    }
  } else {
    const unsigned blocks = (unsigned)(kvh * ((p.tiles + 3) / 4));
    if (a->head_dim == 64) attention_prefill_kernel<64><<<blocks, 256, 0, r->stream>>>(*a, p.tiles);
    else attention_prefill_kernel<128><<<blocks, 256, 0, r->stream>>>(*a, p.tiles);
    BT_LAUNCHED("attention");
  }
  return BT_OK;
}

}  // extern "C"
