// Device arithmetic of the decode step's row kernels, shared by the kernels that run it on stored rows
// (elementwise.hip: bt_rope_put, bt_rms_rows) and the ones that run it on a product's split-K partial sums
// (matmul.hip: bt_matmul_rope_put, bt_matmul_residual_rms), so that fused and unfused give the same bits.
#pragma once
#include "program.h"

namespace bt {

// RoPE of 8 neighbouring pairs (j .. j + 7, j + d/2 .. j + d/2 + 7) of one head: y1 = x1 cos - x2 sin and
// y2 = x2 cos' + x1 sin' in fp32, products and sums rounded one by one (no fused multiply-add), packed to bf16 half
// up. xa, xb: the bf16 inputs at j and j + d/2; ca, cb, sa, sb: the tables at the same places.
__device__ __forceinline__ void rope8(const uint4 &xa, const uint4 &xb, const uint4 &ca, const uint4 &cb,
                                      const uint4 &sa, const uint4 &sb, uint4 &oa, uint4 &ob) {
  const uint32_t xw[2][4] = {{xa.x, xa.y, xa.z, xa.w}, {xb.x, xb.y, xb.z, xb.w}};
  const uint32_t cw[2][4] = {{ca.x, ca.y, ca.z, ca.w}, {cb.x, cb.y, cb.z, cb.w}};
  const uint32_t sw[2][4] = {{sa.x, sa.y, sa.z, sa.w}, {sb.x, sb.y, sb.z, sb.w}};
  uint32_t o[2][4];
#pragma unroll
  for (int w = 0; w < 4; w++) {
    o[0][w] = o[1][w] = 0u;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int sh = 16 * e;
      const float x1 = bf16_value(xw[0][w] >> sh & 0xFFFFu), x2 = bf16_value(xw[1][w] >> sh & 0xFFFFu);
      const float y1 = __fsub_rn(__fmul_rn(x1, bf16_value(cw[0][w] >> sh & 0xFFFFu)),
                                 __fmul_rn(x2, bf16_value(sw[0][w] >> sh & 0xFFFFu)));
      const float y2 = __fadd_rn(__fmul_rn(x2, bf16_value(cw[1][w] >> sh & 0xFFFFu)),
                                 __fmul_rn(x1, bf16_value(sw[1][w] >> sh & 0xFFFFu)));
      o[0][w] |= bf16_packed(y1) << sh;
      o[1][w] |= bf16_packed(y2) << sh;
    }
  }
  oa = make_uint4(o[0][0], o[0][1], o[0][2], o[0][3]);
  ob = make_uint4(o[1][0], o[1][1], o[1][2], o[1][3]);
}

// Where head hh of token i goes: q for a query head, else its cache row at the token's place (nullptr when the place
// is outside the cache), as bt_rope_put lays them out.
__device__ __forceinline__ uint16_t *rope_dst(const bt_rope_args &a, int i, int hh) {
  if (hh < a.heads) return (uint16_t *)(uintptr_t)a.q + (int64_t)i * a.q_sr + (int64_t)hh * a.head_dim;
  const int place = ((const int32_t *)(uintptr_t)a.places)[a.one_place ? 0 : i];
  if (place < 0 || place >= a.cache_rows) return nullptr;
  const int hk = hh - a.heads;
  const bool own = a.vcache && hk >= a.kv;  // a value head with a cache of its own
  return (uint16_t *)(uintptr_t)(own ? a.vcache : a.cache) + (int64_t)(own ? hk - a.kv : hk) * a.cache_sh +
         (int64_t)i * a.cache_tsh + (int64_t)place * a.cache_sr;
}

// RMSNorm of one row by a block of RMS_THREADS threads, the row held in registers: thread t holds columns
// (RMS_THREADS i + t) * 4 .. + 3 of group i < RMS_NV (zeros past k), already rounded to bf16 (half up), so every load
// of the row is issued before the first is used. Returns 1 / sqrt(mean of x^2 + eps); the sum is each thread's groups
// in order, then the wave's lanes (wave_sum), then the waves in order. part: RMS_THREADS / 64 floats of LDS.
constexpr int RMS_THREADS = 1024, RMS_NV = 2;  // 2 x 4 x 1024 = 8192 columns
__device__ __forceinline__ float rms_scale(const float4 (&v)[RMS_NV], int64_t k, float eps, float *part) {
  const int tid = threadIdx.x, lane = tid & 63, wib = tid >> 6;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < RMS_NV; i++) ss += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
  ss = wave_sum(ss);
  if (lane == 0) part[wib] = ss;
  __syncthreads();
  float total = part[0];
#pragma unroll
  for (int w = 1; w < RMS_THREADS / 64; w++) total += part[w];
  return 1.0f / sqrtf(total / (float)k + eps);
}

// The normalized row's bf16 values for group i: x * r * w, in fp32, packed half up.
__device__ __forceinline__ uint2 rms_out(const float4 &v, float r, const uint2 &w) {
  uint2 o;
  o.x = bf16_packed(v.x * r * bf16_value(w.x & 0xFFFFu)) | bf16_packed(v.y * r * bf16_value(w.x >> 16)) << 16;
  o.y = bf16_packed(v.z * r * bf16_value(w.y & 0xFFFFu)) | bf16_packed(v.w * r * bf16_value(w.y >> 16)) << 16;
  return o;
}

}  // namespace bt
