// KV-cache attention: out = softmax(q k^T + mask) v per query row, with the mask taken from each row's place (and a
// sliding window), scores, maxima and sums in fp32, and the output rounded to bf16 once.
//
// Semantics restated from the reference (in code of our own): tensor.py:797-841 (attend), kernels.py:794-1005
// (attention_kernel: fp32 maxima, exp(s - max), sums of p and p v in fp32, keys past a row's place never read),
// tensor.py:837-841 (parts combined by rescaling with e^(m_p - M)). Here the softmax is online: one sweep over the
// keys keeps the running maximum and rescales what has been summed, so K and V are each read once.
#include "common.h"

namespace bt {

// One wavefront a query row. Lanes take 64 keys at a time and score them against q; the wave then folds those scores
// into its running maximum and sum, and multiplies them into the output, each lane owning head_dim / 64 columns.
template <int HD>
__global__ void __launch_bounds__(256) attention_rows_kernel(const bt_attention_args a) {
  constexpr int PER = HD / 64;  // output columns per lane
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (int64_t)a.heads * a.rows) return;
  const int e = (int)(w / a.rows), r = (int)(w % a.rows), kv = e / a.rep;
  const int place = ((const int32_t *)a.places)[(int64_t)e * a.places_sh + r];
  const int lo = a.window > 0 ? max(0, place - a.window + 1) : 0, hi = min(place, a.keys - 1);
  const uint16_t *q = (const uint16_t *)a.q + (int64_t)e * a.q_sh + (int64_t)r * a.q_sr;
  const uint16_t *k = (const uint16_t *)a.k + (int64_t)kv * a.k_sh;
  const uint16_t *v = (const uint16_t *)a.v + (int64_t)kv * a.v_sh;
  float qf[HD];
#pragma unroll
  for (int d = 0; d < HD; d += 8) {
    uint4 x = *(const uint4 *)(q + d);
    uint32_t ws[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; i++) { qf[d + 2 * i] = bf16_value(ws[i] & 0xFFFF); qf[d + 2 * i + 1] = bf16_value(ws[i] >> 16); }
  }
  float m = -__builtin_inff(), l = 0.0f, acc[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) acc[i] = 0.0f;
  for (int j0 = lo; j0 <= hi; j0 += 64) {
    const int j = j0 + lane;
    float s = -__builtin_inff();
    if (j <= hi) {
      const uint16_t *kr = k + (int64_t)j * a.k_sr;
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; d += 8) {
        uint4 x = *(const uint4 *)(kr + d);
        uint32_t ws[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          dot = fmaf(qf[d + 2 * i], bf16_value(ws[i] & 0xFFFF), dot);
          dot = fmaf(qf[d + 2 * i + 1], bf16_value(ws[i] >> 16), dot);
        }
      }
      s = dot;
    }
    float cm = s;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o, 64));
    const float mn = fmaxf(m, cm);
    const float scale = __expf(m - mn);  // 0 on the first chunk, where m is -inf
    const float p = j <= hi ? __expf(s - mn) : 0.0f;
    float ps = p;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o, 64);
    l = l * scale + ps;
#pragma unroll
    for (int i = 0; i < PER; i++) acc[i] *= scale;
    const int n = min(64, hi - j0 + 1);
    for (int t = 0; t < n; t++) {
      const float pt = __shfl(p, t, 64);
      const uint16_t *vr = v + (int64_t)(j0 + t) * a.v_sr + lane * PER;
      if (PER == 2) {
        uint32_t x = *(const uint32_t *)vr;
        acc[0] = fmaf(pt, bf16_value(x & 0xFFFF), acc[0]);
        acc[PER - 1] = fmaf(pt, bf16_value(x >> 16), acc[PER - 1]);
      } else {
#pragma unroll
        for (int i = 0; i < PER; i++) acc[i] = fmaf(pt, bf16_value(vr[i]), acc[i]);
      }
    }
    m = mn;
  }
  uint16_t *o = (uint16_t *)a.out + (int64_t)e * a.o_sh + (int64_t)r * a.o_sr + lane * PER;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int i = 0; i < PER; i++) o[i] = (uint16_t)bf16_packed(acc[i] * inv);
}

}  // namespace bt

using namespace bt;

extern "C" int bt_attention(bt_runtime *rt, const bt_attention_args *a) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!a || !a->q || !a->k || !a->v || !a->out || !a->places) return fail(BT_EINVAL, "attention needs q, k, v, out, places");
  if (a->heads <= 0 || a->rep <= 0 || a->heads % a->rep || a->rows <= 0 || a->keys <= 0 || a->window < 0)
    return fail(BT_EINVAL, "attention shape: %d heads, rep %d, %d rows, %d keys, window %d", a->heads, a->rep, a->rows,
                a->keys, a->window);
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(BT_EINVAL, "attention takes heads 64 or 128 wide, not %d", a->head_dim);
  if ((a->q | a->k | a->v) % 16 || a->q_sr % 8 || a->k_sr % 8 || a->q_sh % 8 || a->k_sh % 8)
    return fail(BT_EINVAL, "attention needs q and k rows on 16-byte boundaries");
  if (a->places_sh != 0 && a->places_sh != a->rows) return fail(BT_EINVAL, "places' head stride is 0 or rows");
  int64_t waves = (int64_t)a->heads * a->rows;
  unsigned blocks = (unsigned)((waves + 3) / 4);
  if (a->head_dim == 64) attention_rows_kernel<64><<<blocks, 256, 0, r->stream>>>(*a);
  else attention_rows_kernel<128><<<blocks, 256, 0, r->stream>>>(*a);
  BT_LAUNCHED("attention");
  return BT_OK;
}
