// Shared definitions of the baretile_amd HIP library: status codes, the per-thread error text, and the number rules
// that every kernel applies (bf16 rounding, block-float fields). gfx950 only.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstdarg>
#include <mutex>
#include <unordered_map>
#include <vector>
#include "../../include/baretile_amd.h"

namespace bt {

// Loads through the global address space, so the compiler emits global_load (vector memory only) rather than flat,
// whose wait also waits for LDS. (The host pass of hipcc also parses device functions, and has no such address space.)
template <class T> __device__ __forceinline__ T gload(const T *p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return *(const __attribute__((address_space(1))) T *)p;
#else
  return *p;
#endif
}

// The sum of x over the wave's 64 lanes, in every lane, with no trip through LDS: lanes l and l ^ 32, then l ^ 16
// (VALU lane swaps, v_permlane32_swap / v_permlane16_swap with both operands x), then within 16-lane rows by DPP
// moves: l ^ 8 (row_ror 8), l and 7 - l of each half-row (row_half_mirror), then l ^ 2 and l ^ 1 (quad_perm). Each
// step pairs lanes symmetrically and adds the pair, so every lane ends with the same bits.
__device__ __forceinline__ float wave_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  x += __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x128, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x141, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0x4E, 0xF, 0xF, false));
  return x + __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), 0xB1, 0xF, 0xF, false));
}

// The last error's text, per host thread. Set by fail(), read through bt_last_error().
void set_error(const char *fmt, ...);
// fail(BT_EINVAL, "...") records the message and returns the code, so entry points can `return fail(...)`.
int fail(int code, const char *fmt, ...);

#define BT_HIP(call)                                                                                           \
  do {                                                                                                         \
    hipError_t e_ = (call);                                                                                    \
    if (e_ != hipSuccess) return ::bt::fail(e_ == hipErrorOutOfMemory ? BT_ENOMEM : BT_ESTATE, "%s: %s (%s:%d)", \
                                            #call, hipGetErrorString(e_), __FILE__, __LINE__);                  \
  } while (0)

// A launch's own error, read right after the <<<>>> so a bad configuration names its kernel.
#define BT_LAUNCHED(name)                                                                                      \
  do {                                                                                                         \
    hipError_t e_ = hipGetLastError();                                                                         \
    if (e_ != hipSuccess) return ::bt::fail(BT_ESTATE, "launching %s: %s", name, hipGetErrorString(e_));       \
  } while (0)

struct Runtime {
  int device = 0;
  hipStream_t stream = nullptr;
  hipStream_t capture_origin = nullptr;  // non-null while bt_graph_begin has the stream in capture
  int closed = 0;
  // Working memory of the library's own kernels (a matmul's B unpacked to bf16), used in stream order. It only
  // grows, outside a capture; a smaller one it replaces is kept until the runtime closes, as a recorded graph may
  // still use it.
  void *scratch = nullptr;
  size_t scratch_bytes = 0;
  std::vector<void *> retired;
  // Every block bt_alloc handed out (bytes: a multiple of 256; plain: made by hipMalloc inside a capture, else taken
  // from the device's stream-ordered pool), and the freed ones kept by size for the next allocation of that size.
  // Every launch of the runtime goes to its one stream, so a block freed after the launches that use it can serve a
  // later allocation at once, in stream order, as the pool would, without the pool's cost on every call (about 10 us
  // a free, which made a one-token decode step bound by its host code).
  struct Block {
    uint64_t bytes;
    bool plain, kept;
  };
  std::mutex blocks_lock;  // ctypes lets go of Python's lock for each call, and a tensor may be freed on any thread
  std::unordered_map<void *, Block> blocks;
  std::unordered_map<uint64_t, std::vector<void *>> kept;
  uint64_t kept_bytes = 0;
};

// The runtime's scratch of at least `bytes`, or null: inside a capture when it would have to grow (the caller then
// takes a way that needs none), or when the device is out of memory.
void *runtime_scratch(Runtime *r, size_t bytes);

// Looks up, with `device` current, the address of that device's copy of bt_attention_noalloc's working memory
// (attention.hip); bt_open calls it once per runtime.
#define BT_MAX_DEVICES 64
void attention_noalloc_init(int device);

// Checks a runtime handle and makes its device current.
int enter(bt_runtime *rt, Runtime **out);

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// ---- number rules (device) -------------------------------------------------------------------------------------

// fp32 -> bf16 bits, round to nearest even, no NaN special case: the host upload rule and the bfp cast's first step.
__device__ __forceinline__ uint32_t bf16_rne(float x) {
  uint32_t b = __float_as_uint(x);
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}
// fp32 -> bf16 bits, round half up in magnitude: how a computed bf16 result is packed.
__device__ __forceinline__ uint32_t bf16_packed(float x) { return (__float_as_uint(x) + 0x8000u) >> 16; }
__device__ __forceinline__ float bf16_value(uint32_t bits) { return __uint_as_float(bits << 16); }
// A value rounded the way a bf16 kernel rounds each result it computes.
__device__ __forceinline__ float round_packed(float x) { return bf16_value(bf16_packed(x)); }

// The block-float magnitude of one bf16 value below its run's largest exponent `top`: bfp8 keeps 7 bits rounded half
// up, bfp4 3 bits rounded to nearest with ties up. The exponent gap saturates at 8, and the result at 127 / 7.
template <int BITS>
__device__ __forceinline__ int bfp_magnitude(uint32_t b, uint32_t top) {
  uint32_t e = (b >> 7) & 255u, m = (b & 127u) | (e ? 128u : 0u);
  uint32_t shift = min(top - e, 8u);
  uint32_t q = BITS == 8 ? (m + (1u << shift)) >> (shift + 1) : (m + (16u << shift)) >> (shift + 5);
  return (int)min(q, BITS == 8 ? 127u : 7u);
}
// The signed q of a value: the magnitude with the value's sign, and 0 without one.
template <int BITS>
__device__ __forceinline__ int bfp_signed(uint32_t b, uint32_t top) {
  int q = bfp_magnitude<BITS>(b, top);
  return (b >> 15) & 1u ? -q : q;
}

// The unpacker's exact bf16 bits for a signed magnitude q (|q| <= 127, bfp4's 3 bits already shifted up by 4) under
// exponent byte e: the magnitude normalized, the exponent (e - shift) mod 256. q == 0 gives +0.
__device__ __forceinline__ uint32_t unpacked_bits(int q, uint32_t e) {
  if (q == 0) return 0;
  uint32_t s = q < 0, mag = (uint32_t)(q < 0 ? -q : q);
  uint32_t m = mag << 1;                       // 8 bits with the top one set once normalized
  uint32_t shift = __clz(m) - 24;              // leading zeros within the byte
  return s << 15 | ((e - shift) & 255u) << 7 | ((m << shift) & 0x7Eu);
}

}  // namespace bt
