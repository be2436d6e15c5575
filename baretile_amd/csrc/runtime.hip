// The runtime facade: a device, one in-order HIP stream per runtime, stream-ordered memory, host copies, a wait with a
// timeout, timing events and graph capture. Each entry point returns a status and leaves its message for
// bt_last_error().
#include "common.h"
#include <chrono>
#include <string>
#include <thread>

namespace bt {

static thread_local std::string last_error;

void set_error(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  last_error = buf;
}

int fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  last_error = buf;
  return code;
}

int enter(bt_runtime *rt, Runtime **out) {
  Runtime *r = reinterpret_cast<Runtime *>(rt);
  if (!r) return fail(BT_EINVAL, "no runtime");
  if (r->closed) return fail(BT_ESTATE, "the runtime is closed");
  BT_HIP(hipSetDevice(r->device));
  (void)hipGetLastError();  // an error left by an earlier call must not be blamed on this one's launch
  *out = r;
  return BT_OK;
}

// Fills words of 32 bits. A kernel rather than hipMemsetAsync, so that a captured graph holds no memset node.
__global__ void fill32_kernel(uint32_t *dst, uint32_t value, uint64_t words) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x, step = (uint64_t)gridDim.x * blockDim.x;
  for (; i < words; i += step) dst[i] = value;
}

// Reads n16 16-byte words once each, four per thread, and folds them into a word that is written only if it equals a
// value the data never gives: the plain streaming read that a measurement compares a kernel's HBM rate against, and the
// known-size read that calibrates the memory counters.
__global__ void __launch_bounds__(256) stream_read_kernel(const uint8_t *p, uint32_t bytes, uint32_t *out) {
  // 16 bytes a lane, four times, through a buffer resource whose range check drops the tail; loaded non-temporal
  // (sc1 nt), as a stream read once is
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p), (short)0, (int)bytes,
                                                                     0x00020000);
  const uint32_t base = (blockIdx.x * 1024u + threadIdx.x) * 16u;
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, base + i * 4096u, 0, 18);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == 0x9E3779B9u && out) out[0] = acc;
}

// One wave waits until `ticks` of the device's constant-rate wall clock have passed since it started, sleeping between
// reads, then ends: a launch that stays busy for a set time and always finishes by itself.
__global__ void sleep_kernel(uint64_t ticks, uint32_t *out) {
  const uint64_t start = wall_clock64();
  uint64_t now = start;
  while (now - start < ticks) {
    __builtin_amdgcn_s_sleep(127);
    now = wall_clock64();
  }
  if (out && now == start) out[0] = 1;  // never taken once ticks > 0; keeps the loop observable
}

// At most this much memory is kept for reuse, in blocks of at most KEEP_BLOCK; larger blocks go back to the pool.
constexpr uint64_t KEEP_BLOCK = 256ull << 20, KEEP_TOTAL = 4ull << 30;

// Gives every kept block back: the pool's in stream order, the plain ones once the stream has drained. Not inside a
// capture, where a free would be recorded into the graph. The caller holds blocks_lock.
int release_kept(Runtime *r) {
  std::vector<void *> plain;
  for (auto &size : r->kept)
    for (void *p : size.second) {
      auto b = r->blocks.find(p);
      if (b == r->blocks.end()) continue;  // every kept block is listed in blocks; this only guards the lookup
      if (b->second.plain) plain.push_back(p);
      else BT_HIP(hipFreeAsync(p, r->stream));
      r->blocks.erase(b);
    }
  r->kept.clear();
  r->kept_bytes = 0;
  if (!plain.empty()) BT_HIP(hipStreamSynchronize(r->stream));
  for (void *p : plain) BT_HIP(hipFree(p));
  return BT_OK;
}

}  // namespace bt

using namespace bt;

extern "C" {

const char *bt_last_error(void) { return last_error.c_str(); }

int bt_sleep(bt_runtime *rt, double seconds) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!(seconds >= 0 && seconds <= 10)) return fail(BT_EINVAL, "sleep takes 0 to 10 seconds, not %g", seconds);
  int khz = 0;
  BT_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, r->device));
  if (khz <= 0) return fail(BT_ESTATE, "the device reports no wall clock rate");
  const uint64_t ticks = (uint64_t)(seconds * 1000.0 * khz);
  if (!ticks) return BT_OK;
  sleep_kernel<<<1, 64, 0, r->stream>>>(ticks, nullptr);
  BT_LAUNCHED("sleep");
  return BT_OK;
}

int bt_stream_read(bt_runtime *rt, uint64_t src, uint64_t bytes, uint64_t scratch_word) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (src % 16 || bytes % 16) return fail(BT_EINVAL, "stream_read takes 16-byte aligned whole words");
  const uint64_t blocks = (bytes + 16383) / 16384;
  if (!blocks) return BT_OK;
  if (bytes > (1ull << 32) - 16384) return fail(BT_EINVAL, "stream_read of %llu bytes: at most 4 GB - 16 KB",
                                                (unsigned long long)bytes);
  stream_read_kernel<<<(unsigned)blocks, 256, 0, r->stream>>>((const uint8_t *)(uintptr_t)src, (uint32_t)bytes,
                                                              (uint32_t *)(uintptr_t)scratch_word);
  BT_LAUNCHED("stream_read");
  return BT_OK;
}

int bt_version(void) { return BT_ABI_VERSION; }

int bt_device_count(int *n) {
  if (!n) return fail(BT_EINVAL, "no result pointer");
  hipError_t e = hipGetDeviceCount(n);
  if (e == hipErrorNoDevice) { *n = 0; return BT_OK; }
  BT_HIP(e);
  return BT_OK;
}

int bt_open(int device, bt_runtime **out) {
  if (!out) return fail(BT_EINVAL, "no result pointer");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(BT_ESTATE, "no GPU is visible: %s", hipGetErrorString(e));
  if (device < 0 || device >= n) return fail(BT_EINVAL, "device %d outside 0..%d", device, n - 1);
  BT_HIP(hipSetDevice(device));
  hipDeviceProp_t p;
  BT_HIP(hipGetDeviceProperties(&p, device));
  if (std::string(p.gcnArchName).rfind("gfx950", 0) != 0)
    return fail(BT_ESTATE, "this library is built for gfx950, and device %d is %s", device, p.gcnArchName);
  attention_noalloc_init(device);  // the no-alloc attention's working memory on this device (a static array)
  Runtime *r = new Runtime;
  r->device = device;
  hipError_t s = hipStreamCreateWithFlags(&r->stream, hipStreamNonBlocking);
  if (s != hipSuccess) { delete r; return fail(BT_ESTATE, "hipStreamCreate: %s", hipGetErrorString(s)); }
  *out = reinterpret_cast<bt_runtime *>(r);
  return BT_OK;
}

int bt_close(bt_runtime *rt) {
  Runtime *r = reinterpret_cast<Runtime *>(rt);
  if (!r) return fail(BT_EINVAL, "no runtime");
  if (r->closed) return BT_OK;
  BT_HIP(hipSetDevice(r->device));
  if (r->capture_origin) return fail(BT_ESTATE, "close a runtime after ending its graph capture");
  {
    std::lock_guard<std::mutex> hold(r->blocks_lock);
    if (int s = release_kept(r)) return s;
  }
  BT_HIP(hipStreamSynchronize(r->stream));
  BT_HIP(hipStreamDestroy(r->stream));
  for (void *p : r->retired) (void)hipFree(p);
  if (r->scratch) (void)hipFree(r->scratch);
  r->closed = 1;
  delete r;
  return BT_OK;
}

}  // extern "C"

namespace bt {
void *runtime_scratch(Runtime *r, size_t bytes) {
  if (bytes <= r->scratch_bytes) return r->scratch;
  if (r->capture_origin) return nullptr;
  const size_t n = (bytes + (1u << 20) - 1) / (1u << 20) * (1u << 20);
  void *p = nullptr;
  if (hipMalloc(&p, n) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (r->scratch) r->retired.push_back(r->scratch);
  r->scratch = p, r->scratch_bytes = n;
  return p;
}
}  // namespace bt

extern "C" {

int bt_alloc(bt_runtime *rt, uint64_t bytes, uint64_t *addr) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!addr) return fail(BT_EINVAL, "no result pointer");
  const uint64_t n = bytes ? (bytes + 255) / 256 * 256 : 256;
  std::lock_guard<std::mutex> hold(r->blocks_lock);
  auto k = r->kept.find(n);
  if (k != r->kept.end() && !k->second.empty()) {  // a freed block of this size, reused in stream order
    void *p = k->second.back();
    k->second.pop_back();
    r->blocks[p].kept = false;
    *addr = (uint64_t)(uintptr_t)p;
    r->kept_bytes -= n;
    return BT_OK;
  }
  // Outside a capture, stream-ordered from the device's pool. Inside a capture, a plain allocation that outlives the
  // graph: the graph keeps using it on every replay.
  void *p = nullptr;
  hipError_t e = r->capture_origin ? hipMalloc(&p, n) : hipMallocAsync(&p, n, r->stream);
  if (e == hipErrorOutOfMemory && !r->capture_origin && r->kept_bytes) {  // give the kept blocks back and try again
    (void)hipGetLastError();
    if (int s = release_kept(r)) return s;
    e = hipMallocAsync(&p, n, r->stream);
  }
  if (e == hipErrorOutOfMemory) return fail(BT_ENOMEM, "out of device memory allocating %llu bytes", (unsigned long long)n);
  if (e != hipSuccess) return fail(BT_ESTATE, "allocating %llu bytes: %s", (unsigned long long)n, hipGetErrorString(e));
  r->blocks[p] = {n, r->capture_origin != nullptr, false};
  *addr = (uint64_t)(uintptr_t)p;
  return BT_OK;
}

int bt_free(bt_runtime *rt, uint64_t addr, int captured) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!addr) return BT_OK;
  void *p = (void *)(uintptr_t)addr;
  std::lock_guard<std::mutex> hold(r->blocks_lock);
  auto b = r->blocks.find(p);
  if (b != r->blocks.end()) {
    const uint64_t n = b->second.bytes;
    if (b->second.kept) return fail(BT_EINVAL, "address %#llx freed twice", (unsigned long long)addr);
    if (n <= KEEP_BLOCK && r->kept_bytes + n <= KEEP_TOTAL) {  // kept for the next allocation of its size
      r->kept[n].push_back(p);
      r->kept_bytes += n;
      b->second.kept = true;
      return BT_OK;
    }
    captured = b->second.plain;
    r->blocks.erase(b);
  }
  if (captured) {  // made while capturing: freed only once the stream has drained
    BT_HIP(hipStreamSynchronize(r->stream));
    BT_HIP(hipFree(p));
  } else {
    BT_HIP(hipFreeAsync(p, r->stream));
  }
  return BT_OK;
}

int bt_upload(bt_runtime *rt, uint64_t dst, const void *src, uint64_t bytes) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (r->capture_origin) return fail(BT_ESTATE, "a graph capture can't copy host memory");
  if (!bytes) return BT_OK;
  BT_HIP(hipMemcpyAsync((void *)(uintptr_t)dst, src, bytes, hipMemcpyHostToDevice, r->stream));
  BT_HIP(hipStreamSynchronize(r->stream));  // the caller's buffer may go away on return
  return BT_OK;
}

int bt_download(bt_runtime *rt, void *dst, uint64_t src, uint64_t bytes) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (r->capture_origin) return fail(BT_ESTATE, "a graph capture can't read back to the host");
  if (!bytes) return BT_OK;
  BT_HIP(hipMemcpyAsync(dst, (const void *)(uintptr_t)src, bytes, hipMemcpyDeviceToHost, r->stream));
  BT_HIP(hipStreamSynchronize(r->stream));
  return BT_OK;
}

int bt_copy(bt_runtime *rt, uint64_t dst, uint64_t src, uint64_t bytes) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!bytes) return BT_OK;
  BT_HIP(hipMemcpyAsync((void *)(uintptr_t)dst, (const void *)(uintptr_t)src, bytes, hipMemcpyDeviceToDevice,
                        r->stream));
  return BT_OK;
}

int bt_fill32(bt_runtime *rt, uint64_t dst, uint32_t value, uint64_t words) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!words) return BT_OK;
  if (dst % 4) return fail(BT_EINVAL, "fill32 needs a 4-byte aligned address");
  uint64_t blocks = (words + 255) / 256;
  fill32_kernel<<<(unsigned)(blocks < 4096 ? blocks : 4096), 256, 0, r->stream>>>((uint32_t *)(uintptr_t)dst, value,
                                                                                  words);
  BT_LAUNCHED("fill32");
  return BT_OK;
}

int bt_wait(bt_runtime *rt, double timeout_s) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (r->capture_origin) return fail(BT_ESTATE, "can't wait while a graph capture is open");
  auto start = std::chrono::steady_clock::now();
  for (int spins = 0;; spins++) {
    hipError_t e = hipStreamQuery(r->stream);
    if (e == hipSuccess) return BT_OK;
    if (e != hipErrorNotReady) return fail(BT_ESTATE, "waiting for the stream: %s", hipGetErrorString(e));
    double waited = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
    if (timeout_s >= 0 && waited > timeout_s)
      return fail(BT_ETIMEOUT, "launches still running after %.1f s", timeout_s);
    if (spins > 64) std::this_thread::sleep_for(std::chrono::microseconds(spins > 4096 ? 1000 : 20));
  }
}

int bt_event_create(bt_runtime *rt, void **ev) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  hipEvent_t e;
  BT_HIP(hipEventCreate(&e));
  *ev = (void *)e;
  return BT_OK;
}

int bt_event_record(bt_runtime *rt, void *ev) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  BT_HIP(hipEventRecord((hipEvent_t)ev, r->stream));
  return BT_OK;
}

int bt_event_elapsed(void *start, void *end, float *ms) {
  BT_HIP(hipEventSynchronize((hipEvent_t)end));
  BT_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
  return BT_OK;
}

int bt_event_destroy(void *ev) {
  BT_HIP(hipEventDestroy((hipEvent_t)ev));
  return BT_OK;
}

int bt_graph_begin(bt_runtime *rt) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (r->capture_origin) return fail(BT_ESTATE, "a graph capture is already open on this runtime");
  BT_HIP(hipStreamBeginCapture(r->stream, hipStreamCaptureModeRelaxed));
  r->capture_origin = r->stream;
  return BT_OK;
}

int bt_graph_end(bt_runtime *rt, void **exec) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (!r->capture_origin) return fail(BT_ESTATE, "no graph capture is open");
  hipGraph_t g = nullptr;
  r->capture_origin = nullptr;
  BT_HIP(hipStreamEndCapture(r->stream, &g));
  hipGraphExec_t x = nullptr;
  hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return fail(BT_ESTATE, "instantiating the graph: %s", hipGetErrorString(e));
  // the executable graph's device-side state (its kernel packets and arguments) goes to the device now, queued on
  // the stream, rather than as part of its first launch
  e = hipGraphUpload(x, r->stream);
  if (e != hipSuccess) {
    (void)hipGraphExecDestroy(x);
    return fail(BT_ESTATE, "uploading the graph: %s", hipGetErrorString(e));
  }
  *exec = (void *)x;
  return BT_OK;
}

int bt_graph_launch(bt_runtime *rt, void *exec) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  if (r->capture_origin) return fail(BT_ESTATE, "can't replay a graph while capturing");
  BT_HIP(hipGraphLaunch((hipGraphExec_t)exec, r->stream));
  return BT_OK;
}

int bt_graph_destroy(void *exec) {
  if (exec) BT_HIP(hipGraphExecDestroy((hipGraphExec_t)exec));
  return BT_OK;
}

int bt_stream(bt_runtime *rt, void **stream) {
  Runtime *r;
  if (int s = enter(rt, &r)) return s;
  *stream = (void *)r->stream;
  return BT_OK;
}

}  // extern "C"
