"""Benchmark of baretile's hot path on one MI355X: the decode GEMV on block-float weights.

A step is one launch of the fused matmul kernel for x [B, 576] @ W [576, 49152] with W packed as bfp4 (the headline,
B = 1) or bfp8, fp32 accumulation and a bf16 result. Inputs are resident in HBM before timing starts. Each step reads a
different copy of W from a pool larger than the 256 MB Infinity Cache, so every step streams its weights from HBM.
Steps are captured into one HIP graph and replayed, and HIP events on the runtime's stream bracket the timed replay.

`value` is the achieved HBM bandwidth of the headline configuration: the algorithmic bytes of one step (packed W, x
and the output) over the measured time per step. The other five configurations (bfp4 and bfp8 at B = 1, 4, 16) are
reported in "configs". The CPU baseline is the NumPy restatement of the reference's path (oracle/), timed on the host
cores on a bounded sample of the same workload.

python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse, ctypes, json, os, sys, time
from ctypes import byref, c_float, c_void_p
import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path: sys.path.insert(0, ROOT)

K_DIM, N_DIM = 576, 49152
PEAK_GBS = 8000.0  # MI355X HBM3E
POOL_BYTES = 320 << 20  # > 256 MB Infinity Cache


def step_bytes(fmt, rows):
  bpv = 1088 / 1024 if fmt == "bfp8" else 576 / 1024
  return int(K_DIM * N_DIM * bpv + rows * K_DIM * 2 + rows * N_DIM * 2)


def weight_bytes(fmt):  # the packed weight alone: 64 x 16 tiles of 1088 (bfp8) or 576 (bfp4) bytes
  return (N_DIM // 16) * (K_DIM // 64) * (1088 if fmt == "bfp8" else 576)


def log(*a):
  print(*a, file=sys.stderr, flush=True)


def gpu_leg(fmt, rows, steps, warmup):
  """Times `steps` GEMV launches on one GPU, then a plain streaming read of the same weight bytes. Returns
  (us per GEMV, its result, x, w, us per streaming read)."""
  from baretile_amd import _lib
  from baretile_amd.runtime import Runtime
  rt = Runtime()
  try:
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, (rows, K_DIM)).astype(np.float32)
    w = rng.normal(0, 0.02, (K_DIM, N_DIM)).astype(np.float32)
    code = _lib.BFP8 if fmt == "bfp8" else _lib.BFP4
    # bf16 of W and x, rounded to nearest even as an upload is
    wb = w.view(np.uint32).astype(np.uint64)
    wb = ((wb + 0x7FFF + (wb >> 16 & 1)) >> 16).astype(np.uint16)
    xb = x.view(np.uint32).astype(np.uint64)
    xb = ((xb + 0x7FFF + (xb >> 16 & 1)) >> 16).astype(np.uint16)
    dw = rt.dram_alloc(wb.nbytes)
    rt.upload(dw, wb.tobytes())
    runs = N_DIM // 16
    exps = rt.dram_alloc(K_DIM * runs)
    vals = rt.dram_alloc(K_DIM * N_DIM // (1 if fmt == "bfp8" else 2))
    rt.run("pack", "bfp_pack", code, dw, _lib.BF16, 1, K_DIM, N_DIM, K_DIM * N_DIM, N_DIM, 1, exps, vals)
    tile = 1088 if fmt == "bfp8" else 576
    wbytes = runs * (K_DIM // 64) * tile
    copies = max(2, -(-POOL_BYTES // wbytes))
    pool = [rt.dram_alloc(wbytes) for _ in range(copies)]
    for p in pool: rt.run("columns", "bfp_columns", code, exps, vals, 1, K_DIM, N_DIM, p)
    dx = rt.dram_alloc(xb.nbytes)
    rt.upload(dx, xb.tobytes())
    out = rt.dram_alloc(rows * N_DIM * 2)
    a = _lib.operand(dx, "bf16", rows * K_DIM, K_DIM, 1)
    o = _lib.operand(out, "bf16", rows * N_DIM, N_DIM, 1)
    rt.wait()

    def launch(i):
      _lib.call("matmul", rt.handle, byref(a), code, pool[i % copies], 1, 1, rows, K_DIM, N_DIM, None, byref(o))

    def timed(fn, warm):
      """us per launch of fn(i) for i < steps, captured into one graph and replayed between two events."""
      for i in range(3): fn(i)  # the first launches load the code object
      rt.wait()
      graph = c_void_p()
      _lib.call("graph_begin", rt.handle)
      for i in range(steps): fn(i)
      _lib.call("graph_end", rt.handle, byref(graph))
      for _ in range(max(1, warm // max(1, steps)) if warm else 0): _lib.call("graph_launch", rt.handle, graph)
      rt.wait()
      start, end = c_void_p(), c_void_p()
      _lib.call("event_create", rt.handle, byref(start))
      _lib.call("event_create", rt.handle, byref(end))
      _lib.call("event_record", rt.handle, start)
      _lib.call("graph_launch", rt.handle, graph)
      _lib.call("event_record", rt.handle, end)
      ms = c_float()
      _lib.call("event_elapsed", start, end, byref(ms))
      rt.wait()
      _lib.call("graph_destroy", graph)
      _lib.call("event_destroy", start)
      _lib.call("event_destroy", end)
      return ms.value * 1000 / steps

    us = timed(launch, warmup)
    # the result is checked against the oracle's values on a few columns, so a fast wrong kernel can't report
    got = np.frombuffer(bytes(rt.download(out, rows * N_DIM * 2)), np.uint16).reshape(rows, N_DIM)
    # the same weight bytes read by a plain streaming kernel, from the same pool: what one launch of this size can get
    word = rt.dram_alloc(256)
    read_us = timed(lambda i: _lib.call("stream_read", rt.handle, pool[i % copies], wbytes // 16 * 16, word), steps)
    return us, got, x, w, read_us
  finally:
    rt.close()


def check(got, x, w, fmt):
  from oracle import bfp as B, ops
  cols = (np.arange(0, N_DIM // 16, 61)[:, None] * 16 + np.arange(16)).reshape(-1)  # whole runs of 16 columns
  xw, wq = B.bf16(x), B.bfp(w[:, cols], fmt)
  want, bound = ops.matmul(xw, wq), ops.matmul_bound(xw, wq)
  val = (got[:, cols].astype(np.uint32) << 16).view(np.float32)
  return bool(np.all(np.abs(val - want) <= bound))


def measured_traffic():
  """HBM bytes per launch of the headline kernel, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
  (profiles/gemv_bfp4_B1_lmhead_traffic.json: per-dispatch counters scaled by a streaming read of known size)."""
  path = os.path.join(ROOT, "profiles", "gemv_bfp4_B1_lmhead_traffic.json")
  try:
    with open(path) as f: return json.load(f)["traffic_bytes_per_launch"]
  except (OSError, KeyError, ValueError):
    return None


def cpu_leg(fmt, rows, seconds=10.0):
  """NumPy float32 x @ Wdeq on the host (the oracle's matmul of the block-float values), W dequantized outside the
  timer. Runs whole GEMVs until `seconds` have passed."""
  from oracle import bfp as B
  rng = np.random.default_rng(0)
  x = B.bf16(rng.normal(0, 1, (rows, K_DIM))).astype(np.float32)
  w = B.bfp(rng.normal(0, 0.02, (K_DIM, N_DIM)).astype(np.float32), fmt).astype(np.float32)
  x @ w
  n, start = 0, time.perf_counter()
  while time.perf_counter() - start < seconds:
    x @ w
    n += 1
  per = (time.perf_counter() - start) / n
  return per * 1e6, n


def blas_threads():
  try:
    from threadpoolctl import threadpool_info
    info = [i for i in threadpool_info() if i.get("user_api") == "blas"]
    if info: return int(info[0].get("num_threads", os.cpu_count())), info[0].get("internal_api", "?")
  except Exception:
    pass
  return os.cpu_count(), "?"


def main():
  ap = argparse.ArgumentParser()
  ap.add_argument("--gpus", type=int, default=1)
  ap.add_argument("--steps", type=int, default=400)
  ap.add_argument("--warmup", type=int, default=400)
  ap.add_argument("--cpu-seconds", type=float, default=10.0)
  ap.add_argument("--no-cpu", action="store_true")
  ap.add_argument("--only", default=None, help="time one configuration, e.g. bfp4_B1 (for profiling runs)")
  args = ap.parse_args()
  if args.gpus != 1:
    print(f"bench.py runs on one GPU: this build has no multi-GPU path, and --gpus {args.gpus} is not supported",
          file=sys.stderr)
    sys.exit(2)
  configs = {}
  for fmt in ("bfp4", "bfp8"):
    for rows in (1, 4, 16):
      if args.only and args.only != f"{fmt}_B{rows}": continue
      steps = args.steps if (fmt, rows) == ("bfp4", 1) else max(50, args.steps // 4)
      us, got, x, w, read_us = gpu_leg(fmt, rows, steps, args.warmup if (fmt, rows) == ("bfp4", 1) else steps)
      ok = check(got, x, w, fmt)
      gbs = step_bytes(fmt, rows) / us / 1e3
      wb = weight_bytes(fmt)
      configs[f"{fmt}_B{rows}"] = {"us_per_step": round(us, 3), "GB/s": round(gbs, 1),
                                   "frac_hbm_peak": round(gbs / PEAK_GBS, 4), "bytes": step_bytes(fmt, rows),
                                   "steps": steps, "parity": ok,
                                   "stream_read_us": round(read_us, 3), "stream_read_GB/s": round(wb / read_us / 1e3, 1),
                                   "frac_of_stream_read": round(read_us / us, 4)}
      log(fmt, rows, configs[f"{fmt}_B{rows}"])
  head = configs.get("bfp4_B1") or next(iter(configs.values()))
  cpu = None
  if not args.no_cpu:
    us_cpu, n = cpu_leg("bfp4", 1, args.cpu_seconds)
    threads, api = blas_threads()
    cpu = {"value": round(step_bytes("bfp4", 1) / us_cpu / 1e3, 3), "unit": "GB/s", "cores": threads,
           "kind": "port", "sample": f"{n} whole GEMVs x[1,576] @ W[576,49152] (bfp4 values dequantized to float32 "
           f"outside the timer) with NumPy float32 ({api} BLAS), {us_cpu:.0f} us each"}
  line = {
    "metric": "bfp4/bfp8 GEMV HBM GB/s (%peak); decode tok/s, SmolLM-135M shape, 1 GPU",
    "value": head["GB/s"], "unit": "GB/s", "n_gpus": 1, "steps": head["steps"], "warmup": args.warmup,
    "ms_per_step": round(head["us_per_step"] / 1000, 6), "higher_is_better": True, "scaling": "weak",
    "vs_baseline": None, "dtype": "bfp4 weights, bf16 activations, fp32 accumulate", "data": "synthetic",
    "config": {"workload": "decode GEMV x[1,576] @ W[576,49152] bfp4 (BASELINE config 2, B=1)", "batch_rows": 1,
               "K": K_DIM, "N": N_DIM, "weight_pool_bytes": POOL_BYTES},
    "roofline": {"bound": "hbm", "achieved": head["GB/s"], "peak": PEAK_GBS, "unit": "GB/s",
                 "frac": head["frac_hbm_peak"], "traffic": measured_traffic()},
    "cpu_baseline": cpu,
    "configs": configs,
  }
  print(json.dumps(line), flush=True)


if __name__ == "__main__":
  main()
