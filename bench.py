"""Benchmark of baretile's hot path on one MI355X.

The headline is the decode GEMV on block-float weights: one launch of the fused matmul kernel for
x [B, 576] @ W [576, 49152] with W packed as bfp4 (B = 1) or bfp8, fp32 accumulation and a bf16 result. Inputs are
resident in HBM before timing starts. Each step reads a different copy of W from a pool larger than the 256 MB
Infinity Cache, so every step streams its weights from HBM. The steps are launched back to back on the runtime's
stream between two HIP events, queued behind a device-side wait that lasts until the host has queued them all, so the
events bracket the launches' device time and not the host's time to queue them. The pool holds 1 GiB of copies, four
times the Infinity Cache, and every launch takes the next copy in a cursor that runs on across the warmup and timed
launches, so a timed launch reads a copy last touched more than 600 MB of traffic earlier, whatever --steps is.
`value` is the achieved HBM bandwidth of the headline configuration: the algorithmic bytes of one step (packed W, x
and the output) over the measured time per step. The other five GEMV configurations (bfp4 and bfp8 at B = 1, 4, 16)
are in "configs". The other legs time HIP graph replays of their steps the same way.

The other BASELINE configurations are reported beside it, each against its own roofline:
  "c1"        config 1, relu(x @ W) with x [128, 576] and W [576, 1536] in bfp8, in one launch;
  "attention" config 4, KV-cache attention alone: decode at 512, 4096 and 16384 keys at batch 1 and 8, and a 2048-row
              causal prefill, 32 query and 8 key heads of 128;
  "layer"     config 5, one Llama-3-8B-shaped block with bfp4 projections: a 2048-token prefill, then a batch-32
              decode step against 4096 cached rows;
  "decode"    config 3, SmolLM-135M-shaped greedy decode: tok/s, and the token streams against the NumPy oracle.
The CPU baselines are the NumPy restatement of the reference's path (oracle/), timed on the host cores on bounded
samples of the same workloads.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME] [--no-cpu]
"""
import argparse, ctypes, json, os, sys, time
from ctypes import byref, c_float, c_void_p
import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path: sys.path.insert(0, ROOT)

K_DIM, N_DIM = 576, 49152
PEAK_GBS = 8000.0  # MI355X HBM3E
POOL_BYTES = 1 << 30  # four times the 256 MB Infinity Cache


def step_bytes(fmt, rows):
  bpv = 1088 / 1024 if fmt == "bfp8" else 576 / 1024
  return int(K_DIM * N_DIM * bpv + rows * K_DIM * 2 + rows * N_DIM * 2)


def weight_bytes(fmt):  # the packed weight alone: 64 x 16 tiles of 1088 (bfp8) or 576 (bfp4) bytes
  return (N_DIM // 16) * (K_DIM // 64) * (1088 if fmt == "bfp8" else 576)


def log(*a):
  print(*a, file=sys.stderr, flush=True)


def gpu_leg(fmt, rows, steps, warmup):
  """Times `steps` GEMV launches on one GPU, then a plain streaming read of the same weight bytes, then a launch that
  does almost nothing, each as `steps` launches back to back. Returns (us per GEMV, its result, x, w, us per streaming
  read, us per near-empty launch)."""
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
    cursor = [0]  # the next copy: runs on across every graph captured here
    dx = rt.dram_alloc(xb.nbytes)
    rt.upload(dx, xb.tobytes())
    out = rt.dram_alloc(rows * N_DIM * 2)
    a = _lib.operand(dx, "bf16", rows * K_DIM, K_DIM, 1)
    o = _lib.operand(out, "bf16", rows * N_DIM, N_DIM, 1)
    rt.wait()

    def launch(i):
      _lib.call("matmul", rt.handle, byref(a), code, pool[cursor[0] % copies], 1, 1, rows, K_DIM, N_DIM, None, byref(o))
      cursor[0] += 1

    def timed(fn, warm):
      """us per launch of fn(i) for i < steps: the launches queued back to back on the runtime's stream, behind a
      device-side hold long enough for the host to queue them all, between two events."""
      for i in range(3): fn(i)  # the first launches load the code object
      rt.wait()
      for i in range(warm): fn(i)  # the untimed steps
      rt.wait()
      start, end = c_void_p(), c_void_p()
      _lib.call("event_create", rt.handle, byref(start))
      _lib.call("event_create", rt.handle, byref(end))
      hold(rt, steps)
      _lib.call("event_record", rt.handle, start)
      for i in range(steps): fn(i)
      _lib.call("event_record", rt.handle, end)
      ms = c_float()
      rt.wait()
      _lib.call("event_elapsed", start, end, byref(ms))
      _lib.call("event_destroy", start)
      _lib.call("event_destroy", end)
      return ms.value * 1000 / steps

    us = timed(launch, warmup)
    # the result is checked against the oracle's values on a few columns, so a fast wrong kernel can't report
    got = np.frombuffer(bytes(rt.download(out, rows * N_DIM * 2)), np.uint16).reshape(rows, N_DIM)
    # the same weight bytes read by a plain streaming kernel, from the same pool: what one launch of this size can get
    word = rt.dram_alloc(256)
    def read(i):
      _lib.call("stream_read", rt.handle, pool[cursor[0] % copies], wbytes // 16 * 16, word)
      cursor[0] += 1
    read_us = timed(read, steps)
    # the fixed cost of a launch in such a graph: a kernel that writes one word and reads nothing
    floor_us = timed(lambda i: _lib.call("fill32", rt.handle, word, 0, 1), steps)
    return us, got, x, w, read_us, floor_us
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


def timed_cpu(fn, seconds, threads=None):
  """(seconds per call, calls) of fn() repeated for `seconds` after one untimed call; with threads, BLAS is held to
  that many threads meanwhile."""
  from contextlib import nullcontext
  try:
    from threadpoolctl import threadpool_limits
    limit = threadpool_limits(threads) if threads else nullcontext()
  except ImportError:
    limit = nullcontext()
  with limit:
    fn()
    n, start = 0, time.perf_counter()
    while time.perf_counter() - start < seconds or n < 1:
      fn()
      n += 1
  return (time.perf_counter() - start) / n, n


def cpu_leg(fmt, rows, seconds=10.0, threads=None):
  """NumPy float32 x @ Wdeq on the host (the oracle's matmul of the block-float values), W dequantized outside the
  timer. Runs whole GEMVs until `seconds` have passed."""
  from oracle import bfp as B
  rng = np.random.default_rng(0)
  x = B.bf16(rng.normal(0, 1, (rows, K_DIM))).astype(np.float32)
  w = B.bfp(rng.normal(0, 0.02, (K_DIM, N_DIM)).astype(np.float32), fmt).astype(np.float32)
  per, n = timed_cpu(lambda: x @ w, seconds, threads)
  return per * 1e6, n


def decode_leg(tokens=128, prompt_len=32, check=True, replay=True):
  """greedy decode of a SmolLM-135M-shaped Llama (30 layers, 576 wide, 9/3 heads of 64, FFN 1536,
  vocab 49152) with random weights (linears N(0, 0.02), norms N(1, 0.1), embedding N(0, 1), seed 0), bfp8 linears
  and tied output layer, bf16 norms, embedding and KV cache, a 32-token uniform prompt and 128 new tokens.

  The device runs the stream twice: autonomously (timed: each step picks its token on the device and feeds it to the
  next, llama.greedy_steps; tok/s counts the tokens after the prompt's pick over their time, and the steady rate is
  the time that the second half of the tokens adds to a stream of the first half) and NumPy-fed (the oracle's picks
  fed, gpt2.py:147-161). The oracle (oracle/llama_ref.py) runs the same decode on the host; its per-token time is the
  CPU baseline. Returns a dict of tok/s, token identity and per-step logit error against the oracle."""
  from oracle import llama_ref as L
  from baretile_amd.models import llama
  from baretile_amd.runtime import Runtime
  size = prompt_len + tokens
  t0 = time.perf_counter()
  c, w = L.smol(np.random.default_rng(0), 30, vocab=49152, places=size)
  prompt = [int(i) for i in np.random.default_rng(1).integers(0, 49152, prompt_len)]
  log("decode: weights made in", round(time.perf_counter() - t0, 1), "s")
  rt = Runtime()
  try:
    dc = llama.model(dim=576, heads=9, kv=3, layers=30, eps=1e-5, theta=10000.0, vocab=49152, ffn=1536,
                     precision=llama.precision(llama.model(layers=30, dim=576), "bfp8"))
    host = {k: v for k, v in w.items() if k not in ("cos", "sin", "turn", "embed.T")}
    dw = llama.upload(rt, host, dc, places=size)
    rt.wait()
    llama.generate(dw, dc, prompt, 4, size, replay=replay)  # loads the code objects
    def stream(n):  # n tokens: (picks, logits, prefill and first pick in s, the other n - 1 tokens in s)
      clock = []
      start = time.perf_counter()
      toks, logits = llama.generate(dw, dc, prompt, n, size, clock=clock, replay=replay)
      return toks, logits, clock[0] - start, clock[-1] - clock[0]
    toks, logits, first, span = stream(tokens)
    half = tokens // 2
    steady = (span - stream(half)[3]) / (tokens - half)  # a token more in a longer stream: one replayed step
    # bytes a token reads: every bfp8 linear and the tied head, the norms, one embedding row, and the keys and values of
    # the positions it attends to (the cache holds prompt_len + step rows at step)
    wb = 30 * (576 * 960 + 576 * 576 + 576 * 3072 + 1536 * 576) * 1088 // 1024 + 576 * 49152 * 1088 // 1024
    ctx = prompt_len + (tokens - 1) / 2
    per_token = wb + 61 * 576 * 2 + 576 * 2 + int(30 * 2 * 3 * 64 * 2 * ctx)
    out = {"tok/s": round((tokens - 1) / span, 1), "steady_tok/s": round(1 / steady, 1),
           "roofline": {"bound": "hbm", "bytes_per_token": per_token, "unit": "GB/s",
                        "achieved": round(per_token / steady / 1e9, 1), "peak": PEAK_GBS,
                        "frac": round(per_token / steady / 1e9 / PEAK_GBS, 4),
                        "note": "the weights fit the 256 MB Infinity Cache, so this bound is loose: the step is "
                                "launch- and latency-bound"},
           "ms_per_token": round(1000 * span / (tokens - 1), 4),
           "prefill_ms": round(1000 * first, 3), "tokens": tokens, "prompt": prompt_len, "graph_replay": replay,
           "kernels_per_token": None}
    caches, stats = llama.kv_cache(rt, dc, size), {}
    if replay:  # what a replayed step holds
      llama.greedy_steps(dw, dc, caches, prompt[0], 0, 1, stats)
      out["kernels_per_token"] = stats["kernels"]
    else:  # the launches of one eager forward (no graph, as under a kernel trace)
      from baretile_amd.tensor import Tensor
      base = rt.launches
      llama.forward(Tensor.of(rt, [[prompt[0]]], "int32"), Tensor.of(rt, [[0]], "int32"), dw, dc, caches).realize()
      out["kernels_per_token"] = rt.launches - base
    del caches
    if not check: return out, None
    t0 = time.perf_counter()
    ref = L.arrays(w, L.precision(c, "bfp8"))
    log("decode: oracle weights in", round(time.perf_counter() - t0, 1), "s")
    t0 = time.perf_counter()
    rtoks, rlogits = L.greedy(prompt, tokens, ref, c, size)
    cpu_s = time.perf_counter() - t0
    fed, flogits = llama.generate(dw, dc, prompt, tokens, size, feed=rtoks)
    errs = [float(np.abs(g - r).max() / np.abs(r).max()) for g, r in zip(flogits, rlogits)]
    margins = [float(np.diff(np.sort(r)[-2:])[0]) for r in rlogits]
    same = next((i for i, (a, b) in enumerate(zip(toks, rtoks)) if a != b), len(toks))
    out.update({"tokens_identical": toks == rtoks, "identical_prefix": same,
                "numpy_fed_agreement": float(np.mean([a == b for a, b in zip(fed, rtoks)])),
                "max_rel_logit_err": round(max(errs), 5), "min_top2_margin": round(min(margins), 4)})
    cpu = {"value": round(tokens / cpu_s, 2), "unit": "tok/s", "cores": blas_threads()[0], "kind": "port",
           "sample": f"the oracle's autonomous greedy decode of the same model: {prompt_len}-token prefill then "
           f"{tokens} tokens, {cpu_s:.1f} s in all, NumPy float32 ({blas_threads()[1]} BLAS), bfp8 weights "
           "dequantized beforehand"}
    return out, cpu
  finally:
    rt.close()


HOLD_S = 0.001  # the device-side wait queued before a timed replay's first event


HOLD_PER_LAUNCH_S = 25e-6  # more than the host takes to queue one launch


def hold(rt, launches=0):
  """Queues a kernel that keeps the device busy for HOLD_S, or HOLD_PER_LAUNCH_S for each of `launches` launches if
  longer, so that the host has queued the whole timed region by the time the device reaches its first event: the
  region then holds the launches' device time alone, not the host's time to queue them (which a serving loop overlaps
  with earlier work)."""
  from baretile_amd import _lib
  _lib.call("sleep", rt.handle, max(HOLD_S, HOLD_PER_LAUNCH_S * launches))


def graph_us(rt, fn, n):
  """us per call of fn() (launches only, no host copies) over n calls captured into one graph and replayed once."""
  from baretile_amd import _lib
  fn()
  rt.wait()
  graph = c_void_p()
  _lib.call("graph_begin", rt.handle)
  for _ in range(n): fn()
  _lib.call("graph_end", rt.handle, byref(graph))
  _lib.call("graph_launch", rt.handle, graph)
  rt.wait()
  start, end = c_void_p(), c_void_p()
  _lib.call("event_create", rt.handle, byref(start))
  _lib.call("event_create", rt.handle, byref(end))
  hold(rt)
  _lib.call("event_record", rt.handle, start)
  _lib.call("graph_launch", rt.handle, graph)
  _lib.call("event_record", rt.handle, end)
  ms = c_float()
  _lib.call("event_elapsed", start, end, byref(ms))
  rt.wait()
  for h in (start, end): _lib.call("event_destroy", h)
  _lib.call("graph_destroy", graph)
  return ms.value * 1000 / n


def replay_us(rt, fn, n):
  """us per call of fn() (which realizes its result) over n calls recorded into one graph (tensor.Recording) and
  replayed once between two events: the device time of the launches, without Python's dispatch."""
  from baretile_amd import _lib
  from baretile_amd.tensor import Recording
  fn()
  rt.wait()
  rec = Recording(rt)
  with rec:
    for _ in range(n): out = fn()
  rec.send()
  rt.wait()
  start, end = c_void_p(), c_void_p()
  _lib.call("event_create", rt.handle, byref(start))
  _lib.call("event_create", rt.handle, byref(end))
  hold(rt)
  _lib.call("event_record", rt.handle, start)
  rec.send()
  _lib.call("event_record", rt.handle, end)
  ms = c_float()
  _lib.call("event_elapsed", start, end, byref(ms))
  rt.wait()
  for h in (start, end): _lib.call("event_destroy", h)
  result = out.tobytes()
  rec.close()
  return ms.value * 1000 / n, result


def bf16_bits(a):
  b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
  return ((b + 0x7FFF + (b >> 16 & 1)) >> 16).astype(np.uint16)


def c1_leg(cpu_seconds, check=True):
  """relu(x @ W), x bf16 [128, 576] N(0, 1), W [576, 1536] N(0, 0.02) in bfp8 (seed 0), in one
  launch of the fused kernel. Roofline: intensity 153 flop/byte is below MI355X's ridge, so the bound is HBM bytes
  (1,480,704 per call), though the 1.48 MB stay in cache."""
  from baretile_amd import _lib
  from baretile_amd.program import Program
  from baretile_amd.runtime import Runtime
  from oracle import bfp as B, ops
  m, k, n = 128, 576, 1536
  rng = np.random.default_rng(0)
  x, w = rng.normal(0, 1, (m, k)).astype(np.float32), rng.normal(0, 0.02, (k, n)).astype(np.float32)
  rt = Runtime()
  try:
    dx, dw = rt.dram_alloc(m * k * 2), rt.dram_alloc(k * n * 2)
    rt.upload(dx, bf16_bits(x).tobytes())
    rt.upload(dw, bf16_bits(w).tobytes())
    exps, vals, cols = rt.dram_alloc(k * n // 16), rt.dram_alloc(k * n), rt.dram_alloc((k // 64) * (n // 16) * 1088)
    rt.run("pack", "bfp_pack", _lib.BFP8, dw, _lib.BF16, 1, k, n, k * n, n, 1, exps, vals)
    rt.run("columns", "bfp_columns", _lib.BFP8, exps, vals, 1, k, n, cols)
    out = rt.dram_alloc(m * n * 2)
    p = Program("bf16", epilogue=True)
    prog = p.build(p.op("relu", p.value()))
    a, o = _lib.operand(dx, "bf16", m * k, k, 1), _lib.operand(out, "bf16", m * n, n, 1)
    us = graph_us(rt, lambda: _lib.call("matmul", rt.handle, byref(a), _lib.BFP8, cols, 1, 1, m, k, n, byref(prog),
                                        byref(o)), 200)
    got = (np.frombuffer(bytes(rt.download(out, m * n * 2)), np.uint16).astype(np.uint32) << 16).view(np.float32)
    got = got.reshape(m, n)
  finally:
    rt.close()
  flops, nbytes = 2 * m * k * n, m * k * 2 + (k // 64) * (n // 16) * 1088 + m * n * 2
  res = {"us": round(us, 3), "TFLOP/s": round(flops / us / 1e6, 2), "GB/s": round(nbytes / us / 1e3, 1),
         "roofline": {"bound": "hbm", "achieved": round(nbytes / us / 1e3, 1), "peak": PEAK_GBS, "unit": "GB/s",
                      "frac": round(nbytes / us / 1e3 / PEAK_GBS, 4)}, "flops": flops, "bytes": nbytes}
  xw, wq = B.bf16(x), B.bfp(w, "bfp8")
  want = ops.matmul(xw, wq)
  res["parity"] = bool(np.all(np.abs(got - np.maximum(want, 0)) <= ops.matmul_bound(xw, wq)))
  cpu = None
  if check:
    xf, wf = xw.astype(np.float32), wq.astype(np.float32)
    np.maximum(xf @ wf, 0)
    t0, reps = time.perf_counter(), 0
    while time.perf_counter() - t0 < cpu_seconds:
      np.maximum(xf @ wf, 0)
      reps += 1
    per = (time.perf_counter() - t0) / reps
    cpu = {"value": round(flops / per / 1e12, 4), "unit": "TFLOP/s", "cores": blas_threads()[0], "kind": "port",
           "sample": f"{reps} calls of np.maximum(x @ Wq, 0) in float32 with Wq the bfp8 values, {per * 1e6:.0f} us each"}
  return res, cpu


def bfp8_cache_leg(rt, args, k, v, kvh, keys, hd, out, E, rows, check):
  """The decode case's K and V as a bfp8 cache (precision's kv entry, llama.py:74-83), read in place by the same
  attention call: bytes are the block floats' (1088 per 1024 values) plus q and out. Parity: bit for bit the bf16
  result on the cache's values."""
  from baretile_amd import _lib
  from baretile_amd.tensor import Tensor
  kc = Tensor.frombytes(rt, keys, hd, bf16_bits(k).tobytes(), kvh).cast("bfp8")
  vc = Tensor.frombytes(rt, keys, hd, bf16_bits(v).tobytes(), kvh).cast("bfp8")
  saved = (args.k, args.v, args.kv_fmt, args.k_exps, args.v_exps, args.scratch, args.scratch_bytes)
  (args.k_exps, args.k), (args.v_exps, args.v) = kc._bfp_planes(), vc._bfp_planes()
  args.kv_fmt = _lib.DTYPES["bfp8"]
  need = ctypes.c_uint64()  # the block-float plan splits the keys its own way
  _lib.call("attention_scratch", byref(args), byref(need))
  scratch = rt.dram_alloc(need.value) if need.value else 0
  args.scratch, args.scratch_bytes = scratch, need.value
  us = graph_us(rt, lambda: _lib.call("attention", rt.handle, byref(args)), 50)
  nbytes = 2 * kvh * keys * hd * 1088 // 1024 + 2 * E * rows * hd * 2
  entry = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1), "frac_hbm_peak": round(nbytes / us / 1e3 / PEAK_GBS, 4),
           "bytes": nbytes}
  if check:  # the same call on the cache's values in bf16, split into the same parts
    got = bytes(rt.download(out, E * rows * hd * 2))
    ks, vs = kc.cast("bf16").realize(), vc.cast("bf16").realize()
    args.k, args.v, args.kv_fmt, args.k_exps, args.v_exps = ks.addr, vs.addr, 0, 0, 0
    args.parts = need.value // (kvh * 4 * (32 + 16 * hd)) if need.value else 1  # one tile a key head
    _lib.call("attention", rt.handle, byref(args))
    rt.wait()
    args.parts = 0
    entry["parity"] = got == bytes(rt.download(out, E * rows * hd * 2))
  args.k, args.v, args.kv_fmt, args.k_exps, args.v_exps, args.scratch, args.scratch_bytes = saved
  rt.wait()
  if scratch: rt.dram_free(scratch)
  log("attention", "decode bfp8 cache", entry)
  return entry


def attention_leg(check=True):
  """bf16 q, k, v N(0, 1), 32 query heads over 8 key heads of 128 (batch entries fold into heads),
  fp32 softmax, bf16 out. Decode: 1 query row against 512, 4096 and 16384 keys at batch 1 and 8, HBM-bound (bytes:
  K and V, 4096 per key per batch entry, plus q and out). Prefill: 2048 causal rows at batch 1, matrix-core bound
  (flops of the visible pairs: 4 * 32 * 128 * 2048 * 2049 / 2)."""
  from baretile_amd import _lib
  from baretile_amd.runtime import Runtime
  from oracle import bfp as B, ops
  rng = np.random.default_rng(0)
  rt = Runtime()
  res = {}
  try:
    cases = [("decode", b, ctx, 1) for b in (1, 8) for ctx in (512, 4096, 16384)] + [("prefill", 1, 2048, 2048)]
    for kind, batch, keys, rows in cases:
      E, kvh, hd = 32 * batch, 8 * batch, 128
      q = rng.standard_normal((E, rows, hd), dtype=np.float32) * np.float32(hd ** -0.5)
      k = rng.standard_normal((kvh, keys, hd), dtype=np.float32)
      v = rng.standard_normal((kvh, keys, hd), dtype=np.float32)
      places = np.broadcast_to(np.arange(rows, dtype=np.int32) if kind == "prefill" else np.full(rows, keys - 1, np.int32),
                               (E, rows)).copy()
      bufs = [rt.dram_alloc(a.size * 2) for a in (q, k, v)]
      for d, a in zip(bufs, (q, k, v)): rt.upload(d, bf16_bits(a).tobytes())
      dp, out = rt.dram_alloc(places.nbytes), rt.dram_alloc(E * rows * hd * 2)
      rt.upload(dp, places.tobytes())
      args = _lib.AttentionArgs(bufs[0], bufs[1], bufs[2], out, dp, rows * hd, hd, keys * hd, hd, keys * hd, hd,
                                rows * hd, hd, rows, E, 4, rows, keys, hd, 0, 0, 0, 0, 0)
      need = ctypes.c_uint64()
      _lib.call("attention_scratch", byref(args), byref(need))
      if need.value: args.scratch, args.scratch_bytes = rt.dram_alloc(need.value), need.value
      us = graph_us(rt, lambda: _lib.call("attention", rt.handle, byref(args)), 50 if kind == "decode" else 10)
      name = f"{kind}_B{batch}_ctx{keys}" if kind == "decode" else f"prefill_{rows}"
      entry = {"us": round(us, 3)}
      if kind == "decode":
        nbytes = 2 * kvh * keys * hd * 2 + 2 * E * rows * hd * 2
        entry.update({"GB/s": round(nbytes / us / 1e3, 1), "frac_hbm_peak": round(nbytes / us / 1e3 / PEAK_GBS, 4),
                      "bytes": nbytes})
      else:
        flops = 4 * 32 * 128 * rows * (rows + 1) // 2
        entry.update({"TFLOP/s": round(flops / us / 1e6, 1), "frac_mfma_peak": round(flops / us / 1e6 / 2500.0, 4),
                      "flops": flops})
      if check:  # key head 0 and its 4 query heads against the oracle
        got = (np.frombuffer(bytes(rt.download(out, 4 * rows * hd * 2)), np.uint16).astype(np.uint32) << 16).view(np.float32)
        want = ops.attention(B.bf16(q[:4]), B.bf16(k[:1]), B.bf16(v[:1]), places[:4, :, None], 0, 4)
        entry["parity"] = bool(np.allclose(got.reshape(4, rows, hd), want, rtol=0.011, atol=0.011))
      res[name] = entry
      log("attention", name, entry)
      if kind == "decode" and batch == 8 and keys == 16384:  # beside it: the same cache in bfp8, read in place
        res[name + "_bfp8_cache"] = bfp8_cache_leg(rt, args, k, v, kvh, keys, hd, out, E, rows, check)
      rt.wait()
      for d in bufs + [dp, out]: rt.dram_free(d)
      if need.value: rt.dram_free(args.scratch)
  finally:
    rt.close()
  cpu = None
  if check:  # the oracle's decode at 4096 keys, batch 1, one query row per head
    q = rng.standard_normal((32, 1, 128)).astype(np.float32)
    k, v = rng.standard_normal((8, 4096, 128)).astype(np.float32), rng.standard_normal((8, 4096, 128)).astype(np.float32)
    pl = np.full((32, 1, 1), 4095)
    t0, reps = time.perf_counter(), 0
    while time.perf_counter() - t0 < 3.0 or reps < 2:
      ops.attention(q, k, v, pl, 0, 4)
      reps += 1
    per = (time.perf_counter() - t0) / reps
    nbytes = 2 * 8 * 4096 * 128 * 2 + 2 * 32 * 128 * 2
    # and the causal prefill, on one key head's 4 query heads (an eighth of the 2048-row case)
    qp = rng.standard_normal((4, 2048, 128)).astype(np.float32)
    kp, vp = rng.standard_normal((1, 2048, 128)).astype(np.float32), rng.standard_normal((1, 2048, 128)).astype(np.float32)
    plp = np.broadcast_to(np.arange(2048)[None, :, None], (4, 2048, 1))
    pper, preps = timed_cpu(lambda: ops.attention(qp, kp, vp, plp, 0, 4), 3.0)
    pflops = 4 * 4 * 128 * 2048 * 2049 // 2
    cpu = {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s", "cores": blas_threads()[0], "kind": "port",
           "sample": f"{reps} calls of the oracle's attention (NumPy float64) at decode, 4096 keys, batch 1: "
           f"{per * 1e3:.1f} ms each", "host_cpus": os.cpu_count(),
           "prefill": {"value": round(pflops / pper / 1e12, 5), "unit": "TFLOP/s",
                       "sample": f"{preps} calls of the oracle's causal attention over 2048 rows for one key head and its "
                       f"4 query heads (an eighth of config 4's prefill), {pper:.2f} s each"}}
  return res, cpu


def _layer_prefill(rt, llama, L, Tensor, c, rc, p, w, ref, shapes, xh, cos, sin, turn, size, tokens, check):
  """The 2048-token prefill of layer_leg: timed, and checked on key rows against the oracle."""
  dim, heads, kv, hd = 4096, 32, 8, 128
  x = Tensor.of(rt, xh[None], "fp32")
  cache = Tensor.zeros(rt, size, hd, batch=2 * kv)
  places = Tensor.of(rt, [list(range(tokens))], "int32")
  rot = (w["cos"].gather(places), w["sin"].gather(places), w["turn"])
  column = places.reshape(1, tokens, 1)
  run = lambda: llama.layer(x, p, c, rot, column, cache, places).realize()
  run()
  rt.wait()
  reps, t0 = 5, time.perf_counter()
  for _ in range(reps): run()
  rt.wait()
  eager = (time.perf_counter() - t0) / reps * 1e6
  us, y = replay_us(rt, run, 5)
  flops = 2 * tokens * sum(a * b for a, b in shapes.values()) + 4 * heads * hd * tokens * (tokens + 1) // 2
  entry = {"us": round(us, 1), "TFLOP/s": round(flops / us / 1e6, 1),
           "frac_mfma_peak": round(flops / us / 1e6 / 2500.0, 4), "flops": flops, "eager_us": round(eager, 1)}
  if check:  # key rows against the oracle's layer, which still computes every row's keys and values
    rows = [0, 1, 255, 1024, 2047]
    got = np.frombuffer(y, np.float32).reshape(tokens, dim)[rows]
    mask = np.where(np.arange(tokens) > np.arange(tokens)[:, None], np.float32(-1e9), np.float32(0))
    t0 = time.perf_counter()
    want = L.layer(xh, ref, rc, (cos[:tokens], sin[:tokens], turn), mask, np.zeros((2 * kv, tokens, hd)),
                   range(tokens), only=rows)
    log("layer prefill oracle rows in", round(time.perf_counter() - t0, 1), "s")
    change, err = np.abs(want - xh[rows]).max(), np.abs(got - want).max()
    entry.update({"parity": bool(err < 0.03 * change), "parity_rows": rows, "max_err_over_change": round(float(err / change), 5)})
  log("layer prefill", entry)
  return entry


def _layer_decode(rt, llama, L, B, Tensor, c, rc, p, w, ref, wbytes, cos, sin, turn, rng, check):
  """The batch-32 decode step of layer_leg: timed, and checked on key slots against the oracle."""
  dim, heads, kv, hd, size, slots = 4096, 32, 8, 128, 4096, 32
  K = B.bf16(rng.standard_normal((slots * kv, size, hd), dtype=np.float32))
  V = B.bf16(rng.standard_normal((slots * kv, size, hd), dtype=np.float32))
  K[:, size - 1:], V[:, size - 1:] = 0, 0
  keys, values = Tensor.of(rt, K), Tensor.of(rt, V)
  xs_h = rng.standard_normal((slots, dim), dtype=np.float32)
  xs = Tensor.of(rt, xs_h[None], "fp32")
  at = Tensor.of(rt, [[size - 1] * slots], "int32")
  rot = (w["cos"].gather(at), w["sin"].gather(at), w["turn"])
  place = Tensor.of(rt, [[size - 1]], "int32")
  # a block of a stack: its input norm made by the block before (h), its down product ending in the norm of the block
  # after (then; this one block stands for it), so that a step holds the block's two norms, as each block of a model
  hs = llama.rms(xs, p["input_layernorm"], c).realize()
  step = lambda: llama.slots_layer(xs, p, c, rot, keys, values, place, h=hs, then=p["input_layernorm"])[0].realize()
  step()
  rt.wait()
  reps, t0 = 20, time.perf_counter()
  for _ in range(reps): step()
  rt.wait()
  eager = (time.perf_counter() - t0) / reps * 1e6
  us, y = replay_us(rt, step, 20)
  nbytes = wbytes + slots * size * kv * hd * 2 * 2
  entry = {"us": round(us, 1), "GB/s": round(nbytes / us / 1e3, 1), "frac_hbm_peak": round(nbytes / us / 1e3 / PEAK_GBS, 4),
           "bytes": nbytes, "tok/s": round(slots / us * 1e6, 1), "eager_us": round(eager, 1)}
  if check:  # key slots against the oracle's layer run on each slot alone
    got = np.frombuffer(y, np.float32).reshape(slots, dim)
    worst, sl = 0.0, [0, 13, 31]
    for s_ in sl:
      cache_s = np.concatenate([K[s_ * kv:(s_ + 1) * kv], V[s_ * kv:(s_ + 1) * kv]]).astype(np.float64)
      want = L.layer(xs_h[s_:s_ + 1], ref, rc, (cos[[size - 1]], sin[[size - 1]], turn), np.zeros((1, size), np.float32),
                     cache_s, [size - 1])[0]
      worst = max(worst, float(np.abs(got[s_] - want).max() / np.abs(want - xs_h[s_]).max()))
    entry.update({"parity": worst < 0.03, "parity_slots": sl, "max_err_over_change": round(worst, 5)})
  log("layer decode", entry)
  return entry, K, V, xs_h


def layer_leg(check=True, cpu_seconds=10.0, parts=("prefill", "decode")):
  """one Llama-3-8B-shaped block (4096 wide, 32 query and 8 key heads of 128, SwiGLU 14336) with
  every projection N(0, 0.02) in bfp4 and bf16 norms: a 2048-token prefill from position 0 (matrix-core bound;
  flops 2 * 2048 * 218,103,808 for the projections plus the causal attention), then one batch-32 decode step, each
  slot at position 4095 of its own 4096-row bf16 cache (HBM-bound: the 122,683,392 bytes of bfp4 weights plus
  32 * 4096 * 8 * 128 * 2 * 2 bytes of K and V).

  Parity: the oracle's layer (oracle/llama_ref.layer) on the same block floats (read back from the device) for key
  rows of the prefill and key slots of the decode step, within the reference's 3% of the block's change to x
  (test_models.py:818-833). CPU baseline: the oracle's layer timed on the host, a prefill of 128 tokens and one slot's
  decode token."""
  from baretile_amd.models import llama
  from baretile_amd.runtime import Runtime
  from baretile_amd.tensor import Tensor
  from oracle import bfp as B, llama_ref as L
  dim, heads, kv, hd, ffn, size, tokens, slots = 4096, 32, 8, 128, 14336, 4096, 2048, 32
  rng = np.random.default_rng(0)
  rt = Runtime()
  res, cpu = {}, None
  try:
    c = llama.model(dim=dim, heads=heads, kv=kv, layers=1, eps=1e-5, theta=500000.0, ffn=ffn, head_dim=hd)
    c.precision = {(op, 0): ("bfp4", 4) for op in ("qkv", "o", "gate_up", "down")}
    rc = L.model(dim=dim, heads=heads, kv=kv, layers=1, eps=1e-5, theta=500000.0, ffn=ffn, head_dim=hd)
    shapes = {"qkv_proj": (dim, (heads + 2 * kv) * hd), "o_proj": (heads * hd, dim), "gate_up_proj": (dim, 2 * ffn),
              "down_proj": (ffn, dim)}
    w, ref = {}, {}
    for name, shape in shapes.items():
      t = Tensor.of(rt, rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).cast("bfp4").columns()
      w[f"layers.0.{name}"] = t
      if check: ref[name] = B.bf16_floats(np.frombuffer(t.tobytes(), np.uint16).reshape(shape))
    for name in ("input_layernorm", "post_attention_layernorm"):
      n = B.bf16(rng.normal(1, 0.1, (1, dim)))
      w[f"layers.0.{name}"], ref[name] = Tensor.of(rt, n), n
    cos, sin, turn = llama.rotary(c, size)
    w["cos"], w["sin"], w["turn"] = Tensor.of(rt, cos), Tensor.of(rt, sin), Tensor.of(rt, turn).columns()
    p = llama.block(w, 0)
    wbytes = sum(shape[0] * shape[1] for shape in shapes.values()) * 576 // 1024
    xh = rng.standard_normal((tokens, dim), dtype=np.float32)
    if "prefill" in parts: res["prefill_2048"] = _layer_prefill(rt, llama, L, Tensor, c, rc, p, w, ref, shapes, xh, cos,
                                                                sin, turn, size, tokens, check)
    if "decode" in parts: res["decode_B32_ctx4096"], K, V, xs_h = _layer_decode(rt, llama, L, B, Tensor, c, rc, p, w, ref,
                                                                                 wbytes, cos, sin, turn, rng, check)
    if check and parts == ("prefill", "decode"):  # the oracle's layer on the host: a 128-token prefill, one slot's token
      n = 128
      mask = np.where(np.arange(n) > np.arange(n)[:, None], np.float32(-1e9), np.float32(0))
      per, reps = timed_cpu(lambda: L.layer(xh[:n], ref, rc, (cos[:n], sin[:n], turn), mask,
                                            np.zeros((2 * kv, n, hd)), range(n)), cpu_seconds / 2)
      pflops = 2 * n * sum(a * b for a, b in shapes.values()) + 4 * heads * hd * n * (n + 1) // 2
      cache_s = np.concatenate([K[:kv], V[:kv]]).astype(np.float64)
      dper, dreps = timed_cpu(lambda: L.layer(xs_h[:1], ref, rc, (cos[[size - 1]], sin[[size - 1]], turn),
                                              np.zeros((1, size), np.float32), cache_s, [size - 1]), cpu_seconds / 2)
      dbytes = wbytes + size * kv * hd * 2 * 2
      threads, api = blas_threads()
      cpu = {"value": round(dbytes / dper / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
             "sample": f"the oracle's layer for one slot's decode token at position 4095 ({dreps} runs, {dper * 1e3:.0f} "
             f"ms each; bytes counted as the GPU figure counts one slot's: bfp4 weights plus its K and V), NumPy "
             f"float32/float64 ({api} BLAS)", "host_cpus": os.cpu_count(),
             "prefill": {"value": round(pflops / per / 1e12, 4), "unit": "TFLOP/s",
                         "sample": f"the oracle's layer on a 128-token prefill, {reps} runs, {per:.2f} s each"}}
  finally:
    rt.close()
  return res, cpu


def gemm_lib_leg(calls=20):
  """For scale, not a BASELINE configuration: the C5 prefill's four product shapes with bf16 B, this library's GEMM
  (bt_matmul on B as bf16 columns tiles, calls replayed from a graph) beside hipBLASLt through torch.matmul (calls
  back to back between two events on torch's stream), both bf16 in, fp32 accumulate, bf16 out. The two results
  are compared (the summation orders differ, so within a relative 2^-7 of the largest output)."""
  import torch
  from baretile_amd import _lib
  from baretile_amd.runtime import Runtime
  rt = Runtime()
  rng = np.random.default_rng(0)
  out = {}
  try:
    for m, k, n in ((2048, 4096, 6144), (2048, 4096, 4096), (2048, 4096, 28672), (2048, 14336, 4096)):
      x = rng.standard_normal((m, k), dtype=np.float32)
      w = rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)
      xb, wb = bf16_bits(x), bf16_bits(w)
      dx, dw, cols, do = rt.dram_alloc(m * k * 2), rt.dram_alloc(k * n * 2), rt.dram_alloc(k * n * 2), rt.dram_alloc(m * n * 2)
      rt.upload(dx, xb.tobytes())
      rt.upload(dw, wb.tobytes())
      rt.run("columns", "bf16_columns", dw, 1, k, n, k * n, n, 1, cols)
      a, o = _lib.operand(dx, "bf16", 0, k, 1), _lib.operand(do, "bf16", 0, n, 1)
      us = graph_us(rt, lambda: _lib.call("matmul", rt.handle, byref(a), _lib.BF16, cols, 1, 1, m, k, n, None, byref(o)),
                    calls)
      got = np.frombuffer(rt.download(do, m * n * 2), np.uint16).astype(np.uint32) << 16
      ta = torch.from_numpy(xb.view(np.int16).reshape(m, k).copy()).to("cuda").view(torch.bfloat16)
      tb = torch.from_numpy(wb.view(np.int16).reshape(k, n).copy()).to("cuda").view(torch.bfloat16)
      for _ in range(5): tc = ta @ tb
      torch.cuda.synchronize()
      start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
      start.record()
      for _ in range(calls): tc = ta @ tb
      end.record()
      torch.cuda.synchronize()
      lib_us = start.elapsed_time(end) * 1000 / calls
      ref = tc.float().cpu().numpy()
      mine = got.view(np.float32).reshape(m, n)
      agree = bool(np.abs(mine - ref).max() <= np.abs(ref).max() * 2.0 ** -7)
      flops = 2.0 * m * k * n
      out[f"{m}x{k}x{n}"] = {"us": round(us, 1), "TFLOP/s": round(flops / us / 1e6, 1),
                             "hipblaslt_us": round(lib_us, 1), "hipblaslt_TFLOP/s": round(flops / lib_us / 1e6, 1),
                             "agree": agree}
      log("gemm", f"{m}x{k}x{n}", out[f"{m}x{k}x{n}"])
      for d in (dx, dw, cols, do): rt.dram_free(d)
      del ta, tb, tc
  finally:
    rt.close()
  return out


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
  ap.add_argument("--only", default=None,
                  help="one part: a GEMV configuration (bfp4_B1 ...), gemv, c1, attention, layer (or layer_prefill, "
                  "layer_decode) or decode; or gemm_lib (not in the default run): the C5 product shapes in bf16, this "
                  "library's GEMM beside hipBLASLt")
  ap.add_argument("--no-decode", action="store_true", help="skip the SmolLM decode (BASELINE config 3)")
  ap.add_argument("--eager", action="store_true", help="decode without graph replay (for kernel-trace profiles)")
  args = ap.parse_args()
  if args.gpus != 1:
    print(f"bench.py runs on one GPU: this build has no multi-GPU path, and --gpus {args.gpus} is not supported",
          file=sys.stderr)
    sys.exit(2)
  if args.only == "gemm_lib":
    print(json.dumps({"gemm_lib": gemm_lib_leg()}), flush=True)
    return
  configs = {}
  for fmt in ("bfp4", "bfp8"):
    for rows in (1, 4, 16):
      if args.only and args.only != f"{fmt}_B{rows}" and args.only != "gemv": continue
      steps = args.steps if (fmt, rows) == ("bfp4", 1) else max(50, args.steps // 4)
      us, got, x, w, read_us, floor_us = gpu_leg(fmt, rows, steps, args.warmup if (fmt, rows) == ("bfp4", 1) else steps)
      ok = check(got, x, w, fmt)
      gbs = step_bytes(fmt, rows) / us / 1e3
      wb = weight_bytes(fmt)
      configs[f"{fmt}_B{rows}"] = {"us_per_step": round(us, 3), "GB/s": round(gbs, 1),
                                   "frac_hbm_peak": round(gbs / PEAK_GBS, 4), "bytes": step_bytes(fmt, rows),
                                   "steps": steps, "parity": ok,
                                   "stream_read_us": round(read_us, 3), "stream_read_GB/s": round(wb / read_us / 1e3, 1),
                                   "frac_of_stream_read": round(read_us / us, 4),
                                   "launch_floor_us": round(floor_us, 3)}
      log(fmt, rows, configs[f"{fmt}_B{rows}"])
  extra = {}
  if args.only in (None, "c1"):
    extra["c1"], extra["c1_cpu_baseline"] = c1_leg(min(args.cpu_seconds, 5.0), check=not args.no_cpu)
    log("c1", extra["c1"])
  if args.only in (None, "attention"):
    extra["attention"], extra["attention_cpu_baseline"] = attention_leg(check=not args.no_cpu)
  if args.only in (None, "layer", "layer_prefill", "layer_decode"):
    parts = {"layer_prefill": ("prefill",), "layer_decode": ("decode",)}.get(args.only, ("prefill", "decode"))
    extra["layer"], extra["layer_cpu_baseline"] = layer_leg(check=not args.no_cpu, cpu_seconds=args.cpu_seconds,
                                                            parts=parts)
  if not args.no_decode and args.only in (None, "decode"):
    extra["decode"], extra["decode_cpu_baseline"] = decode_leg(check=not args.no_cpu, replay=not args.eager)
    log("decode", extra["decode"])
  if args.only in ("c1", "attention", "layer", "layer_prefill", "layer_decode", "decode"):
    print(json.dumps(extra), flush=True)
    return
  head = configs.get("bfp4_B1") or next(iter(configs.values()))
  cpu = None
  if not args.no_cpu:
    us_cpu, n = cpu_leg("bfp4", 1, args.cpu_seconds)
    us_one, n_one = cpu_leg("bfp4", 1, min(3.0, args.cpu_seconds), threads=1)
    threads, api = blas_threads()
    cpu = {"value": round(step_bytes("bfp4", 1) / us_cpu / 1e3, 3), "unit": "GB/s", "cores": threads,
           "kind": "port", "sample": f"{n} whole GEMVs x[1,576] @ W[576,49152] (bfp4 values dequantized to float32 "
           f"outside the timer) with NumPy float32 ({api} BLAS), {us_cpu:.0f} us each",
           "host_cpus": os.cpu_count(), "one_thread": {"value": round(step_bytes("bfp4", 1) / us_one / 1e3, 3),
                                                       "cores": 1, "sample": f"{n_one} GEMVs, {us_one:.0f} us each"}}
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
    **extra,
  }
  print(json.dumps(line), flush=True)


if __name__ == "__main__":
  main()
