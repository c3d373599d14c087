"""Benchmarks of the paged flow-LM KV cache on one MI355X.  Each run prints one JSON line.

--workload decode (default; the headline): batched paged decode attention + KV append.
  1024 concurrent streams, Phonon-40m layers (9 x 8 heads x 64), bf16 K/V in 16-position pages
  handed out from a shuffled free list, cache length per stream uniform in [1, 1024] (numpy seed
  20261202), one bf16 query and one new K/V row per stream per layer, N(0, 1).  A step is one pass
  over all 9 layers: the plan upload, then per layer one fused append + RoPE + decode kernel.
  frames/s = streams / step time; audio-s/s = frames/s * 0.08 (12.5 Hz frames).
  Roofline: algorithmic bytes per decode launch (per stream: 2 (n+1) H D 2 B of K/V read, 1 KB q,
  2 KB new k/v, 1 KB out, 2 KB append write, 4 ceil((n+1)/16) B of page ids) over the kernel's
  average duration, against 8 TB/s.  The duration comes from HIP events that the launches
  themselves record (hipExtLaunchKernel, via xnp_pool_time_next), on the stream the kernels run
  on: on every fifth step, layer 0's launch records the start as its kernel starts and layer 8's
  the stop as its kernel ends; the span / 9 is the mean launch (the nine launches run back to
  back; one event pair per step keeps the event overhead off the steps and off short kernels).
  step_ms: the median and 95th percentile of the step periods, from one event per step start.

--workload prefill: prompt prefill, 64 streams x 256-position prompts, 9 layers, bf16, RoPE
  theta 10000, causal, K/V written into the pages.  Value: prompt positions/s.  Roofline: causal
  flops 2 D T (T+1) H S per layer launch against 2.5 PFLOP/s dense bf16 MFMA.

--workload step: the full per-frame flow-LM layer step, 2048 streams x 9 Phonon-40m layers (512 wide,
  8 heads x 64, FF 2048): LayerNorm, int8 per-channel q8 projections (QKV, out, FF) on MFMA, erf GELU,
  residuals, RoPE, paged bf16 KV append and decode attention over cache lengths U[1, 1500].  Value:
  frames/s.  Roofline: the decode attention kernel (the step's dominant kernel) against 8 TB/s.

--workload flowlm: the single-stream flow LM (Phonon-31m shape, fp32): a 64-token text prompt, then
  greedy frames at temperature 0 through input_linear, the 6 layers, out_norm, the EOS head and the flow
  net.  Value: frames/s at batch 1 with each frame replayed from a hipGraph recording of its launches
  (xnp_flow_lm_step_graph; the launched rate beside it); the CPU oracle of the same stream on 1 thread
  and on all cores.

--workload window: int8 K/V with fp32 scales per (page, head), 1024 streams, a sliding window of
  512 positions on rings of 528 slots whose write heads start at offsets U[0, 4096), each stream
  holding U[64, 2048] rows written so far; per step every stream evicts its oldest row once the
  window is full, appends one and attends over min(n+1, 512) rows.  Value: frames/s.

--workload mimi: Mimi's windowed attention (2 layers x 8 heads x 64, context 250, bf16): 256 streams,
  each step a 250-row chunk (a 10 s voice clip at 25 Hz) into a window that already holds 249 rows.
  Value: positions/s over the whole step (the windowed attention and the window append).  Roofline:
  the windowed attention launch (q, out, the chunk's k and v, the held rows it sees) against 8 TB/s.

--workload vendor_gemm: not this library -- the vendor library's bf16 GEMMs (hipBLASLt through torch)
  at the layer step's four projection shapes and torch's LayerNorm, replayed from a graph, for
  comparison with the q8 projections.  Value: us per layer for the four GEMMs.

CPU baseline: the oracle (the C restatement, OpenMP over streams) on a bounded sample of the same
workload, timed on this host's cores.
"""
import argparse
import gc
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
SEED = 20261201
H, D = 8, 64


def host_threads():
    """The host threads a CPU baseline may use: OMP_NUM_THREADS when set (the GPU box's share of
    its host), else every core."""
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def _load(name, path):
    if name in sys.modules:
        return sys.modules[name]
    is_pkg = os.path.isdir(path)
    spec = importlib.util.spec_from_file_location(
        name, os.path.join(path, "__init__.py") if is_pkg else path,
        submodule_search_locations=[path] if is_pkg else None)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


class HipEvents:
    """hipEvent_t handles from the HIP runtime torch loaded (same soname, so the same library)."""

    def __init__(self):
        import ctypes
        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self):
        ev = self.ct.c_void_p()
        if self.hip.hipEventCreate(self.ct.byref(ev)) != 0:
            raise RuntimeError("hipEventCreate failed")
        return ev.value

    def elapsed_ms(self, a, b):
        ms = self.ct.c_float()
        if self.hip.hipEventElapsedTime(self.ct.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, ev):
        self.hip.hipEventDestroy(ev)


def bf16_np(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32).reshape(a.shape)


def traffic_of(workload, match, bytes_per_launch):
    """HBM bytes per launch of a workload's dominant kernel, from its FETCH_SIZE / WRITE_SIZE counter
    runs (profiles/traffic.json: each counter scaled by what it reads for a 1 GiB copy): the counter
    bytes per algorithmic byte of the profiled run, times this run's algorithmic bytes per launch.
    The ratio belongs to the kernel at that workload, so it carries over to any --steps / --warmup;
    None when the workload (streams, layers, lengths, ...) matches no profiled setting."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        table = json.load(f)
    # one entry per profiled setting: "decode", "decode:kv_heads=1", ...
    for key, entry in table.items():
        if (key == workload or key.startswith(workload + ":")) and entry.get("workload") == match:
            return int(round(entry["traffic_per_algorithmic_byte"] * bytes_per_launch))
    return None


def decode_bytes(lens, elem=2, kvh=H):
    """Bytes one layer's append + decode must move for streams with cached lengths `lens`: each
    stored kv head's K/V rows once (kvh of them), q and out for every query head."""
    lens = np.asarray(lens, np.int64)
    kv = 2 * (lens + 1) * kvh * D * elem
    fixed = (H * D * 2) * 2 + (kvh * D * 2) * 2 + 2 * kvh * D * elem  # q, out; new k/v (bf16); append write
    table = 4 * ((lens + 1 + 15) // 16)
    return int((kv + fixed + table).sum())


def window_bytes(attended, kvh=H):
    """int8 window: K/V rows attended and one scale per (page, kv head) for K and V (kvh stored kv
    heads), bf16 q and out for every query head, the new bf16 k/v rows and their int8 append."""
    a = np.asarray(attended, np.int64)
    pages = (a + 15) // 16 + 1
    return int((2 * a * kvh * D + 2 * kvh * 4 * pages + H * D * 2 * 2 + kvh * D * 2 * 2 + 2 * kvh * D
                + 4 * pages).sum())


class NoGC:
    """Python's cyclic garbage collector off over a timed region, collected just before: its pauses
    belong to this harness, not to the path, and one landing inside a timed step leaves the GPU idle
    for a millisecond or more."""

    def __enter__(self):
        gc.collect()
        gc.disable()

    def __exit__(self, *exc):
        gc.enable()


class StepMarks:
    """A timing event recorded on the current stream at the start of every timed step and after the
    last one: the steps' periods on the GPU's clock, whose median and 95th percentile go in the
    line beside the wall-clock mean."""

    def __init__(self, steps):
        import torch
        self.ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        self.n = 0

    def mark(self):
        self.ev[self.n].record()
        self.n += 1

    def percentiles(self):
        d = np.array([a.elapsed_time(b) for a, b in zip(self.ev[:self.n - 1], self.ev[1:self.n])])
        return {"p50": round(float(np.percentile(d, 50)), 4), "p95": round(float(np.percentile(d, 95)), 4)}


def timed_steps(step, steps, warmup, L, every=5, span=False):
    """Run warmup then `steps` steps; wall ms per step, the durations (ms) of the timed launches,
    and the steps' p50 / p95 periods (StepMarks).

    Every `every`-th step times the kernel with HIP events its launches record (hipExtLaunchKernel):
    a launch that records events issues more slowly (and the steps around it with it), so timing
    every step would slow the very steps the wall clock measures.
    - span=False: one launch, layer (s / every) % L, records both events around its kernel.  Layers
      are alike, so the rotating sample's mean is the mean launch duration.
    - span=True, for steps that launch nothing but the L layers' kernels back to back: layer 0's
      launch records the start and layer L - 1's the stop, and the span / L is the mean launch
      duration.  An event pair costs the kernel it brackets about 5 us; spread over L launches it
      stops inflating short kernels, at the price of the (about 1 us) gaps between launches."""
    import torch
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    hip = HipEvents()
    timed = {s: (s // every) % L for s in range(0, steps, every)}
    ev, pairs = [None] * steps, {}
    for s in timed:
        a, b = hip.create(), hip.create()
        pairs[s] = (a, b)
        ev[s] = [None] * L
        if span:
            ev[s][0] = (a, b) if L == 1 else (a, None)
            if L > 1:
                ev[s][L - 1] = (None, b)
        else:
            ev[s][timed[s]] = (a, b)
    marks = StepMarks(steps)
    with NoGC():
        t0 = time.perf_counter()
        for s in range(steps):
            marks.mark()
            step(ev[s])
        marks.mark()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    kern = np.array([hip.elapsed_ms(*pairs[s]) / (L if span else 1) for s in timed])
    for a, b in pairs.values():
        hip.destroy(a)
        hip.destroy(b)
    return (t1 - t0) * 1000.0 / steps, kern, marks.percentiles()


def line(metric, value, unit, args, ms, dtype, config, roofline, cpu, higher=True, extra=None, pct=None):
    out = {"metric": metric, "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": higher, "scaling": "weak",
           "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": config}
    if pct:
        out["step_ms"] = pct
    if extra:
        out.update(extra)
    out["roofline"] = roofline
    out["cpu_baseline"] = cpu
    return out


# ---- decode (configuration 2; the headline at 1024 streams) -------------------------------------------
def cpu_decode(L, lens_all, seconds, sample=128):
    oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    rng = np.random.default_rng(SEED + 100)
    lens = lens_all[:sample]
    room = 512  # steps the sample's caches have room for
    cap = int(lens.max()) + room
    streams = [oracle.Stream(L, H, D, cap, cache="bf16", act="bf16") for _ in lens]
    rows = bf16_np(rng.standard_normal((int(lens.max()), H, D)))
    for st, n in zip(streams, lens):
        for layer in range(L):
            st.write_rows(layer, 0, 0, vals=rows[:n])
            st.write_rows(layer, 1, 0, vals=rows[:n][::-1].copy())
        st.advance(int(n))
    q, k, v = (bf16_np(rng.standard_normal((len(lens), H, D))) for _ in range(3))
    steps, t0 = 0, time.perf_counter()
    while True:
        for layer in range(L):
            oracle.batch_attend(streams, layer, q, k, v)
        oracle.batch_commit(streams)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds or steps >= room:
            break
    return {"value": round(len(lens) * steps / el, 1), "unit": "frames/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{len(lens)} streams x {L} layers x {steps} steps of the same workload "
                      f"(bf16, lengths from the same U[1,1024] draw), {el:.1f} s"}


def run_decode(args, xnp, torch):
    dev = torch.device("cuda:0")
    S, L = args.streams, args.layers
    rng = np.random.default_rng(SEED + 1)
    lens = rng.integers(1, args.max_len + 1, S)
    if args.fixed_len:
        lens = np.full(S, args.fixed_len)
    total_steps = args.warmup + args.steps
    cap = args.max_len + total_steps + 1
    mbps = (cap + 15) // 16
    nblocks = int(sum((n + total_steps + 16) // 16 + 1 for n in lens)) + 16
    kvh = args.kv_heads or H
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_kv_heads=kvh, num_blocks=nblocks, max_streams=S,
                      max_blocks_per_stream=mbps, cache_dtype="bf16", act_dtype="bf16", max_pos=cap + 16,
                      page_seed=SEED + 2, decode_split=args.split)
    ids = [pool.init_state(cap) for _ in range(S)]
    gen = torch.Generator(device=dev).manual_seed(SEED + 3)
    maxn = int(lens.max())
    for layer in range(L):
        for kvi in (0, 1):
            rows = torch.randn((maxn, kvh, D), generator=gen, device=dev).to(torch.bfloat16)
            for sid, n in zip(ids, lens):
                if layer == 0 and kvi == 0:
                    pool.advance(sid, int(n))
                pool.write_rows(sid, layer, kvi, 0, rows[:n])
    q = [torch.randn((S, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    k = [torch.randn((S, kvh, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    v = [torch.randn((S, kvh, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    out = [torch.empty((S, H, D), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    torch.cuda.synchronize()
    cur = lens.copy()
    bytes_timed = [0, 0]  # bytes of the timed launches, their count

    def step(events):
        if events is not None:
            bytes_timed[0] += decode_bytes(cur, kvh=kvh)  # the one launch this step times
            bytes_timed[1] += 1
        pool.begin(ids)
        for layer in range(L):
            if events is not None and events[layer] is not None:  # recorded by the launch itself
                pool.time_next(*events[layer])
            pool.attend(layer, q[layer], k[layer], v[layer], out[layer], 0.125)
        pool.end()
        cur[:] += 1

    ms, kern, pct = timed_steps(step, args.steps, args.warmup, L, span=True)
    avg_ms = float(kern.mean())
    bytes_per_launch = bytes_timed[0] / bytes_timed[1]  # every layer of a step moves the same bytes
    achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
    fps = S / (ms / 1000.0)
    traffic = traffic_of("decode", {"streams": S, "layers": L, "max_len": args.max_len, "fixed_len": args.fixed_len,
                                    "split": args.split, "kv_heads": kvh}, bytes_per_launch)
    cpu = None if args.no_cpu else cpu_decode(L, lens, args.cpu_seconds)
    grouped = "" if kvh == H else f", {kvh} kv heads stored (grouped query heads)"
    config = {"workload": f"batched paged decode attention + KV append: {S} streams, Phonon-40m layers "
                          f"({L} x {H} heads x {D}{grouped}), bf16 K/V in 16-position pages, shuffled block "
                          f"tables, cache length U[1,{args.max_len}] growing one row per step",
              "streams": S, "layers": L, "heads": H, "kv_heads": kvh, "head_dim": D, "page": 16,
              "mean_cached_len": round(float(cur.mean()) - (args.steps + 1) / 2.0, 1)}
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": ("k_decode<bf16> (fused append + RoPE + decode)" if kvh == H or H // kvh > 16 else
                       "k_decode_gqa (fused append + RoPE + decode, the query heads of a kv head on MFMA)")
                      + ", one launch per layer",
            "avg_kernel_us": round(avg_ms * 1000.0, 2), "bytes_per_launch": int(bytes_per_launch)}
    return line("frames/sec (audio-sec/sec) at 1024 streams; decode-attn HBM GB/s % peak", fps, "frames/s", args,
                ms, "bf16", config, roof, cpu, extra={"audio_sec_per_sec": round(fps * 0.08, 1)}, pct=pct)


# ---- prompt prefill (configuration 3) ---------------------------------------------------------------
def cpu_prefill(L, T, seconds, sample=4):
    oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    rng = np.random.default_rng(SEED + 200)
    q, k, v = (bf16_np(rng.standard_normal((sample, T, H, D))) for _ in range(3))
    done, t0 = 0, time.perf_counter()
    while True:
        for i in range(sample):
            st = oracle.Stream(L, H, D, T, cache="bf16", act="bf16")
            for layer in range(L):
                st.append(layer, k[i], v[i])
                st.attention(layer, q[i])
            done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(done * T / el, 1), "unit": "positions/s", "cores": 1, "kind": "port",
            "sample": f"{done} prompts of {T} positions x {L} layers, one thread (the oracle's prefill is "
                      f"not threaded), {el:.1f} s"}


def run_prefill(args, xnp, torch):
    dev = torch.device("cuda:0")
    S, L, T = args.prefill_streams, args.layers, args.prompt
    mbps = (T + 15) // 16
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * mbps + 16, max_streams=S, max_blocks_per_stream=mbps,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=T + 16, page_seed=SEED + 3)
    gen = torch.Generator(device=dev).manual_seed(SEED + 4)
    q = [torch.randn((S, T, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    k = [torch.randn((S, T, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    v = [torch.randn((S, T, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    out = [torch.empty((S, T, H, D), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    torch.cuda.synchronize()
    ids = [pool.init_state(T) for _ in range(S)]

    def step(events):
        pool.begin(ids, t=T)
        for layer in range(L):
            if events is not None and events[layer] is not None:
                pool.time_next(*events[layer])
            pool.attend(layer, q[layer], k[layer], v[layer], out[layer], 0.125)
        pool.end()
        for i, sid in enumerate(ids):  # a new utterance per stream for the next step
            pool.close(sid)
            ids[i] = pool.init_state(T)

    ms, kern, pct = timed_steps(step, args.steps, args.warmup, L, span=True)
    avg_ms = float(kern.mean())
    flops = 2.0 * D * T * (T + 1) * H * S
    tflops = flops / (avg_ms * 1e-3) / 1e12
    # one launch per layer reads q and the new k, v rows, writes K and V into the pages and the
    # output: 6 S T H D bf16 values, plus 4 B of page id per page touched
    hbm = 6 * S * T * H * D * 2 + 4 * S * ((T + 15) // 16)
    gbs = hbm / (avg_ms * 1e-3) / 1e9
    cpu = None if args.no_cpu else cpu_prefill(L, T, args.cpu_seconds)
    config = {"workload": f"prompt prefill: {S} streams x {T}-position prompts, {L} layers x {H} heads x {D}, "
                          f"bf16, RoPE theta 10000, causal, K/V written into 16-position pages",
              "streams": S, "prompt": T, "layers": L}
    # At this shape the kernel does 2 D T (T+1) H S / (6 S T H D 2) = (T+1)/6 ~ 43 flop per byte,
    # far below the MFMA ridge (2.5 PFLOP/s / 8 TB/s ~ 312), so HBM bounds it; MFMA use is reported
    # beside it.
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_of("prefill", {"streams": S, "prompt": T, "layers": L}, hbm),
            "kernel": ("k_prefill_fast (fused append + RoPE + causal attention on v_mfma_f32_16x16x32_bf16, every "
                       "key of a prompt held in LDS), one launch per layer" if T <= 256 else
                       "k_prefill_mfma (fused append + RoPE + causal attention on v_mfma_f32_16x16x32_bf16, keys "
                       "streamed through LDS), one launch per layer"),
            "avg_kernel_us": round(avg_ms * 1000.0, 2), "bytes_per_launch": hbm,
            "mfma": {"achieved": round(tflops, 2), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4), "flops_per_launch": flops}}
    return line("prompt prefill positions/sec (64 streams x 256); MFMA TFLOP/s % peak", S * T / (ms / 1000.0),
                "positions/s", args, ms, "bf16", config, roof, cpu, pct=pct)


# ---- Mimi's windowed attention (a voice clip through Mimi's transformer) -------------------------------
# Mimi's transformer (the reference's fixture config: d_model 512, 8 heads, 2 layers, context 250):
# each step pushes a chunk of rows through a window of `context` positions per stream
# (transformer.rs:257-318,764-781).
MIMI_LAYERS, MIMI_CONTEXT = 2, 250


def mimi_held(context=MIMI_CONTEXT):
    """Held rows of a full window that the queries of the next chunk see: row i of the chunk sees the
    context - 1 - i before the chunk, so row 0 sees context - 1 of them."""
    return context - 1


def mimi_bytes(S, T, held, kvh=H):
    """One k_prefill_window launch: q and the output (H heads), the chunk's k and v (kvh heads) and the
    held rows any query sees (K and V, kvh heads), each read or written once, all bf16."""
    return S * (2 * T * H * D * 2 + 2 * T * kvh * D * 2 + 2 * held * kvh * D * 2)


def cpu_mimi(T, seconds, sample=2):
    oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    rng = np.random.default_rng(SEED + 700)
    wins = [oracle.Window(MIMI_LAYERS, H, D, MIMI_CONTEXT, rows_max=T, act="bf16") for _ in range(sample)]

    def chunk(w):
        for layer in range(MIMI_LAYERS):
            q, k, v = (bf16_np(rng.standard_normal((T, H, D))) for _ in range(3))
            w.attend(layer, q, k, v)
        w.commit(T)

    for w in wins:  # a full window first, as on the GPU
        chunk(w)
    done, t0 = 0, time.perf_counter()
    while True:
        for w in wins:
            chunk(w)
            done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(done * T / el, 1), "unit": "positions/s", "cores": 1, "kind": "port",
            "sample": f"{done} chunks of {T} rows x {MIMI_LAYERS} layers on {sample} full {MIMI_CONTEXT}-position "
                      f"windows, one thread (the oracle's window is not threaded), {el:.1f} s"}


def run_mimi(args, xnp, torch):
    dev = torch.device("cuda:0")
    S, T, L, C = args.mimi_streams, args.mimi_chunk, MIMI_LAYERS, MIMI_CONTEXT
    mbps = (C + 15) // 16
    chunks = args.warmup + args.steps + 2
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * mbps + 16, max_streams=S, max_blocks_per_stream=mbps,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=T * chunks + 16, page_seed=SEED + 7)
    ids = [pool.init_window(C) for _ in range(S)]
    gen = torch.Generator(device=dev).manual_seed(SEED + 8)
    q = [torch.randn((S, T, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    k = [torch.randn((S, T, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    v = [torch.randn((S, T, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    out = [torch.empty((S, T, H, D), dtype=torch.bfloat16, device=dev) for _ in range(L)]

    def step(events):
        pool.begin(ids, t=T)
        for layer in range(L):
            if events is not None and events[layer] is not None:
                pool.time_next(*events[layer])
            pool.attend(layer, q[layer], k[layer], v[layer], out[layer], 0.125)
        pool.end()

    step(None)  # the first chunk fills every window: the timed chunks see full windows
    torch.cuda.synchronize()
    # each layer's window append runs between the layers' attention launches, so a span would hold it:
    # one launch per timed step records both events around its own kernel
    ms, kern, pct = timed_steps(step, args.steps, args.warmup, L, span=False)
    avg_ms = float(kern.mean())
    held = mimi_held(C)
    hbm = mimi_bytes(S, T, held)
    gbs = hbm / (avg_ms * 1e-3) / 1e9
    # every query row sees `context` keys (its own and the context - 1 before it) once the window is full
    flops = 4.0 * D * T * min(C, held + T) * H * S
    tflops = flops / (avg_ms * 1e-3) / 1e12
    cpu = None if args.no_cpu else cpu_mimi(T, args.cpu_seconds)
    config = {"workload": f"Mimi windowed attention: {S} streams, chunks of {T} rows into full {C}-position windows, "
                          f"{L} layers x {H} heads x {D}, bf16, RoPE theta 10000",
              "streams": S, "chunk": T, "context": C, "layers": L}
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_of("mimi", {"streams": S, "chunk": T}, hbm),
            "kernel": "k_prefill_window (RoPE + windowed attention on v_mfma_f32_32x32x16_bf16, the held rows from "
                      "the pages and the chunk's own from k and v), one launch per layer; the step's k_window_append "
                      "(the rows that stay into their slots) is in the step time, not here",
            "avg_kernel_us": round(avg_ms * 1000.0, 2), "bytes_per_launch": hbm,
            "mfma": {"achieved": round(tflops, 2), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4), "flops_per_launch": flops}}
    return line(f"Mimi windowed attention positions/sec ({S} streams x {T}-row chunks, context {C})", S * T / (ms / 1000.0),
                "positions/s", args, ms, "bf16", config, roof, cpu, pct=pct)


# ---- int8 sliding window (configuration 4) ------------------------------------------------------------
SPAN, WINDOW = 528, 512


def cpu_window(L, lens_all, seconds, sample=64):
    oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    rng = np.random.default_rng(SEED + 300)
    lens = lens_all[:sample]
    streams, nxt = [], []
    for n in lens:
        st = oracle.Stream(L, H, D, SPAN, cache="i8", act="bf16")
        q8 = rng.integers(-127, 128, (SPAN, H, D)).astype(np.int8)
        sc = rng.uniform(0.01, 0.03, (SPAN // 16, H)).astype(np.float32)
        for layer in range(L):
            for kv in (0, 1):
                st.write_rows(layer, kv, 0, q8=q8, scales=sc)
        a = min(int(n), WINDOW)  # rows in view before the next step
        w0 = int(rng.integers(0, SPAN))  # slot of the next row
        valid = np.zeros(SPAN, np.uint8)
        for j in range(a):
            valid[(w0 - 1 - j) % SPAN] = 1
        st.ring_restore("absolute", w0, SPAN, 0, int(n) - a, a, valid)
        streams.append(st)
        nxt.append(w0)
    q, k, v = (bf16_np(rng.standard_normal((len(lens), H, D))) for _ in range(3))
    steps, t0 = 0, time.perf_counter()
    while True:
        for i, st in enumerate(streams):  # the sliding-window policy: s2s.rs:324-333 with drop 1
            if st.current_end == WINDOW:
                st.evict(0, [(nxt[i] - WINDOW) % SPAN])
            st.set_ring_slot(nxt[i])
            nxt[i] = (nxt[i] + 1) % SPAN
        for layer in range(L):
            oracle.batch_attend(streams, layer, q, k, v)
        oracle.batch_commit(streams)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(len(lens) * steps / el, 1), "unit": "frames/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{len(lens)} streams x {L} layers x {steps} steps of the same workload (int8 K/V, window "
                      f"{WINDOW} on {SPAN}-slot rings), {el:.1f} s"}


def run_window(args, xnp, torch):
    dev = torch.device("cuda:0")
    S, L = args.streams, args.layers
    rng = np.random.default_rng(SEED + 4)
    heads = rng.integers(0, 4096, S)
    lens = rng.integers(64, 2049, S)
    mbps = SPAN // 16
    total = int(lens.max()) + args.warmup + args.steps + 2
    kvh = args.kv_heads or H
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_kv_heads=kvh, num_blocks=S * mbps + 16, max_streams=S,
                      max_blocks_per_stream=mbps, cache_dtype="i8", act_dtype="bf16", max_pos=total + 16,
                      page_seed=SEED + 5)
    ids = [pool.init_state(SPAN) for _ in range(S)]
    for sid in ids:
        pool.start_ring(sid, "absolute", prefix=0)
    gen = torch.Generator(device=dev).manual_seed(SEED + 6)
    kv_new = [torch.randn((S, kvh, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(2 * L)]
    q = [torch.randn((S, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    out = [torch.empty((S, H, D), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    torch.cuda.synchronize()
    # write each stream's history: stream i joins at step N - n_i and appends one row per step
    N = int(lens.max())
    start = N - lens
    written = np.zeros(S, np.int64)
    for s in range(N):
        act = np.nonzero(start <= s)[0]
        if len(act) == 0:
            continue
        a_ids = [ids[i] for i in act]
        pool.slide_batch(a_ids, 0, SPAN, WINDOW, 1, heads[act] + written[act])
        pool.begin(a_ids)
        na = len(act)
        for layer in range(L):
            pool.append(layer, kv_new[2 * layer][:na], kv_new[2 * layer + 1][:na])
        pool.end()
        written[act] += 1
    torch.cuda.synchronize()
    bytes_timed = [0, 0]  # bytes of the timed launches, their count

    def step(events):
        att = np.minimum(written + 1, WINDOW)
        if events is not None:
            bytes_timed[0] += window_bytes(att, kvh)  # the one launch this step times
            bytes_timed[1] += 1
        pool.slide_batch(ids, 0, SPAN, WINDOW, 1, heads + written)
        pool.begin(ids)
        for layer in range(L):
            if events is not None and events[layer] is not None:
                pool.time_next(*events[layer])
            pool.attend(layer, q[layer], kv_new[2 * layer], kv_new[2 * layer + 1], out[layer], 0.125)
        pool.end()
        written[:] += 1

    ms, kern, pct = timed_steps(step, args.steps, args.warmup, L, span=True)
    avg_ms = float(kern.mean())
    bytes_per_launch = bytes_timed[0] / bytes_timed[1]  # every layer of a step moves the same bytes
    achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
    fps = S / (ms / 1000.0)
    cpu = None if args.no_cpu or kvh != H else cpu_window(L, lens, args.cpu_seconds)  # the oracle leg keeps H kv heads
    config = {"workload": f"int8 K/V sliding window: {S} streams, {L} layers x {H} heads x {D}, fp32 scales per "
                          f"(page, head), window {WINDOW} on {SPAN}-slot rings, write heads U[0,4096), "
                          f"rows written U[64,2048]; evict + append + dequant-on-gather decode per step",
              "streams": S, "layers": L, "window": WINDOW, "ring_slots": SPAN, "kv_heads": kvh}
    wkey = {"streams": S, "layers": L} if kvh == H else {"streams": S, "layers": L, "kv_heads": kvh}
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_of("window", wkey, bytes_per_launch),
            "kernel": ("k_decode<int8> (fused append + quantize + RoPE + dequant decode)" if kvh == H else
                       "k_decode_gqa<int8> (MFMA over whole kv heads, fused append + quantize + RoPE + dequant "
                       "decode)") + ", one launch per layer",
            "avg_kernel_us": round(avg_ms * 1000.0, 2), "bytes_per_launch": int(bytes_per_launch)}
    return line("frames/sec, int8 KV sliding window (512) at 1024 streams; decode HBM GB/s % peak", fps,
                "frames/s", args, ms, "int8", config, roof, cpu, extra={"audio_sec_per_sec": round(fps * 0.08, 1)},
                pct=pct)


# ---- the full per-frame layer step (configuration 5) ---------------------------------------------
DM, FF = 512, 2048


def gemm_flops(rows):
    """Multiply-adds x 2 of the four q8 projections of one layer over `rows` rows."""
    return 2.0 * rows * DM * ((H + 2 * H) * D + DM + FF) + 2.0 * rows * FF * DM


def step_weights(rng, L):
    xnp = _load("xn_ptts_amd", os.path.join(ROOT, "xn-ptts_amd"))
    ws = []
    for _ in range(L):
        qr = lambda n, k: xnp.quantize_rows(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
        parts = dict(zip(["wqkv", "sqkv"], qr(3 * H * D, DM)))
        parts.update(zip(["wout", "sout"], qr(DM, H * D)))
        parts.update(zip(["w1", "s1"], qr(FF, DM)))
        parts.update(zip(["w2", "s2"], qr(DM, FF)))
        for n in ("ln1", "ln2"):
            parts[n + "_w"] = np.ones(DM, np.float32)
            parts[n + "_b"] = np.zeros(DM, np.float32)
        ws.append(parts)
    return ws


def cpu_step(L, lens_all, weights, seconds, sample=64):
    oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    rng = np.random.default_rng(SEED + 500)
    lens = lens_all[:sample]
    room = 512  # steps the sample's caches have room for
    cap = int(lens.max()) + room
    streams = [oracle.Stream(L, H, D, cap, cache="bf16", act="bf16") for _ in lens]
    rows = bf16_np(rng.standard_normal((int(lens.max()), H, D)))
    for st, n in zip(streams, lens):
        for layer in range(L):
            st.write_rows(layer, 0, 0, vals=rows[:n])
            st.write_rows(layer, 1, 0, vals=rows[:n][::-1].copy())
        st.advance(int(n))
    W = [oracle.LayerWeights(**w) for w in weights]
    x0 = bf16_np(rng.standard_normal((len(lens), 1, DM)))
    steps, t0 = 0, time.perf_counter()
    while True:
        x = x0
        for layer in range(L):
            x = oracle.layer_step(streams, layer, W[layer], x)
        oracle.batch_commit(streams)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds or steps >= room:
            break
    return {"value": round(len(lens) * steps / el, 1), "unit": "frames/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{len(lens)} streams x {L} layers x {steps} steps of the same workload (bf16, lengths from "
                      f"the same U[1,1500] draw, the same q8 weights), {el:.1f} s"}


def run_step(args, xnp, torch):
    dev = torch.device("cuda:0")
    S, L = args.step_streams, args.layers
    rng = np.random.default_rng(SEED + 5)
    lens = rng.integers(1, args.step_max_len + 1, S)
    total_steps = args.warmup + args.steps
    cap = args.step_max_len + total_steps + 1
    mbps = (cap + 15) // 16
    nblocks = int(sum((n + total_steps + 16) // 16 + 1 for n in lens)) + 16
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=nblocks, max_streams=S, max_blocks_per_stream=mbps,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=cap + 16, page_seed=SEED + 6)
    ids = [pool.init_state(cap) for _ in range(S)]
    gen = torch.Generator(device=dev).manual_seed(SEED + 7)
    maxn = int(lens.max())
    for layer in range(L):
        for kvi in (0, 1):
            rows = torch.randn((maxn, H, D), generator=gen, device=dev).to(torch.bfloat16)
            for sid, n in zip(ids, lens):
                if layer == 0 and kvi == 0:
                    pool.advance(sid, int(n))
                pool.write_rows(sid, layer, kvi, 0, rows[:n])
    wnp = step_weights(np.random.default_rng(SEED + 8), L)
    W = []
    for w in wnp:
        d = {k: torch.from_numpy(v).to(dev) for k, v in w.items()}
        W.append(xnp.LayerWeights(**d))
    x0 = torch.randn((S, 1, DM), generator=gen, device=dev).to(torch.bfloat16)
    x = torch.empty_like(x0)
    ws = torch.empty(pool.layer_workspace(S, DM, FF), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    cur = lens.copy()
    bytes_timed = [0, 0]  # bytes of the timed launches, their count

    def step(events):
        if events is not None:
            bytes_timed[0] += decode_bytes(cur)  # the one launch this step times
            bytes_timed[1] += 1
        x.copy_(x0)  # the step's input rows (synthetic; the model's would come from its embeddings)
        pool.begin(ids)
        for layer in range(L):
            if events is not None and events[layer] is not None:
                pool.time_next(*events[layer])
            pool.layer_step(layer, W[layer], x, ws)
        pool.end()
        cur[:] += 1

    ms, kern, pct = timed_steps(step, args.steps, args.warmup, L)
    avg_ms = float(kern.mean())
    bytes_per_launch = bytes_timed[0] / bytes_timed[1]  # every layer of a step moves the same bytes
    achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
    fps = S / (ms / 1000.0)
    rest_ms = ms / L - avg_ms  # per layer: norms, projections, plan, launch gaps
    flops = gemm_flops(S)
    cpu = None if args.no_cpu else cpu_step(L, lens, wnp, args.cpu_seconds)
    config = {"workload": f"full per-frame flow-LM layer step: {S} streams, Phonon-40m layers ({L} x {DM} wide, "
                          f"{H} heads x {D}, FF {FF}), int8 per-channel q8 projections (QKV, out, FF) on MFMA, "
                          f"LayerNorm, erf GELU, residuals, RoPE, paged bf16 KV append and decode attention, cache "
                          f"length U[1,{args.step_max_len}]",
              "streams": S, "layers": L, "d_model": DM, "ff": FF}
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_of("step", {"streams": S, "layers": L, "max_len": args.step_max_len}, bytes_per_launch),
            "kernel": "k_decode<bf16> (fused append + RoPE + decode), one launch per layer",
            "avg_kernel_us": round(avg_ms * 1000.0, 2), "bytes_per_launch": int(bytes_per_launch),
            "rest_of_layer_us": round(rest_ms * 1000.0, 2), "gemm_gop_per_layer": round(flops / 1e9, 2),
            "gemm_tops_upper_bound": round(flops / (rest_ms * 1e-3) / 1e12, 2)}
    return line("frames/sec, full per-frame layer step at 2048 streams; decode-attn HBM GB/s % peak", fps,
                "frames/s", args, ms, "bf16", config, roof, cpu, extra={"audio_sec_per_sec": round(fps * 0.08, 1)},
                pct=pct)


# ---- the batched frame: the q8 flow LM at 2048 streams ----------------------------------------------
def cpu_frame(cfg, blob, lens, seconds, threads):
    """The oracle's q8 frame on a sample of the streams, one stream per host thread (each call
    releases the interpreter lock): frames/s over the sample."""
    from concurrent.futures import ThreadPoolExecutor
    oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    m = oracle.FlowLM(cfg, blob)
    rng = np.random.default_rng(SEED + 11)
    sample = [int(n) for n in lens[:2 * threads]]
    sts = []
    for n in sample:
        st = m.stream(n + 256)
        for layer in range(cfg.num_layers):
            for kv in (0, 1):
                st.write_rows(layer, kv, 0, rng.standard_normal((n, H, D)).astype(np.float32))
        st.advance(n)
        sts.append(st)
    zero = np.zeros(cfg.ldim, np.float32)

    def run(i):
        m.step(sts[i], None, zero)

    frames, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        while time.perf_counter() - t0 < seconds and frames < 200 * len(sts):
            list(ex.map(run, range(len(sts))))
            frames += len(sts)
    el = time.perf_counter() - t0
    return {"value": round(frames / el, 2), "unit": "frames/s", "cores": threads, "kind": "port",
            "sample": f"{len(sts)} streams of the same length draw, {frames // len(sts)} frames each, the q8 frame "
                      f"(oracle, one stream per thread), {el:.1f} s"}


def run_frame(args, xnp, torch):
    dev = torch.device("cuda:0")
    fl = xnp.flow_lm
    S, L = args.step_streams, args.layers
    cfg = fl.FlowLMConfig(num_layers=L, precision="q8")  # 9 x 512, 8 heads, FF 2048; flow net 512 x 6; ldim 32
    blob = fl.random_weights(cfg, SEED + 10)
    rng = np.random.default_rng(SEED + 5)
    lens = rng.integers(1, args.step_max_len + 1, S)
    total = args.warmup + 2 * args.steps + 8
    cap = args.step_max_len + total + 1
    mbps = (cap + 15) // 16
    nblocks = int(sum((n + total + 16) // 16 + 1 for n in lens)) + 16
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=nblocks, max_streams=S, max_blocks_per_stream=mbps,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=cap + 16, page_seed=SEED + 6)
    ids = [pool.init_state(cap) for _ in range(S)]
    gen = torch.Generator(device=dev).manual_seed(SEED + 7)
    maxn = int(lens.max())
    for layer in range(L):
        for kvi in (0, 1):
            rows = torch.randn((maxn, H, D), generator=gen, device=dev).to(torch.bfloat16)
            for sid, n in zip(ids, lens):
                if layer == 0 and kvi == 0:
                    pool.advance(sid, int(n))
                pool.write_rows(sid, layer, kvi, 0, rows[:n])
    lm = xnp.FlowLM(pool, cfg, blob, max_rows=S)
    lat = torch.zeros((S, cfg.ldim), dtype=torch.float32, device=dev)
    eos = torch.empty(S, dtype=torch.float32, device=dev)
    noise = torch.zeros((S, cfg.ldim), dtype=torch.float32, device=dev)  # temperature 0
    stream = torch.cuda.Stream()
    cur = lens.copy()
    with torch.cuda.stream(stream):
        lm.step(ids, None, noise, lat, eos, graph=True)  # the bos frame, then frames from the latents
        cur += 1
        for _ in range(args.warmup):
            lm.step(ids, lat, noise, lat, eos, graph=True)
            cur += 1
        stream.synchronize()
        bytes0 = decode_bytes(cur)
        marks = StepMarks(args.steps)
        with NoGC():
            t0 = time.perf_counter()
            for _ in range(args.steps):
                marks.mark()
                lm.step(ids, lat, noise, lat, eos, graph=True)
            marks.mark()
            stream.synchronize()
        ms = (time.perf_counter() - t0) * 1000.0 / args.steps
        cur += args.steps
        # the dominant kernel: layer 0's fused append + decode, timed by its launch's events over
        # eager frames (an event recorded inside a graph replay is not the launch's own)
        hip = HipEvents()
        evs, bts = [], []
        for _ in range(args.steps):
            e = (hip.create(), hip.create())
            bts.append(decode_bytes(cur))
            pool.time_next(*e)
            lm.step(ids, lat, noise, lat, eos)
            evs.append(e)
            cur += 1
        stream.synchronize()
        kern = np.array([hip.elapsed_ms(*e) for e in evs])
        for e in evs:
            hip.destroy(e[0])
            hip.destroy(e[1])
    avg_ms = float(kern.mean())
    achieved = float(np.mean(bts)) / (avg_ms * 1e-3) / 1e9
    fps = S / (ms / 1000.0)
    cpu = None if args.no_cpu else cpu_frame(cfg, blob, lens, args.cpu_seconds, host_threads())
    config = {"workload": f"full batched flow-LM frame at {S} streams, q8: input_linear, {L} transformer layers "
                          f"({DM} wide, {H} heads x {D}, FF {FF}, int8 per-channel weights on MFMA, bf16 activations, "
                          f"paged bf16 KV append + decode over cache lengths U[1,{args.step_max_len}]), out_norm, the "
                          f"EOS head and the flow net (512 x 6, one LSD step) at temperature 0; every frame replayed "
                          f"from one hipGraph after its plan upload",
              "streams": S, "layers": L, "d_model": DM, "ff": FF, "flow": "512 x 6"}
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_of("frame", {"streams": S, "layers": L, "max_len": args.step_max_len}, float(np.mean(bts))),
            "kernel": "k_decode<bf16> (fused append + RoPE + decode) of layer 0, timed in eager frames",
            "avg_kernel_us": round(avg_ms * 1000.0, 2), "bytes_per_launch": int(np.mean(bts)),
            "decode_share_of_frame": round(L * avg_ms / ms, 3)}
    return line("frames/sec, full batched flow-LM frame at 2048 streams (q8 transformer + flow net)", fps,
                "frames/s", args, ms, "bf16", config, roof, cpu, extra={"audio_sec_per_sec": round(fps * 0.08, 1)},
                pct=marks.percentiles())


# ---- the single-stream flow LM (configuration 1) ----------------------------------------------------
def flow_bytes(cfg, n):
    """Algorithmic bytes of one frame at batch 1: every f32 weight of the transformer, the heads and
    the flow net read once, plus the K/V rows attended (n cached before the step), in f32."""
    d, F, ld, ff = cfg.d_model, cfg.flow_dim, cfg.ldim, cfg.dim_feedforward
    w = d * ld + cfg.num_layers * (4 * d * d + 2 * d * ff + 4 * d) + 2 * d + d + 1
    w += F * d + F + F * ld + F + cfg.flow_depth * (5 * F * F + 8 * F) + 2 * F * F + 2 * F + ld * F + ld
    kv = cfg.num_layers * 2 * (n + 1) * d
    return 4 * (w + kv)


def cpu_flowlm(cfg, blob, tokens, seconds, threads):
    oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    oracle.set_threads(threads)
    m = oracle.FlowLM(cfg, blob)
    st = m.stream(len(tokens) + 512)
    m.prompt_text(st, tokens)
    zero = np.zeros(cfg.ldim, np.float32)
    lat, frames, t0 = None, 0, time.perf_counter()
    while True:
        lat, _ = m.step(st, lat, zero)
        frames += 1
        el = time.perf_counter() - t0
        if el >= seconds or frames >= 512:
            break
    return {"value": round(frames / el, 1), "unit": "frames/s", "cores": threads, "kind": "port",
            "sample": f"the same stream: {len(tokens)}-token prompt, then {frames} frames at temperature 0, "
                      f"{el:.1f} s on {threads} thread{'s' if threads > 1 else ''}"}


def run_vendor_gemm(args, xnp, torch):
    """The vendor library's bf16 GEMMs (torch.nn.functional.linear: hipBLASLt) and LayerNorm at the
    layer step's shapes, for comparison with the q8 projections: bf16 weights (no widening), no
    epilogue.  Each op is replayed from a torch graph of 20 calls, so the host's launch rate is out
    of the time."""
    dev = torch.device("cuda:0")
    M = args.step_streams
    shapes = {"in_proj": (3 * H * D, DM), "out_proj": (DM, H * D), "linear1": (FF, DM), "linear2": (DM, FF)}
    gen = torch.Generator(device=dev).manual_seed(SEED + 12)
    stream = torch.cuda.Stream()
    per, flops = {}, {}

    def time_op(fn, reps=20):
        with torch.cuda.stream(stream):
            for _ in range(3):
                fn()
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(reps):
                fn()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / (args.steps * reps)

    for name, (N, K) in shapes.items():
        x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
        w = torch.randn((N, K), generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        per[name] = round(time_op(lambda: torch.matmul(x, w.t(), out=y)), 2)
        flops[name] = 2.0 * M * N * K
    x = torch.randn((M, DM), generator=gen, device=dev).to(torch.bfloat16)
    ln = torch.nn.LayerNorm(DM, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        ln_us = round(time_op(lambda: ln(x)), 2)
    total = sum(per.values())
    config = {"workload": f"the vendor library at the layer step's shapes: {M} rows, bf16 x[M, K] W[N, K]^T for "
                          f"in_proj, out_proj, linear1, linear2 (d_model {DM}, FF {FF}); LayerNorm of {M} x {DM}",
              "rows": M, "d_model": DM, "ff": FF}
    roof = {"bound": "mfma", "achieved": round(sum(flops.values()) / (total * 1e-6) / 1e12, 1),
            "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(sum(flops.values()) / (total * 1e-6) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4), "traffic": None,
            "kernel": "torch.matmul (hipBLASLt) bf16, one call per projection; torch LayerNorm",
            "per_projection_us": per, "layer_norm_us": ln_us}
    return line("us per layer for the four projections' bf16 GEMMs in the vendor library (comparison only)",
                total, "us", args, total / 1000.0, "bf16", config, roof, None, higher=False)


def run_flowlm(args, xnp, torch):
    dev = torch.device("cuda:0")
    fl = xnp.flow_lm
    cfg = fl.FlowLMConfig()  # Phonon-31m: 6 x 512, 8 heads, FF 2048, ldim 32, n_bins 4000, flow 512 x 6
    blob = fl.random_weights(cfg, SEED)
    rng = np.random.default_rng(SEED)
    tokens = rng.integers(0, cfg.n_bins + 1, 64).astype(np.int32)
    frames = args.warmup + args.steps
    cap = xnp.seq_budget(64, xnp.frame_budget(64))  # plan.rs:52-54: 868
    if 64 + 2 * frames > cap:
        raise SystemExit(f"{frames} frames twice do not fit the {cap}-position budget of a 64-token prompt")
    mbps = (cap + 15) // 16
    pool = xnp.KvPool(num_layers=cfg.num_layers, num_heads=cfg.num_heads, num_blocks=mbps + 4, max_streams=1,
                      max_blocks_per_stream=mbps, cache_dtype="f32", act_dtype="f32", max_pos=cap + 16,
                      page_seed=SEED + 9)
    sid = pool.init_state(cap)
    lm = xnp.FlowLM(pool, cfg, blob, max_rows=64)
    noise = torch.zeros((1, cfg.ldim), dtype=torch.float32, device=dev)  # temperature 0
    lat = torch.zeros((1, cfg.ldim), dtype=torch.float32, device=dev)  # read and overwritten in place
    eos = torch.empty(1, dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream()  # a recorded frame replays on a stream of the caller's
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        t0 = time.perf_counter()
        lm.prompt_text([sid], tokens[None, :])
        stream.synchronize()
        prompt_ms = (time.perf_counter() - t0) * 1000.0

        def frames_ms(first, count, graph, marks=None):
            with NoGC():
                t = time.perf_counter()
                for f in range(first, first + count):
                    if marks:
                        marks.mark()
                    lm.step([sid], None if f == 0 else lat, noise, lat, eos, graph=graph)
                if marks:
                    marks.mark()
                stream.synchronize()
                return (time.perf_counter() - t) * 1000.0 / max(count, 1)

        frames_ms(0, args.warmup, True)
        ms = frames_ms(args.warmup, args.steps, True)  # the value: frames replayed from a recording
        n_eager = min(args.steps, cap - 64 - frames)
        eager_ms = frames_ms(frames, n_eager, False)  # the same frames, launched
        # the frame periods' percentiles come from a replayed pass of their own: an event recorded
        # between frames costs a visible share of a 0.2 ms frame at batch 1
        n_pct = min(args.steps, cap - 64 - frames - n_eager)
        marks = StepMarks(n_pct)
        frames_ms(frames + n_eager, n_pct, True, marks)
    fps = 1000.0 / ms
    bytes_mean = np.mean([flow_bytes(cfg, 64 + f) for f in range(args.warmup, frames)])
    gbs = bytes_mean / (ms * 1e-3) / 1e9
    cpu = None if args.no_cpu else cpu_flowlm(cfg, blob, tokens, args.cpu_seconds, 1)
    extra = {"audio_sec_per_sec": round(fps * 0.08, 2), "prompt_ms": round(prompt_ms, 3),
             "eager_frames_per_s": round(1000.0 / eager_ms, 1)}
    if not args.no_cpu:
        oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
        extra["cpu_baseline_all_cores"] = cpu_flowlm(cfg, blob, tokens, args.cpu_seconds, host_threads())
        oracle.set_threads(host_threads())
    config = {"workload": "single-stream flow LM, Phonon-31m shape (6 x 512, 8 heads x 64, FF 2048, ldim 32, "
                          "n_bins 4000, flow net 512 x 6, 1 LSD step), random-init f32 weights N(0, 0.02), unit "
                          "norms; 64 seeded tokens, then greedy frames at temperature 0 on an f32 paged cache",
              "streams": 1, "layers": cfg.num_layers, "prompt_tokens": 64, "frames_timed": args.steps}
    # batch 1 is bound by its chain of about 50 dependent kernels: the roofline is the frame's bytes
    # (every f32 weight once plus the K/V attended) over its wall time, not one kernel's
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "whole frame replayed from a hipGraph: f32 linears (LayerNorms fused), k_decode<f32>, flow "
                      "net (batch 1, bound by its chain of about 50 dependent kernels)",
            "bytes_per_frame": int(bytes_mean)}
    return line("frames/sec, single-stream flow LM (Phonon-31m shape, fp32)", fps, "frames/s", args, ms, "f32",
                config, roof, cpu, extra=extra, pct=marks.percentiles() if n_pct >= 2 else None)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=["decode", "prefill", "window", "step", "flowlm", "frame", "mimi",
                                           "vendor_gemm"],
                    default="decode")
    ap.add_argument("--step-streams", type=int, default=2048)
    ap.add_argument("--step-max-len", type=int, default=1500)
    ap.add_argument("--streams", type=int, default=1024)
    ap.add_argument("--layers", type=int, default=9)
    ap.add_argument("--max-len", type=int, default=1024)
    ap.add_argument("--fixed-len", type=int, default=0,
                    help="decode: every stream at this cached length instead of U[1, max-len] (a balance check)")
    ap.add_argument("--split", type=int, default=0, help="decode: waves per (stream, head): 1, 2, 4, 8 (0: default)")
    ap.add_argument("--kv-heads", type=int, default=0,
                    help="decode: kv heads stored (grouped query heads; 0: one per query head)")
    ap.add_argument("--prefill-streams", type=int, default=64)
    ap.add_argument("--prompt", type=int, default=256)
    ap.add_argument("--mimi-streams", type=int, default=256)
    ap.add_argument("--mimi-chunk", type=int, default=250)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="decode: only the headline, without the other configurations' entries")
    ap.add_argument("--nested-steps", type=int, default=20, help="timed steps of each nested configuration")
    ap.add_argument("--nested-cpu-seconds", type=float, default=5.0)
    ap.add_argument("--calibrate", action="store_true",
                    help="only copy 1 GiB device to device 5 times: the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.calibrate:
        import torch
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": src.numel() * src.element_size(), "copies": 5}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: streams are independent and would shard "
                                   "by stream across GPUs, but no multi-GPU run is part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    xnp = _load("xn_ptts_amd", os.path.join(ROOT, "xn-ptts_amd"))
    xnp.load_library()
    runs = {"decode": run_decode, "prefill": run_prefill, "window": run_window, "step": run_step,
            "flowlm": run_flowlm, "frame": run_frame, "mimi": run_mimi, "vendor_gemm": run_vendor_gemm}
    out = runs[args.workload](args, xnp, torch)
    if args.workload == "decode" and not args.headline_only and headline_args(args):
        out["configs"] = nested_configs(args, xnp, torch, runs)
    print(json.dumps(out))


# The other configurations of the same run, each an entry of the headline's line: the workload's
# own value, step time, roofline and CPU baseline, timed as its own --workload run times it.
NESTED = [("flowlm", 1, "single-stream flow LM, Phonon-31m shape, f32 (batch 1)"),
          ("prefill", 3, "prompt prefill, 64 streams x 256 positions"),
          ("window", 4, "int8 KV sliding window (512), 1024 streams"),
          ("step", 5, "full per-frame layer step, 2048 streams"),
          ("frame", 5, "the batched q8 flow-LM frame around configuration 5's layers (flow net and heads included)"),
          ("mimi", None, "Mimi's windowed attention (no configuration of its own): 256 streams x 250-row chunks, context 250")]


def headline_args(args):
    """The default headline workload (the nested entries describe the configurations as drawn)."""
    return (args.streams, args.layers, args.max_len, args.fixed_len, args.split, args.kv_heads) == (1024, 9, 1024, 0, 0, 0)


def nested_configs(args, xnp, torch, runs):
    entries = {}
    for name, cfg_index, what in NESTED:
        sub = argparse.Namespace(**vars(args))
        sub.workload, sub.steps, sub.cpu_seconds = name, args.nested_steps, args.nested_cpu_seconds
        gc.collect()
        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        res = runs[name](sub, xnp, torch)
        keep = {k: v for k, v in res.items() if k not in ("n_gpus", "scaling", "vs_baseline", "data")}
        keep["configuration"] = cfg_index
        keep["what"] = what
        keep["wall_s"] = round(time.perf_counter() - t0, 1)
        entries[name] = keep
        print(f"# {name}: {res['value']} {res['unit']} ({keep['wall_s']} s)", file=sys.stderr, flush=True)
    return entries


if __name__ == "__main__":
    main()
