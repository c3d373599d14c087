"""Batched paged decode attention + KV append for many Phonon-40m-shaped streams on one MI355X.

Workload (default): 1024 concurrent streams, 9 layers x 8 heads x 64, bf16 K/V in 16-position
pages handed out from a shuffled free list, cache length per stream drawn uniform in [1, 1024]
(seed 20261202), one bf16 query and one new K/V row per stream per layer, N(0, 1).  A step is one
pass over all 9 layers: plan upload, then per layer one fused append + RoPE + decode kernel.  frames/s = streams / step time; audio-s/s = frames/s * 0.08 (12.5 Hz frames).

Roofline: algorithmic bytes per decode kernel launch (per stream: 2 (n+1) H D 2 B of K/V read,
1 KB q, 2 KB new k/v, 1 KB out, 2 KB append write, 4 ceil((n+1)/16) B of block table) over the
kernel's average duration, against 8 TB/s.  The duration comes from HIP events that the launch
itself records as the kernel starts and ends (hipExtLaunchKernel, via xnp_pool_time_next), on
the stream the kernel runs on.

CPU baseline: the oracle (the C restatement, OpenMP over streams) on a bounded sample of the same
workload -- 128 streams, the same length distribution -- timed on this host's cores.
"""
import argparse
import importlib.util
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
SEED = 20261201


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


def algorithmic_bytes(lens, H=8, D=64, elem=2):
    """Bytes one layer's append + decode must move for streams with cached lengths `lens`."""
    lens = np.asarray(lens, np.int64)
    kv = 2 * (lens + 1) * H * D * elem
    fixed = (H * D * elem) * (1 + 2 + 1 + 2)  # q, new k/v, out, append write
    table = 4 * ((lens + 1 + 15) // 16)
    return int((kv + fixed + table).sum())


def cpu_baseline(L, H, lens_all, seconds=10.0, sample=128):
    """The oracle on `sample` streams of the workload, all layers per step, until `seconds`."""
    oracle = _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
    rng = np.random.default_rng(SEED + 100)
    lens = lens_all[:sample]
    cap = int(lens.max()) + 64
    streams = [oracle.Stream(L, H, 64, cap, cache="bf16", act="bf16") for _ in lens]

    def bf16(a):
        u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32).reshape(a.shape)

    pool_rows = bf16(rng.standard_normal((int(lens.max()), H, 64)))
    for st, n in zip(streams, lens):
        for layer in range(L):
            st.write_rows(layer, 0, 0, vals=pool_rows[:n])
            st.write_rows(layer, 1, 0, vals=pool_rows[:n][::-1].copy())
        st.advance(int(n))
    q, k, v = (bf16(rng.standard_normal((len(lens), H, 64))) for _ in range(3))
    steps, t0 = 0, time.perf_counter()
    while True:
        for layer in range(L):
            oracle.batch_attend(streams, layer, q, k, v)
        oracle.batch_commit(streams)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds or steps >= 64:
            break
    fps = len(lens) * steps / el
    return {"value": round(fps, 1), "unit": "frames/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{len(lens)} streams x {L} layers x {steps} steps of the same workload "
                      f"(bf16, lengths from the same U[1,1024] draw), {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--streams", type=int, default=1024)
    ap.add_argument("--layers", type=int, default=9)
    ap.add_argument("--max-len", type=int, default=1024)
    ap.add_argument("--fixed-len", type=int, default=0,
                    help="every stream at this cached length instead of U[1, max-len] (a balance check)")
    ap.add_argument("--split", type=int, default=0, help="waves per (stream, head) in decode: 2, 4, 8 (0: default)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
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
    dev = torch.device("cuda:0")
    S, L, H, D = args.streams, args.layers, 8, 64
    rng = np.random.default_rng(SEED + 1)
    lens = rng.integers(1, args.max_len + 1, S)
    if args.fixed_len:
        lens = np.full(S, args.fixed_len)
    total_steps = args.warmup + args.steps
    cap = args.max_len + total_steps + 1
    mbps = (cap + 15) // 16
    nblocks = int(sum((n + total_steps + 16) // 16 + 1 for n in lens)) + 16
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=nblocks, max_streams=S, max_blocks_per_stream=mbps,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=cap + 16, page_seed=SEED + 2,
                      decode_split=args.split)
    ids = [pool.init_state(cap) for _ in range(S)]
    gen = torch.Generator(device=dev).manual_seed(SEED + 3)
    maxn = int(lens.max())
    for layer in range(L):
        for kvi in (0, 1):
            rows = torch.randn((maxn, H, D), generator=gen, device=dev).to(torch.bfloat16)
            for sid, n in zip(ids, lens):
                if layer == 0 and kvi == 0:
                    pool.advance(sid, int(n))
                pool.write_rows(sid, layer, kvi, 0, rows[:n])
    q = [torch.randn((S, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    k = [torch.randn((S, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    v = [torch.randn((S, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
    out = [torch.empty((S, H, D), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    torch.cuda.synchronize()

    cur = lens.copy()

    def step(events=None):
        pool.begin(ids)
        for layer in range(L):
            if events is not None:  # recorded by the launch itself, around the kernel alone
                pool.time_next(events[layer][0], events[layer][1])
            pool.attend(layer, q[layer], k[layer], v[layer], out[layer], 0.125)
        pool.end()

    for _ in range(args.warmup):
        step()
        cur += 1
    torch.cuda.synchronize()
    hip = HipEvents()
    ev = [[[hip.create() for _ in range(2)] for _ in range(L)] for _ in range(args.steps)]
    bytes_total = 0
    t0 = time.perf_counter()
    for s in range(args.steps):
        bytes_total += L * algorithmic_bytes(cur, H, D)
        step(ev[s])
        cur += 1
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1000.0 / args.steps
    call_ms = np.array([[hip.elapsed_ms(ev[s][l][0], ev[s][l][1]) for l in range(L)] for s in range(args.steps)])
    for e in (e for s_ in ev for l_ in s_ for e in l_):
        hip.destroy(e)
    avg_call_ms = float(call_ms.mean())
    calls = args.steps * L
    bytes_per_call = bytes_total / calls
    achieved = bytes_per_call / (avg_call_ms * 1e-3) / 1e9
    fps = S / (ms_per_step / 1000.0)

    # HBM traffic per launch from the FETCH_SIZE / WRITE_SIZE counter runs of this same command,
    # scaled by the factors a copy of known size gives (profiles/decode_traffic.json).
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tr = json.load(f)
        same = tr.get("workload") == {"streams": S, "layers": L, "max_len": args.max_len, "steps": args.steps,
                                      "warmup": args.warmup, "fixed_len": args.fixed_len, "split": args.split}
        if same:
            traffic = int(tr["traffic_bytes_per_launch"])

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(L, H, lens, seconds=args.cpu_seconds)

    line = {
        "metric": "frames/sec (audio-sec/sec) at 1024 streams; decode-attn HBM GB/s % peak",
        "value": round(fps, 1),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"batched paged decode attention + KV append: {S} streams, Phonon-40m layers "
                        f"({L} x {H} heads x {D}), bf16 K/V in 16-position pages, shuffled block tables, "
                        f"cache length U[1,{args.max_len}] growing one row per step",
            "streams": S, "layers": L, "heads": H, "head_dim": D, "page": 16,
            "mean_cached_len": round(float(cur.mean()) - (args.steps + 1) / 2.0, 1),
        },
        "audio_sec_per_sec": round(fps * 0.08, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "k_decode<bf16> (fused append + RoPE + decode), one launch per layer",
            "avg_kernel_us": round(avg_call_ms * 1000.0, 2),
            "bytes_per_launch": int(bytes_per_call),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
