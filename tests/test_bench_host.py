"""Host logic of bench.py, on the CPU: the algorithmic byte counts its roofline divides by (checked
at sizes small enough to count by hand), the counter-ratio lookup behind `roofline.traffic`, which
runs carry the nested configurations, and the refusal of more than one GPU."""
import argparse
import importlib.util
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_decode_bytes_count_what_one_layer_moves():
    b = _bench()
    # 15 cached rows + the new one = 16 rows, one page: K and V of 8 heads x 64 dims in bf16
    # (2 x 16 x 8 x 64 x 2 = 32768), q and out (2 x 1024), the new k/v rows read (2048) and written
    # (2048), one page id (4)
    assert b.decode_bytes([15]) == 32768 + 2048 + 2048 + 2048 + 4
    # 16 cached rows: 17 rows over two pages, two page ids
    assert b.decode_bytes([16]) == 2 * 17 * 8 * 64 * 2 + 3 * 2048 + 8
    assert b.decode_bytes([15, 16]) == b.decode_bytes([15]) + b.decode_bytes([16])
    # int8 cache: one byte per K/V element and per appended element; q, out and new rows stay bf16
    assert b.decode_bytes([15], elem=1) == 16384 + 2048 + 2048 + 1024 + 4
    # one stored kv head under 8 query heads: K/V and the new rows once, q and out per query head
    assert b.decode_bytes([15], kvh=1) == 4096 + 2048 + 256 + 256 + 4


def test_window_bytes_count_rows_scales_and_page_ids():
    b = _bench()
    # 16 attended rows of int8 K and V (2 x 16 x 8 x 64), K and V scales of 2 pages (the attended
    # one and the write page) per kv head (2 x 8 x 4 x 2), bf16 q and out (2048), new bf16 k/v
    # rows (2048), their int8 append (1024), 2 page ids (8)
    assert b.window_bytes([16]) == 16384 + 128 + 2048 + 2048 + 1024 + 8


def test_mimi_bytes_count_the_chunk_and_the_held_rows_it_sees():
    b = _bench()
    # a full window of context 250 holds 249 rows between chunks; row 0 of the next chunk sees all
    assert b.mimi_held(250) == 249 and b.mimi_held(6) == 5
    # one stream, a 250-row chunk: q and out (2 x 250 x 8 x 64 x 2 = 512000), the chunk's k and v
    # (512000), K and V of the 249 held rows (2 x 249 x 8 x 64 x 2 = 509952)
    assert b.mimi_bytes(1, 250, 249) == 512000 + 512000 + 509952
    assert b.mimi_bytes(3, 250, 249) == 3 * b.mimi_bytes(1, 250, 249)
    # two kv heads under 8 query heads: q and out per query head, the rest per kv head
    assert b.mimi_bytes(1, 4, 5, kvh=2) == 2 * 4 * 8 * 64 * 2 + 2 * 4 * 2 * 64 * 2 + 2 * 5 * 2 * 64 * 2


def test_mimi_cpu_baseline_runs_chunks_of_the_oracle_window():
    b = _bench()
    cpu = b.cpu_mimi(16, 0.01, sample=1)
    assert cpu["unit"] == "positions/s" and cpu["value"] > 0 and cpu["kind"] == "port"


def test_traffic_comes_from_the_profiled_workload_only():
    b = _bench()
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        entry = json.load(f)["decode"]
    ratio, match = entry["traffic_per_algorithmic_byte"], entry["workload"]
    assert 1.0 <= ratio < 1.1  # the kernel reads each byte about once
    assert b.traffic_of("decode", match, 10 ** 9) == round(ratio * 10 ** 9)
    assert b.traffic_of("decode", dict(match, streams=512), 10 ** 9) is None
    assert b.traffic_of("no such workload", match, 10 ** 9) is None


def test_only_the_default_headline_carries_the_nested_configurations():
    b = _bench()
    base = dict(streams=1024, layers=9, max_len=1024, fixed_len=0, split=0, kv_heads=0)
    assert b.headline_args(argparse.Namespace(**base))
    for key, value in (("streams", 512), ("max_len", 2048), ("split", 2), ("kv_heads", 1)):
        assert not b.headline_args(argparse.Namespace(**dict(base, **{key: value})))
    assert sorted({cfg for _, cfg, _ in b.NESTED if cfg is not None}) == [1, 3, 4, 5]
    assert {name for name, _, _ in b.NESTED} == {"flowlm", "prefill", "window", "step", "frame", "mimi"}


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert msg["n_gpus"] == 2 and "one GPU" in msg["error"]
