"""GPU parity: the HIP path (through the C ABI) against the oracle on the same seeded inputs.

Bars (stated per test): cache contents -- every stored row, and int8 codes and scales -- equal the
oracle's bit for bit; attention outputs are within 1e-5 relative (f32) or 2e-2 relative (bf16,
int8 KV) of the oracle's f32 outputs, where relative error is max|got - want| / max|want| over
each (row, head) vector.
"""
import os
import types

import numpy as np
import pytest
import torch

from conftest import oracle, xnp
from helpers import bf16_round, exact_attend, rel_err

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-5, "bf16": 2e-2, "i8": 2e-2}
TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16}
CACHE_TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "i8": torch.int8}
DEV = "cuda:0"


def dev(a, act):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(TORCH_DT[act])


def host(t):
    return t.float().cpu().numpy()


class Pair:
    """A GPU pool and one oracle stream per GPU stream, driven in lockstep."""

    def __init__(self, *, L=2, H=8, KVH=None, cache="bf16", act="bf16", streams=8, cap=256,
                 split=0, seed=0, page_seed=0, max_pos=8192):
        self.L, self.H, self.KVH = L, H, KVH or H
        self.cache, self.act = cache, act
        self.rng = np.random.default_rng(seed)
        mbps = (cap + 15) // 16
        self.pool = xnp.KvPool(num_layers=L, num_heads=H, num_kv_heads=self.KVH, num_blocks=streams * mbps * 2 + 8,
                               max_streams=streams * 2 + 2, max_blocks_per_stream=mbps, cache_dtype=cache,
                               act_dtype=act, max_pos=max_pos, page_seed=page_seed, decode_split=split)
        self.ids, self.orc = [], []
        for _ in range(streams):
            self.add(cap)

    def add(self, cap):
        self.ids.append(self.pool.init_state(cap))
        self.orc.append(oracle.Stream(self.L, self.H, 64, cap, cache=self.cache, act=self.act, kv_heads=self.KVH))

    def x(self, *shape):
        a = self.rng.standard_normal(shape).astype(np.float32)
        return bf16_round(a) if self.act == "bf16" else a

    def fill(self, i, n):
        """Append n rows to stream i through the multi-row append kernel (no attention)."""
        if n == 0:
            return
        self.pool.begin([self.ids[i]], t=n)
        for layer in range(self.L):
            k, v = self.x(n, self.KVH, 64), self.x(n, self.KVH, 64)
            self.pool.append(layer, dev(k, self.act), dev(v, self.act))
            self.orc[i].append(layer, k, v)
        self.pool.end()
        self.orc[i].commit(n)

    def prefill(self, t, which=None, qscale=1.0):
        """A prompt step: t rows on every stream in `which`, through xnp_attend (append + causal);
        qscale (a power of two) scales the queries."""
        which = list(range(len(self.ids))) if which is None else which
        n = len(which)
        self.pool.begin([self.ids[i] for i in which], t=t)
        worst = 0.0
        for layer in range(self.L):
            q, k, v = self.x(n, t, self.H, 64) * qscale, self.x(n, t, self.KVH, 64), self.x(n, t, self.KVH, 64)
            out = torch.empty((n, t, self.H, 64), dtype=TORCH_DT[self.act], device=DEV)
            self.pool.attend(layer, dev(q, self.act), dev(k, self.act), dev(v, self.act), out, 0.125)
            torch.cuda.synchronize()
            got = host(out)
            for j, i in enumerate(which):
                want, _ = self.orc[i].attend(layer, q[j], k[j], v[j])
                err = rel_err(got[j], want)
                worst = max(worst, err)
                assert err <= TOL[self.cache], (layer, i, err)
        self.pool.end()
        for i in which:
            self.orc[i].commit(t)
        return worst

    def prefill_split(self, t, which=None):
        """A prompt step through xnp_append then xnp_prefill (two calls, keys read back from the pages)."""
        which = list(range(len(self.ids))) if which is None else which
        n = len(which)
        self.pool.begin([self.ids[i] for i in which], t=t)
        worst = 0.0
        for layer in range(self.L):
            q, k, v = self.x(n, t, self.H, 64), self.x(n, t, self.KVH, 64), self.x(n, t, self.KVH, 64)
            out = torch.empty((n, t, self.H, 64), dtype=TORCH_DT[self.act], device=DEV)
            self.pool.append(layer, dev(k, self.act), dev(v, self.act))
            self.pool.prefill(layer, dev(q, self.act), out, 0.125)
            torch.cuda.synchronize()
            got = host(out)
            for j, i in enumerate(which):
                want, _ = self.orc[i].attend(layer, q[j], k[j], v[j])
                err = rel_err(got[j], want)
                worst = max(worst, err)
                assert err <= TOL[self.cache], (layer, i, err)
        self.pool.end()
        for i in which:
            self.orc[i].commit(t)
        return worst

    def step(self, which=None, fused=True, check=True, qscale=1.0):
        which = list(range(len(self.ids))) if which is None else which
        n = len(which)
        self.pool.begin([self.ids[i] for i in which])
        errs = []
        for layer in range(self.L):
            q, k, v = self.x(n, self.H, 64) * qscale, self.x(n, self.KVH, 64), self.x(n, self.KVH, 64)
            out = torch.empty((n, self.H, 64), dtype=TORCH_DT[self.act], device=DEV)
            if fused:
                self.pool.attend(layer, dev(q, self.act), dev(k, self.act), dev(v, self.act), out, 0.125)
            else:
                self.pool.append(layer, dev(k, self.act), dev(v, self.act))
                self.pool.decode(layer, dev(q, self.act), out, 0.125)
            torch.cuda.synchronize()
            got = host(out)
            for j, i in enumerate(which):
                want, want64 = self.orc[i].attend(layer, q[j:j + 1], k[j:j + 1], v[j:j + 1])
                errs.append(rel_err(got[j:j + 1], want))
                if check:
                    assert rel_err(got[j:j + 1], want) <= TOL[self.cache], (layer, i)
        self.pool.end()
        for i in which:
            self.orc[i].commit(1)
        return max(errs) if errs else 0.0

    def assert_cache_equal(self, i, upto=None):
        sid, st = self.ids[i], self.orc[i]
        n = st.current_end if upto is None else upto
        if st.ring_info()["mode"]:
            n = st.ring_info()["filled"]
        if n == 0:
            return
        valid = st.ring_info()["valid"] if st.ring_info()["mode"] else np.ones(st.capacity, bool)
        G = self.H // self.KVH  # the pool stores kv head j once; the oracle repeats it at heads j*G ..
        for layer in range(self.L):
            for kv in (0, 1):
                rows = torch.empty((n, self.KVH, 64), dtype=CACHE_TORCH[self.cache], device=DEV)
                nb = (n - 1) // 16 + 1
                scales = torch.zeros((nb, self.KVH), dtype=torch.float32, device=DEV)
                self.pool.read_rows(sid, layer, kv, 0, rows, scales if self.cache == "i8" else None)
                torch.cuda.synchronize()
                vals, q8, osc = st.read_rows(layer, kv, 0, n)
                vals, q8, osc = vals[:, ::G], q8[:, ::G], osc[:, ::G]
                m = valid[:n]
                if self.cache == "i8":
                    g = rows.cpu().numpy()
                    assert np.array_equal(g[m], q8[m]), (i, layer, kv)
                    gs = scales.cpu().numpy()
                    live = np.array([m[16 * b:16 * b + 16].any() for b in range(nb)])
                    assert np.array_equal(gs[live].view(np.uint32), osc[live].view(np.uint32)), (i, layer, kv)
                else:
                    g = rows.float().cpu().numpy()
                    assert np.array_equal(g[m].view(np.uint32), vals[m].view(np.uint32)), (i, layer, kv)


# ---- linear caches -----------------------------------------------------------------------------
# split 0 lets the library choose: 8 waves per (stream, head) for batches as small as these
@pytest.mark.parametrize("split", [0, 2])
@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("f32", "f32"), ("i8", "bf16"), ("i8", "f32")])
def test_append_and_decode_match_the_oracle(cache, act, split):
    p = Pair(cache=cache, act=act, streams=8, cap=300, seed=1, page_seed=7, split=split)
    lens = [0, 1, 15, 16, 17, 100, 200, 255]
    for i, n in enumerate(lens):
        p.fill(i, n)
    for i in range(8):
        p.assert_cache_equal(i)
    for _ in range(3):
        p.step()
    for i in range(8):
        p.assert_cache_equal(i)


def test_one_row_returns_its_value_exactly():
    p = Pair(cache="bf16", act="bf16", streams=2, cap=32, seed=2)
    p.pool.begin(p.ids)
    q, k, v = p.x(2, 8, 64), p.x(2, 8, 64), p.x(2, 8, 64)
    out = torch.empty((2, 8, 64), dtype=torch.bfloat16, device=DEV)
    p.pool.attend(0, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, 0.125)
    torch.cuda.synchronize()
    p.pool.abort()
    assert np.array_equal(host(out), v)


def test_split_chunks_and_separate_calls_agree():
    outs = []
    for split, fused in [(2, True), (4, True), (8, True), (4, False)]:
        p = Pair(cache="bf16", act="bf16", streams=4, cap=600, seed=3, split=split)
        for i, n in enumerate([1, 37, 300, 590]):
            p.fill(i, n)
        p.pool.begin(p.ids)
        q, k, v = p.x(4, 8, 64), p.x(4, 8, 64), p.x(4, 8, 64)
        out = torch.empty((4, 8, 64), dtype=torch.bfloat16, device=DEV)
        if fused:
            p.pool.attend(0, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, 0.125)
        else:
            p.pool.append(0, dev(k, "bf16"), dev(v, "bf16"))
            p.pool.decode(0, dev(q, "bf16"), out, 0.125)
        torch.cuda.synchronize()
        p.pool.end()
        outs.append(host(out))
        want = np.concatenate([p.orc[i].attend(0, q[i:i + 1], k[i:i + 1], v[i:i + 1])[0] for i in range(4)])
        assert rel_err(outs[-1], want) <= 2e-2
    assert np.array_equal(outs[1], outs[3])  # the fused append changes nothing but the launch


# ---- grouped heads, stored once per kv head (transformer.rs:199-211) ----------------------------
@pytest.mark.parametrize("kvh", [4, 2, 1])
@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("f32", "f32"), ("i8", "bf16")])
def test_grouped_kv_heads(cache, act, kvh):
    # 8 query heads over 4, 2 or 1 stored kv heads: appends of t rows, prompts, then decode steps
    # (an int8 pool appends in a kernel of its own before each decode)
    p = Pair(cache=cache, act=act, H=8, KVH=kvh, streams=5, cap=160, seed=4 + kvh)
    for i, n in enumerate([0, 3, 40, 64, 100]):
        p.fill(i, n)
    p.prefill(9, which=[0, 2])
    for _ in range(3):
        p.step()
    for i in range(5):
        p.assert_cache_equal(i)


@pytest.mark.parametrize("h,kvh", [(6, 2), (12, 2), (12, 3), (8, 8), (8, 2)])
@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("f32", "f32"), ("i8", "bf16")])
def test_grouped_heads_of_other_ratios(cache, act, h, kvh):
    # 3, 6, 4, 1 and 4 query heads per kv head: a decode work group then takes one, two or four of
    # them (or, bf16 and int8, the whole kv head on MFMA).  13 streams: the grid's XCD runs of 8
    # streams, one whole run and a tail of 5.
    lens = [0, 5, 16, 17, 40, 63, 90, 1, 33, 48, 2, 79, 15]
    p = Pair(cache=cache, act=act, H=h, KVH=kvh, streams=len(lens), cap=96, seed=40 + h + kvh)
    for i, n in enumerate(lens):
        p.fill(i, n)
    for _ in range(3):
        p.step()
    for i in range(len(lens)):
        p.assert_cache_equal(i)


def test_grouped_heads_store_a_kv_head_once():
    # the pages hold KVH heads: a pool of 2 kv heads takes a quarter of one of 8
    def pages_bytes(kvh):
        pool = xnp.KvPool(num_layers=2, num_heads=8, num_kv_heads=kvh, num_blocks=64, max_streams=4,
                          max_blocks_per_stream=8, cache_dtype="bf16", act_dtype="bf16", max_pos=256)
        return pool.stats()["device_bytes"]
    page = 2 * 2 * 64 * 16 * 64 * 2  # layers x (K, V) x blocks x 16 rows x 64 dims x 2 bytes, per kv head
    assert pages_bytes(8) - pages_bytes(2) == 6 * page


@pytest.mark.parametrize("cache,act,mode", [("bf16", "bf16", "shift"), ("i8", "bf16", "absolute"),
                                            ("bf16", "bf16", "absolute"), ("f32", "f32", "absolute")])
def test_grouped_heads_on_rings(cache, act, mode):
    # 4 query heads per kv head; an absolute ring's prefix gives the batch a second query position,
    # with which bf16 and f32 decode take two heads per work group instead of four
    p = Pair(cache=cache, act=act, H=8, KVH=2, streams=2, cap=48, seed=31)
    context = 20
    for i in range(2):
        p.fill(i, 4)
        p.pool.start_ring(p.ids[i], mode, prefix=4)
        p.orc[i].start_ring(mode, prefix=4)
    for steps in range(50):
        for i in range(2):  # a 4-row prefix, then frames sliding over 20 slots, the oldest evicted
            slot = 4 + steps % context
            if p.orc[i].ring_info()["valid"][slot]:
                p.orc[i].evict(4, [slot])
                p.pool.evict(p.ids[i], 4, [slot])
            p.orc[i].set_ring_slot(slot)
            p.pool.set_ring_slot(p.ids[i], slot)
        p.step()
    for i in range(2):
        p.assert_cache_equal(i)


@pytest.mark.parametrize("cache", ["bf16", "i8"])
@pytest.mark.parametrize("h", [8, 16])
def test_grouped_heads_on_prefix_rings_take_the_mfma_decode(cache, h):
    # 8 and 16 query heads over one kv head (the MFMA decode of a whole kv head) on absolute rings
    # with voice prefixes of 0, 5 and 20 rows (20: the prefix ends inside the second page), so that
    # the batch keeps a second query position: keys before a stream's prefix are scored against its
    # query at pos_pre (transformer.rs:879-929 restated as the absolute ring), the others at pos.
    # int8 pages score both positions in f16, each query with its own power of two and sum.
    # Frames slide over a context of 40 slots with the oldest evicted, 60 steps, every output held to
    # the oracle and every cache row (int8: codes and scales) bit-exact.
    p = Pair(cache=cache, act="bf16", H=h, KVH=1, streams=3, cap=96, seed=70 + h)
    prefixes, context = [0, 5, 20], 40
    for i, pre in enumerate(prefixes):
        p.fill(i, pre)
        p.pool.start_ring(p.ids[i], "absolute", prefix=pre)
        p.orc[i].start_ring("absolute", prefix=pre)
    worst = 0.0
    for steps in range(60):
        for i, pre in enumerate(prefixes):
            slot = pre + steps % context
            if p.orc[i].ring_info()["valid"][slot]:
                p.orc[i].evict(pre, [slot])
                p.pool.evict(p.ids[i], pre, [slot])
            p.orc[i].set_ring_slot(slot)
            p.pool.set_ring_slot(p.ids[i], slot)
        worst = max(worst, p.step())
    for i in range(3):
        p.assert_cache_equal(i)
    assert worst <= TOL[cache]


def test_empty_batch_is_a_no_op():
    p = Pair(streams=1, cap=16)
    p.pool.begin([])
    out = torch.empty((0, 8, 64), dtype=torch.bfloat16, device=DEV)
    p.pool.attend(0, out, out, out, out, 0.125)
    p.pool.end()
    assert p.pool.current_end(p.ids[0]) == 0


# ---- Mimi's window cache (transformer.rs:257-318, 428-468, 764-781) ------------------------------
def _window_batch(pool, ids, orcs, t, L, H, act, cache, rng, twins=()):
    """One step of t rows on `ids`, every layer checked against the oracle caches `orcs` (None:
    not checked).  twins: (i, j) pairs whose stream j gets stream i's inputs and must answer alike."""
    n = len(ids)
    pool.begin(ids, t=t)
    for layer in range(L):
        q, k, v = (rng.standard_normal((n, t, H, 64)).astype(np.float32) for _ in range(3))
        if act == "bf16":
            q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
        for i, j in twins:
            q[j], k[j], v[j] = q[i], k[i], v[i]
        out = torch.empty((n, t, H, 64), dtype=TORCH_DT[act], device=DEV)
        pool.attend(layer, dev(q, act), dev(k, act), dev(v, act), out, 0.125)
        torch.cuda.synchronize()
        got = host(out)
        for j, o in enumerate(orcs):
            if o is not None:
                want, _ = o.attend(layer, q[j], k[j], v[j])
                assert rel_err(got[j], want) <= TOL[cache], (layer, j, t)
        for i, j in twins:
            assert np.array_equal(got[i], got[j]), (layer, i, j)
    pool.end()
    for o in orcs:
        if o is not None:
            o.commit(t)


def _assert_window_rows(pool, sid, win, window, L, H, cache):
    # the oracle keeps positions [offset - len, offset); the pool holds position p in slot p % window
    filled = min(win.offset, window)
    for layer in range(L):
        for kv in (0, 1):
            rows = torch.empty((filled, H, 64), dtype=CACHE_TORCH[cache], device=DEV)
            pool.read_rows(sid, layer, kv, 0, rows)
            torch.cuda.synchronize()
            g = rows.float().cpu().numpy()
            want = win.rows(layer, kv)
            for i, p in enumerate(range(win.offset - win.len, win.offset)):
                assert np.array_equal(g[p % window].view(np.uint32), want[i].view(np.uint32)), (layer, kv, p)


@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("f32", "f32")])
def test_window_caches_match_mimis_kv_cache(cache, act):
    # Three windows (KvCache::new(24), (24), (40)) and a plain stream in the same batches for 60
    # single rows; then 15 steps of two rows (Mimi's decoder: two 25 Hz rows per 80 ms frame) on the
    # windows and a clone of the first (with_seq_budget clones a window as it is), fed its inputs.
    L, H = 2, 8
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=64, max_streams=8, max_blocks_per_stream=8,
                      cache_dtype=cache, act_dtype=act, max_pos=4096, page_seed=3)
    contexts = [24, 24, 40]
    ids = [pool.init_window(c) for c in contexts]
    orcs = [oracle.Window(L, H, 64, c, act=act) for c in contexts]
    ids.append(pool.init_state(128))
    orcs.append(oracle.Stream(L, H, 64, 128, cache=cache, act=act))
    assert pool.info(ids[0])["window"] == 24 and pool.info(ids[3])["window"] == 0
    rng = np.random.default_rng(50)
    for s_ in range(60):
        _window_batch(pool, ids, orcs, 1, L, H, act, cache, rng)
        if s_ in (10, 23, 24, 59):
            for i in range(3):
                _assert_window_rows(pool, ids[i], orcs[i], contexts[i], L, H, cache)
    clone = pool.with_seq_budget(ids[0], 999)
    assert pool.info(clone)["window"] == 24
    wids = ids[:3] + [clone]
    for _ in range(15):
        _window_batch(pool, wids, orcs[:3] + [None], 2, L, H, act, cache, rng, twins=[(0, 3)])
    for i in range(3):
        _assert_window_rows(pool, wids[i], orcs[i], contexts[i], L, H, cache)
        assert pool.current_end(wids[i]) == contexts[i]  # rows held: the window, full


def test_int8_rows_holding_infinities_quantize_as_the_oracle():
    # An int8 page's scale is its rows' amax / 127, taken with IEEE maxima: a row holding an
    # infinity gives the page an infinite scale, its infinite elements code -127 (rint(inf / inf) is
    # NaN, clamped) and every other code of the page 0, the oracle's arithmetic step for step.
    # Planted through the multi-row append (prompt rows) and the fused single-row append of a
    # decode step; the outputs are NaN by then and not compared, the cache bytes are, bit for bit.
    p = Pair(cache="i8", act="bf16", streams=2, cap=64, seed=61, L=1)
    p.fill(0, 20)
    p.fill(1, 7)
    n = 5
    p.pool.begin([p.ids[0]], t=n)
    k, v = p.x(n, p.KVH, 64), p.x(n, p.KVH, 64)
    k[2, 3, 10] = np.inf
    v[4, 5, 0] = -np.inf
    p.pool.append(0, dev(k, "bf16"), dev(v, "bf16"))
    p.orc[0].append(0, k, v)
    p.pool.end()
    p.orc[0].commit(n)
    p.pool.begin(p.ids)
    q, k, v = p.x(2, p.H, 64), p.x(2, p.KVH, 64), p.x(2, p.KVH, 64)
    k[1, 0, 7] = -np.inf
    v[1, 2, 63] = np.inf
    out = torch.empty((2, p.H, 64), dtype=torch.bfloat16, device=DEV)
    p.pool.attend(0, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, 0.125)
    torch.cuda.synchronize()
    for j in range(2):
        p.orc[j].attend(0, q[j:j + 1], k[j:j + 1], v[j:j + 1])
    p.pool.end()
    for j in range(2):
        p.orc[j].commit(1)
        p.assert_cache_equal(j)


def test_int8_window_cache_matches_the_ring_it_stands_for():
    # An int8 window has no counterpart in the reference; it is an absolute ring of `context`
    # slots whose every row evicts the oldest, so the oracle's ring driven that way is its bar:
    # bit-exact codes and scales, outputs within 2e-2.  Two windows of one batch with different
    # histories (the second joins 17 rows later, so the held rows and the oldest slot differ
    # within each launch): single rows, rows in pairs, steps of 5 rows and steps of 30 rows (more
    # than the window holds: the later rows of a step overwrite the earlier ones, in the same
    # pages, whose scales then requantize).
    L, H, context = 2, 8, 24
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=16, max_streams=2, max_blocks_per_stream=2,
                      cache_dtype="i8", act_dtype="bf16", max_pos=4096, page_seed=4)
    wins = [pool.init_window(context) for _ in range(2)]
    sts = [oracle.Stream(L, H, 64, context, cache="i8", act="bf16") for _ in range(2)]
    for st in sts:
        st.start_ring("absolute", prefix=0)
    rng = np.random.default_rng(51)
    pos = [0, 0]

    def check(j):
        n = min(pos[j], context)
        for layer in range(L):
            for kv in (0, 1):
                rows = torch.empty((n, H, 64), dtype=torch.int8, device=DEV)
                nb = (n - 1) // 16 + 1
                sc = torch.zeros((nb, H), dtype=torch.float32, device=DEV)
                pool.read_rows(wins[j], layer, kv, 0, rows, sc)
                torch.cuda.synchronize()
                _, q8, osc = sts[j].read_rows(layer, kv, 0, n)
                assert np.array_equal(rows.cpu().numpy(), q8), (j, pos[j], layer, kv)
                assert np.array_equal(sc.cpu().numpy().view(np.uint32), osc.view(np.uint32)), (j, pos[j], layer, kv)

    steps = [((0,), 1)] * 17 + [((0, 1), 1)] * 40 + [((0, 1), 2)] * 12 + [((0, 1), 5)] * 6 + [((0, 1), 30)] * 3 \
        + [((1,), 5)] + [((0, 1), 1)] * 5
    for which, t in steps:
        q, k, v = (bf16_round(rng.standard_normal((L, len(which), t, H, 64)).astype(np.float32) * 2) for _ in range(3))
        pool.begin([wins[j] for j in which], t=t)
        got = []
        for layer in range(L):
            out = torch.empty((len(which), t, H, 64), dtype=torch.bfloat16, device=DEV)
            pool.attend(layer, dev(q[layer], "bf16"), dev(k[layer], "bf16"), dev(v[layer], "bf16"), out, 0.125)
            torch.cuda.synchronize()
            got.append(host(out))
        pool.end()
        for b, j in enumerate(which):
            st = sts[j]
            for i in range(t):  # the oracle's ring, one row at a time over every layer
                if st.ring_info()["filled"] == context:
                    st.evict(0, [pos[j] % context])
                st.set_ring_slot(pos[j] % context)
                for layer in range(L):
                    want, _ = st.attend(layer, q[layer][b, i:i + 1], k[layer][b, i:i + 1], v[layer][b, i:i + 1])
                    assert rel_err(got[layer][b, i:i + 1], want) <= TOL["i8"], (j, pos[j], layer)
                st.commit(1)
                pos[j] += 1
            if pos[j] % 7 == 0 or t > 1:
                check(j)
    assert pos == [17 + 40 + 24 + 30 + 90 + 5, 40 + 24 + 30 + 90 + 5 + 5]
    for j in range(2):
        check(j)


@pytest.mark.parametrize("cache,act,kvh", [("bf16", "bf16", 8), ("bf16", "bf16", 2), ("f32", "f32", 8)])
def test_a_long_mimi_chunk_matches_the_kv_cache(cache, act, kvh):
    # Mimi's encoder pushes a whole voice clip through its transformer in one call
    # (tts_model.rs:509-515, mimi.rs:162-167): a chunk longer than the window (context 250) attends
    # under the window mask of transformer.rs:764-781, then KvCache::trim keeps the last rows
    # (transformer.rs:302-317).  Here: a 300-row chunk, 40 single rows, 10 steps of 2 rows and a
    # 100-row chunk over the held rows, on two windows of the same batch, each against the oracle's
    # KvCache: outputs within the dtype's bar every step, every held row bit for bit at the end.
    # bf16 chunks of more than 4 rows take the windowed MFMA prefill and its append; f32 runs row
    # by row.  With grouped heads the pool stores each kv head once; the oracle gets it repeated.
    L, H, context = 2, 8, 250
    G = H // kvh
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_kv_heads=kvh, num_blocks=48, max_streams=4,
                      max_blocks_per_stream=16, cache_dtype=cache, act_dtype=act, max_pos=1024, page_seed=6)
    ids = [pool.init_window(context) for _ in range(2)]
    orcs = [oracle.Window(L, H, 64, context, rows_max=300, act=act) for _ in range(2)]
    rng = np.random.default_rng(53 + kvh)

    def step(t, which=(0, 1)):
        n = len(which)
        pool.begin([ids[j] for j in which], t=t)
        for layer in range(L):
            q = rng.standard_normal((n, t, H, 64)).astype(np.float32)
            k = rng.standard_normal((n, t, kvh, 64)).astype(np.float32)
            v = rng.standard_normal((n, t, kvh, 64)).astype(np.float32)
            if act == "bf16":
                q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
            out = torch.empty((n, t, H, 64), dtype=TORCH_DT[act], device=DEV)
            pool.attend(layer, dev(q, act), dev(k, act), dev(v, act), out, 0.125)
            torch.cuda.synchronize()
            got = host(out)
            for b, j in enumerate(which):
                want, _ = orcs[j].attend(layer, q[b], np.repeat(k[b], G, axis=1), np.repeat(v[b], G, axis=1))
                assert rel_err(got[b], want) <= TOL[cache], (t, layer, j)
        pool.end()
        for j in which:
            orcs[j].commit(t)

    # window 0 takes a 37-row chunk of its own first: every later launch holds two windows with
    # different held rows and different oldest slots
    step(37, which=(0,))
    for t in [300] + [1] * 40 + [2] * 10 + [100]:
        step(t)
    for j in range(2):
        assert orcs[j].offset == 460 + (37 if j == 0 else 0) and pool.current_end(ids[j]) == context
        win = orcs[j]
        for layer in range(L):
            for kv in (0, 1):
                rows = torch.empty((context, kvh, 64), dtype=CACHE_TORCH[cache], device=DEV)
                pool.read_rows(ids[j], layer, kv, 0, rows)
                torch.cuda.synchronize()
                g = rows.float().cpu().numpy()
                want = win.rows(layer, kv)[:, ::G]
                for i, p in enumerate(range(win.offset - win.len, win.offset)):
                    assert np.array_equal(g[p % context].view(np.uint32), want[i].view(np.uint32)), (j, layer, kv, p)


def test_the_mimi_configuration_at_full_size_spot_checked():
    # The bench's Mimi workload at its size: 256 windows of context 250, 2 layers x 8 heads x 64,
    # bf16; a first 250-row chunk into empty windows, then a second over the 249 held rows (the
    # shape the bench times).  Every window's layer 0 is held to the oracle's KvCache (a one-layer
    # window per stream, run on the host's threads); both layers of a sample of windows, and the
    # sample's held rows bit for bit at the end.
    from concurrent.futures import ThreadPoolExecutor
    S, L, H, context, T = 256, 2, 8, 250, 250
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * 16 + 8, max_streams=S, max_blocks_per_stream=16,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=1024, page_seed=18)
    ids = [pool.init_window(context) for _ in range(S)]
    sample = [0, 1, 130, 255]
    full = {i: oracle.Window(L, H, 64, context, rows_max=T, act="bf16") for i in sample}
    every = [oracle.Window(1, H, 64, context, rows_max=T, act="bf16") for _ in range(S)]
    rng = np.random.default_rng(71)
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        for chunk in range(2):
            pool.begin(ids, t=T)
            for layer in range(L):
                q, k, v = (bf16_round(rng.standard_normal((S, T, H, 64)).astype(np.float32)) for _ in range(3))
                out = torch.empty((S, T, H, 64), dtype=torch.bfloat16, device=DEV)
                pool.attend(layer, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, 0.125)
                torch.cuda.synchronize()
                got = host(out)
                if layer == 0:
                    wants = list(ex.map(lambda j: every[j].attend(0, q[j], k[j], v[j])[0], range(S)))
                    worst = max(rel_err(got[j], wants[j]) for j in range(S))
                    assert worst <= TOL["bf16"], (chunk, worst)
                for i in sample:
                    want, _ = full[i].attend(layer, q[i], k[i], v[i])
                    assert rel_err(got[i], want) <= TOL["bf16"], (chunk, layer, i)
            pool.end()
            for w in every:
                w.commit(T)
            for i in sample:
                full[i].commit(T)
    for i in sample:
        win = full[i]
        assert pool.current_end(ids[i]) == context
        for layer in range(L):
            for kv in (0, 1):
                rows = torch.empty((context, H, 64), dtype=torch.bfloat16, device=DEV)
                pool.read_rows(ids[i], layer, kv, 0, rows)
                torch.cuda.synchronize()
                g = rows.float().cpu().numpy()
                want = win.rows(layer, kv)
                for r, pos in enumerate(range(win.offset - win.len, win.offset)):
                    assert np.array_equal(g[pos % context].view(np.uint32), want[r].view(np.uint32)), (i, layer, kv, pos)


def test_window_misuse_is_refused():
    pool = xnp.KvPool(num_layers=1, num_heads=8, num_blocks=16, max_streams=4, max_blocks_per_stream=4,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=1024)
    wid, pid = pool.init_window(16), pool.init_state(64)
    with pytest.raises(xnp.XnpError, match="window of 0"):
        pool.init_window(0)
    with pytest.raises(xnp.XnpError, match="window caches only"):
        pool.begin([wid, pid], t=2)
    with pytest.raises(xnp.XnpError, match="places its rows itself"):
        pool.set_ring_slot(wid, 3)
    with pytest.raises(xnp.XnpError, match="places its rows itself"):
        pool.evict(wid, 0, [0])
    with pytest.raises(xnp.XnpError, match="not a ring"):
        pool.load_kv(wid, 0, torch.zeros((2, 0, 8, 64), dtype=torch.float32, device=DEV))
    pool.begin([wid], t=2)
    x = torch.zeros((1, 2, 8, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(xnp.XnpError, match="through xnp_attend alone"):
        pool.decode(0, x, x, 0.125)
    with pytest.raises(xnp.XnpError, match="through xnp_attend alone"):
        pool.append(0, x, x)
    pool.abort()
    assert pool.current_end(wid) == 0


# ---- voices stored as the KV cache (ptts-wasm/src/lib.rs:291-325) -------------------------------
@pytest.mark.parametrize("cache,act", [("f32", "f32"), ("bf16", "bf16"), ("i8", "bf16")])
def test_a_voice_file_loads_into_pages_and_its_forks_share_them(cache, act, tmp_path):
    # An `embeddings_v2/` voice: per layer an f32 [2, 1, 37, H, D] cache (keys already rotated).
    # Loaded once, then forked per generation (with_seq_budget): the forks share the two full
    # pages, copy the 5-row tail page, and decode 20 frames each against the oracle.
    from safetensors.numpy import save_file
    p = Pair(cache=cache, act=act, streams=2, cap=128, seed=21)  # room for the voice and 3 forks
    rng = np.random.default_rng(22)
    n = 37
    tensors = {xnp.voice_kv_name(l): (rng.standard_normal((2, 1, n, 8, 64)) * 2).astype(np.float32)
               for l in range(p.L)}
    path = tmp_path / "voice.safetensors"
    save_file(tensors, str(path))
    vid = p.pool.load_voice(str(path))
    o = oracle.Stream(p.L, p.H, 64, n, cache=cache, act=act)
    o.advance(n)
    for l in range(p.L):
        o.load_kv(l, tensors[xnp.voice_kv_name(l)][:, 0])
    p.ids.append(vid)
    p.orc.append(o)
    assert p.pool.current_end(vid) == n
    p.assert_cache_equal(2)
    free0 = p.pool.stats()["free_blocks"]
    for _ in range(3):
        p.ids.append(p.pool.with_seq_budget(vid, 128))
        p.orc.append(o.with_seq_budget(128))
    assert free0 - p.pool.stats()["free_blocks"] == 3  # one copied tail page per fork
    for _ in range(20):  # past the tail page: the forks take pages of their own
        p.step(which=[3, 4, 5])
    for i in range(2, 6):
        p.assert_cache_equal(i)
    # refusals: a stream of another length, and a ring
    with pytest.raises(xnp.XnpError, match="exactly as many rows"):
        p.pool.load_kv(p.ids[3], 0, torch.zeros((2, n, 8, 64), dtype=torch.float32, device=DEV))
    with pytest.raises(ValueError, match="first dim of size 2"):
        p.pool.load_voice({k: v[:1] for k, v in tensors.items()})


# ---- with_seq_budget: shared pages ----------------------------------------------------------------
def test_fork_shares_the_prefix_and_diverges():
    p = Pair(cache="bf16", act="bf16", streams=1, cap=128, seed=5)
    p.fill(0, 40)
    fid = p.pool.with_seq_budget(p.ids[0], 128)
    p.ids.append(fid)
    p.orc.append(p.orc[0].with_seq_budget(128))
    for _ in range(3):
        p.step()  # both append; the source's partial page must be left alone by the fork
    p.assert_cache_equal(0)
    p.assert_cache_equal(1)


# ---- rings (transformer.rs:842-929) ----------------------------------------------------------------
@pytest.mark.parametrize("cache,act,mode", [("f32", "f32", "shift"), ("bf16", "bf16", "shift"),
                                            ("bf16", "bf16", "absolute"), ("i8", "bf16", "absolute")])
@pytest.mark.parametrize("split", [0, 2])
def test_ring_sessions_match_the_oracle(cache, act, mode, split):
    # The s2s policy on several streams at once: a voice prefix, then frames in a context of 24
    # slots whose oldest third goes whenever it is full (s2s.rs:318-333).
    p = Pair(cache=cache, act=act, streams=3, cap=64, seed=6, split=split)
    v, context = [5, 16, 0], 24
    for i in range(3):
        p.fill(i, v[i])
        p.pool.start_ring(p.ids[i], mode, prefix=v[i])
        p.orc[i].start_ring(mode, prefix=v[i])
    in_view = [0, 0, 0]
    for steps in range(70):
        for i in range(3):
            if in_view[i] == context:
                oldest = steps - in_view[i]
                slots = [v[i] + (oldest + j) % context for j in range(context // 3)]
                p.orc[i].evict(v[i], slots)
                in_view[i] -= context // 3
            p.orc[i].set_ring_slot(v[i] + steps % context)
            p.pool.slide(p.ids[i], v[i], context, context, context // 3, steps)
            assert p.pool.info(p.ids[i])["ring_write"] == p.orc[i].ring_info()["write"]
        p.step()
        for i in range(3):
            in_view[i] += 1
        if steps % 23 == 0 or steps == 69:
            for i in range(3):
                p.assert_cache_equal(i)


@pytest.mark.parametrize("kvh", [8, 2])
@pytest.mark.parametrize("qscale", [2.0 ** 17, 2.0 ** -20])
def test_int8_pools_take_queries_beyond_the_f16_range(kvh, qscale):
    # int8 pages with bf16 activations take the query as f16, scaled by a power of two that fits
    # it: queries of N(0, 1) x 2^17 (components past f16's 65504) and x 2^-20 (below its normal
    # range) on the VALU decode (8 kv heads) and the MFMA one (2 kv heads, 4 query heads each),
    # after a 9-row prompt through the MFMA prefill (f16 scores, each query row's own power of two):
    # outputs to the oracle, caches bit-exact
    p = Pair(cache="i8", act="bf16", H=8, KVH=kvh, streams=3, cap=96, seed=50)
    for i, n in enumerate([0, 20, 47]):
        p.fill(i, n)
    p.prefill(9, qscale=qscale)
    for _ in range(3):
        p.step(qscale=qscale)
    for i in range(3):
        p.assert_cache_equal(i)


@pytest.mark.parametrize("kvh", [8, 2, 1])
def test_int8_sliding_window_with_random_write_heads(kvh):
    # A window of 64 rows on a ring of 80 slots (window + one page), write heads at random
    # offsets, one eviction per step once the window is full.  8 kv heads: the VALU decode; 2 and
    # 1 (4 and 8 query heads per kv head): the MFMA decode of whole kv heads, which appends once
    # per kv head and requantizes the write page as its scales grow.
    p = Pair(cache="i8", act="bf16", H=8, KVH=kvh, streams=4, cap=80, seed=7, L=1)
    heads = [0, 5, 33, 79]
    for i in range(4):
        p.pool.start_ring(p.ids[i], "absolute", prefix=0)
        p.orc[i].start_ring("absolute", prefix=0)
    in_view = [0] * 4
    for n in range(150):
        for i in range(4):
            step = heads[i] + n
            if in_view[i] == 64:
                p.orc[i].evict(0, [(step - 64) % 80])
                in_view[i] -= 1
            p.orc[i].set_ring_slot(step % 80)
            p.pool.slide(p.ids[i], 0, 80, 64, 1, step)
        p.step()
        for i in range(4):
            in_view[i] += 1
    for i in range(4):
        p.assert_cache_equal(i)


def test_shifting_and_absolute_rings_agree_over_a_long_session():
    # The s2s policy (s2s.rs:318-333) for 1000 frames on a bf16 ring of each mode, fed the same
    # inputs: a voice prefix, a context of 96 slots, the oldest third evicted whenever it is full.
    # The shifting ring is the reference's (keys rotated back in place on every eviction,
    # transformer.rs:905-926); the absolute one keeps keys as written and rotates the query twice.
    # Each is held to its own oracle -- outputs within 2e-2, cache rows bit-exact.
    # Both stand for one mathematical object: after evictions the cache is that of the sequence
    # without the evicted rows (transformer.rs:1359-1395), so at every frame the exact output is the
    # f64 attention of the query over the kept rows at their compacted positions (exact_attend, from
    # the bf16 inputs before any rotation or rounding).  Each mode differs from it by its own
    # roundings (the shifting ring re-rounds its keys on every rotation, the absolute one rounds a
    # query rotated elsewhere, both round the stored keys and the output).  The bar: neither GPU
    # mode is further from the exact output over the session than the reference's own shifting ring
    # computed in f32 (the oracle's), plus one bf16 rounding of the output (2^-8 of its largest
    # value); and each frame's two GPU modes differ by no more than their two distances to exact.
    v, context, drop, frames = [16, 5, 0], 96, 32, 1000
    pairs = {m: Pair(cache="bf16", act="bf16", streams=3, cap=128, seed=12, L=2) for m in ("shift", "absolute")}
    rng = np.random.default_rng(13)
    seq = {}  # (stream, layer) -> the kept rows (k, v) in sequence order, prefix first
    for i in range(3):
        for layer in range(2):
            k_, v2 = (bf16_round(rng.standard_normal((v[i], 8, 64)).astype(np.float32)) for _ in range(2))
            seq[i, layer] = [k_, v2]
    for m, p in pairs.items():
        for i in range(3):
            if v[i]:
                p.pool.begin([p.ids[i]], t=v[i])
                for layer in range(2):
                    k_, v2 = seq[i, layer]
                    p.pool.append(layer, dev(k_, "bf16"), dev(v2, "bf16"))
                    p.orc[i].append(layer, k_, v2)
                p.pool.end()
                p.orc[i].commit(v[i])
            p.pool.start_ring(p.ids[i], m, prefix=v[i])
            p.orc[i].start_ring(m, prefix=v[i])
    in_view, worst_between = [0, 0, 0], 0.0
    dist = {(src, m): [] for src in ("gpu", "oracle") for m in pairs}
    for step in range(frames):
        for p in pairs.values():
            for i in range(3):
                if in_view[i] == context:
                    oldest = step - in_view[i]
                    p.orc[i].evict(v[i], [v[i] + (oldest + j) % context for j in range(drop)])
                p.orc[i].set_ring_slot(v[i] + step % context)
                p.pool.slide(p.ids[i], v[i], context, context, drop, step)
        for i in range(3):
            if in_view[i] == context:
                in_view[i] -= drop
                for layer in range(2):  # the sequence without the evicted rows: the oldest after the prefix
                    k_, v2 = seq[i, layer]
                    seq[i, layer] = [np.concatenate([k_[:v[i]], k_[v[i] + drop:]]),
                                     np.concatenate([v2[:v[i]], v2[v[i] + drop:]])]
        for p in pairs.values():
            p.pool.begin(p.ids)
        for layer in range(2):
            q, k, v_ = (bf16_round(rng.standard_normal((3, 8, 64)).astype(np.float32)) for _ in range(3))
            outs, wants = {}, {}
            for m, p in pairs.items():
                out = torch.empty((3, 8, 64), dtype=torch.bfloat16, device=DEV)
                p.pool.attend(layer, dev(q, "bf16"), dev(k, "bf16"), dev(v_, "bf16"), out, 0.125)
                torch.cuda.synchronize()
                outs[m] = host(out)
                wants[m] = np.concatenate([p.orc[i].attend(layer, q[i:i + 1], k[i:i + 1], v_[i:i + 1])[0]
                                           for i in range(3)])
                for i in range(3):
                    assert rel_err(outs[m][i:i + 1], wants[m][i:i + 1]) <= 2e-2, (m, step, layer, i)
            for i in range(3):
                k_, v2 = seq[i, layer]
                seq[i, layer] = [np.concatenate([k_, k[i:i + 1]]), np.concatenate([v2, v_[i:i + 1]])]
                ex = exact_attend(q[i], *seq[i, layer])[None]
                d = {}
                for m in pairs:
                    d[m] = rel_err(outs[m][i:i + 1], ex)
                    dist["gpu", m].append(d[m])
                    dist["oracle", m].append(rel_err(wants[m][i:i + 1], ex))
                e = rel_err(outs["shift"][i:i + 1], outs["absolute"][i:i + 1])
                worst_between = max(worst_between, e)
                assert e <= 1.01 * (d["shift"] + d["absolute"]) + 1e-6, (step, layer, i, e, d)
        for p in pairs.values():
            p.pool.end()
            for i in range(3):
                p.orc[i].commit(1)
        for i in range(3):
            in_view[i] += 1
        if step % 250 == 249:
            for p in pairs.values():
                for i in range(3):
                    p.assert_cache_equal(i)
    assert pairs["absolute"].pool.info(pairs["absolute"].ids[2])["ring_shift"] == frames - in_view[2]
    ref = max(dist["oracle", "shift"])
    for m in pairs:
        assert max(dist["gpu", m]) <= ref + 2.0 ** -8, (m, max(dist["gpu", m]), ref)
    # measured: the absolute ring sits closer to the exact session than the shifting one (one
    # rounding of each key instead of one per rotation), in the worst frame and on average
    assert np.mean(dist["gpu", "absolute"]) <= np.mean(dist["oracle", "shift"]) + 2.0 ** -9
    summary = ", ".join(f"{src} {m}: worst {max(d):.2e} mean {np.mean(d):.2e}" for (src, m), d in dist.items())
    print(f"distance to the exact session over {frames} frames: {summary}; GPU shift vs absolute: worst "
          f"{worst_between:.2e}")


def test_an_int8_absolute_ring_runs_past_the_initial_rope_table():
    # An absolute ring counts positions on after its evictions (the reference rotates at any
    # offset, transformer.rs:794-803): a 64-row table grows as the ring's positions pass it, and the
    # ring stays bit-exact with the oracle, outputs within 2e-2.
    p = Pair(cache="i8", act="bf16", streams=3, cap=80, seed=14, L=2, max_pos=64)
    heads = [0, 17, 70]
    for i in range(3):
        p.pool.start_ring(p.ids[i], "absolute", prefix=0)
        p.orc[i].start_ring("absolute", prefix=0)
    in_view = [0] * 3
    for n in range(300):
        for i in range(3):
            step = heads[i] + n
            if in_view[i] == 64:
                p.orc[i].evict(0, [(step - 64) % 80])
                in_view[i] -= 1
            p.orc[i].set_ring_slot(step % 80)
            p.pool.slide(p.ids[i], 0, 80, 64, 1, step)
        p.step()
        for i in range(3):
            in_view[i] += 1
        if n in (63, 64, 130, 299):
            for i in range(3):
                p.assert_cache_equal(i)
    assert p.pool.stats()["rope_rows"] == 512  # positions up to 299: 64 -> 128 -> 256 -> 512


@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("f32", "f32")])
def test_a_window_cache_runs_past_the_initial_rope_table(cache, act):
    # Mimi's KvCache builds RoPE rows at its absolute offset on every call (transformer.rs:794-803):
    # a window's positions grow without bound.  A 32-row table grows under a 24-row window over
    # 120 rows, single then paired, held to the oracle's KvCache.
    L, H = 2, 8
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=16, max_streams=2, max_blocks_per_stream=2,
                      cache_dtype=cache, act_dtype=act, max_pos=32, page_seed=5)
    wid = pool.init_window(24)
    win = oracle.Window(L, H, 64, 24, act=act)
    rng = np.random.default_rng(52)
    for t in [1] * 80 + [2] * 20:
        _window_batch(pool, [wid], [win], t, L, H, act, cache, rng)
    _assert_window_rows(pool, wid, win, 24, L, H, cache)
    assert win.offset == 120 and pool.stats()["rope_rows"] == 128


def test_the_int8_window_configuration_at_full_size_spot_checked():
    # The int8 sliding-window workload at its full size: 1024 streams x 9 layers x 8 heads x 64, int8
    # pages with a scale per (page, head), window 512 on 528-slot absolute rings, write heads
    # U[0,4096), histories of U[64,2048] rows as the workload draws them (the long ones wrap their
    # ring four times, each page's scale only growing once the ring has wrapped), each row through
    # the batched append with one slide per step, then two attend steps.  Layer 0 of every stream is
    # mirrored on a one-layer oracle ring of its own (outputs of both attend steps within 2e-2, then
    # every live code and scale of one stream in 64 bit-exact); 10 streams spread over the lengths
    # (the longest and the shortest included) are mirrored on all 9 layers: outputs within 2e-2,
    # then every live cache row, code and scale bit-exact.
    S, L, H, SPAN, WIN = 1024, 9, 8, 528, 512
    rng = np.random.default_rng(20261204)
    heads = rng.integers(0, 4096, S)
    lens = rng.integers(64, 2049, S)
    order = np.argsort(-lens, kind="stable")
    sample = sorted(set(order[::128].tolist()) | {int(order[0]), int(order[-1])})
    mbps = SPAN // 16
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * mbps + 16, max_streams=S, max_blocks_per_stream=mbps,
                      cache_dtype="i8", act_dtype="bf16", max_pos=int(lens.max()) + 8, page_seed=17)
    ids = [pool.init_state(SPAN) for _ in range(S)]
    for sid in ids:
        pool.start_ring(sid, "absolute", prefix=0)
    orc = {i: oracle.Stream(L, H, 64, SPAN, cache="i8", act="bf16") for i in sample}
    for i in sample:
        orc[i].start_ring("absolute", prefix=0)
    in_view = {i: 0 for i in sample}
    every = [oracle.Stream(1, H, 64, SPAN, cache="i8", act="bf16") for _ in range(S)]
    for st in every:
        st.start_ring("absolute", prefix=0)
    every_view = np.zeros(S, np.int64)

    def every_step(act, k, v, q=None):  # slide, then append (or attend) row j on layer 0 of stream act[j]
        pos = heads[act] + written[act]
        drop = np.where(every_view[act] == WIN, (pos - WIN) % SPAN, -1)
        out = oracle.batch_ring_step([every[i] for i in act], 0, drop, pos % SPAN, k, v, q=q)
        every_view[act] = np.minimum(every_view[act] + 1, WIN)
        return out

    written = np.zeros(S, np.int64)
    g = torch.Generator(device=DEV).manual_seed(20261204)

    def randn(*shape):
        return torch.randn(shape, device=DEV, generator=g).to(torch.bfloat16)

    def slide(i):  # xnp_ring_slide(prefix 0, span 528, window 512, drop 1, step) restated on the oracle
        step = int(heads[i] + written[i])
        if in_view[i] == WIN:
            orc[i].evict(0, [(step - WIN) % SPAN])
            in_view[i] -= 1
        orc[i].set_ring_slot(step % SPAN)

    kv = [randn(S, H, 64) for _ in range(2 * L)]
    kvh = [host(t) for t in kv]
    N = int(lens.max())
    start = N - lens
    for s in range(N):  # stream i joins at step N - lens[i] and appends one row per step
        act = np.nonzero(start <= s)[0]
        pool.slide_batch([ids[i] for i in act], 0, SPAN, WIN, 1, heads[act] + written[act])
        pool.begin([ids[i] for i in act])
        for layer in range(L):
            pool.append(layer, kv[2 * layer][:len(act)], kv[2 * layer + 1][:len(act)])
        pool.end()
        every_step(act, kvh[0][:len(act)], kvh[1][:len(act)])
        for i in sample:
            if start[i] <= s:
                slide(i)
                j = int(np.searchsorted(act, i))
                for layer in range(L):
                    orc[i].append(layer, kvh[2 * layer][j:j + 1], kvh[2 * layer + 1][j:j + 1])
                orc[i].commit(1)
                in_view[i] += 1
        written[act] += 1
    torch.cuda.synchronize()
    everyone = np.arange(S)
    for _ in range(2):
        pool.slide_batch(ids, 0, SPAN, WIN, 1, heads + written)
        for i in sample:
            slide(i)
        pool.begin(ids)
        for layer in range(L):
            q, k, v = randn(S, H, 64), randn(S, H, 64), randn(S, H, 64)
            out = torch.empty((S, H, 64), dtype=torch.bfloat16, device=DEV)
            pool.attend(layer, q, k, v, out, 0.125)
            torch.cuda.synchronize()
            if layer == 0:  # every stream
                want = every_step(everyone, host(k), host(v), q=host(q))
                per = np.abs(host(out) - want).max(axis=-1) / np.maximum(np.abs(want).max(axis=-1), 1e-30)
                worst = int(per.max(axis=-1).argmax())
                assert per.max() <= 2e-2, (worst, int(lens[worst]), float(per.max()))
            got, qh, kh, vh = host(out[sample]), host(q[sample]), host(k[sample]), host(v[sample])
            for j, i in enumerate(sample):
                want, _ = orc[i].attend(layer, qh[j:j + 1], kh[j:j + 1], vh[j:j + 1])
                assert rel_err(got[j:j + 1], want) <= 2e-2, (layer, i, int(lens[i]))
        pool.end()
        for i in sample:
            orc[i].commit(1)
            in_view[i] += 1
        written += 1
    # page by page: a ring written from an arbitrary head holds pages only where it has written
    for i in sample:
        valid = orc[i].ring_info()["valid"]
        for pg in range(mbps):
            live = valid[16 * pg:16 * pg + 16]
            if not live.any():
                continue
            for layer in range(L):
                for kvi in (0, 1):
                    rows = torch.empty((16, H, 64), dtype=torch.int8, device=DEV)
                    sc = torch.zeros((1, H), dtype=torch.float32, device=DEV)
                    pool.read_rows(ids[i], layer, kvi, 16 * pg, rows, sc)
                    torch.cuda.synchronize()
                    _, q8, osc = orc[i].read_rows(layer, kvi, 16 * pg, 16)
                    assert np.array_equal(rows.cpu().numpy()[live], q8[live]), (i, pg, layer, kvi)
                    assert np.array_equal(sc.cpu().numpy().view(np.uint32), osc.view(np.uint32)), (i, pg, layer, kvi)
    # layer 0 of one stream in 64 (besides the sample), every live slot's code and every live
    # page's scale against its one-layer oracle ring
    for i in range(0, S, 64):
        valid = every[i].ring_info()["valid"]
        for pg in range(mbps):  # only the pages the ring has written exist
            live = valid[16 * pg:16 * pg + 16]
            if not live.any():
                continue
            for kvi in (0, 1):
                rows = torch.empty((16, H, 64), dtype=torch.int8, device=DEV)
                sc = torch.zeros((1, H), dtype=torch.float32, device=DEV)
                pool.read_rows(ids[i], 0, kvi, 16 * pg, rows, sc)
                torch.cuda.synchronize()
                _, q8, osc = every[i].read_rows(0, kvi, 16 * pg, 16)
                assert np.array_equal(rows.cpu().numpy()[live], q8[live]), (i, pg, kvi)
                assert np.array_equal(sc.cpu().numpy().view(np.uint32), osc.view(np.uint32)), (i, pg, kvi)
    assert pool.check_tables() == 0


# ---- raw rows ------------------------------------------------------------------------------------
@pytest.mark.parametrize("cache", ["bf16", "i8"])
def test_rows_written_raw_read_back_the_same(cache):
    act = "bf16"
    pool = xnp.KvPool(num_layers=2, num_heads=8, num_blocks=16, max_streams=2, max_blocks_per_stream=8,
                      cache_dtype=cache, act_dtype=act, page_seed=3)
    sid = pool.init_state(100)
    pool.advance(sid, 70)
    g = torch.Generator(device="cpu").manual_seed(0)
    if cache == "i8":
        rows = torch.randint(-127, 128, (50, 8, 64), generator=g, dtype=torch.int8).to(DEV)
        scales = torch.rand((4, 8), generator=g).to(DEV)  # rows 13..62 touch pages 0..3
    else:
        rows = torch.randn((50, 8, 64), generator=g).to(torch.bfloat16).to(DEV)
        scales = None
    pool.write_rows(sid, 1, 1, 13, rows, scales)
    back = torch.empty_like(rows)
    sback = torch.zeros((4, 8), device=DEV) if cache == "i8" else None
    pool.read_rows(sid, 1, 1, 13, back, sback)
    torch.cuda.synchronize()
    assert torch.equal(back, rows)
    if cache == "i8":
        assert torch.equal(sback, scales)


@pytest.mark.parametrize("cache,act,maxlen", [("bf16", "bf16", 500), ("f32", "f32", 250), ("i8", "bf16", 900)])
def test_one_wave_per_stream_and_head_at_batch_scale(cache, act, maxlen):
    # Enough streams (160 x 8 heads) that the batch keeps the pool's default of one wave per
    # (stream, head): caches whose K and V tiles of one head hold at most 128 KB.  Every stream's
    # output against the oracle, two steps, and the cache rows of a sample bit for bit.
    S, L = 160, 1
    rng = np.random.default_rng(20261203)
    lens = rng.integers(1, maxlen + 1, S)
    p = Pair(cache=cache, act=act, streams=S, cap=maxlen + 4, seed=41, L=L, page_seed=17)
    for i, n in enumerate(lens):
        p.fill(i, int(n))
    p.pool.begin(p.ids)
    assert p.pool.stats()["decode_waves"] == 1
    p.pool.abort()
    for _ in range(2):
        assert p.step() <= TOL[cache]
    for i in range(0, S, 23):
        p.assert_cache_equal(i)


@pytest.mark.parametrize("split", [2, 8])
def test_256_streams_with_lengths_uniform_up_to_1024(split):
    # 256 streams with cache lengths U[1, 1024] on shuffled pages, each head's pages shared out
    # over `split` waves that merge in LDS.  Every stream is checked against the oracle.
    S, L = 256, 1
    rng = np.random.default_rng(20261202)
    lens = rng.integers(1, 1025, S)
    p = Pair(cache="bf16", act="bf16", streams=S, cap=1040, seed=11, L=L, split=split, page_seed=99)
    for i, n in enumerate(lens):
        n = int(n)
        kk, vv = p.x(n, 8, 64), p.x(n, 8, 64)
        p.pool.advance(p.ids[i], n)
        # the oracle stores the pre-rotated rows raw too: load the same rows on both sides
        p.pool.write_rows(p.ids[i], 0, 0, 0, dev(kk, "bf16"))
        p.pool.write_rows(p.ids[i], 0, 1, 0, dev(vv, "bf16"))
        p.orc[i].write_rows(0, 0, 0, vals=kk)
        p.orc[i].write_rows(0, 1, 0, vals=vv)
        p.orc[i].advance(n)
    for _ in range(2):
        assert p.step() <= 2e-2
    for i in range(0, S, 37):
        p.assert_cache_equal(i)


def test_the_decode_configuration_at_full_size_spot_checked():
    # The batched decode workload at its full size: 1024 streams x 9 layers x 8 heads x 64, bf16
    # pages of 16 on shuffled block tables, cache lengths U[1, 1024], the library's own split.
    # Every stream runs, and every stream's layer 0 is held to a one-layer oracle of its own over
    # both steps (outputs within 2e-2); 18 of them, spread over the longest-first order (the
    # longest and the shortest included), are checked on all 9 layers: outputs within 2e-2, then
    # every cache row bit-exact.
    S, L, H, cap = 1024, 9, 8, 1040
    rng = np.random.default_rng(20261203)
    lens = rng.integers(1, 1025, S)
    order = np.argsort(-lens, kind="stable")
    sample = sorted(set(order[::64].tolist()) | {int(order[0]), int(order[-1])})
    mbps = (cap + 15) // 16
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * mbps + 8, max_streams=S, max_blocks_per_stream=mbps,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=8192, page_seed=13)
    ids = [pool.init_state(cap) for _ in range(S)]
    orc = {i: oracle.Stream(L, H, 64, cap, cache="bf16", act="bf16") for i in sample}
    every = [oracle.Stream(1, H, 64, n + 4, cache="bf16", act="bf16") for n in lens.tolist()]
    g = torch.Generator(device=DEV).manual_seed(20261203)

    def randn(*shape):
        return torch.randn(shape, device=DEV, generator=g).to(torch.bfloat16)

    for i, n in enumerate(lens.tolist()):
        # each stream's history through the voice load (f32 rows rounded to bf16 on the device)
        pool.advance(ids[i], n)
        every[i].advance(n)
        if i in orc:
            orc[i].advance(n)
        for layer in range(L):
            kv = torch.randn((2, n, H, 64), device=DEV, generator=g)
            pool.load_kv(ids[i], layer, kv)
            if i in orc or layer == 0:
                kvh = host(kv)
                if layer == 0:
                    every[i].load_kv(0, kvh)
                if i in orc:
                    orc[i].load_kv(layer, kvh)
        torch.cuda.synchronize()  # the staged rows are freed on the next iteration
    for _ in range(2):
        pool.begin(ids)
        for layer in range(L):
            q, k, v = randn(S, H, 64), randn(S, H, 64), randn(S, H, 64)
            out = torch.empty((S, H, 64), dtype=torch.bfloat16, device=DEV)
            pool.attend(layer, q, k, v, out, 0.125)
            torch.cuda.synchronize()
            if layer == 0:  # every stream
                want = oracle.batch_attend(every, 0, host(q), host(k), host(v))
                got_all = host(out)
                per = np.abs(got_all - want).max(axis=-1) / np.maximum(np.abs(want).max(axis=-1), 1e-30)
                worst = int(per.max(axis=-1).argmax())
                assert per.max() <= 2e-2, (worst, int(lens[worst]), float(per.max()))
            got, qh, kh, vh = host(out[sample]), host(q[sample]), host(k[sample]), host(v[sample])
            for j, i in enumerate(sample):
                want, _ = orc[i].attend(layer, qh[j:j + 1], kh[j:j + 1], vh[j:j + 1])
                assert rel_err(got[j:j + 1], want) <= 2e-2, (layer, i, int(lens[i]))
        pool.end()
        oracle.batch_commit(every)
        for i in sample:
            orc[i].commit(1)
    shim = types.SimpleNamespace(pool=pool, ids=ids, orc=orc, L=L, H=H, KVH=H, cache="bf16")
    for i in sample:
        Pair.assert_cache_equal(shim, i)
    assert pool.check_tables() == 0


# ---- prompt prefill (transformer.rs:231-248) ------------------------------------------------------
@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("f32", "f32"), ("i8", "bf16")])
def test_prefill_matches_the_oracle(cache, act):
    # prior caches of 0..37 rows, then a 20-row prompt on all of them (crossing pages), then
    # single steps: outputs within tolerance, every cache row bit-exact.
    p = Pair(cache=cache, act=act, streams=4, cap=128, seed=21, page_seed=5)
    for i, n in enumerate([0, 5, 16, 37]):
        p.fill(i, n)
    p.prefill(20)
    for i in range(4):
        p.assert_cache_equal(i)
    p.step()
    p.prefill(3, which=[1, 2])
    p.step()
    for i in range(4):
        p.assert_cache_equal(i)


@pytest.mark.parametrize("cache", ["bf16", "i8"])
def test_prefill_of_256_position_grouped_head_prompts_on_8_streams(cache):
    # 8 streams x 256-position prompts (the 64-stream prefill workload's shape, fewer streams); int8
    # pages take the append, then the MFMA prefill reading every key back from the pages
    p = Pair(cache=cache, act="bf16", streams=8, cap=272, seed=22, L=1, page_seed=6)
    assert p.prefill(256) <= 2e-2
    for i in range(0, 8, 3):
        p.assert_cache_equal(i)


def test_the_prefill_configuration_at_full_size_spot_checked():
    # The prefill workload at its full size: 64 streams x 256-position prompts x 9 layers, bf16,
    # shuffled pages; every stream runs, 8 of them go through the oracle on every layer, and every
    # stream's layer 0 goes through a one-layer oracle stream of its own: outputs within 2e-2, then
    # every cache row the prompt wrote bit-exact (all layers of the sample, layer 0 of every stream).
    S, L, H, T = 64, 9, 8, 256
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * 17 + 8, max_streams=S, max_blocks_per_stream=17,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=1024, page_seed=21)
    ids = [pool.init_state(272) for _ in range(S)]
    sample = list(range(0, S, 9))
    orc = {i: oracle.Stream(L, H, 64, 272, cache="bf16", act="bf16") for i in sample}
    every = {i: oracle.Stream(1, H, 64, 272, cache="bf16", act="bf16") for i in range(S)}
    g = torch.Generator(device=DEV).manual_seed(20261206)
    pool.begin(ids, t=T)
    for layer in range(L):
        q, k, v = (torch.randn((S, T, H, 64), device=DEV, generator=g).to(torch.bfloat16) for _ in range(3))
        out = torch.empty((S, T, H, 64), dtype=torch.bfloat16, device=DEV)
        pool.attend(layer, q, k, v, out, 0.125)
        torch.cuda.synchronize()
        rows = range(S) if layer == 0 else sample
        got, qh, kh, vh = host(out), host(q), host(k), host(v)
        for i in rows:
            if i in orc:
                want, _ = orc[i].attend(layer, qh[i], kh[i], vh[i])
                assert rel_err(got[i], want) <= 2e-2, (layer, i)
            if layer == 0:
                want, _ = every[i].attend(0, qh[i], kh[i], vh[i])
                assert rel_err(got[i], want) <= 2e-2, (layer, i, "every")
    pool.end()
    for i in sample:
        orc[i].commit(T)
    for i in range(S):
        every[i].commit(T)
    shim = types.SimpleNamespace(pool=pool, ids=ids, orc=orc, L=L, H=H, KVH=H, cache="bf16")
    for i in sample:
        Pair.assert_cache_equal(shim, i)
    shim0 = types.SimpleNamespace(pool=pool, ids=ids, orc=every, L=1, H=H, KVH=H, cache="bf16")
    for i in range(S):
        Pair.assert_cache_equal(shim0, i)


def test_prompts_on_reopened_streams_use_live_pages():
    # A new utterance per stream each round (close, reopen, prompt): the device tables must hold
    # the live pages (a stale -1 would send the append and prefill kernels out of the pool).
    p = Pair(cache="bf16", act="bf16", streams=4, cap=64, seed=23, L=2, page_seed=8)
    for _ in range(3):
        p.prefill(40)
        assert p.pool.check_tables() == 0
        for i in range(4):
            p.assert_cache_equal(i)
            p.pool.close(p.ids[i])
            p.ids[i] = p.pool.init_state(64)
            p.orc[i] = oracle.Stream(p.L, p.H, 64, 64, cache="bf16", act="bf16")
    assert p.pool.check_tables() == 0


@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("i8", "bf16")])
def test_prefill_after_a_separate_append(cache, act):
    # xnp_append then xnp_prefill: the prompt's keys are read back from the pages
    p = Pair(cache=cache, act=act, streams=3, cap=128, seed=24, page_seed=9)
    for i, n in enumerate([0, 7, 33]):
        p.fill(i, n)
    p.prefill_split(45)
    for i in range(3):
        p.assert_cache_equal(i)
    p.step()


@pytest.mark.parametrize("cache", ["bf16", "i8"])
def test_long_prompts_take_several_rounds(cache):
    # 300- and 530-row prompts: more than one round of 256 query rows per work group, on top of
    # prior rows that end mid-page; grouped heads.  int8 pages: the MFMA prefill after the append,
    # scores in f16 against the codes, each page's scales applied per 16-key group
    p = Pair(cache=cache, act="bf16", H=8, KVH=2, streams=2, cap=640, seed=25, L=1, page_seed=10)
    p.fill(1, 21)
    assert p.prefill(300, which=[0]) <= 2e-2
    assert p.prefill(530, which=[1]) <= 2e-2
    for i in range(2):
        p.assert_cache_equal(i)
    p.step()


# The longest stream a pool takes: 480 pages of 16 rows (60 page ids per wave's lanes, 8 waves per
# (stream, head)).  Streams one row short of full and one page short of full decode their last row
# into the last slot and into a fresh last page; a short stream rides along in the same batch.
# The grouped-head rows take the MFMA decode.
@pytest.mark.parametrize("cache,act,kvh", [("bf16", "bf16", 8), ("i8", "bf16", 8), ("f32", "f32", 8),
                                           ("bf16", "bf16", 1), ("i8", "bf16", 2)])
def test_streams_at_the_longest_a_pool_takes(cache, act, kvh):
    cap = 480 * 16
    p = Pair(cache=cache, act=act, KVH=kvh, streams=3, cap=cap, seed=31, L=1, page_seed=12)
    for i, n in enumerate([cap - 1, cap - 16, 3]):
        p.fill(i, n)
    assert p.step() <= TOL[cache]
    for i in range(3):
        p.assert_cache_equal(i)
    assert p.orc[0].current_end == cap


@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("i8", "bf16"), ("f32", "f32")])
def test_a_prompt_that_fills_the_longest_stream(cache, act):
    # 7580 rows (ending mid-page), then a 100-row prompt ending on the last slot of page 480: the
    # prompt reads every page id of the stream (the MFMA prefill keeps them in LDS; int8 runs it
    # after the append, f32 takes the row-by-row prompt kernel after the append)
    cap = 480 * 16
    p = Pair(cache=cache, act=act, streams=1, cap=cap, seed=32, L=1, page_seed=13)
    p.fill(0, cap - 100)
    assert p.prefill(100) <= TOL[cache]
    p.assert_cache_equal(0)
    assert p.orc[0].current_end == cap


@pytest.mark.parametrize("cache,act", [("bf16", "bf16"), ("f32", "f32")])
def test_unwritten_rows_holding_nan_bytes_do_not_reach_the_output(cache, act):
    # A page's rows past current_end are never attended, but the kernels read whole tiles: rows
    # holding NaN bit patterns (left by an earlier user of the memory) must weigh exactly nothing.
    p = Pair(cache=cache, act=act, streams=2, cap=64, seed=26, L=1, page_seed=11)
    for i, n in enumerate([20, 37]):
        sid, st = p.ids[i], p.orc[i]
        p.pool.advance(sid, n)
        st.advance(n)
        full = (n + 15) // 16 * 16  # every row of the pages the stream holds
        for kv in (0, 1):
            vals = p.x(n, p.H, 64)
            st.write_rows(0, kv, 0, vals=vals)
            rows = np.full((full, p.H, 64), np.nan, np.float32)
            rows[:n] = vals
            p.pool.write_rows(sid, 0, kv, 0, dev(rows, act))
    torch.cuda.synchronize()
    assert p.step() <= TOL[cache]
    for i in range(2):
        p.assert_cache_equal(i)


def test_a_step_captured_in_a_hip_graph_replays_like_eager_steps():
    # The per-layer launches of a batch allocate nothing and read positions and pages from the
    # plan the step uploads, as DeviceStep keeps the position on the device (transformer.rs:111-140)
    # so that StepGraph can record one step and replay it (step_graph.rs:111-307).  Capture the L
    # attend launches once; each later step is begin (eager plan upload) + replay + end.  A twin
    # pool runs the same steps eagerly: outputs and caches must agree bit for bit, every replay.
    L, H, S = 2, 8, 6
    lens = [0, 3, 15, 16, 40, 70]
    rng = np.random.default_rng(27)
    pools, idss = [], []
    for _ in range(2):
        pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * 8 + 8, max_streams=S, max_blocks_per_stream=8,
                          cache_dtype="bf16", act_dtype="bf16", max_pos=256, page_seed=13)
        pools.append(pool)
        idss.append([pool.init_state(128) for _ in range(S)])
    for i, n in enumerate(lens):
        if n == 0:
            continue
        k, v = dev(bf16_round(rng.standard_normal((n, H, 64))), "bf16"), dev(bf16_round(rng.standard_normal((n, H, 64))), "bf16")
        for pool, ids in zip(pools, idss):
            pool.begin([ids[i]], t=n)
            for layer in range(L):
                pool.append(layer, k, v)
            pool.end()
    s = torch.cuda.Stream()
    q, k, v = ([torch.empty((S, H, 64), dtype=torch.bfloat16, device=DEV) for _ in range(L)] for _ in range(3))
    outs = [[torch.empty((S, H, 64), dtype=torch.bfloat16, device=DEV) for _ in range(L)] for _ in range(2)]

    def refill():
        for t in q + k + v:
            t.copy_(torch.from_numpy(bf16_round(rng.standard_normal((S, H, 64)))).to(DEV))

    def launches(pool, out):
        for layer in range(L):
            pool.attend(layer, q[layer], k[layer], v[layer], out[layer], 0.125)

    g = torch.cuda.CUDAGraph()
    for step in range(6):
        with torch.cuda.stream(s):
            refill()
            for p, (pool, ids) in enumerate(zip(pools, idss)):
                pool.begin(ids, stream=s.cuda_stream)
                if p == 0:
                    launches(pool, outs[0])
                elif step == 0:
                    with torch.cuda.graph(g, stream=s):
                        launches(pool, outs[1])
                    g.replay()
                else:
                    g.replay()
                pool.end()
        s.synchronize()
        for layer in range(L):
            a, b = outs[0][layer].view(torch.int16), outs[1][layer].view(torch.int16)
            assert torch.equal(a, b), (step, layer)
        torch.cuda.synchronize()
    for i in range(S):
        n = lens[i] + 6
        for layer in range(L):
            for kvi in (0, 1):
                rows = [torch.empty((n, H, 64), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
                for pool, ids, r in zip(pools, idss, rows):
                    pool.read_rows(ids[i], layer, kvi, 0, r)
                torch.cuda.synchronize()
                assert torch.equal(rows[0].view(torch.int16), rows[1].view(torch.int16)), (i, layer, kvi)
