"""Pins of the oracle (the CPU restatement) that do not go through the oracle's own formulas:
closed forms, textbook definitions computed independently (numpy f64, torch's bf16 cast), and
restatements of the reference's relational tests (transformer.rs:1022-1417).

The reference holds no golden vectors for this path (its hot-path tests are relational), and its
Rust code cannot run here, so these are what fix the oracle's numbers.
"""
import math

import numpy as np
import pytest
import torch

from conftest import oracle
from helpers import bf16_round, exact_attend, lcg, normal, rel_err

THETA = 10000.0


# ---- bf16 rounding ------------------------------------------------------------------------
def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-20, 20, 4000),
                        np.float32([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 0.0, -0.0,
                                    3.4e38, 1e-40])])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    got = np.array([oracle.bf16_round(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(bf16_round(x).view(np.uint32), want.view(np.uint32))


# ---- RoPE (rope.rs:37-95) -------------------------------------------------------------------
@pytest.mark.parametrize("pos", [1, 7, 100, 4095])
def test_rope_rotates_each_interleaved_pair_by_pos_times_freq(pos):
    # x = e_{2i}: rotate gives (cos a, sin a) in pair i with a = pos * theta^(-i/32); e_{2i+1}
    # gives (-sin a, cos a).  This fixes the pairing (2i, 2i+1), the sign and the frequencies.
    D = 64
    c, s = oracle.rope_row(D, THETA, float(pos), "f32")
    for i in range(D // 2):
        a = pos * THETA ** (-i / 32)
        e0 = np.zeros(D, np.float32)
        e0[2 * i] = 1.0
        r0 = oracle.rotate(e0, c, s)
        e1 = np.zeros(D, np.float32)
        e1[2 * i + 1] = 1.0
        r1 = oracle.rotate(e1, c, s)
        tol = 2e-6 * max(1.0, a)  # f32 angle pos * inv_freq carries ~1 ulp of a
        assert abs(r0[2 * i] - math.cos(a)) < tol and abs(r0[2 * i + 1] - math.sin(a)) < tol
        assert abs(r1[2 * i] + math.sin(a)) < tol and abs(r1[2 * i + 1] - math.cos(a)) < tol
        others = np.delete(r0, [2 * i, 2 * i + 1])
        assert not others.any()


def test_rope_position_zero_is_the_identity_exactly():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(64).astype(np.float32)
    c, s = oracle.rope_row(64, THETA, 0.0, "f32")
    assert np.array_equal(oracle.rotate(x, c, s), x)


def test_rope_preserves_pair_norms_and_composes():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(64).astype(np.float32)
    ca, sa = oracle.rope_row(64, THETA, 37.0, "f32")
    cb, sb = oracle.rope_row(64, THETA, 18.0, "f32")
    cab, sab = oracle.rope_row(64, THETA, 55.0, "f32")
    y = oracle.rotate(x, ca, sa)
    pn = lambda v: np.hypot(v[0::2].astype(np.float64), v[1::2].astype(np.float64))
    np.testing.assert_allclose(pn(y), pn(x), rtol=1e-6)
    np.testing.assert_allclose(oracle.rotate(y, cb, sb), oracle.rotate(x, cab, sab), atol=2e-5)
    # shift_back (rope.rs:26-35) is the rotation by -count: it undoes a rotation by count
    cm, sm = oracle.rope_row(64, THETA, -18.0, "f32")
    np.testing.assert_allclose(oracle.rotate(oracle.rotate(x, cab, sab), cm, sm), y, atol=2e-5)


def test_rope_bf16_tables_are_the_f32_values_rounded():
    c32, s32 = oracle.rope_row(64, THETA, 1234.0, "f32")
    c16, s16 = oracle.rope_row(64, THETA, 1234.0, "bf16")
    assert np.array_equal(c16, bf16_round(c32)) and np.array_equal(s16, bf16_round(s32))


# ---- decode attention (sdpa_decode, transformer.rs:223,230) -----------------------------------
def sdpa_f64(q, K, V, scale):
    """Textbook softmax(q K^T * scale) V in f64 (numpy), q [D], K/V [n][D]."""
    s = (K.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    return (p / p.sum()) @ V.astype(np.float64)


def rotated(x, pos, act="f32"):
    c, s = oracle.rope_row(x.shape[-1], THETA, float(pos), act)
    return oracle.rotate(x, c, s, act)


def fill(st, rows_k, rows_v, layer=0):
    for i in range(rows_k.shape[0]):
        st.append(layer, rows_k[i:i + 1], rows_v[i:i + 1])
        st.commit(1)


def test_one_key_returns_its_value():
    rng = np.random.default_rng(3)
    st = oracle.Stream(1, 2, 64, 8)
    q, k, v = (rng.standard_normal((1, 2, 64)).astype(np.float32) for _ in range(3))
    out, out64 = st.attend(0, q, k, v)
    assert np.array_equal(out, v)  # softmax of a single score is exactly 1
    np.testing.assert_array_equal(out64, v.astype(np.float64))


def test_zero_query_or_identical_keys_give_the_mean_of_values():
    rng = np.random.default_rng(4)
    vals = rng.standard_normal((20, 1, 64)).astype(np.float32)
    # q = 0: every score is exactly 0
    st = oracle.Stream(1, 1, 64, 32)
    ks = rng.standard_normal((20, 1, 64)).astype(np.float32)
    fill(st, ks[:19], vals[:19])
    out, out64 = st.attend(0, np.zeros((1, 1, 64), np.float32), ks[19:], vals[19:])
    assert rel_err(out64[0, 0], vals[:, 0].astype(np.float64).mean(axis=0)) < 1e-12
    assert rel_err(out[0, 0], vals[:, 0].astype(np.float64).mean(axis=0)) < 1e-5
    # the same stored key in every slot (the new one rotated into place, to rounding)
    st = oracle.Stream(1, 1, 64, 32)
    key = rng.standard_normal((1, 1, 64)).astype(np.float32)
    st.write_rows(0, 0, 0, vals=np.repeat(key, 19, axis=0))
    st.write_rows(0, 1, 0, vals=vals[:19])
    st.advance(19)
    c, s = oracle.rope_row(64, THETA, -19.0, "f32")
    k_in = oracle.rotate(key[0, 0], c, s)[None, None]
    out, out64 = st.attend(0, rng.standard_normal((1, 1, 64)).astype(np.float32), k_in, vals[19:])
    assert rel_err(out64[0, 0], vals[:, 0].astype(np.float64).mean(axis=0)) < 1e-5


def test_a_dominant_score_returns_that_value():
    rng = np.random.default_rng(5)
    st = oracle.Stream(1, 1, 64, 32)
    ks = rng.standard_normal((10, 1, 64)).astype(np.float32) * 0.01
    vs = rng.standard_normal((10, 1, 64)).astype(np.float32)
    q = np.zeros((1, 1, 64), np.float32)
    q[0, 0, 0] = 1.0
    # key 3 is a large multiple of the query's direction once both are rotated into place:
    # stored key 3 = rotate(k_in, 3) and rotated q = rotate(q, 10), so k_in = rotate(4000 q, 7)
    c, s = oracle.rope_row(64, THETA, 7.0, "f32")
    ks[3] = oracle.rotate(q[0, 0] * 4000.0, c, s)[None]
    fill(st, ks, vs)
    out, _ = st.attend(0, q, np.zeros((1, 1, 64), np.float32), np.zeros((1, 1, 64), np.float32))
    np.testing.assert_allclose(out[0, 0], vs[3, 0], atol=1e-5)


@pytest.mark.parametrize("n", [1, 2, 17, 300])
def test_decode_matches_textbook_attention(n):
    rng = np.random.default_rng(10 + n)
    H, D = 2, 64
    st = oracle.Stream(2, H, D, n + 4)
    K = rng.standard_normal((n, H, D)).astype(np.float32)
    V = rng.standard_normal((n, H, D)).astype(np.float32)
    fill(st, K[:-1], V[:-1], layer=1)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    out, out64 = st.attend(1, q, K[-1:], V[-1:])
    for h in range(H):
        Kr = np.stack([rotated(K[i, h], i) for i in range(n)])
        want = sdpa_f64(rotated(q[0, h], n - 1), Kr, V[:, h], 0.125)
        assert rel_err(out64[0, h], want) < 1e-9
        assert rel_err(out[0, h], want) < 1e-5


def test_prefill_is_causal_textbook_attention():
    rng = np.random.default_rng(6)
    H, D, t, cur = 2, 64, 24, 5
    st = oracle.Stream(1, H, D, 64)
    K = rng.standard_normal((cur + t, H, D)).astype(np.float32)
    V = rng.standard_normal((cur + t, H, D)).astype(np.float32)
    Q = rng.standard_normal((t, H, D)).astype(np.float32)
    fill(st, K[:cur], V[:cur])
    out, out64 = st.attend(0, Q, K[cur:], V[cur:])
    for i in range(t):
        for h in range(H):
            Kr = np.stack([rotated(K[j, h], j) for j in range(cur + i + 1)])
            want = sdpa_f64(rotated(Q[i, h], cur + i), Kr, V[:cur + i + 1, h], 0.125)
            assert rel_err(out64[i, h], want) < 1e-9


def test_bf16_outputs_are_rounded_and_close_to_f64():
    rng = np.random.default_rng(7)
    st = oracle.Stream(1, 2, 64, 64, cache="bf16", act="bf16")
    for i in range(40):
        k, v = (bf16_round(rng.standard_normal((1, 2, 64))) for _ in range(2))
        st.append(0, k, v)
        st.commit(1)
    q = bf16_round(rng.standard_normal((1, 2, 64)))
    k, v = (bf16_round(rng.standard_normal((1, 2, 64))) for _ in range(2))
    out, out64 = st.attend(0, q, k, v)
    assert np.array_equal(out, bf16_round(out))
    assert rel_err(out, out64) < 2e-2
    vals, _, _ = st.read_rows(0, 0, 0, 41)
    assert np.array_equal(vals, bf16_round(vals))


# ---- grouped-query heads (transformer.rs:1112-1164) -----------------------------------------
def test_grouped_kv_heads_equal_repeated_heads():
    rand = lcg(1)
    H, KVH, D = 4, 2, 64
    a = oracle.Stream(1, H, D, 16, kv_heads=KVH)
    b = oracle.Stream(1, H, D, 16)
    for (start, t) in [(0, 3), (3, 1), (4, 1)]:
        q = rand(t * H * D).reshape(t, H, D)
        k = rand(t * KVH * D).reshape(t, KVH, D)
        v = rand(t * KVH * D).reshape(t, KVH, D)
        oa, _ = a.attend(0, q, k, v)
        ob, _ = b.attend(0, q, np.repeat(k, H // KVH, axis=1), np.repeat(v, H // KVH, axis=1))
        a.commit(t)
        b.commit(t)
        assert np.array_equal(oa, ob)


# ---- with_seq_budget (transformer.rs:1022-1099) ----------------------------------------------
def filled(seq, used):
    # k[s, h, d] = s + 100 h, v = -k, as the reference's test pattern
    st = oracle.Stream(1, 2, 64, seq)
    k = np.fromfunction(lambda s, h, d: s + 100 * h, (seq, 2, 64), dtype=np.float32).astype(np.float32)
    st.write_rows(0, 0, 0, vals=k)
    st.write_rows(0, 1, 0, vals=-k)
    st.advance(used)
    return st, k


def test_with_seq_budget_copies_the_used_prefix_and_zero_fills_the_rest():
    small, k = filled(4, 3)
    big = small.with_seq_budget(10)
    assert big.current_end == 3 and big.capacity == 10
    kb, _, _ = big.read_rows(0, 0, 0, 10)
    assert np.array_equal(kb[:3], k[:3]) and not kb[3:].any()
    vb, _, _ = big.read_rows(0, 1, 0, 3)
    assert np.array_equal(vb, -k[:3])


def test_the_copy_does_not_share_storage_with_the_source():
    small, k = filled(4, 2)
    big = small.with_seq_budget(8)
    big.write_rows(0, 0, 0, vals=np.full((1, 2, 64), 9e9, np.float32))
    ks, _, _ = small.read_rows(0, 0, 0, 1)
    assert ks[0, 1, 0] == 100.0


def test_a_budget_smaller_than_the_prefix_is_refused():
    st, _ = filled(4, 3)
    with pytest.raises(oracle.OracleError, match="3.*2"):
        st.with_seq_budget(2)
    st.with_seq_budget(3)


# ---- ring (transformer.rs:1347-1416) ----------------------------------------------------------
def rows(n, phase, H=4, D=64):
    # transformer.rs:1350-1354: sin(i * 0.37 + phase), here already split in heads
    return np.sin(np.arange(n * H * D, dtype=np.float32) * np.float32(0.37) + np.float32(phase)).reshape(n, H, D)


@pytest.mark.parametrize("mode", ["shift", "absolute"])
def test_evicting_leaves_the_cache_of_a_sequence_without_them(mode):
    # A 5-row prompt and 6 frame slots whose oldest 3 frames go whenever they are full: three
    # evictions over 15 frames, the later ones wrapping round the ring.  Every frame must see what
    # it would have seen had the evicted frames never been there (1e-4, as the reference).
    H, D = 4, 64
    qs, ks, vs = rows(15, 1.0), rows(15, 2.0), rows(15, 3.0)
    pk, pv, pq = rows(5, 0.0), rows(5, 0.5), rows(5, 0.25)
    ring = oracle.Stream(1, H, D, 11)
    ring.attend(0, pq, pk, pv)
    ring.commit(5)
    ring.start_ring(mode, prefix=5)
    in_view = 0
    for i in range(15):
        if in_view == 6:
            oldest = i - in_view
            ring.evict(5, [5 + (oldest + j) % 6 for j in range(3)])
            in_view -= 3
            assert ring.current_end == 5 + in_view
        ring.set_ring_slot(5 + i % 6)
        got, _ = ring.attend(0, qs[i:i + 1], ks[i:i + 1], vs[i:i + 1])
        ring.commit(1)
        in_view += 1
        plain = oracle.Stream(1, H, D, 11)
        plain.attend(0, pq, pk, pv)
        plain.commit(5)
        for j in range(i + 1 - in_view, i + 1):
            want, _ = plain.attend(0, qs[j:j + 1], ks[j:j + 1], vs[j:j + 1])
            plain.commit(1)
        assert np.abs(got - want).max() < 1e-4, f"frame {i}"


def test_absolute_ring_equals_shifting_ring():
    # Evicting with the keys left where they were written and the query rotated twice gives what
    # rotating the kept keys back gives (bf16: to the rounding of the rotations).
    rng = np.random.default_rng(8)
    H, D, cap, pre = 2, 64, 40, 6
    st = {m: oracle.Stream(1, H, D, cap, cache="bf16", act="bf16") for m in ("shift", "absolute")}
    q0, k0, v0 = (bf16_round(rng.standard_normal((pre, H, D))) for _ in range(3))
    for s in st.values():
        s.attend(0, q0, k0, v0)
        s.commit(pre)
    for m, s in st.items():
        s.start_ring(m, prefix=pre)
    outs = {m: [] for m in st}
    in_view, ctx = 0, 20
    for i in range(90):
        q, k, v = (bf16_round(rng.standard_normal((1, H, D))) for _ in range(3))
        for m, s in st.items():
            if in_view == ctx:
                s.evict(pre, [pre + (i - in_view + j) % ctx for j in range(7)])
            s.set_ring_slot(pre + i % ctx)
            o, _ = s.attend(0, q, k, v)
            s.commit(1)
            outs[m].append(o)
        in_view = in_view - 7 + 1 if in_view == ctx else in_view + 1
    a, b = np.concatenate(outs["shift"]), np.concatenate(outs["absolute"])
    assert rel_err(a, b) < 5e-2
    assert st["shift"].ring_info()["shift"] == 0 and st["absolute"].ring_info()["shift"] > 0
    assert st["shift"].current_end == st["absolute"].current_end


def test_the_batched_ring_step_is_its_per_stream_calls():
    # orc_batch_ring_step composes evict, set_ring_slot, append or attend, and commit: the same
    # outputs and cache bytes as those calls made stream by stream (int8 absolute rings on a
    # 20-slot window of 24 slots, heads at different offsets, 70 steps, the last 5 attending).
    rng = np.random.default_rng(31)
    S, H, D, span, win = 5, 2, 64, 24, 20
    heads = rng.integers(0, 100, S)
    one = [oracle.Stream(1, H, D, span, cache="i8", act="bf16") for _ in range(S)]
    bat = [oracle.Stream(1, H, D, span, cache="i8", act="bf16") for _ in range(S)]
    for st in one + bat:
        st.start_ring("absolute", prefix=0)
    in_view = np.zeros(S, np.int64)
    for step in range(70):
        pos = heads + step
        drop = np.where(in_view == win, (pos - win) % span, -1)
        k, v, q = (bf16_round(rng.standard_normal((S, H, D))) for _ in range(3))
        attend = step >= 65
        want = []
        for i, st in enumerate(one):
            if drop[i] >= 0:
                st.evict(0, [int(drop[i])])
            st.set_ring_slot(int(pos[i] % span))
            if attend:
                want.append(st.attend(0, q[i:i + 1], k[i:i + 1], v[i:i + 1])[0][0])
            else:
                st.append(0, k[i:i + 1], v[i:i + 1])
            st.commit(1)
        got = oracle.batch_ring_step(bat, 0, drop, pos % span, k, v, q=q if attend else None)
        if attend:
            assert np.array_equal(got, np.stack(want))
        in_view = np.minimum(in_view + 1, win)
    for a, b in zip(one, bat):
        assert a.ring_info()["write"] == b.ring_info()["write"]
        assert np.array_equal(a.ring_info()["valid"], b.ring_info()["valid"])
        for kv in (0, 1):
            va, qa, sa = a.read_rows(0, kv, 0, span)
            vb, qb, sb = b.read_rows(0, kv, 0, span)
            assert np.array_equal(qa, qb) and np.array_equal(sa.view(np.uint32), sb.view(np.uint32))


def test_a_shifting_ring_in_f32_is_the_exact_sequence_without_the_evicted_rows():
    # The invariant of transformer.rs:1359-1395, against exact arithmetic: an f32 shifting ring run
    # by the s2s policy (a 7-row prefix, a context of 24 slots, the oldest 8 evicted when full) gives
    # at every frame the f64 attention of the query over the kept rows at their compacted positions
    # (exact_attend, RoPE in f64 from the inputs), to f32 rounding; 100 frames.
    rng = np.random.default_rng(41)
    H, D, pre, context, drop = 4, 64, 7, 24, 8
    st = oracle.Stream(1, H, D, pre + context)
    keys, vals = rng.standard_normal((pre, H, D)).astype(np.float32), rng.standard_normal((pre, H, D)).astype(np.float32)
    st.append(0, keys, vals)
    st.commit(pre)
    st.start_ring("shift", prefix=pre)
    in_view, worst = 0, 0.0
    for step in range(100):
        if in_view == context:
            oldest = step - in_view
            st.evict(pre, [pre + (oldest + j) % context for j in range(drop)])
            keys, vals = np.concatenate([keys[:pre], keys[pre + drop:]]), np.concatenate([vals[:pre], vals[pre + drop:]])
            in_view -= drop
        st.set_ring_slot(pre + step % context)
        q, k, v = (rng.standard_normal((1, H, D)).astype(np.float32) for _ in range(3))
        out, _ = st.attend(0, q, k, v)
        st.commit(1)
        in_view += 1
        keys, vals = np.concatenate([keys, k]), np.concatenate([vals, v])
        worst = max(worst, rel_err(out, exact_attend(q[0], keys, vals)[None]))
    assert worst <= 2e-5, worst


def test_misuse_of_a_ring_is_refused():
    st = oracle.Stream(1, 4, 64, 8)
    st.attend(0, rows(4, 0.0), rows(4, 0.1), rows(4, 0.2))
    st.commit(4)
    with pytest.raises(oracle.OracleError, match="not a ring"):
        st.set_ring_slot(4)
    st.start_ring("shift")
    with pytest.raises(oracle.OracleError, match="cannot be resized"):
        st.with_seq_budget(10)
    st.set_ring_slot(4)
    st.attend(0, rows(1, 1.0), rows(1, 1.1), rows(1, 1.2))
    st.commit(1)
    with pytest.raises(oracle.OracleError):
        st.evict(4, [2])
    with pytest.raises(oracle.OracleError):
        st.evict(4, [5])
    with pytest.raises(oracle.OracleError):  # refused as a whole: slot 4 stays
        st.evict(4, [4, 5])
    assert st.ring_info()["valid"][4]
    st.set_ring_slot(4)
    with pytest.raises(oracle.OracleError, match="still holds a row"):
        st.attend(0, rows(1, 2.0), rows(1, 2.1), rows(1, 2.2))
    st.evict(4, [4])
    st.attend(0, rows(1, 2.0), rows(1, 2.1), rows(1, 2.2))
    with pytest.raises(oracle.OracleError, match="one row at a time"):
        st.attend(0, rows(2, 2.0), rows(2, 2.1), rows(2, 2.2))


# ---- int8 (per-(page, head) scales) -------------------------------------------------------------
def test_int8_rows_quantize_within_half_a_step():
    rng = np.random.default_rng(9)
    st = oracle.Stream(1, 2, 64, 48, cache="i8", act="bf16")
    V = bf16_round(rng.standard_normal((40, 2, 64)) * rng.uniform(0.1, 3.0, (40, 1, 1)))
    for i in range(40):
        st.append(0, np.zeros((1, 2, 64), np.float32), V[i:i + 1])
        st.commit(1)
    vals, q8, scales = st.read_rows(0, 1, 0, 40)
    for b in range(3):
        blk = V[16 * b:16 * b + 16]
        amax = np.abs(blk).max(axis=(0, 2))
        # the final scale is the block's amax / 127 (every row seen by the running max)
        np.testing.assert_array_equal(scales[b], (amax / np.float32(127)).astype(np.float32))
        # A row is rounded once when written and once more each time a later row raises the
        # page's scale: its error is at most (1 + raises after it) half steps of the final scale.
        run = np.maximum.accumulate(np.abs(blk).max(axis=2), axis=0)  # [rows, H]
        raises = (run[1:] > run[:-1]).astype(int)
        later = np.concatenate([np.cumsum(raises[::-1], axis=0)[::-1], np.zeros((1, 2), int)])
        bound = (1 + later)[:, :, None] * scales[b][None, :, None] / 2
        err = np.abs(vals[16 * b:16 * b + 16] - blk)
        assert (err <= bound * (1 + 1e-5)).all()
        # rows written at the final scale (no raise after them) are within half a step
        assert (err[later[:, 0] == 0, 0] <= scales[b][0] / 2 * (1 + 1e-5)).all()
    assert np.abs(q8).max() <= 127
    # a fresh page (first row) takes its scale from that row alone
    st2 = oracle.Stream(1, 1, 64, 16, cache="i8", act="f32")
    x = np.linspace(-2, 3, 64, dtype=np.float32)[None, None]
    st2.append(0, np.zeros_like(x), x)
    vals, q8, scales = st2.read_rows(0, 1, 0, 1)
    assert scales[0, 0] == np.float32(3.0) / np.float32(127.0)
    assert q8[0, 0, -1] == 127 and np.abs(vals[0, 0] - x[0, 0]).max() <= scales[0, 0] / 2 + 1e-7


# ---- voices stored as the KV cache (ptts-wasm/src/lib.rs:291-325) -----------------------------
@pytest.mark.parametrize("cache", ["f32", "bf16", "i8"])
def test_a_voice_loads_as_its_rows_in_the_cache_dtype(cache):
    rng = np.random.default_rng(31)
    n, H = 37, 3  # two full blocks and a tail block of 5 rows
    kv = (rng.standard_normal((2, n, H, 64)) * rng.uniform(0.1, 4.0, (1, n, H, 1))).astype(np.float32)
    st = oracle.Stream(2, H, 64, 64, cache=cache, act="f32" if cache == "f32" else "bf16")
    st.advance(n)
    st.load_kv(1, kv)
    assert st.current_end == n
    for which in (0, 1):
        vals, q8, scales = st.read_rows(1, which, 0, n)
        x = kv[which]
        if cache == "f32":
            assert np.array_equal(vals.view(np.uint32), x.view(np.uint32))
        elif cache == "bf16":
            want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
            assert np.array_equal(vals.view(np.uint32), want.view(np.uint32))
        else:
            for b in range(3):
                blk, q = x[16 * b:16 * b + 16], q8[16 * b:16 * b + 16]
                amax = np.abs(blk.astype(np.float64)).max(axis=(0, 2))  # [H], over the block's rows only
                np.testing.assert_allclose(scales[b], amax / 127.0, rtol=1e-7)
                # the largest magnitude of each (block, head) lands on code +-127, and every value
                # is within half a step of what it dequantizes to
                assert (np.abs(q.astype(int)).max(axis=(0, 2)) == 127).all()
                err = np.abs(vals[16 * b:16 * b + 16].astype(np.float64) - blk)
                assert (err <= scales[b][None, :, None] / 2 * (1 + 1e-6)).all()
                np.testing.assert_array_equal(vals[16 * b:16 * b + 16], q * scales[b][None, :, None])
    vals, _, _ = st.read_rows(0, 0, 0, n)  # layer 0 was not loaded
    assert not vals.any()


def test_a_voice_loads_only_into_a_plain_stream_of_its_length():
    kv = np.zeros((2, 4, 2, 64), np.float32)
    st = oracle.Stream(1, 2, 64, 32, cache="bf16", act="bf16")
    with pytest.raises(oracle.OracleError, match="exactly as many rows"):
        st.load_kv(0, kv)
    st.advance(4)
    st.start_ring("absolute")
    with pytest.raises(oracle.OracleError, match="not a ring"):
        st.load_kv(0, kv)


# ---- Mimi's window cache (transformer.rs:257-318, 428-468, 764-781) ----------------------------
def _window_run(win, steps, rng, H, act):
    """Feed `steps` (rows per step) of seeded q, k, v through an oracle window; the outputs."""
    outs = []
    for t in steps:
        q, k, v = (rng.standard_normal((t, H, 64)).astype(np.float32) for _ in range(3))
        if act == "bf16":
            q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
        outs.append(win.attend(0, q, k, v))
        win.commit(t)
    return outs


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_a_window_wider_than_the_stream_is_plain_causal_attention(act):
    # With context above every position the mask is the causal one: the flow LM's linear cache
    # (pinned against textbook attention above) gives the same outputs bit for bit.
    steps = [3, 1, 1, 2, 1, 4] + [1] * 10
    win = oracle.Window(1, 2, 64, 200, act=act)
    st = oracle.Stream(1, 2, 64, 64, cache=act, act=act)
    got = _window_run(win, steps, np.random.default_rng(40), 2, act)
    rng = np.random.default_rng(40)
    for t, (o, _) in zip(steps, got):
        q, k, v = (rng.standard_normal((t, 2, 64)).astype(np.float32) for _ in range(3))
        if act == "bf16":
            q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
        want, _ = st.attend(0, q, k, v)
        st.commit(t)
        assert np.array_equal(o.view(np.uint32), want.view(np.uint32))
    n = sum(steps)
    assert win.len == n and win.offset == n
    np.testing.assert_array_equal(win.rows(0, 0), st.read_rows(0, 0, 0, n)[0])


def test_a_window_matches_textbook_windowed_attention():
    # f64 RoPE from math.cos/sin at absolute positions, then softmax over keys p - context < j <= p
    context, H = 5, 2
    steps = [1, 2, 1, 3, 1, 1, 2, 1, 1, 1, 3]
    win = oracle.Window(1, H, 64, context, act="f32")
    rng = np.random.default_rng(41)
    inv = np.array([THETA ** (-i / 32) for i in range(32)])

    def rot(x, pos):
        a = pos * inv
        c, s_ = np.cos(a), np.sin(a)
        x0, x1 = x[..., 0::2].astype(np.float64), x[..., 1::2].astype(np.float64)
        y = np.empty(x.shape, np.float64)
        y[..., 0::2], y[..., 1::2] = x0 * c - x1 * s_, x0 * s_ + x1 * c
        return y

    keys, vals, p = [], [], 0
    for t in steps:
        q, k, v = (rng.standard_normal((t, H, 64)).astype(np.float32) for _ in range(3))
        _, out64 = win.attend(0, q, k, v, scale=0.125)
        win.commit(t)
        for i in range(t):
            keys.append(rot(k[i], p + i))
            vals.append(v[i].astype(np.float64))
        for i in range(t):
            pos = p + i
            lo = max(0, pos - context + 1)
            K, V = np.stack(keys[lo:pos + 1]), np.stack(vals[lo:pos + 1])  # [n][H][D]
            sc = np.einsum("hd,nhd->hn", rot(q[i], pos), K) * 0.125
            w = np.exp(sc - sc.max(axis=1, keepdims=True))
            w /= w.sum(axis=1, keepdims=True)
            want = np.einsum("hn,nhd->hd", w, V)
            assert rel_err(out64[i], want) <= 1e-5, (p, i)
        p += t
    assert win.len == context - 1 and win.offset == p


def test_a_chunk_attends_as_its_rows_one_at_a_time():
    # Row i of a chunk sees what it would see as a step of its own, so a chunk of 3 equals three
    # single rows, bit for bit, and leaves the same kept rows.
    a = oracle.Window(1, 2, 64, 6, act="bf16")
    b = oracle.Window(1, 2, 64, 6, act="bf16")
    ra, rb = np.random.default_rng(42), np.random.default_rng(42)
    for _ in range(7):
        qa, ka, va = (bf16_round(ra.standard_normal((3, 2, 64)).astype(np.float32)) for _ in range(3))
        qb, kb, vb = (bf16_round(rb.standard_normal((3, 2, 64)).astype(np.float32)) for _ in range(3))
        oa, _ = a.attend(0, qa, ka, va)
        a.commit(3)
        for i in range(3):
            ob, _ = b.attend(0, qb[i:i + 1], kb[i:i + 1], vb[i:i + 1])
            b.commit(1)
            assert np.array_equal(oa[i].view(np.uint32), ob[0].view(np.uint32))
    assert a.len == b.len == 5
    np.testing.assert_array_equal(a.rows(0, 1), b.rows(0, 1))


# ---- the rest of the layer (transformer.rs:591-634) -------------------------------------------
def test_layer_norm_matches_torch():
    # torch.nn.functional.layer_norm in f64 is the textbook definition (biased variance, eps inside
    # the root, affine after); a constant row normalizes to the bias exactly.
    rng = np.random.default_rng(40)
    x = rng.standard_normal((7, 512)).astype(np.float32) * 3 + 1
    w = rng.standard_normal(512).astype(np.float32)
    b = rng.standard_normal(512).astype(np.float32)
    got = oracle.layer_norm(x, w, b)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (512,), torch.from_numpy(w).double(),
                                          torch.from_numpy(b).double(), eps=1e-5).numpy()
    assert rel_err(got, want) < 2e-6
    const = oracle.layer_norm(np.full((2, 512), 4.25, np.float32), w, b)
    assert np.array_equal(const, np.stack([b, b]))
    got16 = oracle.layer_norm(x, w, b, act="bf16")
    assert np.array_equal(got16, bf16_round(got))


def test_quantize_rows_keeps_every_weight_within_half_a_step():
    rng = np.random.default_rng(41)
    w = rng.standard_normal((33, 100)).astype(np.float32) * 0.02
    w[5] = 0.0
    q, s = oracle.quantize_rows(w)
    assert s[5] == 0 and not q[5].any()
    live = np.arange(33) != 5
    assert np.allclose(s[live], np.abs(w[live]).max(axis=1) / 127, rtol=1e-7)
    assert (np.abs(q[live]).max(axis=1) == 127).all()
    err = np.abs(w[live] - q[live].astype(np.float64) * s[live, None])
    assert (err <= s[live, None] / 2 * (1 + 1e-6)).all()


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_linear_q8_is_the_matmul_with_the_dequantized_weights(act):
    rng = np.random.default_rng(42)
    x = normal(rng, (9, 512), act)
    q, s = oracle.quantize_rows(rng.standard_normal((96, 512)).astype(np.float32) * 0.02)
    got = oracle.linear_q8(x, q, s, act)
    want = x.astype(np.float64) @ (q.astype(np.float64) * s[:, None].astype(np.float64)).T
    assert rel_err(got, want) < (1e-5 if act == "f32" else 2 ** -8)


@pytest.mark.parametrize("kind", ["erf", "tanh"])
def test_gelu_matches_torch(kind):
    x = np.linspace(-6, 6, 241, dtype=np.float32)
    want = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="none" if kind == "erf" else "tanh")
    got = np.array([oracle.gelu(float(v), kind) for v in x])
    assert np.abs(got - want.numpy()).max() < 2e-6


def _torch_layer(x, hist, layer_w, pos, H, KVH, D, theta=THETA):
    """The layer (transformer.rs:591-634) in torch f64 from library routines: layer_norm, matmul,
    gelu, softmax; RoPE with the pinned rope rows; hist holds the rotated K and V rows so far."""
    t64 = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    W = layer_w
    deq = lambda q, s: t64(q) * t64(s)[:, None]
    X = t64(x)
    T = X.shape[0]
    h = torch.nn.functional.layer_norm(X, (X.shape[1],), t64(W.ln1_w), t64(W.ln1_b), eps=1e-5)
    qkv = h @ deq(W.wqkv, W.sqkv).T
    q = qkv[:, :H * D].reshape(T, H, D)
    k = qkv[:, H * D:H * D + KVH * D].reshape(T, KVH, D).repeat_interleave(H // KVH, dim=1)
    v = qkv[:, H * D + KVH * D:].reshape(T, KVH, D).repeat_interleave(H // KVH, dim=1)

    def rope(a, p):
        c, s = oracle.rope_row(D, theta, float(p), "f32")
        c, s = t64(c), t64(s)
        out = a.clone()
        out[..., 0::2] = a[..., 0::2] * c - a[..., 1::2] * s
        out[..., 1::2] = a[..., 0::2] * s + a[..., 1::2] * c
        return out

    q = torch.stack([rope(q[i], pos + i) for i in range(T)])
    k = torch.stack([rope(k[i], pos + i) for i in range(T)])
    hist["k"] = torch.cat([hist["k"], k]) if "k" in hist else k
    hist["v"] = torch.cat([hist["v"], v]) if "v" in hist else v
    K, V = hist["k"], hist["v"]
    n = K.shape[0]
    att = torch.einsum("thd,nhd->thn", q, K) * (1.0 / math.sqrt(D))
    causal = torch.arange(n)[None, :] <= (n - T + torch.arange(T))[:, None]
    att = att.masked_fill(~causal[:, None, :], float("-inf")).softmax(-1)
    o = torch.einsum("thn,nhd->thd", att, V).reshape(T, H * D)
    X = X + o @ deq(W.wout, W.sout).T
    h2 = torch.nn.functional.layer_norm(X, (X.shape[1],), t64(W.ln2_w), t64(W.ln2_b), eps=1e-5)
    f = torch.nn.functional.gelu(h2 @ deq(W.w1, W.s1).T, approximate="none")
    X = X + f @ deq(W.w2, W.s2).T
    return X.numpy()


def random_layer_weights(rng, d_model=512, H=8, KVH=8, D=64, ff=2048, std=0.02):
    qr = lambda n, k: oracle.quantize_rows(rng.standard_normal((n, k)).astype(np.float32) * std)
    wqkv, sqkv = qr((H + 2 * KVH) * D, d_model)
    wout, sout = qr(d_model, H * D)
    w1, s1 = qr(ff, d_model)
    w2, s2 = qr(d_model, ff)
    g = lambda: (1 + 0.1 * rng.standard_normal(d_model)).astype(np.float32)
    b = lambda: (0.1 * rng.standard_normal(d_model)).astype(np.float32)
    return oracle.LayerWeights(wqkv, sqkv, wout, sout, w1, s1, w2, s2, g(), b(), g(), b())


@pytest.mark.parametrize("KVH", [8, 2])
def test_layer_step_is_the_reference_layer(KVH):
    # a 6-row prompt, then 3 single-row steps, on two streams; f32 activations and cache
    rng = np.random.default_rng(43 + KVH)
    H, D, dm = 8, 64, 512
    W = random_layer_weights(rng, H=H, KVH=KVH, ff=1024)
    sts = [oracle.Stream(1, H, D, 64, cache="f32", act="f32", kv_heads=KVH) for _ in range(2)]
    hists = [{}, {}]
    pos = 0
    for t in (6, 1, 1, 1):
        x = rng.standard_normal((2, t, dm)).astype(np.float32)
        got = oracle.layer_step(sts, 0, W, x)
        for i in range(2):
            want = _torch_layer(x[i], hists[i], W, pos, H, KVH, D)
            assert rel_err(got[i], want) < 2e-5, (t, i)
        oracle.batch_commit_t(sts, t)
        pos += t


# ---- the flow LM around the transformer (flow_lm.rs, mlp.rs, conditioners.rs) -------------------
flow_lm = __import__("xn_ptts_amd.flow_lm", fromlist=["flow_lm"])


def _small_flow_cfg(**kw):
    base = dict(d_model=512, num_heads=8, num_layers=2, dim_feedforward=1024, ldim=32, n_bins=100,
                flow_dim=256, flow_depth=2, lsd_decode_steps=1)
    base.update(kw)
    return flow_lm.FlowLMConfig(**base)


def _t(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def _torch_time_embed(W, i, t, kind):
    p = f"time_embed.{i}."
    args = t * _t(W[p + "freqs"])
    emb = torch.cat([torch.cos(args), torch.sin(args)])
    h = torch.nn.functional.silu(torch.nn.functional.linear(emb, _t(W[p + "mlp0.w"]), _t(W[p + "mlp0.b"])))
    h = torch.nn.functional.linear(h, _t(W[p + "mlp2.w"]), _t(W[p + "mlp2.b"]))
    if kind == "rms":
        return torch.nn.functional.rms_norm(h, (h.shape[-1],), _t(W[p + "alpha"]), eps=1e-5)
    return h / torch.sqrt(torch.var(h, unbiased=True) + 1e-5) * _t(W[p + "alpha"])


def _torch_flow_net(W, cfg, c, temb, x0):
    lin = lambda x, n: torch.nn.functional.linear(x, _t(W[n + ".w"]), _t(W[n + ".b"]))
    F = cfg.flow_dim
    x = lin(_t(x0), "input_proj")
    y = lin(c, "cond_embed")
    ya = torch.nn.functional.silu(y if temb is None else temb + y)  # no time conditions: c alone
    for j in range(cfg.flow_depth):
        p = f"res_blocks.{j}."
        ada = lin(ya, p + "ada")
        h = torch.nn.functional.layer_norm(x, (F,), _t(W[p + "in_ln.w"]), _t(W[p + "in_ln.b"]), eps=1e-6)
        h = h * (1 + ada[F:2 * F]) + ada[:F]
        h = lin(torch.nn.functional.silu(lin(h, p + "mlp0")), p + "mlp2")
        x = x + ada[2 * F:] * h
    ada = lin(ya, "final.ada")
    h = torch.nn.functional.layer_norm(x, (F,), eps=1e-6) * (1 + ada[F:]) + ada[:F]
    return lin(h, "final.linear")


@pytest.mark.parametrize("kind", ["rms", "rms_var"])
def test_flow_time_embedding_matches_torch(kind):
    cfg = _small_flow_cfg(time_rms_norm=kind)
    blob = flow_lm.random_weights(cfg, 80, unit_norms=False)
    W = flow_lm.split(cfg, blob)
    m = oracle.FlowLM(cfg, blob)
    for s, t in [(0.0, 1.0), (0.25, 0.5)]:
        want = (_torch_time_embed(W, 0, s, kind) + _torch_time_embed(W, 1, t, kind)) / 2
        assert rel_err(m.time_embedding(s, t), want.numpy()) < 1e-5


def test_flow_net_matches_torch():
    cfg = _small_flow_cfg()
    blob = flow_lm.random_weights(cfg, 81, std=0.05, unit_norms=False)
    W = flow_lm.split(cfg, blob)
    m = oracle.FlowLM(cfg, blob)
    rng = np.random.default_rng(82)
    c, x0 = rng.standard_normal(cfg.d_model), rng.standard_normal(cfg.ldim)
    temb = m.time_embedding(0.0, 1.0)
    want = _torch_flow_net(W, cfg, _t(c), _t(temb), x0)
    assert rel_err(m.flow_net(c, temb, x0), want.numpy()) < 1e-5


def _torch_flow_lm(cfg, W, ids, frames, noise, cond=None):
    """prompt_text then `frames` generate steps (flow_lm.rs:296-432, tts_model.rs:297-378) in torch f64;
    cond [frames][d_model]: the conditions added to each step's input (flow_lm.rs:304-307)."""
    H, dm = cfg.num_heads, cfg.d_model
    ad = cfg.attn_dim or dm  # StreamingMultiheadAttention::load (transformer.rs:155-166)
    KVH = cfg.num_kv_heads or H
    D, kd = ad // H, ad // H * KVH
    hist = [{} for _ in range(cfg.num_layers)]

    def rope(a, p):
        c, s = oracle.rope_row(D, cfg.max_period, float(p), "f32")
        out = a.clone()
        out[..., 0::2] = a[..., 0::2] * _t(c) - a[..., 1::2] * _t(s)
        out[..., 1::2] = a[..., 0::2] * _t(s) + a[..., 1::2] * _t(c)
        return out

    def transformer(x, pos):
        T = x.shape[0]
        for l in range(cfg.num_layers):
            p = f"layers.{l}."
            h = torch.nn.functional.layer_norm(x, (dm,), _t(W[p + "norm1.w"]), _t(W[p + "norm1.b"]), eps=1e-5)
            qkv = h @ _t(W[p + "in_proj"]).T
            q = qkv[:, :ad].reshape(T, H, D)  # then each kv head serves H / KVH query heads (:199-211)
            k = qkv[:, ad:ad + kd].reshape(T, KVH, D).repeat_interleave(H // KVH, dim=1)
            v = qkv[:, ad + kd:].reshape(T, KVH, D).repeat_interleave(H // KVH, dim=1)
            q = torch.stack([rope(q[i], pos + i) for i in range(T)])
            k = torch.stack([rope(k[i], pos + i) for i in range(T)])
            hs = hist[l]
            hs["k"] = torch.cat([hs["k"], k]) if "k" in hs else k
            hs["v"] = torch.cat([hs["v"], v]) if "v" in hs else v
            n = hs["k"].shape[0]
            att = torch.einsum("thd,nhd->thn", q, hs["k"]) / math.sqrt(D)
            causal = torch.arange(n)[None, :] <= (n - T + torch.arange(T))[:, None]
            att = att.masked_fill(~causal[:, None, :], float("-inf")).softmax(-1)
            x = x + torch.einsum("thn,nhd->thd", att, hs["v"]).reshape(T, ad) @ _t(W[p + "out_proj"]).T
            h = torch.nn.functional.layer_norm(x, (dm,), _t(W[p + "norm2.w"]), _t(W[p + "norm2.b"]), eps=1e-5)
            f = torch.nn.functional.gelu(h @ _t(W[p + "linear1"]).T)
            x = x + f @ _t(W[p + "linear2"]).T
        return x

    transformer(_t(W["conditioner.embed"][ids]), 0)
    pos, latent, outs = len(ids), _t(W["bos_emb"]), []
    lsd = cfg.flow_type == "lsd"
    assert not lsd or cfg.lsd_decode_steps == 1
    temb = None
    if lsd:
        temb = (_torch_time_embed(W, 0, 0.0, cfg.time_rms_norm) + _torch_time_embed(W, 1, 1.0, cfg.time_rms_norm)) / 2
    for f in range(frames):
        inp = _t(W["input_linear"]) @ latent
        if cond is not None:
            inp = inp + _t(cond[f])
        x = transformer(inp[None, :], pos)[0]
        pos += 1
        t_out = torch.nn.functional.layer_norm(x, (dm,), _t(W["out_norm.w"]), _t(W["out_norm.b"]), eps=1e-5)
        if cfg.z_dim:  # z_proj, bias-free (flow_lm.rs:320-323)
            t_out = _t(W["z_proj"]) @ t_out
        eos = float(_t(W["out_eos.w"])[0] @ t_out + _t(W["out_eos.b"])[0])
        v = _torch_flow_net(W, cfg, t_out, temb, noise[f])
        # one LSD step: noise + v / 1; Drifting: v; Pointwise: noise + v (flow_lm.rs:372-381)
        latent = v if cfg.flow_type == "drifting" else _t(noise[f]) + v
        outs.append((latent.numpy().copy(), eos))
    return outs


@pytest.mark.parametrize("flow_type,z_dim,extra", [
    ("lsd", 0, {}), ("lsd", 48, {}), ("drifting", 0, {}), ("pointwise", 32, {}),
    ("lsd", 0, dict(num_kv_heads=2, cond=True)),                    # grouped heads, conditions
    ("pointwise", 32, dict(num_heads=4, attn_dim=256, num_kv_heads=1, cond=True))])  # attn_dim < d_model
def test_flow_lm_prompt_and_frames_match_torch(flow_type, z_dim, extra):
    # a 5-token prompt, then 4 frames (from bos_emb, then each frame's latent), noise N(0, 0.5);
    # with conditions, a different condition row N(0, 0.5) added to each frame's input
    extra = dict(extra)
    with_cond = extra.pop("cond", False)
    cfg = _small_flow_cfg(flow_type=flow_type, z_dim=z_dim, **extra)
    blob = flow_lm.random_weights(cfg, 83, std=0.05, unit_norms=False)
    W = flow_lm.split(cfg, blob)
    m = oracle.FlowLM(cfg, blob)
    rng = np.random.default_rng(84)
    ids = rng.integers(0, cfg.n_bins + 1, 5)
    noise = (0.5 * rng.standard_normal((4, cfg.ldim))).astype(np.float32)
    cond = (0.5 * rng.standard_normal((4, cfg.d_model))).astype(np.float32) if with_cond else None
    want = _torch_flow_lm(cfg, W, ids, 4, noise, cond)
    st = m.stream(32)
    m.prompt_text(st, ids)
    lat = None
    for f in range(4):
        lat, eos = m.step(st, lat, noise[f], cond=None if cond is None else cond[f])
        wl, we = want[f]
        assert rel_err(lat, wl) < 2e-5, f
        assert abs(eos - we) <= 2e-5 * max(1.0, abs(we)), f
    assert st.current_end == 9


def _q8_exact(cfg, blob):
    """The blob with every linear's rows replaced by their int8 dequantization, so that quantizing
    it again gives the same codes: the q8 precision then differs from f32 only in its bf16 rounding."""
    blob = blob.copy()
    W = flow_lm.split(cfg, blob)
    for name, t in W.items():  # every linear the q8 precision quantizes: not the LUT, not the time embedders
        if t.ndim == 2 and name != "conditioner.embed" and not name.startswith("time_embed"):
            q, s = oracle.quantize_rows(t)
            t[:] = q.astype(np.float32) * s[:, None]
    return blob


@pytest.mark.parametrize("flow_type,z_dim,extra", [("lsd", 0, {}), ("pointwise", 64, {}),
                                                   ("lsd", 0, dict(num_heads=4, attn_dim=256, num_kv_heads=2, cond=True))])
def test_q8_flow_lm_is_the_f32_one_within_bf16_rounding(flow_type, z_dim, extra):
    # The q8 precision on weights its quantization reproduces exactly, against the f32 path (pinned
    # against torch above): only the bf16 rounding of every activation separates them.  With grouped
    # heads, an attention narrower than d_model and a condition row added to every frame's input.
    extra = dict(extra)
    with_cond = extra.pop("cond", False)
    kw = dict(d_model=512, num_heads=8, num_layers=2, dim_feedforward=1024, flow_dim=512, flow_depth=2, n_bins=50,
              flow_type=flow_type, z_dim=z_dim)
    kw.update(extra)
    c32 = flow_lm.FlowLMConfig(**kw)
    cq8 = flow_lm.FlowLMConfig(**kw, precision="q8")
    blob = _q8_exact(c32, flow_lm.random_weights(c32, 85, std=0.05, unit_norms=False))
    f32, q8 = oracle.FlowLM(c32, blob), oracle.FlowLM(cq8, blob)
    s32, sq8 = f32.stream(64), q8.stream(64)
    rng = np.random.default_rng(86)
    ids = rng.integers(0, 51, 6)
    f32.prompt_text(s32, ids)
    q8.prompt_text(sq8, ids)
    lat = None
    worst = 0.0
    for f in range(8):
        noise = (0.5 * rng.standard_normal(c32.ldim)).astype(np.float32)
        cond = bf16_round(0.5 * rng.standard_normal(c32.d_model)) if with_cond else None
        want, we = f32.step(s32, lat, noise, cond=cond)
        got, ge = q8.step(sq8, lat, noise, cond=cond)  # both from the f32 path's latent: no drift between them
        err = rel_err(got, want)
        worst = max(worst, err)
        assert err < 4e-2, (f, err)
        assert abs(ge - we) <= 4e-2 * max(1.0, abs(we)), (f, ge, we)
        assert np.array_equal(got, bf16_round(got))  # q8 latents are bf16 values
        lat = want
    assert worst > 1e-4  # the precisions do differ: the q8 path is not the f32 one


def _ulps(got, want):
    """|got - want| in units of the bf16 spacing at want (both bf16 values)."""
    want64 = np.abs(want.astype(np.float64))
    spacing = np.exp2(np.floor(np.log2(np.maximum(want64, 1e-30))) - 7)
    return np.abs(got.astype(np.float64) - want) / spacing


def test_flow_linear_q8_and_its_epilogues_match_torch_bf16_ops():
    # y against an f64 product rounded by torch's cast; each epilogue against the same operation on
    # torch bf16 tensors, which round every result once, from the oracle's own y
    rng = np.random.default_rng(87)
    rows, k, n = 9, 48, 40
    x = bf16_round(rng.standard_normal((rows, k)).astype(np.float32))
    q, s = oracle.quantize_rows(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    bt = lambda a: torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)
    y = oracle.flow_linear_q8(x, q, s, "store", bias=b)
    ref = (torch.from_numpy(x.astype(np.float64)) @ torch.from_numpy(q.astype(np.float64) * s[:, None].astype(np.float64)).T
           + torch.from_numpy(b.astype(np.float64))).to(torch.bfloat16).float().numpy()
    assert (_ulps(y, ref) <= 1).all() and (y == ref).mean() > 0.97
    assert np.array_equal(oracle.flow_linear_q8(x, q, s, "store_f32", bias=b), y)
    yt = bt(y)
    f = lambda t: t.float().numpy()
    got = oracle.flow_linear_q8(x, q, s, "silu", bias=b)
    assert (_ulps(got, f(torch.nn.functional.silu(yt))) <= 1).all()
    temb = bf16_round(rng.standard_normal(n).astype(np.float32))
    got = oracle.flow_linear_q8(x, q, s, "silu_add", bias=b, aux=temb)
    assert (_ulps(got, f(torch.nn.functional.silu(yt + bt(temb)))) <= 1).all()
    gate = bf16_round(rng.standard_normal((rows, n)).astype(np.float32))
    x0 = bf16_round(rng.standard_normal((rows, n)).astype(np.float32))
    got = oracle.flow_linear_q8(x, q, s, "gated", bias=b, aux=gate, out=x0)
    assert np.array_equal(got, f(bt(x0) + bt(gate) * yt))
    cur = rng.standard_normal((rows, n)).astype(np.float32)
    got = oracle.flow_linear_q8(x, q, s, "axpy_f32", bias=b, aux=cur, alpha=0.25)
    assert np.array_equal(got, f(bt(cur) + yt * 0.25))


def test_layer_norm_mod_matches_torch_bf16_ops():
    rng = np.random.default_rng(88)
    rows, dim = 6, 512
    x = bf16_round((2 + 3 * rng.standard_normal((rows, dim))).astype(np.float32))
    w, b = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32), (0.1 * rng.standard_normal(dim)).astype(np.float32)
    mod = bf16_round(rng.standard_normal((rows, 3 * dim)).astype(np.float32))
    shift, scale = mod[:, :dim], mod[:, dim:2 * dim]
    bt = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)
    ln = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), (dim,), torch.from_numpy(w.astype(np.float64)),
                                        torch.from_numpy(b.astype(np.float64)), eps=1e-6).to(torch.bfloat16)
    want = ((ln * (bt(scale) + 1)) + bt(shift)).float().numpy()
    got = oracle.layer_norm_mod(x, w, b, shift, scale)
    assert (_ulps(got, want) <= 1).all() and (got == want).mean() > 0.97
    ln0 = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), (dim,), eps=1e-6).to(torch.bfloat16)
    got = oracle.layer_norm_mod(x, shift=shift, scale=scale)
    assert (_ulps(got, ((ln0 * (bt(scale) + 1)) + bt(shift)).float().numpy()) <= 1).all()
