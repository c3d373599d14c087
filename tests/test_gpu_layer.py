"""GPU parity of the rest of the flow-LM layer (transformer.rs:591-634): LayerNorm, the q8
projections and a whole layer step, through the C ABI, against the oracle on the same inputs.

Bars: 2e-2 relative (bf16 activations; relative error per row as in tests/helpers.py:rel_err).
Cache rows written by a layer step come from projections the GPU sums in its own order, so they
are compared within the same bar rather than bit for bit (the append's own bit-exactness is pinned
in test_gpu_parity.py with identical inputs).
"""
import numpy as np
import pytest
import torch

from conftest import oracle, xnp
from helpers import bf16_round, normal, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


def dev(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dtype)


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("rows,dim", [(1, 512), (37, 512), (130, 1024), (9, 2048)])
def test_layer_norm_matches_the_oracle(rows, dim):
    rng = np.random.default_rng(50 + rows)
    x = normal(rng, (rows, dim), "bf16") * 3 + 0.5
    x = bf16_round(x)
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    b = (0.1 * rng.standard_normal(dim)).astype(np.float32)
    out = torch.empty((rows, dim), dtype=torch.bfloat16, device=DEV)
    xnp.layer_norm(dev(x), dev(w, torch.float32), dev(b, torch.float32), out)
    torch.cuda.synchronize()
    assert rel_err(host(out), oracle.layer_norm(x, w, b, act="bf16")) <= TOL


@pytest.mark.parametrize("rows,k,n", [(1, 512, 64), (37, 512, 1536), (200, 512, 2048), (300, 1024, 512), (70, 2048, 512)])
@pytest.mark.parametrize("epi", ["store", "gelu_erf", "gelu_tanh", "residual"])
def test_linear_q8_matches_the_oracle(rows, k, n, epi):
    check_linear_q8(rows, k, n, epi)


@pytest.mark.parametrize("epi", ["store", "gelu_erf", "residual"])
def test_linear_q8_on_128_row_tiles_matches_the_oracle(epi):
    # Wide projections whose 128 x 64 tiles still make 512 work groups take 128-row tiles (linear1
    # at 2048 rows): here 257 column tiles by 2 row tiles, the last of one row.  Ragged N and K on
    # those tiles are in test_gpu_flow_pieces.py.
    check_linear_q8(129, 512, 16448, epi)


def check_linear_q8(rows, k, n, epi):
    rng = np.random.default_rng(rows * 7 + n)
    x = normal(rng, (rows, k), "bf16")
    q, s = xnp.quantize_rows(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
    y0 = normal(rng, (rows, n), "bf16")
    y = dev(y0)
    ls = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32) if epi == "residual" else None
    xnp.linear_q8(dev(x), dev(q, torch.int8), dev(s, torch.float32), y, epi,
                  ls=dev(ls, torch.float32) if ls is not None else None)
    torch.cuda.synchronize()
    want = oracle.linear_q8(x, q, s, "bf16")
    if epi.startswith("gelu"):
        kind = epi.split("_")[1]
        want = bf16_round(np.vectorize(lambda v: oracle.gelu(float(v), kind))(want).astype(np.float32))
    elif epi == "residual":
        want = bf16_round(y0 + bf16_round(want * ls[None, :]))
    assert rel_err(host(y), want) <= TOL, epi


def test_quantize_rows_matches_the_oracle_bit_for_bit():
    rng = np.random.default_rng(60)
    w = rng.standard_normal((70, 300)).astype(np.float32) * 0.02
    w[3] = 0
    q, s = xnp.quantize_rows(w)
    oq, os_ = oracle.quantize_rows(w)
    assert np.array_equal(q, oq) and np.array_equal(s.view(np.uint32), os_.view(np.uint32))


def make_weights(rng, H=8, KVH=8, D=64, dm=512, ff=2048, ls=False):
    qr = lambda n, k: xnp.quantize_rows(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
    parts = dict(zip(["wqkv", "sqkv"], qr((H + 2 * KVH) * D, dm)))
    parts.update(zip(["wout", "sout"], qr(dm, H * D)))
    parts.update(zip(["w1", "s1"], qr(ff, dm)))
    parts.update(zip(["w2", "s2"], qr(dm, ff)))
    for n in ("ln1", "ln2"):
        parts[n + "_w"] = (1 + 0.1 * rng.standard_normal(dm)).astype(np.float32)
        parts[n + "_b"] = (0.1 * rng.standard_normal(dm)).astype(np.float32)
    parts["ls1"] = (0.5 + 0.1 * rng.standard_normal(dm)).astype(np.float32) if ls else None
    parts["ls2"] = (0.5 + 0.1 * rng.standard_normal(dm)).astype(np.float32) if ls else None
    orc = oracle.LayerWeights(**parts)
    d = {k_: (dev(v, torch.int8 if v.dtype == np.int8 else torch.float32) if v is not None else None)
         for k_, v in parts.items()}
    return orc, xnp.LayerWeights(**d)


# ff 2048 (Phonon-40m's): linear2's K = 2048 runs the GEMM's two-half groups
@pytest.mark.parametrize("cache,KVH,ls,ff", [("bf16", 8, False, 1024), ("bf16", 2, True, 1024), ("i8", 8, False, 1024),
                                             ("bf16", 8, False, 2048)])
def test_layer_steps_match_the_oracle(cache, KVH, ls, ff):
    # 5 streams with prior caches of 0..40 rows; a 7-row prompt on all, then 3 single-row steps,
    # through 2 layers each
    rng = np.random.default_rng(61 + KVH + ff)
    L, H, D, dm = 2, 8, 64, 512
    W = [make_weights(rng, H=H, KVH=KVH, ff=ff, ls=ls) for _ in range(L)]
    S, cap = 5, 96
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_kv_heads=KVH, num_blocks=S * 8 + 8, max_streams=S,
                      max_blocks_per_stream=cap // 16, cache_dtype=cache, act_dtype="bf16", max_pos=256,
                      page_seed=12)
    ids = [pool.init_state(cap) for _ in range(S)]
    sts = [oracle.Stream(L, H, D, cap, cache=cache, act="bf16", kv_heads=KVH) for _ in range(S)]
    for i, n in enumerate([0, 5, 16, 40, 3]):
        if n == 0:
            continue
        pool.begin([ids[i]], t=n)
        for layer in range(L):
            k, v = normal(rng, (n, KVH, D), "bf16"), normal(rng, (n, KVH, D), "bf16")
            pool.append(layer, dev(k), dev(v))
            sts[i].append(layer, k, v)
        pool.end()
        sts[i].commit(n)
    ws = torch.empty(pool.layer_workspace(S * 7, dm, ff), dtype=torch.uint8, device=DEV)
    for t in (7, 1, 1, 1):
        x = normal(rng, (S, t, dm), "bf16")
        xg = dev(x)
        pool.begin(ids, t=t)
        want = x
        for layer in range(L):
            pool.layer_step(layer, W[layer][1], xg, ws)
            want = oracle.layer_step(sts, layer, W[layer][0], want)
        pool.end()
        torch.cuda.synchronize()
        for st in sts:
            st.commit(t)
        got = host(xg)
        for i in range(S):
            assert rel_err(got[i], want[i]) <= TOL, (t, i)
    # the cache rows the steps wrote, within the same bar
    for i in range(S):
        n = sts[i].current_end
        for layer in range(L):
            for kv in (0, 1):
                # the pool stores each kv head once; the oracle repeats it over its group
                rows = torch.empty((n, KVH, D), dtype=torch.bfloat16 if cache == "bf16" else torch.int8, device=DEV)
                nb = (n + 15) // 16
                sc = torch.zeros((nb, KVH), dtype=torch.float32, device=DEV)
                pool.read_rows(ids[i], layer, kv, 0, rows, sc if cache == "i8" else None)
                torch.cuda.synchronize()
                vals = sts[i].read_rows(layer, kv, 0, n)[0][:, ::H // KVH]
                if cache == "i8":
                    got_rows = rows.float().cpu().numpy() * np.repeat(sc.cpu().numpy(), 16, axis=0)[:n, :, None]
                    bar = 6e-2  # one int8 step of a row whose scale came from slightly different inputs
                else:
                    got_rows, bar = host(rows), TOL
                assert rel_err(got_rows, vals) <= bar, (i, layer, kv)


def test_the_layer_step_configuration_at_full_size_spot_checked():
    # The layer-step workload at its full size: 2048 streams x 9 Phonon-40m layers (512 wide, 8 heads
    # x 64, FF 2048, int8 per-channel projections), bf16 caches of U[1,1500] rows loaded as KV, one
    # single-row step through all 9 layers.  Every stream runs, and every stream's layer 0 goes
    # through the oracle's layer step on a one-layer cache of its own; 13 of them, spread over the
    # lengths (the longest and the shortest included), go through the oracle's layer step on all 9
    # layers (a layer is per row, and per stream for attention), each layer from the GPU's input to
    # it, so that every layer is held to the 2e-2 bar on its own.
    S, L, H, D, dm, ff, cap = 2048, 9, 8, 64, 512, 2048, 1504
    rng = np.random.default_rng(20261205)
    W = [make_weights(rng, ff=ff) for _ in range(L)]
    lens = rng.integers(1, 1501, S)
    order = np.argsort(-lens, kind="stable")
    sample = sorted(set(order[::200].tolist()) | {int(order[0]), int(order[-1])})
    mbps = cap // 16
    pool = xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * mbps + 8, max_streams=S, max_blocks_per_stream=mbps,
                      cache_dtype="bf16", act_dtype="bf16", max_pos=2048, page_seed=19)
    ids = [pool.init_state(cap) for _ in range(S)]
    sts = {i: oracle.Stream(L, H, D, cap, cache="bf16", act="bf16") for i in sample}
    every = [oracle.Stream(1, H, D, n + 2, cache="bf16", act="bf16") for n in lens.tolist()]
    g = torch.Generator(device=DEV).manual_seed(20261205)
    for i, n in enumerate(lens.tolist()):
        pool.advance(ids[i], n)
        every[i].advance(n)
        if i in sts:
            sts[i].advance(n)
        for layer in range(L):
            kv = torch.randn((2, n, H, D), device=DEV, generator=g)
            pool.load_kv(ids[i], layer, kv)
            if i in sts or layer == 0:
                kvh = host(kv)
                if layer == 0:
                    every[i].load_kv(0, kvh)
                if i in sts:
                    sts[i].load_kv(layer, kvh)
        torch.cuda.synchronize()  # the staged rows are freed on the next iteration
    ws = torch.empty(pool.layer_workspace(S, dm, ff), dtype=torch.uint8, device=DEV)
    xg = dev(normal(rng, (S, 1, dm), "bf16"))
    sub = [sts[i] for i in sample]
    pool.begin(ids, t=1)
    for layer in range(L):
        torch.cuda.synchronize()
        xall = host(xg)
        xin = xall[sample]
        pool.layer_step(layer, W[layer][1], xg, ws)
        want = oracle.layer_step(sub, layer, W[layer][0], xin)
        torch.cuda.synchronize()
        gall = host(xg)
        got = gall[sample]
        for j, i in enumerate(sample):
            assert rel_err(got[j], want[j]) <= TOL, (layer, i, int(lens[i]))
        if layer == 0:  # every stream
            wall = oracle.layer_step(every, 0, W[0][0], xall)
            per = np.abs(gall - wall).max(axis=-1) / np.maximum(np.abs(wall).max(axis=-1), 1e-30)
            worst = int(per.max(axis=-1).argmax())
            assert per.max() <= TOL, (worst, int(lens[worst]), float(per.max()))
    pool.end()
    assert pool.check_tables() == 0


@pytest.mark.parametrize("ls", [False, True])
def test_the_layer_step_equals_its_pieces_bit_for_bit(ls):
    # xnp_layer_step against the same layer composed of the public pieces on a second, identical
    # pool: layer_norm, linear_q8 (store, residual, gelu) and attend.  The step is those launches in
    # that order on its own workspace, so every bit must agree: the residual stream and the cache
    # rows compared as integers.  Row counts that no 16-row band divides (37 single rows, a 7-row
    # prompt on 5 streams), 300 rows, with and without layer scales.
    rng = np.random.default_rng(71 + ls)
    L, H, KVH, D, dm, ff = 1, 8, 8, 64, 512, 2048
    qd, kd = H * D, KVH * D
    orc, lw = make_weights(rng, H=H, KVH=KVH, ff=ff, ls=ls)
    dw = {k: dev(getattr(orc, k), torch.int8 if getattr(orc, k).dtype == np.int8 else torch.float32)
          for k in ("wqkv", "sqkv", "wout", "sout", "w1", "s1", "w2", "s2", "ln1_w", "ln1_b", "ln2_w", "ln2_b")}
    dw["ls1"] = dev(orc.ls1, torch.float32) if ls else None
    dw["ls2"] = dev(orc.ls2, torch.float32) if ls else None
    S, cap = 300, 48
    pools = [xnp.KvPool(num_layers=L, num_heads=H, num_kv_heads=KVH, num_blocks=S * (cap // 16) + 8, max_streams=S,
                        max_blocks_per_stream=cap // 16, cache_dtype="bf16", act_dtype="bf16", max_pos=256,
                        page_seed=13) for _ in range(2)]
    ids = [[p.init_state(cap) for _ in range(S)] for p in pools]
    ws = torch.empty(pools[0].layer_workspace(S * 7, dm, ff), dtype=torch.uint8, device=DEV)
    for which, t in ((list(range(37)), 1), (list(range(5)), 7), (list(range(S)), 1)):
        n, M = len(which), len(which) * t
        x0 = normal(rng, (n, t, dm), "bf16")
        xa, xb = dev(x0), dev(x0)
        pools[0].begin([ids[0][i] for i in which], t=t)
        pools[0].layer_step(0, lw, xa, ws)
        pools[0].end()
        pools[1].begin([ids[1][i] for i in which], t=t)
        h = torch.empty((M, dm), dtype=torch.bfloat16, device=DEV)
        qkv = torch.empty((M, qd + 2 * kd), dtype=torch.bfloat16, device=DEV)
        att = torch.empty((M, qd), dtype=torch.bfloat16, device=DEV)
        f = torch.empty((M, ff), dtype=torch.bfloat16, device=DEV)
        xv = xb.view(M, dm)
        xnp.layer_norm(xv, dw["ln1_w"], dw["ln1_b"], h)
        xnp.linear_q8(h, dw["wqkv"], dw["sqkv"], qkv, "store")
        q, k, v = (qkv[:, a:b].contiguous() for a, b in ((0, qd), (qd, qd + kd), (qd + kd, qd + 2 * kd)))
        pools[1].attend(0, q, k, v, att, 1.0 / np.sqrt(D))
        xnp.linear_q8(att, dw["wout"], dw["sout"], xv, "residual", ls=dw["ls1"])
        xnp.layer_norm(xv, dw["ln2_w"], dw["ln2_b"], h)
        xnp.linear_q8(h, dw["w1"], dw["s1"], f, "gelu_erf")
        xnp.linear_q8(f, dw["w2"], dw["s2"], xv, "residual", ls=dw["ls2"])
        pools[1].end()
        torch.cuda.synchronize()
        assert torch.equal(xa.view(torch.int16), xb.view(torch.int16)), (n, t)
    for i in (0, 4, 36, 299):
        n = pools[0].info(ids[0][i])["current_end"]
        for kv in (0, 1):
            got = [torch.empty((n, KVH, D), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
            for p, sid, r in zip(pools, (ids[0][i], ids[1][i]), got):
                p.read_rows(sid, 0, kv, 0, r)
            torch.cuda.synchronize()
            assert torch.equal(got[0].view(torch.int16), got[1].view(torch.int16)), (i, kv)
