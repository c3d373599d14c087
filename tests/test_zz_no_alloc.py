"""GPU test of xnp_layer_step_static, the layer step that takes its scratch from the library's static
device array instead of a caller's workspace: through the C ABI, its outputs and cache rows equal
xnp_layer_step's bit for bit (the same kernels on the same inputs), over two calls in a row, the
second with a smaller batch; a step too large for the array is refused and changes nothing.
"""
import numpy as np
import pytest
import torch

from conftest import xnp
from helpers import normal

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
L, H, D, DM, FF = 2, 8, 64, 512, 2048


def dev(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dtype)


def weights(rng):
    qr = lambda n, k: xnp.quantize_rows(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
    parts = dict(zip(["wqkv", "sqkv"], qr(3 * H * D, DM)))
    parts.update(zip(["wout", "sout"], qr(DM, H * D)))
    parts.update(zip(["w1", "s1"], qr(FF, DM)))
    parts.update(zip(["w2", "s2"], qr(DM, FF)))
    for n in ("ln1", "ln2"):
        parts[n + "_w"] = (1 + 0.1 * rng.standard_normal(DM)).astype(np.float32)
        parts[n + "_b"] = (0.1 * rng.standard_normal(DM)).astype(np.float32)
    d = {k: dev(v, torch.int8 if v.dtype == np.int8 else torch.float32) for k, v in parts.items()}
    return xnp.LayerWeights(**d)


def make_pool(S, cap):
    return xnp.KvPool(num_layers=L, num_heads=H, num_blocks=S * (cap // 16) + 8, max_streams=S,
                      max_blocks_per_stream=cap // 16, cache_dtype="bf16", act_dtype="bf16", max_pos=cap + 16,
                      page_seed=7)


def read_all(pool, sid, n):
    out = []
    for layer in range(L):
        for kv in (0, 1):
            rows = torch.empty((n, H, D), dtype=torch.bfloat16, device=DEV)
            pool.read_rows(sid, layer, kv, 0, rows)
            out.append(rows)
    torch.cuda.synchronize()
    return [r.view(torch.int16).cpu().numpy() for r in out]


def test_the_static_scratch_step_equals_the_workspace_step_twice_then_smaller():
    rng = np.random.default_rng(20261207)
    W = [weights(rng) for _ in range(L)]
    S, cap = 48, 512
    a, b = make_pool(S, cap), make_pool(S, cap)
    ia = [a.init_state(cap) for _ in range(S)]
    ib = [b.init_state(cap) for _ in range(S)]
    lens = rng.integers(0, 300, S)
    for i, n in enumerate(lens.tolist()):  # the same histories in both pools
        if n == 0:
            continue
        for pool, ids in ((a, ia), (b, ib)):
            pool.advance(ids[i], n)
        for layer in range(L):
            kv = torch.from_numpy(rng.standard_normal((2, n, H, D)).astype(np.float32)).to(DEV)
            a.load_kv(ia[i], layer, kv)
            b.load_kv(ib[i], layer, kv)
        torch.cuda.synchronize()
    ws = torch.empty(a.layer_workspace(S * 4, DM, FF), dtype=torch.uint8, device=DEV)
    # a prompt of 4 rows on every stream, then one row on a smaller batch: the second call reads a
    # static scratch that still holds the first call's contents
    for batch, t in ((list(range(S)), 4), (list(range(0, S, 5)), 1)):
        x0 = normal(rng, (len(batch), t, DM), "bf16")
        xa, xb = dev(x0), dev(x0)
        a.begin([ia[i] for i in batch], t=t)
        b.begin([ib[i] for i in batch], t=t)
        for layer in range(L):
            a.layer_step(layer, W[layer], xa, ws)
            b.layer_step_static(layer, W[layer], xb)
        a.end()
        b.end()
        torch.cuda.synchronize()
        assert torch.equal(xa.view(torch.int16), xb.view(torch.int16)), (len(batch), t)
    for i in range(S):
        n = a.info(ia[i])["current_end"]
        assert n == b.info(ib[i])["current_end"]
        for ra, rb in zip(read_all(a, ia[i], n), read_all(b, ib[i], n)):
            assert np.array_equal(ra, rb), i


def test_a_step_too_large_for_the_static_scratch_is_refused_and_changes_nothing():
    rng = np.random.default_rng(20261208)
    W = [weights(rng) for _ in range(L)]
    S, cap, t = 64, 64, 48  # 3072 rows: about 27 MiB of scratch, more than the array holds
    pool = make_pool(S, cap)
    ids = [pool.init_state(cap) for _ in range(S)]
    x = dev(normal(rng, (S, t, DM), "bf16"))
    before = x.clone()
    pool.begin(ids, t=t)
    with pytest.raises(xnp.XnpError) as e:
        pool.layer_step_static(0, W[0], x)
    assert e.value.name == "XNP_E_INVALID" and "static scratch" in e.value.message
    pool.abort()
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int16), before.view(torch.int16))
    assert all(pool.info(i)["current_end"] == 0 for i in ids)


def test_a_call_that_fails_inside_the_step_lets_go_of_the_static_scratch():
    # A call holds the device's array from its claim to its release, so that no other call (another
    # host thread's, on any stream) interleaves launches with it.  A call that fails after its claim
    # (no batch open; a layer out of range) releases it too: the next call takes it and its step
    # equals the workspace step of an identical pool.
    rng = np.random.default_rng(20261210)
    W = [weights(rng) for _ in range(L)]
    S, cap = 8, 64
    a, c = make_pool(S, cap), make_pool(S, cap)
    ia, ic = ([p.init_state(cap) for _ in range(S)] for p in (a, c))
    x0 = normal(rng, (S, 1, DM), "bf16")
    xa, xc = dev(x0), dev(x0)
    torch.cuda.synchronize()
    a.begin(ia, t=1)
    a.abort()
    with pytest.raises(xnp.XnpError) as e:
        a.layer_step_static(0, W[0], xa)  # no batch is open
    assert e.value.name == "XNP_E_STATE" and "no batch" in e.value.message
    a.begin(ia, t=1)
    with pytest.raises(xnp.XnpError) as e:
        a.layer_step_static(L, W[0], xa)  # no such layer
    assert e.value.name == "XNP_E_INVALID" and "layer" in e.value.message
    a.layer_step_static(0, W[0], xa)
    a.end()
    ws = torch.empty(c.layer_workspace(S, DM, FF), dtype=torch.uint8, device=DEV)
    c.begin(ic, t=1)
    c.layer_step(0, W[0], xc, ws)
    c.end()
    torch.cuda.synchronize()
    assert torch.equal(xa.view(torch.int16), xc.view(torch.int16))


def test_a_call_on_another_stream_is_refused_while_the_last_one_may_still_run():
    # One array per device: pool b's call on HIP stream B, made while pool a's call on stream A is
    # still queued behind a sleep, is refused (XNP_E_STATE) and runs nothing; once A's work is done,
    # B takes the array over, and its step equals the workspace step of a third, identical pool.
    rng = np.random.default_rng(20261209)
    W = [weights(rng) for _ in range(L)]
    S, cap = 8, 64
    a, b, c = make_pool(S, cap), make_pool(S, cap), make_pool(S, cap)
    ia, ib, ic = ([p.init_state(cap) for _ in range(S)] for p in (a, b, c))
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    xa = dev(normal(rng, (S, 1, DM), "bf16"))
    x0 = normal(rng, (S, 1, DM), "bf16")
    xb, xc = dev(x0), dev(x0)
    torch.cuda.synchronize()
    a.begin(ia, t=1, stream=sa.cuda_stream)
    with torch.cuda.stream(sa):
        torch.cuda._sleep(50_000_000)  # a bounded spin that keeps stream A busy for a while
    a.layer_step_static(0, W[0], xa)  # queued behind the spin
    b.begin(ib, t=1, stream=sb.cuda_stream)
    with pytest.raises(xnp.XnpError) as e:
        b.layer_step_static(0, W[0], xb)
    assert e.value.name == "XNP_E_STATE" and "another HIP stream" in e.value.message
    torch.cuda.synchronize()
    assert torch.equal(xb.view(torch.int16), dev(x0).view(torch.int16))  # nothing ran on B
    b.layer_step_static(0, W[0], xb)  # A's work is done: B takes the array over
    a.end()
    b.end()
    ws = torch.empty(c.layer_workspace(S, DM, FF), dtype=torch.uint8, device=DEV)
    c.begin(ic, t=1)
    c.layer_step(0, W[0], xc, ws)
    c.end()
    torch.cuda.synchronize()
    assert torch.equal(xb.view(torch.int16), xc.view(torch.int16))
