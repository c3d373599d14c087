"""GPU parity of the flow LM around the transformer (flow_lm.rs, mlp.rs, conditioners.rs,
tts_model.rs:297-378), through the C ABI, against the oracle on the same weights, tokens and noise.

Bar: f32 precision (f32 kernels, f32 pool): 1e-5 relative (latents per frame, EOS logits against
max(1, |logit|)); cache rows come from projections the GPU sums in its own order, so they are held
to the same bar.  q8 precision (int8 weights on MFMA, bf16 activations and pool): 4e-2 relative,
each frame started from the oracle's previous latent.  Both sides round at the same points, but a
bf16 rounding that the GPU's summation order moves by one step (test_gpu_flow_pieces.py bounds how
often) reaches every later activation of a deep bf16 network, so the two frames differ as two bf16
evaluations do: as much as the q8 precision differs from f32 (1.4e-2 to 2.5e-2 in the oracle,
test_q8_flow_lm_is_the_f32_one_within_bf16_rounding).  A dropped term or a wrong sign moves them by
O(1).
"""
import numpy as np
import pytest
import torch

from conftest import oracle, xnp
from helpers import bf16_round, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
fl = xnp.flow_lm


def run_pair(cfg, blob, tokens, frames, noise, cap, cond=None, model_cond=None):
    """cond [frames][n][d_model]: each stream's conditions per frame; model_cond [d_model]: the
    model's (used when cond is None)."""
    n = tokens.shape[0]
    H = cfg.num_heads
    mbps = (cap + 15) // 16
    q8 = cfg.precision == "q8"
    dt = "bf16" if q8 else "f32"
    tol = 4e-2 if q8 else 1e-5
    pool = xnp.KvPool(num_layers=cfg.num_layers, num_heads=H, num_kv_heads=cfg.num_kv_heads or H,
                      num_blocks=n * mbps + 8, max_streams=n, max_blocks_per_stream=mbps, cache_dtype=dt, act_dtype=dt,
                      max_pos=cap + 16, page_seed=3)
    ids = [pool.init_state(cap) for _ in range(n)]
    lm = xnp.FlowLM(pool, cfg, blob, max_rows=n * tokens.shape[1])
    if model_cond is not None:
        lm.set_condition(model_cond)
    orc = oracle.FlowLM(cfg, blob)
    sts = [orc.stream(cap) for _ in range(n)]
    lm.prompt_text(ids, tokens)
    for i in range(n):
        orc.prompt_text(sts[i], tokens[i])
    lat_in = None
    out = torch.empty((n, cfg.ldim), dtype=torch.float32, device=DEV)
    eos = torch.empty(n, dtype=torch.float32, device=DEV)
    nz = torch.from_numpy(noise).to(DEV)
    want_lat = [None] * n
    worst = 0.0
    cdev = None if cond is None else torch.from_numpy(np.ascontiguousarray(cond, np.float32)).to(DEV)
    for f in range(frames):
        lm.step(ids, lat_in, nz[f], out, eos, conditions=None if cdev is None else cdev[f])
        torch.cuda.synchronize()
        got_lat, got_eos = out.cpu().numpy(), eos.cpu().numpy()
        for i in range(n):
            c = cond[f, i] if cond is not None else model_cond
            wl, we = orc.step(sts[i], want_lat[i], noise[f, i], cond=c)
            want_lat[i] = wl
            e = max(rel_err(got_lat[i], wl), abs(got_eos[i] - we) / max(1.0, abs(we)))
            worst = max(worst, e)
            assert e <= tol, (f, i, e)
        # f32: each side continues from its own latent; q8: both from the oracle's
        lat_in = torch.from_numpy(np.stack(want_lat)).to(DEV) if q8 else out.clone()
    return pool, ids, sts, worst


def test_flow_lm_prompt_and_frames_match_the_oracle():
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=256, dim_feedforward=1024, n_bins=100)
    blob = fl.random_weights(cfg, 90, std=0.05, unit_norms=False)
    rng = np.random.default_rng(91)
    tokens = rng.integers(0, cfg.n_bins + 1, (2, 5)).astype(np.int32)
    noise = (0.5 * rng.standard_normal((6, 2, cfg.ldim))).astype(np.float32)
    pool, ids, sts, _ = run_pair(cfg, blob, tokens, 6, noise, 32)
    # the cache rows the prompt and the frames wrote, within the same bar
    for i in range(2):
        n = sts[i].current_end
        assert n == 11
        for layer in range(cfg.num_layers):
            for kv in (0, 1):
                rows = torch.empty((n, cfg.num_heads, 64), dtype=torch.float32, device=DEV)
                pool.read_rows(ids[i], layer, kv, 0, rows)
                torch.cuda.synchronize()
                vals, _, _ = sts[i].read_rows(layer, kv, 0, n)
                assert rel_err(rows.cpu().numpy(), vals) <= 1e-5, (i, layer, kv)


def test_phonon_31m_shape_64_tokens_then_200_frames_at_temperature_0():
    # the single-stream configuration: 6 layers x 512, 8 heads, FF 2048, ldim 32, 4001-row LUT,
    # flow net 512 x 6, 1 LSD step; N(0, 0.02) linears, unit norms; 64 tokens, 200 greedy frames
    cfg = fl.FlowLMConfig()
    blob = fl.random_weights(cfg, 20261201)
    rng = np.random.default_rng(20261201)
    tokens = rng.integers(0, cfg.n_bins + 1, (1, 64)).astype(np.int32)
    noise = np.zeros((200, 1, cfg.ldim), np.float32)  # temperature 0 (flow_lm.rs:494-500)
    _, _, sts, worst = run_pair(cfg, blob, tokens, 200, noise, 868)
    assert sts[0].current_end == 264
    print(f"worst relative error over 200 frames: {worst:.2e}")


def test_bad_tokens_are_refused_and_change_nothing():
    cfg = fl.FlowLMConfig(num_layers=1, flow_depth=1, flow_dim=256, dim_feedforward=512, n_bins=10)
    blob = fl.random_weights(cfg, 92)
    pool = xnp.KvPool(num_layers=1, num_heads=8, num_blocks=8, max_streams=1, max_blocks_per_stream=4,
                      cache_dtype="f32", act_dtype="f32")
    sid = pool.init_state(64)
    lm = xnp.FlowLM(pool, cfg, blob, max_rows=8)
    with pytest.raises(xnp.XnpError):
        lm.prompt_text([sid], np.array([[1, 2, 11]], np.int32))
    assert pool.current_end(sid) == 0


def test_graph_recorded_frames_equal_eager_frames():
    # StepGraph's analog (step_graph.rs:111-307): the frame's launches recorded once and replayed
    # after each eager plan upload, against a twin model stepping eagerly -- bit for bit, every
    # frame, with the host reading results back between replays.  The latent buffer is updated in
    # place, so after the first frame (bos) one recording serves every later frame.
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=256, dim_feedforward=1024, n_bins=100)
    blob = fl.random_weights(cfg, 93, std=0.05, unit_norms=False)
    rng = np.random.default_rng(94)
    n = 2
    tokens = rng.integers(0, cfg.n_bins + 1, (n, 4)).astype(np.int32)
    s = torch.cuda.Stream()
    runs = []
    for _ in range(2):
        pool = xnp.KvPool(num_layers=2, num_heads=8, num_blocks=16, max_streams=n, max_blocks_per_stream=4,
                          cache_dtype="f32", act_dtype="f32", max_pos=128, page_seed=4)
        ids = [pool.init_state(64) for _ in range(n)]
        lm = xnp.FlowLM(pool, cfg, blob, max_rows=n * 4)
        with torch.cuda.stream(s):
            lm.prompt_text(ids, tokens)
        lat = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
        eos = torch.zeros(n, dtype=torch.float32, device=DEV)
        runs.append((pool, ids, lm, lat, eos))
    noise = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
    for f in range(8):
        with torch.cuda.stream(s):
            noise.copy_(torch.from_numpy((0.5 * rng.standard_normal((n, cfg.ldim))).astype(np.float32)).to(DEV))
            for g, (pool, ids, lm, lat, eos) in enumerate(runs):
                lm.step(ids, None if f == 0 else lat, noise, lat, eos, stream=s.cuda_stream, graph=(g == 1))
        s.synchronize()
        assert torch.equal(runs[0][3], runs[1][3]) and torch.equal(runs[0][4], runs[1][4]), f
    assert runs[1][0].current_end(runs[1][1][0]) == 12


@pytest.mark.parametrize("flow_type,z_dim", [("lsd", 64), ("drifting", 0), ("pointwise", 48)])
def test_flow_lm_variants_match_the_oracle(flow_type, z_dim):
    # z_proj after out_norm (flow_lm.rs:320-323) and the heads without time conditions
    # (flow_lm.rs:380-381), two streams, 2 LSD steps where the solver runs
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=256, dim_feedforward=1024, n_bins=100,
                          flow_type=flow_type, z_dim=z_dim, lsd_decode_steps=2)
    blob = fl.random_weights(cfg, 95, std=0.05, unit_norms=False)
    rng = np.random.default_rng(96)
    tokens = rng.integers(0, cfg.n_bins + 1, (2, 5)).astype(np.int32)
    noise = (0.5 * rng.standard_normal((5, 2, cfg.ldim))).astype(np.float32)
    _, _, sts, worst = run_pair(cfg, blob, tokens, 5, noise, 32)
    assert sts[0].current_end == 10
    print(f"{flow_type} z_dim {z_dim}: worst relative error {worst:.2e}")


@pytest.mark.parametrize("precision", ["f32", "q8"])
@pytest.mark.parametrize("heads,kv_heads,attn_dim,cond", [(8, 2, 0, "stream"), (4, 1, 256, "model"),
                                                          (4, 2, 256, "stream")])
def test_grouped_heads_attn_dim_and_conditions_match_the_oracle(precision, heads, kv_heads, attn_dim, cond):
    # FlowLMConfig's num_kv_heads (flow_lm.rs:143-145, 253: the pool stores kv_heads heads), attn_dim
    # (flow_lm.rs:139-141, 252: in_proj [a + 2 kv][d], out_proj [d][a], 64-wide heads) and the
    # conditions broadcast-added to the step input (flow_lm.rs:304-307): each stream's own row per
    # frame (FlowLMState::conditions, as s2s.rs:334 sets it), or the model's summed conditions
    # (condition_providers, flow_lm.rs:218-222).  Three streams, a 6-token prompt, 8 frames.
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=512, dim_feedforward=1024, n_bins=100, d_model=512,
                          num_heads=heads, num_kv_heads=kv_heads, attn_dim=attn_dim, lsd_decode_steps=2,
                          precision=precision)
    blob = fl.random_weights(cfg, 107, std=0.05, unit_norms=False)
    rng = np.random.default_rng(108)
    tokens = rng.integers(0, cfg.n_bins + 1, (3, 6)).astype(np.int32)
    noise = (0.5 * rng.standard_normal((8, 3, cfg.ldim))).astype(np.float32)
    c = (0.5 * rng.standard_normal((8, 3, cfg.d_model))).astype(np.float32)
    if precision == "q8":
        c = bf16_round(c)
    kw = dict(cond=c) if cond == "stream" else dict(model_cond=c[0, 0])
    pool, ids, sts, worst = run_pair(cfg, blob, tokens, 8, noise, 32, **kw)
    assert sts[0].current_end == 14 and pool.current_end(ids[0]) == 14
    print(f"{precision} {heads} heads over {kv_heads}, attn_dim {attn_dim or 512}, {cond} conditions: "
          f"worst relative error {worst:.2e}")


def test_q8_graph_is_recorded_again_when_the_condition_source_changes():
    # Frames replayed from a graph equal eager frames bit for bit while the conditions come from the
    # step's own rows, then from the model's, then from nowhere: each change of source records again.
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=512, dim_feedforward=1024, n_bins=100,
                          num_heads=8, num_kv_heads=2, precision="q8")
    blob = fl.random_weights(cfg, 109, std=0.05, unit_norms=False)
    rng = np.random.default_rng(110)
    n, P = 3, 4
    tokens = rng.integers(0, cfg.n_bins + 1, (n, P)).astype(np.int32)
    s = torch.cuda.Stream()
    runs = []
    for _ in range(2):
        pool = xnp.KvPool(num_layers=2, num_heads=8, num_kv_heads=2, num_blocks=24, max_streams=n,
                          max_blocks_per_stream=4, cache_dtype="bf16", act_dtype="bf16", max_pos=128, page_seed=6)
        ids = [pool.init_state(64) for _ in range(n)]
        lm = xnp.FlowLM(pool, cfg, blob, max_rows=n * P)
        with torch.cuda.stream(s):
            lm.prompt_text(ids, tokens)
        lat = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
        eos = torch.zeros(n, dtype=torch.float32, device=DEV)
        runs.append((pool, ids, lm, lat, eos))
    noise = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
    cond = torch.zeros((n, cfg.d_model), dtype=torch.float32, device=DEV)
    model = bf16_round(0.5 * rng.standard_normal(cfg.d_model).astype(np.float32))
    for f in range(18):
        with torch.cuda.stream(s):
            noise.copy_(torch.from_numpy((0.5 * rng.standard_normal((n, cfg.ldim))).astype(np.float32)).to(DEV))
            cond.copy_(torch.from_numpy(bf16_round(0.5 * rng.standard_normal((n, cfg.d_model)))).to(DEV))
            for g, (pool, ids, lm, lat, eos) in enumerate(runs):
                if f == 6:
                    lm.set_condition(model)
                if f == 12:
                    lm.set_condition(None)
                lm.step(ids, None if f == 0 else lat, noise, lat, eos, stream=s.cuda_stream, graph=(g == 1),
                        conditions=cond if f < 6 else None)
        s.synchronize()
        assert torch.equal(runs[0][3], runs[1][3]) and torch.equal(runs[0][4], runs[1][4]), f


@pytest.mark.parametrize("flow_type,z_dim,steps", [("lsd", 0, 1), ("lsd", 64, 2), ("drifting", 0, 1),
                                                   ("pointwise", 64, 1)])
def test_q8_flow_lm_matches_the_q8_oracle(flow_type, z_dim, steps):
    # Three streams of a 7-token prompt, then 12 frames: every linear on the MFMA GEMM (rows past
    # the batch, N = 1 and N = 32 tiles, K = 32), the bf16 LayerNorm with the AdaLN modulation.
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=512, dim_feedforward=1024, n_bins=100,
                          flow_type=flow_type, z_dim=z_dim, lsd_decode_steps=steps, precision="q8")
    blob = fl.random_weights(cfg, 97, std=0.05, unit_norms=False)
    rng = np.random.default_rng(98)
    tokens = rng.integers(0, cfg.n_bins + 1, (3, 7)).astype(np.int32)
    noise = (0.5 * rng.standard_normal((12, 3, cfg.ldim))).astype(np.float32)
    _, _, sts, worst = run_pair(cfg, blob, tokens, 12, noise, 64)
    assert sts[0].current_end == 19
    print(f"q8 {flow_type} z_dim {z_dim} steps {steps}: worst relative error {worst:.2e}")


def test_q8_graph_recorded_frames_equal_eager_frames():
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=512, dim_feedforward=1024, n_bins=100, precision="q8")
    blob = fl.random_weights(cfg, 99, std=0.05, unit_norms=False)
    rng = np.random.default_rng(100)
    n = 3
    tokens = rng.integers(0, cfg.n_bins + 1, (n, 4)).astype(np.int32)
    s = torch.cuda.Stream()
    runs = []
    for _ in range(2):
        pool = xnp.KvPool(num_layers=2, num_heads=8, num_blocks=24, max_streams=n, max_blocks_per_stream=4,
                          cache_dtype="bf16", act_dtype="bf16", max_pos=128, page_seed=5)
        ids = [pool.init_state(64) for _ in range(n)]
        lm = xnp.FlowLM(pool, cfg, blob, max_rows=n * 4)
        with torch.cuda.stream(s):
            lm.prompt_text(ids, tokens)
        lat = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
        eos = torch.zeros(n, dtype=torch.float32, device=DEV)
        runs.append((pool, ids, lm, lat, eos))
    noise = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
    for f in range(8):
        with torch.cuda.stream(s):
            noise.copy_(torch.from_numpy((0.5 * rng.standard_normal((n, cfg.ldim))).astype(np.float32)).to(DEV))
            for g, (pool, ids, lm, lat, eos) in enumerate(runs):
                lm.step(ids, None if f == 0 else lat, noise, lat, eos, stream=s.cuda_stream, graph=(g == 1))
        s.synchronize()
        assert torch.equal(runs[0][3], runs[1][3]) and torch.equal(runs[0][4], runs[1][4]), f


def test_q8_graph_is_recorded_again_when_a_stream_takes_up_a_ring_prefix():
    # A recording made while no stream keeps a ring prefix holds the decode built without the
    # prefix's second query rotation.  When one stream then turns into an absolute ring that keeps
    # its prompt (s2s.rs:174) and evicts (s2s.rs:324-333), replayed frames must still equal eager
    # frames bit for bit: the plan picks the prefix decode, and the graph is recorded again.
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=512, dim_feedforward=1024, n_bins=100, precision="q8")
    blob = fl.random_weights(cfg, 103, std=0.05, unit_norms=False)
    rng = np.random.default_rng(104)
    n, P, span, drop = 3, 4, 12, 4
    tokens = rng.integers(0, cfg.n_bins + 1, (n, P)).astype(np.int32)
    s = torch.cuda.Stream()
    runs = []
    for _ in range(2):
        pool = xnp.KvPool(num_layers=2, num_heads=8, num_blocks=24, max_streams=n, max_blocks_per_stream=4,
                          cache_dtype="bf16", act_dtype="bf16", max_pos=128, page_seed=6)
        ids = [pool.init_state(64) for _ in range(n)]
        lm = xnp.FlowLM(pool, cfg, blob, max_rows=n * P)
        with torch.cuda.stream(s):
            lm.prompt_text(ids, tokens)
        lat = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
        eos = torch.zeros(n, dtype=torch.float32, device=DEV)
        runs.append((pool, ids, lm, lat, eos))
    noise = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
    plain = 3  # frames before stream 0 becomes a ring; its frames sit at slots P, P + 1, ...
    for f in range(plain + 21):
        with torch.cuda.stream(s):
            noise.copy_(torch.from_numpy((0.5 * rng.standard_normal((n, cfg.ldim))).astype(np.float32)).to(DEV))
            for g, (pool, ids, lm, lat, eos) in enumerate(runs):
                if f == plain:
                    pool.start_ring(ids[0], "absolute", prefix=P, stream=s.cuda_stream)
                if f >= plain:
                    pool.slide(ids[0], P, span, span, drop, f, stream=s.cuda_stream)
                lm.step(ids, None if f == 0 else lat, noise, lat, eos, stream=s.cuda_stream, graph=(g == 1))
        s.synchronize()
        assert torch.equal(runs[0][3], runs[1][3]) and torch.equal(runs[0][4], runs[1][4]), f
    info = runs[1][0].info(runs[1][1][0])
    assert info["ring_shift"] == 12 and info["ring_prefix"] == P  # three evictions of 4 rows


def test_q8_graph_is_recorded_again_when_the_rope_tables_grow():
    # A pool whose RoPE tables start at 16 rows: the prompt and the frames reach positions past 16
    # and then past 32, and each growth frees the tables a recorded frame's kernels read.  Replayed
    # frames must still equal eager frames bit for bit: the growth changes the launch key, and the
    # graph is recorded again against the new tables.
    cfg = fl.FlowLMConfig(num_layers=2, flow_depth=2, flow_dim=512, dim_feedforward=1024, n_bins=100, precision="q8")
    blob = fl.random_weights(cfg, 105, std=0.05, unit_norms=False)
    rng = np.random.default_rng(106)
    n, P, frames = 3, 6, 40
    tokens = rng.integers(0, cfg.n_bins + 1, (n, P)).astype(np.int32)
    s = torch.cuda.Stream()
    runs = []
    for _ in range(2):
        pool = xnp.KvPool(num_layers=2, num_heads=8, num_blocks=24, max_streams=n, max_blocks_per_stream=4,
                          cache_dtype="bf16", act_dtype="bf16", max_pos=16, page_seed=6)
        ids = [pool.init_state(64) for _ in range(n)]
        lm = xnp.FlowLM(pool, cfg, blob, max_rows=n * P)
        with torch.cuda.stream(s):
            lm.prompt_text(ids, tokens)
        lat = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
        eos = torch.zeros(n, dtype=torch.float32, device=DEV)
        runs.append((pool, ids, lm, lat, eos))
    noise = torch.zeros((n, cfg.ldim), dtype=torch.float32, device=DEV)
    rows = []
    for f in range(frames):
        with torch.cuda.stream(s):
            noise.copy_(torch.from_numpy((0.5 * rng.standard_normal((n, cfg.ldim))).astype(np.float32)).to(DEV))
            for g, (pool, ids, lm, lat, eos) in enumerate(runs):
                lm.step(ids, None if f == 0 else lat, noise, lat, eos, stream=s.cuda_stream, graph=(g == 1))
        s.synchronize()
        assert torch.equal(runs[0][3], runs[1][3]) and torch.equal(runs[0][4], runs[1][4]), f
        rows.append(runs[1][0].stats()["rope_rows"])
    assert rows[0] == 16 and rows[-1] >= 64 and len(set(rows)) >= 3  # grown twice while replaying


def test_q8_refuses_an_f32_pool_and_odd_widths():
    cfg = fl.FlowLMConfig(num_layers=1, flow_depth=1, flow_dim=512, dim_feedforward=512, n_bins=10, precision="q8")
    blob = fl.random_weights(cfg, 101)
    f32 = xnp.KvPool(num_layers=1, num_heads=8, num_blocks=8, max_streams=1, max_blocks_per_stream=4,
                     cache_dtype="f32", act_dtype="f32")
    with pytest.raises(xnp.XnpError, match="bf16 pool"):
        xnp.FlowLM(f32, cfg, blob)
    bad = fl.FlowLMConfig(num_layers=1, flow_depth=1, flow_dim=256, dim_feedforward=512, n_bins=10, precision="q8")
    bf = xnp.KvPool(num_layers=1, num_heads=8, num_blocks=8, max_streams=1, max_blocks_per_stream=4,
                    cache_dtype="bf16", act_dtype="bf16")
    with pytest.raises(xnp.XnpError, match="multiples of 512"):
        xnp.FlowLM(bf, bad, fl.random_weights(bad, 102))
