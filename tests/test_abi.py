"""CPU tests of the C ABI (libxnp_kv.so) that run no kernel: exported symbols, and the host
logic -- page allocator, stream state, ring state machine, batch bookkeeping, refusals -- through
a host-only pool (XNP_POOL_HOST_ONLY), checked against the oracle and the reference's rules."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT, oracle, xnp

HEADER = os.path.join(ROOT, "include", "xnp_kv.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const char \*|xnp_status|int32_t)\s*(xnp_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(xnp.LIB_PATH)
    names = declared_symbols()
    assert len(names) == len(xnp.kv.SIGNATURES)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers each one
    assert set(names) <= set(xnp.kv.SIGNATURES)


def pool(**kw):
    args = dict(num_layers=2, num_heads=4, num_blocks=64, max_streams=8, max_blocks_per_stream=8,
                cache_dtype="f32", act_dtype="f32", host_only=True, max_pos=512)
    args.update(kw)
    return xnp.KvPool(**args)


def test_budgets_follow_plan_rs():
    # plan.rs:43-54: frame_budget(64 tokens) = ceil((64/3 + 2) * 12.5) = 292; seq = 64 + 512 + 292
    assert xnp.frame_budget(64, 12.5) == 292
    assert xnp.seq_budget(64, 292) == 868
    assert xnp.frame_budget(0, 12.5) == 25


def test_bad_configs_are_refused():
    for heads, kvh in [(3, 2), (4, 3), (4, 0)]:
        with pytest.raises(xnp.XnpError) as e:
            pool(num_heads=heads, num_kv_heads=kvh)
        assert e.value.name == "XNP_E_HEADS" and "heads" in e.value.message
    with pytest.raises(xnp.XnpError, match="head_dim"):
        pool(head_dim=32)
    with pytest.raises(xnp.XnpError, match="not supported"):
        pool(cache_dtype="bf16", act_dtype="f32")


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_rope_table_is_the_oracles_bit_for_bit(act):
    p = pool(cache_dtype=act, act_dtype=act, max_pos=4096)
    table = p.rope_rows(0, 4096)
    for pos in [0, 1, 2, 17, 255, 1000, 2047, 4095]:
        c, s = oracle.rope_row(64, 10000.0, float(pos), act)
        assert np.array_equal(table[pos, :, 0].view(np.uint32), c.view(np.uint32))
        assert np.array_equal(table[pos, :, 1].view(np.uint32), s.view(np.uint32))


@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_rope_tables_grow_when_positions_reach_their_end(act):
    # An absolute ring counts positions on after its evictions (the reference rotates at any offset,
    # transformer.rs:794-803): a batch reaching past the table's rows grows it, doubling, and the new
    # rows are the oracle's bit for bit.
    p = pool(cache_dtype=act, act_dtype=act, max_pos=64)
    s = p.init_state(48)
    p.begin([s], t=32)
    p.end()
    p.start_ring(s, "absolute", prefix=0)
    for step in range(32, 232):  # a window of 32 on 48 slots, one row evicted per step
        p.slide(s, 0, 48, 32, 1, step)
        p.begin([s])
        p.end()
    info = p.info(s)
    assert info["current_end"] == 32 and info["ring_shift"] == 200  # the last step wrote position 231
    assert p.stats()["rope_rows"] == 256
    table = p.rope_rows(0, 256)
    for pos in [0, 63, 64, 127, 128, 200, 231, 255]:
        c, sn = oracle.rope_row(64, 10000.0, float(pos), act)
        assert np.array_equal(table[pos, :, 0].view(np.uint32), c.view(np.uint32)), pos
        assert np.array_equal(table[pos, :, 1].view(np.uint32), sn.view(np.uint32)), pos
    with pytest.raises(xnp.XnpError, match="256-row table"):
        p.rope_rows(200, 100)


def test_a_broken_page_map_is_refused_before_anything_changes():
    # Every block a step writes must hold a page of the stream's own: planted on a host-only pool, an
    # id past the pool, a free page, a page shared with a fork (with_seq_budget shares full pages,
    # transformer.rs:350-392) and the page another stream of the batch takes for its own row (pages
    # are handed out in order: a's next is page 2) are each refused, the pool left as it was; the
    # repaired map steps.
    p = pool()
    a = p.init_state(64)
    p.begin([a], t=32)
    p.end()
    b = p.with_seq_budget(a, 64)
    shared = p.blocks(a)[1]
    assert p.blocks(b)[:2] == p.blocks(a)[:2] and p.info(b)["shared"] == 2
    free0 = p.stats()["free_blocks"]
    for page in (64 + 5, 60, shared, 2):
        p.debug_set_block(b, 2, page)
        with pytest.raises(xnp.XnpError) as e:
            p.begin([a, b], t=1)
        assert e.value.name == "XNP_E_STATE" and "page map is broken" in e.value.message, page
        p.debug_set_block(b, 2, -1)  # put back before anything reads the map
        assert p.stats()["free_blocks"] == free0 and p.stats()["batch_open"] == 0
        assert p.current_end(a) == 32 and p.current_end(b) == 32
    p.begin([a, b], t=1)
    p.end()
    assert p.current_end(b) == 33 and p.stats()["free_blocks"] == free0 - 2


def test_pages_are_taken_as_rows_arrive_and_returned_on_close():
    p = pool()
    a = p.init_state(100)
    assert p.stats()["free_blocks"] == 64 and p.blocks(a) == [-1] * 7
    p.begin([a], t=20)
    assert p.stats()["free_blocks"] == 62
    p.end()
    assert p.current_end(a) == 20
    p.begin([a], t=1)
    p.end()
    assert p.stats()["free_blocks"] == 62  # row 20 lands in page 1
    p.advance(a, 12)  # rows 21..32: page 2 for row 32
    assert p.current_end(a) == 33 and p.stats()["free_blocks"] == 61
    p.close(a)
    assert p.stats()["free_blocks"] == 64 and p.stats()["open_streams"] == 0


def test_shuffled_pages_are_a_permutation():
    p = pool(num_blocks=32, page_seed=20261201, max_blocks_per_stream=32)
    a = p.init_state(32 * 16)
    p.advance(a, 32 * 16)
    pages = p.blocks(a)
    assert sorted(pages) == list(range(32)) and pages != list(range(32))


def test_capacity_and_out_of_blocks_are_refused_and_change_nothing():
    p = pool(num_blocks=4)
    a, b = p.init_state(40), p.init_state(40)
    with pytest.raises(xnp.XnpError) as e:
        p.begin([a], t=41)
    assert e.value.name == "XNP_E_NO_ROOM" and "no room left" in e.value.message
    p.begin([a], t=40)  # 3 pages
    p.end()
    with pytest.raises(xnp.XnpError) as e:
        p.begin([b], t=17)  # 2 pages, 1 free
    assert e.value.name == "XNP_E_OUT_OF_BLOCKS"
    assert p.stats()["free_blocks"] == 1 and p.current_end(b) == 0 and p.stats()["batch_open"] == 0
    with pytest.raises(xnp.XnpError) as e:
        p.begin([b, 99], t=1)
    assert e.value.name == "XNP_E_STREAM"
    with pytest.raises(xnp.XnpError, match="twice"):
        p.begin([b, b], t=1)
    with pytest.raises(xnp.XnpError) as e:
        p.init_state(8 * 16 + 1)
    assert e.value.name == "XNP_E_INVALID"


def test_abort_gives_back_the_pages_and_keeps_the_state():
    p = pool()
    a, b = p.init_state(64), p.init_state(64)
    p.begin([a, b], t=1)
    assert p.stats()["free_blocks"] == 62
    p.abort()
    assert p.stats()["free_blocks"] == 64 and p.current_end(a) == 0
    with pytest.raises(xnp.XnpError) as e:
        p.end()
    assert e.value.name == "XNP_E_STATE"


def test_kernel_calls_on_a_host_only_pool_are_refused():
    p = pool()
    a = p.init_state(16)
    p.begin([a])
    for call in (lambda: p.append(0, None, None), lambda: p.decode(0, None, None, 0.125)):
        with pytest.raises(xnp.XnpError) as e:
            call()
        assert e.value.name == "XNP_E_STATE"
    with pytest.raises(xnp.XnpError) as e:
        p.close(a)  # a batch is open
    assert e.value.name == "XNP_E_STATE"
    p.abort()


def test_decode_runs_one_work_group_per_stream_and_head():
    p = pool(max_blocks_per_stream=64, num_blocks=256, max_pos=2048)
    ids = [p.init_state(1024) for _ in range(3)]
    for sid, n in zip(ids, [0, 64, 1000]):
        p.advance(sid, n)
    p.begin(ids)
    assert p.stats()["work_items"] == 3 * 4
    p.abort()
    p.begin(ids[:1], t=5)  # a prompt step decodes nothing
    assert p.stats()["work_items"] == 0
    p.abort()
    with pytest.raises(xnp.XnpError, match="decode_split"):
        pool(decode_split=3)
    with pytest.raises(xnp.XnpError, match="pages per stream"):
        pool(decode_split=2, max_blocks_per_stream=121)


def test_decode_waves_per_group_follow_the_pages_a_wave_indexes():
    # by default: the fewest waves whose lanes index a stream's pages (two up to 120 pages, four up
    # to 240, then eight), one while a head's K and V tiles hold at most 128 KB (32 bf16 pages, 60
    # int8 ones: a wave's lanes index 60); at least two on the MFMA decode of grouped bf16 heads;
    # more for a batch too small to fill the GPU (about 1024 waves); a fixed split stays fixed
    def waves(streams=160, **kw):
        args = dict(num_heads=8, num_blocks=streams + 8, max_streams=streams, cache_dtype="bf16", act_dtype="bf16")
        args.update(kw)
        p = pool(**args)
        ids = [p.init_state(16) for _ in range(streams)]
        p.begin(ids)
        w = p.stats()["decode_waves"]
        p.abort()
        assert p.stats()["decode_waves"] == 0
        return w

    assert waves(max_blocks_per_stream=32) == 1
    assert waves(max_blocks_per_stream=33) == 2
    assert waves(max_blocks_per_stream=60, cache_dtype="i8") == 1
    assert waves(max_blocks_per_stream=61, cache_dtype="i8") == 2
    assert waves(max_blocks_per_stream=16, cache_dtype="f32", act_dtype="f32") == 1
    assert waves(max_blocks_per_stream=17, cache_dtype="f32", act_dtype="f32") == 2
    assert waves(max_blocks_per_stream=121) == 4
    assert waves(max_blocks_per_stream=241) == 8
    assert waves(max_blocks_per_stream=8, cache_dtype="i8") == 1
    # 4 query heads per kv head, 600 streams: 1200 groups of a kv head on MFMA (two waves), or of
    # four query heads each on the VALU (f32: one wave)
    assert waves(streams=600, max_blocks_per_stream=8, num_kv_heads=2) == 2
    assert waves(streams=600, max_blocks_per_stream=8, num_kv_heads=2, cache_dtype="f32", act_dtype="f32") == 1
    assert waves(streams=160, max_blocks_per_stream=8, num_kv_heads=2) == 4  # 320 groups: grown
    assert waves(streams=16, max_blocks_per_stream=8) == 8                  # 128 groups: grown to 8
    assert waves(streams=160, max_blocks_per_stream=8, decode_split=1) == 1
    p = pool(max_blocks_per_stream=8)
    p.begin([p.init_state(16)], t=4)  # a prompt step decodes nothing
    assert p.stats()["decode_waves"] == 0
    p.abort()


# ---- with_seq_budget (transformer.rs:350-392) ------------------------------------------------
def test_fork_shares_full_pages_and_copies_the_partial_one():
    p = pool()
    a = p.init_state(128)
    p.advance(a, 40)  # pages 0, 1 full; 2 partial
    free = p.stats()["free_blocks"]
    b = p.with_seq_budget(a, 100)
    ia, ib = p.info(a), p.info(b)
    assert ib["current_end"] == 40 and ib["capacity"] == 100
    assert p.blocks(b)[:2] == p.blocks(a)[:2] and p.blocks(b)[2] != p.blocks(a)[2]
    assert ia["shared"] == 2 and ib["shared"] == 2 and p.stats()["free_blocks"] == free - 1
    p.close(a)
    assert p.info(b)["shared"] == 0 and p.stats()["free_blocks"] == free - 1 + 1
    with pytest.raises(xnp.XnpError) as e:
        p.with_seq_budget(b, 39)
    assert e.value.name == "XNP_E_BUDGET" and "40" in e.value.message and "39" in e.value.message
    p.with_seq_budget(b, 40)


def test_a_ring_cannot_be_forked_and_starting_one_unshares():
    p = pool()
    a = p.init_state(64)
    p.advance(a, 32)
    b = p.with_seq_budget(a, 64)
    assert p.info(b)["shared"] == 2
    p.start_ring(b)
    assert p.info(b)["shared"] == 0 and p.info(a)["shared"] == 0
    with pytest.raises(xnp.XnpError) as e:
        p.with_seq_budget(b, 64)
    assert e.value.name == "XNP_E_BUDGET" and "ring" in e.value.message


# ---- ring state machine vs the oracle (transformer.rs:842-929, 1397-1416) ----------------------
def test_misuse_of_a_ring_is_refused_like_the_oracle():
    p = pool(num_heads=4)
    st = oracle.Stream(2, 4, 64, 8)
    a = p.init_state(8)
    p.begin([a], t=4)
    p.end()
    st.advance(4)
    both = [(lambda f: f(p, a), lambda g: g(st))]

    def same(fp, fo):
        errs = []
        for f in (lambda: fp(), lambda: fo()):
            try:
                f()
                errs.append(None)
            except (xnp.XnpError, oracle.OracleError) as e:
                errs.append(str(e).split(": ", 1)[-1])
        assert errs[0] == errs[1], errs
        return errs[0]

    assert "not a ring" in same(lambda: p.set_ring_slot(a, 4), lambda: st.set_ring_slot(4))
    same(lambda: p.start_ring(a), lambda: st.start_ring("shift"))
    same(lambda: p.set_ring_slot(a, 4), lambda: st.set_ring_slot(4))
    assert "slot 8 of a 8-slot ring" in same(lambda: p.set_ring_slot(a, 8), lambda: st.set_ring_slot(8))

    def step():
        p.begin([a])
        p.end()

    def ostep():
        st.append(0, np.zeros((1, 4, 64)), np.zeros((1, 4, 64)))
        st.commit(1)

    same(step, ostep)
    for slots in ([2], [5], [4, 5]):
        assert "holds no row past the prefix" in same(lambda: p.evict(a, 4, slots), lambda: st.evict(4, slots))
    assert p.valid(a)[4]
    same(lambda: p.set_ring_slot(a, 4), lambda: st.set_ring_slot(4))
    assert "still holds a row" in same(step, ostep)
    assert "cannot evict 6 of 5" in same(lambda: p.evict(a, 0, [0, 1, 2, 3, 4, 4]), lambda: st.evict(0, [0, 1, 2, 3, 4, 4]))
    same(lambda: p.evict(a, 4, [4]), lambda: st.evict(4, [4]))
    same(step, ostep)
    info, oinfo = p.info(a), st.ring_info()
    assert (info["ring_write"], info["ring_filled"], info["current_end"]) == (oinfo["write"], oinfo["filled"], st.current_end)
    assert p.valid(a) == list(oinfo["valid"])
    with pytest.raises(xnp.XnpError, match="one row at a time"):
        p.begin([a], t=2)


@pytest.mark.parametrize("mode", ["shift", "absolute"])
def test_slide_is_the_s2s_session_policy(mode):
    # s2s.rs:318-333 with a voice prefix of v = 5 and a context of 6: evict the oldest third when
    # the context is full, then write at v + steps % context.  Restated in Python here.
    p = pool(num_heads=4)
    a = p.init_state(11)
    p.begin([a], t=5)
    p.end()
    p.start_ring(a, mode, prefix=5)
    v, context, in_view = 5, 6, 0
    valid = [True] * 5 + [False] * 6
    for steps in range(40):
        if in_view == context:
            oldest = steps - in_view
            for j in range(context // 3):
                valid[v + (oldest + j) % context] = False
            in_view -= context // 3
        write = v + steps % context
        p.slide(a, v, context, context, context // 3, steps)
        assert p.info(a)["ring_write"] == write and p.valid(a) == valid
        p.begin([a])
        p.end()
        valid[write] = True
        in_view += 1
        assert p.info(a)["current_end"] == 5 + in_view


def test_sliding_window_keeps_the_last_window_rows():
    p = pool(num_heads=4, max_blocks_per_stream=40, num_blocks=128, max_pos=4096)
    a = p.init_state(528)
    p.start_ring(a, "absolute", prefix=0)
    h0 = 1234
    for n in range(700):
        p.slide(a, 0, 528, 512, 1, h0 + n)
        p.begin([a])
        p.end()
        info = p.info(a)
        assert info["in_view"] == min(n + 1, 512)
        assert info["ring_write"] == (h0 + n) % 528
    assert info["ring_shift"] == 700 - 512 and info["current_end"] == 512


def test_table_patches_of_reopened_streams_leave_the_live_pages():
    # Closing a stream queues -1 for its entries; reopening it and taking pages queues the new
    # ids for the same entries.  The device applies a flush's patches in no particular order
    # (the host-only shadow applies them in reverse), so each entry must be flushed once, with
    # its current value.
    p = pool(num_blocks=64, max_streams=8, max_blocks_per_stream=8)
    ids = [p.init_state(128) for _ in range(4)]
    for _ in range(3):
        p.begin(ids, t=100)
        p.end()
        assert p.check_tables() == 0
        for i, sid in enumerate(ids):
            p.close(sid)
            ids[i] = p.init_state(128)
    p.begin(ids, t=37)
    p.abort()
    p.begin(ids, t=50)
    p.end()
    a = p.with_seq_budget(ids[0], 128)
    p.close(ids[1])
    p.advance(a, 20)
    assert p.check_tables() == 0


def test_quantize_rows_is_the_oracles_bit_for_bit():
    # a host function of the library: no GPU needed
    rng = np.random.default_rng(70)
    w = rng.standard_normal((40, 200)).astype(np.float32) * 0.05
    w[7] = 0.0
    q, s = xnp.quantize_rows(w)
    oq, os_ = oracle.quantize_rows(w)
    assert np.array_equal(q, oq) and np.array_equal(s.view(np.uint32), os_.view(np.uint32))


def test_layer_calls_refuse_bad_shapes_without_running_a_kernel():
    lib = xnp.load_library()
    assert lib.xnp_linear_q8(None, 4, 100, None, None, 64, 0, None, None, None) == 1  # k not a multiple of 64
    assert lib.xnp_linear_q8(None, 4, 64, None, None, 64, 9, None, None, None) == 1   # no such epilogue
    assert lib.xnp_layer_norm(None, 4, 300, None, None, 1e-5, None, None) == 1        # dim not a multiple of 512
    pool = xnp.KvPool(num_layers=1, num_heads=8, num_blocks=8, max_streams=2, max_blocks_per_stream=4,
                      host_only=True)
    w = xnp.kv.LayerWeightsC()
    assert lib.xnp_layer_step(pool._h, 0, ctypes.byref(w), None, None, 0, None) == 1  # null x
    x = ctypes.c_uint16()
    assert lib.xnp_layer_step(pool._h, 0, ctypes.byref(w), ctypes.byref(x), None, 0, None) == 9  # no batch open
    assert pool.layer_workspace(2048, 512, 2048) >= 2048 * (512 * 5 + 2048) * 2


def test_flow_lm_layout_agrees_between_the_library_and_the_package():
    cfg = xnp.FlowLMConfig()
    d = xnp.flow_lm.desc_of(cfg)
    n = ctypes.c_int64()
    assert xnp.load_library().xnp_flow_lm_weights_size(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == xnp.flow_lm.blob_size(cfg)
    small = xnp.FlowLMConfig(num_layers=2, flow_depth=3, n_bins=10, flow_dim=256, dim_feedforward=1024)
    d = xnp.flow_lm.desc_of(small)
    assert xnp.load_library().xnp_flow_lm_weights_size(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value == xnp.flow_lm.blob_size(small)


def test_flow_lm_refuses_a_pool_it_does_not_fit():
    cfg = xnp.FlowLMConfig(num_layers=2, flow_depth=1, n_bins=10)
    pool = xnp.KvPool(num_layers=2, num_heads=8, num_blocks=8, max_streams=2, max_blocks_per_stream=4,
                      host_only=True, cache_dtype="f32", act_dtype="f32")
    with pytest.raises(xnp.XnpError):  # a host-only pool has no device
        xnp.FlowLM(pool, cfg, np.zeros(xnp.flow_lm.blob_size(cfg), np.float32))
    with pytest.raises(xnp.XnpError):  # the blob does not match the layout
        xnp.FlowLM(pool, cfg, np.zeros(10, np.float32))


# ---- voice files (ptts-wasm/src/lib.rs:291-325, 394-396) ------------------------------------------
def test_voice_files_are_read_and_checked_as_the_reference_checks_them(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(3)
    names = [xnp.voice_kv_name(i) for i in range(2)]
    assert names[1] == "transformer.layers.1.self_attn/cache"
    good = {nm: rng.standard_normal((2, 1, 5, 4, 64)).astype(np.float32) for nm in names}
    path = tmp_path / "voice.safetensors"
    save_file(good, str(path))
    frames, layers = xnp.voice_layers(xnp.read_voice_file(str(path)), 2, 4)
    assert frames == 5
    assert np.array_equal(layers[1], good[names[1]][:, 0])

    def bad(name, arr, match):
        t = dict(good)
        if arr is None:
            del t[name]
        else:
            t[name] = arr
        with pytest.raises(ValueError, match=match):
            xnp.voice_layers(t, 2, 4)

    bad(names[1], None, "expected f32 tensor: transformer.layers.1.self_attn/cache")
    bad(names[0], good[names[0]].astype(np.float16), "expected f32 tensor")
    bad(names[0], np.zeros((3, 1, 5, 4, 64), np.float32), "expected a first dim of size 2, got 3")
    bad(names[0], np.zeros((2, 2, 5, 4, 64), np.float32), "batch of 2")
    bad(names[0], np.zeros((2, 1, 5, 8, 64), np.float32), "8 heads of 64, the pool holds 4")
    bad(names[1], np.zeros((2, 1, 6, 4, 64), np.float32), "6 frames, layer 0 holds 5")
    bad(names[0], np.zeros((2, 5, 4, 64), np.float32), "expected 5 dims")


def test_random_stream_lifecycles_keep_the_page_accounting():
    # Seeded random sequences of open, advance, batched appends (ended or aborted), forks
    # (with_seq_budget: full pages shared, the partial one copied) and closes on a small pool, so
    # that refusals (no free page, no free stream, capacity) are frequent.  After every call: the
    # free pages are the pool's pages minus the distinct pages the streams hold; a stream holds
    # exactly ceil(end / 16) pages, in [0, NB); a page held twice is a full page of both holders; a
    # refused call changes neither ends nor the free count.
    NB, S, MB = 24, 6, 6
    rng = np.random.default_rng(20261202)
    p = pool(num_blocks=NB, max_streams=S, max_blocks_per_stream=MB)
    model = {}  # sid -> [end, capacity]

    def pages_needed(end, t):
        return (end + t + 15) // 16 - (end + 15) // 16

    def check():
        held = {}
        for sid, (end, cap) in model.items():
            assert p.current_end(sid) == end
            blk = p.blocks(sid)
            live = [(b, pg) for b, pg in enumerate(blk) if pg >= 0]
            assert len(live) == (end + 15) // 16 and [b for b, _ in live] == list(range(len(live))), (sid, blk, end)
            for b, pg in live:
                assert 0 <= pg < NB
                held.setdefault(pg, []).append((sid, b, end))
        for pg, owners in held.items():
            if len(owners) > 1:  # shared by a fork: a full page for every holder
                assert all((b + 1) * 16 <= end for _, b, end in owners), (pg, owners)
        assert p.stats()["free_blocks"] == NB - len(held)
        assert p.stats()["open_streams"] == len(model)

    def refused(call):
        before = ({s: p.current_end(s) for s in model}, p.stats()["free_blocks"])
        with pytest.raises(xnp.XnpError):
            call()
        assert before == ({s: p.current_end(s) for s in model}, p.stats()["free_blocks"])

    for _ in range(3000):
        op = rng.integers(0, 6)
        free = p.stats()["free_blocks"]
        sids = list(model)
        if op == 0 or not sids:  # open
            cap = int(rng.integers(1, MB * 16 + 1))
            if len(model) < S:
                model[p.init_state(cap)] = [0, cap]
            else:
                refused(lambda: p.init_state(cap))
        elif op == 1:  # advance
            sid = sids[rng.integers(len(sids))]
            end, cap = model[sid]
            n = int(rng.integers(0, cap - end + 1))
            if pages_needed(end, n) <= free:
                p.advance(sid, n)
                model[sid][0] += n
            else:
                refused(lambda: p.advance(sid, n))
        elif op == 2:  # a batch of t rows on some streams, ended or aborted
            pick = [s for s in sids if rng.random() < 0.5] or sids[:1]
            t = int(rng.integers(1, 40))
            need = sum(pages_needed(model[s][0], t) for s in pick)
            if any(model[s][0] + t > model[s][1] for s in pick) or need > free:
                refused(lambda: p.begin(pick, t=t))
            else:
                p.begin(pick, t=t)
                assert p.stats()["free_blocks"] == free - need
                if rng.random() < 0.3:
                    p.abort()
                else:
                    p.end()
                    for s in pick:
                        model[s][0] += t
        elif op == 3:  # fork
            sid = sids[rng.integers(len(sids))]
            end = model[sid][0]
            budget = int(rng.integers(end, MB * 16 + 1)) if end <= MB * 16 else end
            tail = end % 16 != 0
            if len(model) < S and (not tail or free > 0):
                model[p.with_seq_budget(sid, budget)] = [end, budget]
            else:
                refused(lambda: p.with_seq_budget(sid, budget))
        elif op == 4:  # a budget below the filled rows is refused
            sid = sids[rng.integers(len(sids))]
            if model[sid][0] > 0:
                refused(lambda: p.with_seq_budget(sid, model[sid][0] - 1))
        else:  # close
            sid = sids[rng.integers(len(sids))]
            p.close(sid)
            del model[sid]
        check()
    for sid in list(model):
        p.close(sid)
    assert p.stats()["free_blocks"] == NB
