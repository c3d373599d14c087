"""Python binding of the C ABI in include/xnp_kv.h (libxnp_kv.so, built next to this file).

The method names follow the reference's Rust API for the flow-LM cache, so a caller ported
from ptts reads the same:

    StreamingMultiheadAttention::init_state   transformer.rs:169-180   KvPool.init_state
    StreamingTransformerState::with_seq_budget transformer.rs:350-392  KvPool.with_seq_budget
    StreamingTransformerState::advance        transformer.rs:337-344   KvPool.advance
    StreamingTransformer::start_ring          transformer.rs:842-852   KvPool.start_ring
    StreamingTransformer::set_ring_slot       transformer.rs:855-871   KvPool.set_ring_slot
    StreamingTransformer::evict               transformer.rs:879-929   KvPool.evict
    complete_kv + sdpa_decode / prefill       transformer.rs:61-92,183-251  KvPool.attend

Device buffers are torch tensors (plumbing only: every computation runs in the library's HIP
kernels).  A refused call raises XnpError carrying the library's status and message.
"""
from __future__ import annotations

import ctypes
import os
from typing import Iterable, Optional, Sequence

_HERE = os.path.dirname(os.path.abspath(__file__))
# XNP_KV_LIB names another build of the same library: the host-sanitizer build that
# `make -C xn-ptts_amd/csrc asan-check` runs the CPU tests against.
LIB_PATH = os.environ.get("XNP_KV_LIB") or os.path.join(_HERE, "libxnp_kv.so")

F32, BF16, I8 = 0, 1, 2
DTYPES = {"f32": F32, "bf16": BF16, "i8": I8}
RING_SHIFT, RING_ABSOLUTE = 1, 2
RING_MODES = {"shift": RING_SHIFT, "absolute": RING_ABSOLUTE}
POOL_HOST_ONLY = 1
BLOCK = 16

STATUS = {
    0: "XNP_OK", 1: "XNP_E_INVALID", 2: "XNP_E_STREAM", 3: "XNP_E_NO_ROOM",
    4: "XNP_E_OUT_OF_BLOCKS", 5: "XNP_E_RING", 6: "XNP_E_EVICT", 7: "XNP_E_BUDGET",
    8: "XNP_E_HEADS", 9: "XNP_E_STATE", 10: "XNP_E_HIP",
}

# Every entry point include/xnp_kv.h declares, with its ctypes signature.
_c = ctypes
_p = _c.c_void_p
_i32 = _c.c_int32
_i32p = _c.POINTER(_c.c_int32)


class PoolDesc(_c.Structure):
    _fields_ = [
        ("num_layers", _i32), ("num_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("num_blocks", _i32), ("max_streams", _i32), ("max_blocks_per_stream", _i32),
        ("cache_dtype", _i32), ("act_dtype", _i32), ("max_period", _c.c_float),
        ("max_pos", _i32), ("flags", _i32), ("page_seed", _c.c_uint64), ("device", _i32),
        ("decode_split", _i32),
    ]


class LayerWeightsC(_c.Structure):
    """xnp_layer_weights: device pointers of one layer's q8 projections, norms and layer scales."""
    _fields_ = [("d_model", _i32), ("ff", _i32), ("gelu", _i32),
                ("wqkv", _p), ("sqkv", _p), ("wout", _p), ("sout", _p), ("w1", _p), ("s1", _p),
                ("w2", _p), ("s2", _p), ("ln1_w", _p), ("ln1_b", _p), ("ln2_w", _p), ("ln2_b", _p),
                ("ls1", _p), ("ls2", _p)]


class StreamInfo(_c.Structure):
    _fields_ = [(n, _i32) for n in (
        "current_end", "capacity", "ring_mode", "ring_write", "ring_filled", "ring_prefix",
        "ring_shift", "in_view", "blocks", "shared", "window")]


class PoolStats(_c.Structure):
    _fields_ = [("free_blocks", _i32), ("open_streams", _i32), ("batch_open", _i32),
                ("work_items", _i32), ("device_bytes", _c.c_int64), ("rope_rows", _i32),
                ("decode_waves", _i32)]


SIGNATURES = {
    "xnp_pool_create": (_i32, [_c.POINTER(PoolDesc), _c.POINTER(_p)]),
    "xnp_pool_destroy": (_i32, [_p]),
    "xnp_pool_stats_get": (_i32, [_p, _c.POINTER(PoolStats)]),
    "xnp_pool_rope_rows": (_i32, [_p, _i32, _i32, _c.POINTER(_c.c_float)]),
    "xnp_pool_time_next": (_i32, [_p, _p, _p]),
    "xnp_pool_check_tables": (_i32, [_p, _i32p, _p]),
    "xnp_stream_open": (_i32, [_p, _i32, _i32p]),
    "xnp_stream_close": (_i32, [_p, _i32]),
    "xnp_stream_fork": (_i32, [_p, _i32, _i32, _i32p, _p]),
    "xnp_stream_info_get": (_i32, [_p, _i32, _c.POINTER(StreamInfo)]),
    "xnp_stream_advance": (_i32, [_p, _i32, _i32]),
    "xnp_stream_blocks": (_i32, [_p, _i32, _i32p, _i32, _i32p]),
    "xnp_ring_valid": (_i32, [_p, _i32, _c.POINTER(_c.c_uint8), _i32]),
    "xnp_write_rows": (_i32, [_p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p]),
    "xnp_stream_load_kv": (_i32, [_p, _i32, _i32, _p, _i32, _p]),
    "xnp_window_open": (_i32, [_p, _i32, _i32p]),
    "xnp_flow_linear_q8": (_i32, [_p, _i32, _i32, _i32, _p, _p, _p, _i32, _i32, _p, _i32, _p, _i32, _c.c_float, _p]),
    "xnp_layer_norm_mod": (_i32, [_p, _i32, _i32, _p, _p, _c.c_float, _p, _p, _i32, _p, _p]),
    "xnp_read_rows": (_i32, [_p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p]),
    "xnp_ring_start": (_i32, [_p, _i32, _i32, _i32, _p]),
    "xnp_ring_set_slot": (_i32, [_p, _i32, _i32]),
    "xnp_ring_evict": (_i32, [_p, _i32, _i32, _i32p, _i32, _p]),
    "xnp_ring_slide": (_i32, [_p, _i32, _i32, _i32, _i32, _i32, _c.c_int64, _p]),
    "xnp_ring_slide_batch": (_i32, [_p, _i32p, _i32, _i32, _i32, _i32, _i32, _c.POINTER(_c.c_int64), _i32p, _p]),
    "xnp_batch_begin": (_i32, [_p, _i32p, _i32, _i32, _p]),
    "xnp_append": (_i32, [_p, _i32, _p, _p, _p]),
    "xnp_decode": (_i32, [_p, _i32, _p, _p, _c.c_float, _p]),
    "xnp_prefill": (_i32, [_p, _i32, _p, _p, _c.c_float, _p]),
    "xnp_attend": (_i32, [_p, _i32, _p, _p, _p, _p, _c.c_float, _p]),
    "xnp_batch_end": (_i32, [_p]),
    "xnp_batch_abort": (_i32, [_p]),
    "xnp_layer_workspace": (_i32, [_p, _i32, _i32, _i32, _c.POINTER(_c.c_uint64)]),
    "xnp_layer_step": (_i32, [_p, _i32, _p, _p, _p, _c.c_uint64, _p]),
    "xnp_layer_step_static": (_i32, [_p, _i32, _p, _p, _p]),
    "xnp_debug_set_block": (_i32, [_p, _i32, _i32, _i32]),
    "xnp_layer_norm": (_i32, [_p, _i32, _i32, _p, _p, _c.c_float, _p, _p]),
    "xnp_linear_q8": (_i32, [_p, _i32, _i32, _p, _p, _i32, _i32, _p, _p, _p]),
    "xnp_quantize_rows": (_i32, [_p, _i32, _i32, _p, _p]),
    "xnp_flow_lm_weights_size": (_i32, [_p, _c.POINTER(_c.c_int64)]),
    "xnp_flow_lm_create": (_i32, [_p, _p, _p, _c.c_int64, _c.POINTER(_p)]),
    "xnp_flow_lm_destroy": (_i32, [_p]),
    "xnp_flow_lm_prompt_text": (_i32, [_p, _i32p, _i32, _p, _i32, _p]),
    "xnp_flow_lm_set_condition": (_i32, [_p, _p, _i32]),
    "xnp_flow_lm_step": (_i32, [_p, _i32p, _i32, _p, _p, _p, _p, _p, _p]),
    "xnp_flow_lm_step_graph": (_i32, [_p, _i32p, _i32, _p, _p, _p, _p, _p, _p]),
    "xnp_frame_budget": (_i32, [_i32, _c.c_double]),
    "xnp_seq_budget": (_i32, [_i32, _i32]),
    "xnp_last_error": (_c.c_char_p, []),
}

_lib = None


def load_library(path: str = LIB_PATH):
    """Load libxnp_kv.so; raise if it is missing (there is no fallback path)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build() (make -C xn-ptts_amd/csrc)")
    # torch ships its own HIP runtime under the same soname (libamdhip64.so.7).  Loading torch
    # first makes the library bind to that one; loaded the other way round, the process would
    # hold two HIP runtimes and torch's would find no device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class XnpError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.name = STATUS.get(status, str(status))
        self.message = message


def _check(status: int):
    if status != 0:
        raise XnpError(status, _lib.xnp_last_error().decode())


def frame_budget(num_tokens: int, frame_rate: float = 12.5) -> int:
    return load_library().xnp_frame_budget(num_tokens, frame_rate)


def seq_budget(num_tokens: int, frame_budget_: int) -> int:
    return load_library().xnp_seq_budget(num_tokens, frame_budget_)


def voice_kv_name(layer: int) -> str:
    """The tensor holding layer `layer` of a voice stored as the KV cache (ptts-wasm/src/lib.rs:394-396)."""
    return f"transformer.layers.{layer}.self_attn/cache"


def voice_layers(tensors, num_layers: int, num_heads: int, head_dim: int = 64):
    """Check a KV-cache voice (voice_from_kv_cache, ptts-wasm/src/lib.rs:291-325) and return
    (frames, [per layer: the f32 [2, frames, heads, head_dim] tensor]).  `tensors` maps names to
    numpy arrays or torch tensors, as a safetensors file loads.  The errors are the reference's."""
    layers, frames = [], None
    for i in range(num_layers):
        name = voice_kv_name(i)
        t = tensors.get(name)
        if t is None or str(t.dtype) not in ("float32", "torch.float32"):
            raise ValueError(f"expected f32 tensor: {name}")
        if len(t.shape) != 5:
            raise ValueError(f"{name}: expected 5 dims [2, batch, seq, heads, head_dim], got {tuple(t.shape)}")
        two, batch, seq, heads, hd = (int(d) for d in t.shape)
        if two != 2:
            raise ValueError(f"{name}: expected a first dim of size 2, got {two}")
        if batch != 1:
            raise ValueError(f"{name}: a stream holds one voice, got a batch of {batch}")
        if heads != num_heads or hd != head_dim:
            raise ValueError(f"{name}: {heads} heads of {hd}, the pool holds {num_heads} of {head_dim}")
        if frames is not None and seq != frames:
            raise ValueError(f"{name}: {seq} frames, layer 0 holds {frames}")
        frames = seq
        layers.append(t.reshape(2, seq, heads, hd))
    return frames, layers


def read_voice_file(path: str):
    """The tensors of a safetensors voice file, as numpy arrays (read on the host)."""
    from safetensors.numpy import load_file
    return load_file(path)


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is not None:
        return stream
    import torch
    if torch.cuda.is_available() and torch.cuda.is_initialized():
        return torch.cuda.current_stream().cuda_stream
    return None


class KvPool:
    """A paged K/V store for `num_layers` flow-LM layers, shared by many streams on one GPU."""

    def __init__(self, *, num_layers: int, num_heads: int, num_blocks: int, max_streams: int,
                 max_blocks_per_stream: int, head_dim: int = 64, num_kv_heads: Optional[int] = None,
                 cache_dtype: str = "bf16", act_dtype: str = "bf16", max_period: float = 10000.0,
                 max_pos: int = 4096, page_seed: int = 0, host_only: bool = False, device: int = 0,
                 decode_split: int = 0):
        lib = load_library()
        self.desc = PoolDesc(
            num_layers=num_layers, num_heads=num_heads,
            num_kv_heads=num_kv_heads if num_kv_heads is not None else num_heads,
            head_dim=head_dim, num_blocks=num_blocks, max_streams=max_streams,
            max_blocks_per_stream=max_blocks_per_stream, cache_dtype=DTYPES[cache_dtype],
            act_dtype=DTYPES[act_dtype], max_period=max_period, max_pos=max_pos,
            flags=POOL_HOST_ONLY if host_only else 0, page_seed=page_seed, device=device,
            decode_split=decode_split)
        self.cache_dtype, self.act_dtype = cache_dtype, act_dtype
        self.host_only = host_only
        h = _p()
        _check(lib.xnp_pool_create(ctypes.byref(self.desc), ctypes.byref(h)))
        self._h = h
        self._lib = lib

    # -- pool ---------------------------------------------------------------------------------
    def close_pool(self):
        if self._h:
            self._lib.xnp_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close_pool()
        except Exception:
            pass

    def stats(self) -> dict:
        s = PoolStats()
        _check(self._lib.xnp_pool_stats_get(self._h, ctypes.byref(s)))
        return {n: getattr(s, n) for n, _ in PoolStats._fields_}

    def check_tables(self, stream=None) -> int:
        """Device block-table entries that differ from the host's page map (0 when consistent)."""
        bad = _i32()
        _check(self._lib.xnp_pool_check_tables(self._h, ctypes.byref(bad), _stream(stream)))
        return bad.value

    def time_next(self, start_event, stop_event):
        """Have the next decode/prefill launch record these hipEvent_t handles around its kernel
        (either may be None: a start from one launch and a stop from a later one)."""
        _check(self._lib.xnp_pool_time_next(self._h, start_event, stop_event))

    def debug_set_block(self, sid: int, blk: int, page: int):
        """Test hook, host-only pools: plant a page map entry (xnp_debug_set_block)."""
        _check(self._lib.xnp_debug_set_block(self._h, sid, blk, page))

    def rope_rows(self, pos0: int, n: int):
        import numpy as np
        out = np.zeros((n, self.desc.head_dim // 2, 2), np.float32)
        _check(self._lib.xnp_pool_rope_rows(self._h, pos0, n, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    # -- streams (transformer.rs:169-180, 337-392) --------------------------------------------
    def init_state(self, capacity: int) -> int:
        sid = _i32()
        _check(self._lib.xnp_stream_open(self._h, capacity, ctypes.byref(sid)))
        return sid.value

    def close(self, sid: int):
        _check(self._lib.xnp_stream_close(self._h, sid))

    def init_window(self, context: int) -> int:
        """MimiStreamingMultiheadAttention::init_state (transformer.rs:416-418): a stream whose
        steps attend the last `context` positions (KvCache::new(context)), rows placing themselves."""
        sid = _i32()
        _check(self._lib.xnp_window_open(self._h, context, ctypes.byref(sid)))
        return sid.value

    def with_seq_budget(self, sid: int, budget: int, stream=None) -> int:
        out = _i32()
        _check(self._lib.xnp_stream_fork(self._h, sid, budget, ctypes.byref(out), _stream(stream)))
        return out.value

    def advance(self, sid: int, n: int):
        _check(self._lib.xnp_stream_advance(self._h, sid, n))

    def info(self, sid: int) -> dict:
        s = StreamInfo()
        _check(self._lib.xnp_stream_info_get(self._h, sid, ctypes.byref(s)))
        return {n: getattr(s, n) for n, _ in StreamInfo._fields_}

    def current_end(self, sid: int) -> int:
        return self.info(sid)["current_end"]

    def blocks(self, sid: int) -> list:
        cnt = _i32()
        _check(self._lib.xnp_stream_blocks(self._h, sid, None, 0, ctypes.byref(cnt)))
        arr = (_i32 * max(cnt.value, 1))()
        _check(self._lib.xnp_stream_blocks(self._h, sid, arr, cnt.value, ctypes.byref(cnt)))
        return list(arr[:cnt.value])

    def valid(self, sid: int) -> list:
        cap = self.info(sid)["capacity"]
        arr = (ctypes.c_uint8 * max(cap, 1))()
        _check(self._lib.xnp_ring_valid(self._h, sid, arr, cap))
        return [bool(x) for x in arr[:cap]]

    def write_rows(self, sid: int, layer: int, kv: int, slot0: int, rows, scales=None, stream=None):
        n = rows.shape[0] if rows is not None else 0
        _check(self._lib.xnp_write_rows(self._h, sid, layer, kv, slot0, n, _ptr(rows), _ptr(scales),
                                        _stream(stream)))

    def load_kv(self, sid: int, layer: int, kv, stream=None):
        """Rows [0, n) of one layer from a device f32 [2, n, H, D] tensor (xnp_stream_load_kv)."""
        n = kv.shape[1]
        _check(self._lib.xnp_stream_load_kv(self._h, sid, layer, _ptr(kv), n, _stream(stream)))

    def load_voice(self, voice, capacity: Optional[int] = None, stream=None) -> int:
        """A stream holding a voice stored as the KV cache (`embeddings_v2/` voices): a path to a
        safetensors file, or its tensors by name.  The stream's capacity is the voice's length
        unless given; give each generation its own budget with with_seq_budget, which shares
        the voice's full pages instead of copying them (transformer.rs:350-392)."""
        import torch
        tensors = read_voice_file(voice) if isinstance(voice, (str, os.PathLike)) else voice
        frames, layers = voice_layers(tensors, self.desc.num_layers, self.desc.num_heads, self.desc.head_dim)
        sid = self.init_state(frames if capacity is None else capacity)
        try:
            self.advance(sid, frames)
            dev = torch.device("cuda", self.desc.device)
            staged = [torch.as_tensor(t).to(dev, torch.float32).contiguous() for t in layers]
            for layer, t in enumerate(staged):
                self.load_kv(sid, layer, t, stream)
            torch.cuda.synchronize(dev)  # the staged copies are freed on return
        except BaseException:
            self.close(sid)
            raise
        return sid

    def read_rows(self, sid: int, layer: int, kv: int, slot0: int, rows, scales=None, stream=None):
        n = rows.shape[0]
        _check(self._lib.xnp_read_rows(self._h, sid, layer, kv, slot0, n, _ptr(rows), _ptr(scales),
                                       _stream(stream)))

    # -- ring (transformer.rs:842-929, s2s.rs:318-333) ----------------------------------------
    def start_ring(self, sid: int, mode: str = "shift", prefix: int = 0, stream=None):
        _check(self._lib.xnp_ring_start(self._h, sid, RING_MODES[mode], prefix, _stream(stream)))

    def set_ring_slot(self, sid: int, slot: int):
        _check(self._lib.xnp_ring_set_slot(self._h, sid, slot))

    def evict(self, sid: int, prefix: int, slots: Sequence[int], stream=None):
        arr = (_i32 * max(len(slots), 1))(*slots)
        _check(self._lib.xnp_ring_evict(self._h, sid, prefix, arr, len(slots), _stream(stream)))

    def slide(self, sid: int, prefix: int, span: int, window: int, drop: int, step: int, stream=None):
        _check(self._lib.xnp_ring_slide(self._h, sid, prefix, span, window, drop, step, _stream(stream)))

    def slide_batch(self, ids, prefix: int, span: int, window: int, drop: int, steps, stream=None):
        """slide() over many streams, stream i at steps[i], in one call."""
        ids = list(ids)
        n = len(ids)
        arr = (_i32 * max(n, 1))(*ids)
        st = (ctypes.c_int64 * max(n, 1))(*[int(x) for x in steps])
        failed = _i32(-1)
        _check(self._lib.xnp_ring_slide_batch(self._h, arr, n, prefix, span, window, drop, st,
                                              ctypes.byref(failed), _stream(stream)))

    # -- a batched step -----------------------------------------------------------------------
    def begin(self, ids: Iterable[int], t: int = 1, stream=None):
        ids = list(ids)
        arr = (_i32 * max(len(ids), 1))(*ids)
        self._stream_h = _stream(stream)
        _check(self._lib.xnp_batch_begin(self._h, arr, len(ids), t, self._stream_h))

    def append(self, layer: int, k, v):
        _check(self._lib.xnp_append(self._h, layer, _ptr(k), _ptr(v), self._stream_h))

    def decode(self, layer: int, q, out, scale: float):
        _check(self._lib.xnp_decode(self._h, layer, _ptr(q), _ptr(out), scale, self._stream_h))

    def prefill(self, layer: int, q, out, scale: float):
        _check(self._lib.xnp_prefill(self._h, layer, _ptr(q), _ptr(out), scale, self._stream_h))

    def attend(self, layer: int, q, k, v, out, scale: float):
        _check(self._lib.xnp_attend(self._h, layer, _ptr(q), _ptr(k), _ptr(v), _ptr(out), scale,
                                    self._stream_h))

    def layer_workspace(self, rows: int, d_model: int, ff: int) -> int:
        out = _c.c_uint64()
        _check(self._lib.xnp_layer_workspace(self._h, rows, d_model, ff, _c.byref(out)))
        return out.value

    def layer_step(self, layer: int, weights: "LayerWeights", x, workspace):
        """StreamingTransformerLayer::forward (transformer.rs:591-634) on every row of the open
        batch: x [n][t][d_model] bf16 is the residual stream, updated in place."""
        _check(self._lib.xnp_layer_step(self._h, layer, _c.byref(weights.c), _ptr(x), _ptr(workspace),
                                        workspace.numel() * workspace.element_size(), self._stream_h))

    def layer_step_static(self, layer: int, weights: "LayerWeights", x):
        """layer_step with the library's static scratch instead of a workspace: allocates nothing."""
        _check(self._lib.xnp_layer_step_static(self._h, layer, _c.byref(weights.c), _ptr(x), self._stream_h))

    def end(self):
        _check(self._lib.xnp_batch_end(self._h))

    def abort(self):
        _check(self._lib.xnp_batch_abort(self._h))


# ---- the rest of the layer (transformer.rs:591-634) ---------------------------------------------
GELU = {"erf": 0, "tanh": 1}
EPILOGUES = {"store": 0, "gelu_erf": 1, "gelu_tanh": 2, "residual": 3, "silu": 4, "silu_add": 5, "gated": 6,
             "axpy_f32": 7, "store_f32": 8, "add_f32": 9}


class LayerWeights:
    """One layer's weights on the device (torch tensors): int8 projections with per-channel f32
    scales, f32 norm weights and biases, optional layer scales."""

    def __init__(self, wqkv, sqkv, wout, sout, w1, s1, w2, s2, ln1_w, ln1_b, ln2_w, ln2_b,
                 ls1=None, ls2=None, gelu: str = "erf"):
        self.tensors = [wqkv, sqkv, wout, sout, w1, s1, w2, s2, ln1_w, ln1_b, ln2_w, ln2_b, ls1, ls2]
        self.c = LayerWeightsC(d_model=wout.shape[0], ff=w1.shape[0], gelu=GELU[gelu],
                               wqkv=_ptr(wqkv), sqkv=_ptr(sqkv), wout=_ptr(wout), sout=_ptr(sout),
                               w1=_ptr(w1), s1=_ptr(s1), w2=_ptr(w2), s2=_ptr(s2), ln1_w=_ptr(ln1_w),
                               ln1_b=_ptr(ln1_b), ln2_w=_ptr(ln2_w), ln2_b=_ptr(ln2_b), ls1=_ptr(ls1),
                               ls2=_ptr(ls2))


def quantize_rows(w):
    """Per-row int8 weights of a float32 numpy matrix: (q int8, scales f32), computed by the library."""
    import numpy as np
    w = np.ascontiguousarray(w, np.float32)
    q = np.zeros(w.shape, np.int8)
    s = np.zeros(w.shape[0], np.float32)
    _check(load_library().xnp_quantize_rows(w.ctypes.data, w.shape[0], w.shape[1], q.ctypes.data, s.ctypes.data))
    return q, s


def layer_norm(x, w, b, out, eps: float = 1e-5, stream=None):
    dim = x.shape[-1]
    _check(load_library().xnp_layer_norm(_ptr(x), x.numel() // dim, dim, _ptr(w), _ptr(b), eps, _ptr(out),
                                         _stream(stream)))


def linear_q8(x, w, s, y, epilogue: str = "store", ls=None, stream=None):
    k = x.shape[-1]
    _check(load_library().xnp_linear_q8(_ptr(x), x.numel() // k, k, _ptr(w), _ptr(s), w.shape[0],
                                        EPILOGUES[epilogue], _ptr(y), _ptr(ls), _stream(stream)))


def flow_linear_q8(x, w, s, y, epilogue: str = "store", bias=None, aux=None, alpha: float = 1.0, stream=None):
    """xnp_flow_linear_q8: x [rows][k] bf16 or f32 (f32: rounded as read; store or add_f32), w [n][k] int8,
    s [n], y [rows][>= n] (bf16, or f32 for axpy_f32 / store_f32); aux per the epilogue."""
    k = x.shape[-1]
    rows = x.numel() // k
    n = w.shape[0]
    ld_aux = aux.shape[-1] if aux is not None and aux.dim() > 1 else 0
    _check(load_library().xnp_flow_linear_q8(_ptr(x), int(x.dtype.is_floating_point and x.element_size() == 4),
                                             rows, k, _ptr(w), _ptr(s), _ptr(bias), n, EPILOGUES[epilogue], _ptr(y),
                                             y.shape[-1], _ptr(aux), ld_aux, alpha, _stream(stream)))


def layer_norm_mod(x, out, w=None, b=None, shift=None, scale=None, eps: float = 1e-6, stream=None):
    """xnp_layer_norm_mod on bf16 rows: LayerNorm (affine optional), then the AdaLN modulation when
    shift and scale (bf16 views whose rows have the stride of their base tensor) are given."""
    dim = x.shape[-1]
    ld_mod = shift.stride(0) if shift is not None else 0
    _check(load_library().xnp_layer_norm_mod(_ptr(x), x.numel() // dim, dim, _ptr(w), _ptr(b), eps, _ptr(shift),
                                             _ptr(scale), ld_mod, _ptr(out), _stream(stream)))
