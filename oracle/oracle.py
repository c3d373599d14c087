"""ctypes wrapper of liboracle.so, the CPU restatement of the reference's KV-cache path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU
baseline leg, as the checker.  The product (xn-ptts_amd/) never imports it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# XNP_ORACLE_LIB names another build of the oracle (the sanitizer build of `make -C oracle asan`)
LIB_PATH = os.environ.get("XNP_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
F32, BF16, I8 = 0, 1, 2
RING_NONE, RING_SHIFT, RING_ABSOLUTE = 0, 1, 2
DT = {"f32": F32, "bf16": BF16, "i8": I8}
MODES = {"shift": RING_SHIFT, "absolute": RING_ABSOLUTE}

_lib = None
_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: make -C oracle")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_bf16_round": (ctypes.c_float, [ctypes.c_float]),
            "orc_quant": (ctypes.c_int8, [ctypes.c_float, ctypes.c_float]),
            "orc_rope_row": (None, [ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int, _fp, _fp]),
            "orc_rotate": (None, [ctypes.c_int, _fp, _fp, _fp, ctypes.c_int]),
            "orc_open": (ctypes.c_void_p, [ctypes.c_int] * 7 + [ctypes.c_float]),
            "orc_close": (None, [ctypes.c_void_p]),
            "orc_current_end": (ctypes.c_int, [ctypes.c_void_p]),
            "orc_capacity": (ctypes.c_int, [ctypes.c_void_p]),
            "orc_ring_info": (None, [ctypes.c_void_p, _ip, _ip, _ip, _ip, _ip, _u8p]),
            "orc_attend": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _fp, _fp, _fp,
                                          ctypes.c_float, _fp, _dp]),
            "orc_append": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _fp, _fp]),
            "orc_attention": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _fp,
                                             ctypes.c_float, _fp, _dp]),
            "orc_commit": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
            "orc_advance": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
            "orc_start_ring": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
            "orc_set_ring_slot": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
            "orc_ring_restore": (ctypes.c_int, [ctypes.c_void_p] + [ctypes.c_int] * 6 + [_u8p]),
            "orc_evict": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _ip, ctypes.c_int]),
            "orc_with_seq_budget": (ctypes.c_void_p, [ctypes.c_void_p, ctypes.c_int]),
            "orc_read_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, _fp, _i8p, _fp]),
            "orc_write_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int, _fp, _i8p, _fp]),
            "orc_load_kv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _fp, ctypes.c_int]),
            "orc_window_open": (ctypes.c_void_p, [ctypes.c_int] * 6 + [ctypes.c_float]),
            "orc_window_close": (None, [ctypes.c_void_p]),
            "orc_window_attend": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _fp, _fp, _fp,
                                                 ctypes.c_float, _fp, _dp]),
            "orc_window_commit": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
            "orc_window_len": (ctypes.c_int, [ctypes.c_void_p]),
            "orc_window_offset": (ctypes.c_int, [ctypes.c_void_p]),
            "orc_window_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _fp]),
            "orc_batch_attend": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.c_int,
                                                _fp, _fp, _fp, ctypes.c_float, _fp]),
            "orc_batch_commit": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int]),
            "orc_batch_ring_step": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.c_int,
                                                   _ip, _ip, _fp, _fp, _fp, ctypes.c_float, _fp]),
            "orc_threads": (ctypes.c_int, []),
            "orc_set_threads": (None, [ctypes.c_int]),
            "orc_flow_lm_size": (ctypes.c_longlong, [ctypes.c_void_p]),
            "orc_linear_f32": (None, [_fp, ctypes.c_int, ctypes.c_int, _fp, _fp, ctypes.c_int, _fp]),
            "orc_flow_time_embedding": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_float, ctypes.c_float, _fp]),
            "orc_flow_net": (ctypes.c_int, [ctypes.c_void_p, _fp, _fp, _fp, _fp, _fp]),
            "orc_flow_lm_prompt_text": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_void_p, _ip, ctypes.c_int]),
            "orc_flow_lm_step": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_void_p, _fp, _fp, _fp, _fp, _fp]),
            "orc_flow_linear_q8": (None, [_fp, ctypes.c_int, ctypes.c_int, _i8p, _fp, _fp, ctypes.c_int, ctypes.c_int,
                                          _fp, ctypes.c_int, _fp, ctypes.c_int, ctypes.c_float]),
            "orc_layer_norm_mod": (None, [_fp, ctypes.c_int, ctypes.c_int, _fp, _fp, ctypes.c_float, _fp, _fp,
                                          ctypes.c_int, _fp]),
            "orc_flow_q8_prepare": (ctypes.c_void_p, [ctypes.c_void_p, _fp]),
            "orc_flow_q8_free": (None, [ctypes.c_void_p]),
            "orc_flow_q8_prompt_text": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _ip, ctypes.c_int]),
            "orc_flow_q8_step": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _fp, _fp, _fp, _fp, _fp]),
            "orc_layer_norm": (None, [_fp, ctypes.c_int, ctypes.c_int, _fp, _fp, ctypes.c_float, ctypes.c_int, _fp]),
            "orc_quantize_rows": (None, [_fp, ctypes.c_int, ctypes.c_int, _i8p, _fp]),
            "orc_linear_q8": (None, [_fp, ctypes.c_int, ctypes.c_int, _i8p, _fp, ctypes.c_int, ctypes.c_int, _fp]),
            "orc_gelu": (ctypes.c_float, [ctypes.c_float, ctypes.c_int]),
            "orc_layer_step": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_void_p, ctypes.c_float, _fp]),
            "orc_last_error": (ctypes.c_char_p, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


class OracleError(RuntimeError):
    pass


def _ok(rc):
    if rc != 0:
        raise OracleError(lib().orc_last_error().decode())


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_fp)


def bf16_round(x: float) -> float:
    return lib().orc_bf16_round(x)


def quant(y: float, s: float) -> int:
    return lib().orc_quant(y, s)


def rope_row(head_dim: int, max_period: float, pos: float, act: str = "f32"):
    c = np.zeros(head_dim // 2, np.float32)
    s = np.zeros(head_dim // 2, np.float32)
    lib().orc_rope_row(head_dim, max_period, pos, DT[act], c.ctypes.data_as(_fp), s.ctypes.data_as(_fp))
    return c, s


def rotate(x, cos_row, sin_row, act: str = "f32"):
    x, xp = _f32(np.array(x, np.float32, copy=True))
    c, cp = _f32(cos_row)
    s, sp = _f32(sin_row)
    lib().orc_rotate(x.shape[-1], xp, cp, sp, DT[act])
    return x


class Stream:
    """One stream's StreamingMHAState over all layers, contiguous [S_cap][H][D] per layer."""

    def __init__(self, layers, heads, head_dim, capacity, cache="f32", act="f32", kv_heads=None,
                 max_period=10000.0, _handle=None):
        self.L, self.H, self.D = layers, heads, head_dim
        self.KVH = kv_heads or heads
        self.cache, self.act = cache, act
        self.max_period = max_period
        if _handle is None:
            _handle = lib().orc_open(layers, heads, self.KVH, head_dim, capacity, DT[cache], DT[act], max_period)
            if not _handle:
                raise OracleError(lib().orc_last_error().decode())
        self.h = _handle

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_close(self.h)
            self.h = None

    @property
    def current_end(self):
        return lib().orc_current_end(self.h)

    @property
    def capacity(self):
        return lib().orc_capacity(self.h)

    def ring_info(self):
        vals = [ctypes.c_int() for _ in range(5)]
        valid = np.zeros(max(self.capacity, 1), np.uint8)
        lib().orc_ring_info(self.h, *[ctypes.byref(v) for v in vals], valid.ctypes.data_as(_u8p))
        mode, write, filled, prefix, shift = [v.value for v in vals]
        return dict(mode=mode, write=write, filled=filled, prefix=prefix, shift=shift,
                    valid=valid[:self.capacity].astype(bool))

    def attend(self, layer, q, k, v, scale=0.125):
        q, qp = _f32(q)
        k, kp = _f32(k)
        v, vp = _f32(v)
        t = q.shape[0]
        out = np.zeros((t, self.H, self.D), np.float32)
        out64 = np.zeros((t, self.H, self.D), np.float64)
        _ok(lib().orc_attend(self.h, layer, t, qp, kp, vp, scale, out.ctypes.data_as(_fp),
                             out64.ctypes.data_as(_dp)))
        return out, out64

    def append(self, layer, k, v):
        k, kp = _f32(k)
        v, vp = _f32(v)
        _ok(lib().orc_append(self.h, layer, k.shape[0], kp, vp))

    def attention(self, layer, q, scale=0.125):
        q, qp = _f32(q)
        t = q.shape[0]
        out = np.zeros((t, self.H, self.D), np.float32)
        out64 = np.zeros((t, self.H, self.D), np.float64)
        _ok(lib().orc_attention(self.h, layer, t, qp, scale, out.ctypes.data_as(_fp),
                                out64.ctypes.data_as(_dp)))
        return out, out64

    def commit(self, t=1):
        _ok(lib().orc_commit(self.h, t))

    def advance(self, n):
        _ok(lib().orc_advance(self.h, n))

    def start_ring(self, mode="shift", prefix=0):
        _ok(lib().orc_start_ring(self.h, MODES[mode], prefix))

    def ring_restore(self, mode, write, filled, prefix, shift, current_end, valid):
        v = np.ascontiguousarray(valid, np.uint8)
        _ok(lib().orc_ring_restore(self.h, MODES[mode], write, filled, prefix, shift, current_end,
                                   v.ctypes.data_as(_u8p)))

    def set_ring_slot(self, slot):
        _ok(lib().orc_set_ring_slot(self.h, slot))

    def evict(self, prefix, slots):
        arr = (ctypes.c_int * max(len(slots), 1))(*slots)
        _ok(lib().orc_evict(self.h, prefix, arr, len(slots)))

    def with_seq_budget(self, budget):
        h = lib().orc_with_seq_budget(self.h, budget)
        if not h:
            raise OracleError(lib().orc_last_error().decode())
        return Stream(self.L, self.H, self.D, budget, self.cache, self.act, self.KVH, self.max_period, _handle=h)

    def read_rows(self, layer, kv, slot0, n):
        vals = np.zeros((n, self.H, self.D), np.float32)
        q8 = np.zeros((n, self.H, self.D), np.int8)
        nb = ((slot0 + n - 1) // 16 - slot0 // 16 + 1) if n > 0 else 0
        scales = np.zeros((max(nb, 1), self.H), np.float32)
        _ok(lib().orc_read_rows(self.h, layer, kv, slot0, n, vals.ctypes.data_as(_fp),
                                q8.ctypes.data_as(_i8p), scales.ctypes.data_as(_fp)))
        return vals, q8, scales[:nb]

    def write_rows(self, layer, kv, slot0, vals=None, q8=None, scales=None):
        n = (vals if vals is not None else q8).shape[0]
        v, vp = _f32(vals if vals is not None else np.zeros((n, self.H, self.D), np.float32))
        q = np.ascontiguousarray(q8 if q8 is not None else np.zeros((n, self.H, self.D), np.int8), np.int8)
        s, sp = _f32(scales if scales is not None else np.zeros((max(n // 16 + 2, 1), self.H), np.float32))
        _ok(lib().orc_write_rows(self.h, layer, kv, slot0, n, vp, q.ctypes.data_as(_i8p), sp))

    def load_kv(self, layer, kv):
        """voice_from_kv_cache (ptts-wasm/src/lib.rs:291-325): kv [2][n][H][D] f32 -> rows [0, n)."""
        kv = np.ascontiguousarray(kv, np.float32)
        assert kv.ndim == 4 and kv.shape[0] == 2, kv.shape
        a, ap = _f32(kv)
        _ok(lib().orc_load_kv(self.h, layer, ap, kv.shape[1]))


class Window:
    """Mimi's KvCache over all layers (transformer.rs:257-318): the last context - 1 rows kept
    between steps, a step of t rows attending the causal window of `context` positions."""

    def __init__(self, layers, heads, head_dim, context, rows_max=4, act="f32", max_period=10000.0):
        self.L, self.H, self.D, self.context = layers, heads, head_dim, context
        self.h = lib().orc_window_open(layers, heads, head_dim, context, rows_max, DT[act], max_period)
        if not self.h:
            raise OracleError(lib().orc_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_window_close(self.h)
            self.h = None

    @property
    def len(self):
        return lib().orc_window_len(self.h)

    @property
    def offset(self):
        return lib().orc_window_offset(self.h)

    def attend(self, layer, q, k, v, scale=0.125):
        """q, k, v [t][H][D]; returns (out, out64)."""
        q, qp = _f32(q)
        k, kp = _f32(k)
        v, vp = _f32(v)
        t = q.shape[0]
        out = np.zeros((t, self.H, self.D), np.float32)
        out64 = np.zeros((t, self.H, self.D), np.float64)
        _ok(lib().orc_window_attend(self.h, layer, t, qp, kp, vp, scale, out.ctypes.data_as(_fp),
                                    out64.ctypes.data_as(_dp)))
        return out, out64

    def commit(self, t):
        _ok(lib().orc_window_commit(self.h, t))

    def rows(self, layer, kv):
        """The kept rows [len][H][D], oldest first (keys rotated)."""
        out = np.zeros((max(self.len, 1), self.H, self.D), np.float32)
        _ok(lib().orc_window_rows(self.h, layer, kv, out.ctypes.data_as(_fp)))
        return out[:self.len]


def batch_attend(streams, layer, q, k, v, scale=0.125):
    """One layer of a batched decode step over `streams`, OpenMP across streams."""
    n = len(streams)
    arr = (ctypes.c_void_p * n)(*[s.h for s in streams])
    q, qp = _f32(q)
    k, kp = _f32(k)
    v, vp = _f32(v)
    out = np.zeros_like(q)
    _ok(lib().orc_batch_attend(arr, n, layer, qp, kp, vp, scale, out.ctypes.data_as(_fp)))
    return out


def batch_commit(streams):
    n = len(streams)
    arr = (ctypes.c_void_p * n)(*[s.h for s in streams])
    _ok(lib().orc_batch_commit(arr, n))


def batch_ring_step(streams, layer, drop, slot, k, v, q=None, scale=0.125):
    """Each stream i: evict slot drop[i] (if >= 0, prefix 0), take slot slot[i], then append row i of
    k, v to `layer` (q None) or attend with row i of q as well, and commit the row (OpenMP across
    streams).  Returns the attention outputs [n][H][D] when q is given."""
    n = len(streams)
    arr = (ctypes.c_void_p * n)(*[s.h for s in streams])
    d = np.ascontiguousarray(drop, np.int32)
    sl = np.ascontiguousarray(slot, np.int32)
    k, kp = _f32(k)
    v, vp = _f32(v)
    out = None
    if q is not None:
        q, qp = _f32(q)
        out = np.zeros_like(q)
        op = out.ctypes.data_as(_fp)
    else:
        qp = op = None
    _ok(lib().orc_batch_ring_step(arr, n, layer, d.ctypes.data_as(_ip), sl.ctypes.data_as(_ip), qp, kp, vp, scale, op))
    return out


def batch_commit_t(streams, t):
    """Commit t rows on every stream (a prompt step)."""
    for st in streams:
        st.commit(t)


def threads() -> int:
    return lib().orc_threads()


def set_threads(n: int):
    lib().orc_set_threads(n)


# ---- the rest of the layer (transformer.rs:591-634) ------------------------------------------------
def layer_norm(x, w, b, eps=1e-5, act="f32"):
    x, xp = _f32(x)
    out = np.zeros_like(x)
    w, wp = _f32(w)
    b, bp = _f32(b)
    dim = x.shape[-1]
    lib().orc_layer_norm(xp, x.size // dim, dim, wp, bp, eps, DT[act], out.ctypes.data_as(_fp))
    return out


def quantize_rows(w):
    """Per-row int8 weights: (q [rows][cols] int8, scales [rows] f32)."""
    w, wp = _f32(w)
    q = np.zeros(w.shape, np.int8)
    s = np.zeros(w.shape[0], np.float32)
    lib().orc_quantize_rows(wp, w.shape[0], w.shape[1], q.ctypes.data_as(_i8p), s.ctypes.data_as(_fp))
    return q, s


def linear_q8(x, q, s, act="f32"):
    x, xp = _f32(x)
    q = np.ascontiguousarray(q, np.int8)
    s, sp = _f32(s)
    k = x.shape[-1]
    rows = x.size // k
    y = np.zeros(x.shape[:-1] + (q.shape[0],), np.float32)
    lib().orc_linear_q8(xp, rows, k, q.ctypes.data_as(_i8p), sp, q.shape[0], DT[act], y.ctypes.data_as(_fp))
    return y


def gelu(x: float, kind: str = "erf") -> float:
    return lib().orc_gelu(x, 0 if kind == "erf" else 1)


class _LayerWeightsC(ctypes.Structure):
    _fields_ = [("d_model", ctypes.c_int), ("ff", ctypes.c_int), ("gelu", ctypes.c_int),
                ("wqkv", _i8p), ("sqkv", _fp), ("wout", _i8p), ("sout", _fp),
                ("w1", _i8p), ("s1", _fp), ("w2", _i8p), ("s2", _fp),
                ("ln1_w", _fp), ("ln1_b", _fp), ("ln2_w", _fp), ("ln2_b", _fp),
                ("ls1", _fp), ("ls2", _fp)]


class LayerWeights:
    """One layer's q8 projections, norms and optional layer scales, as numpy arrays."""

    def __init__(self, wqkv, sqkv, wout, sout, w1, s1, w2, s2, ln1_w, ln1_b, ln2_w, ln2_b,
                 ls1=None, ls2=None, gelu="erf"):
        i8 = lambda a: np.ascontiguousarray(a, np.int8)
        f = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
        self.wqkv, self.wout, self.w1, self.w2 = i8(wqkv), i8(wout), i8(w1), i8(w2)
        self.sqkv, self.sout, self.s1, self.s2 = f(sqkv), f(sout), f(s1), f(s2)
        self.ln1_w, self.ln1_b, self.ln2_w, self.ln2_b = f(ln1_w), f(ln1_b), f(ln2_w), f(ln2_b)
        self.ls1, self.ls2 = f(ls1), f(ls2)
        self.gelu = gelu
        self.d_model = self.wout.shape[0]
        self.ff = self.w1.shape[0]

    def c(self):
        P = lambda a, t: a.ctypes.data_as(t) if a is not None else ctypes.cast(None, t)
        return _LayerWeightsC(self.d_model, self.ff, 0 if self.gelu == "erf" else 1,
                              P(self.wqkv, _i8p), P(self.sqkv, _fp), P(self.wout, _i8p), P(self.sout, _fp),
                              P(self.w1, _i8p), P(self.s1, _fp), P(self.w2, _i8p), P(self.s2, _fp),
                              P(self.ln1_w, _fp), P(self.ln1_b, _fp), P(self.ln2_w, _fp), P(self.ln2_b, _fp),
                              P(self.ls1, _fp), P(self.ls2, _fp))


def layer_step(streams, layer, weights: LayerWeights, x, scale=0.125):
    """One transformer layer on t rows of each stream: x [n][t][d_model] -> the updated x."""
    x = np.array(x, np.float32, copy=True, order="C")
    n, t = x.shape[0], x.shape[1]
    arr = (ctypes.c_void_p * n)(*[s_.h for s_ in streams])
    cw = weights.c()
    _ok(lib().orc_layer_step(arr, n, t, layer, ctypes.cast(ctypes.pointer(cw), ctypes.c_void_p), scale,
                             x.ctypes.data_as(_fp)))
    return x


FLOW_EPILOGUES = {"store": 0, "silu": 4, "silu_add": 5, "gated": 6, "axpy_f32": 7, "store_f32": 8, "add_f32": 9}


def flow_linear_q8(x, q, s, epilogue="store", bias=None, aux=None, out=None, alpha=1.0):
    """The flow net's q8 linear (oracle.h): x [rows][k] (rounded to bf16 as read), q [n][k] int8,
    s [n]; out [rows][n] is read by "gated" and returned."""
    x, xp = _f32(x)
    rows, k = x.shape
    n = q.shape[0]
    q = np.ascontiguousarray(q, np.int8)
    o = np.zeros((rows, n), np.float32) if out is None else np.array(out, np.float32, copy=True, order="C")
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    a = None if aux is None else np.ascontiguousarray(aux, np.float32)
    sv, sp = _f32(s)
    lib().orc_flow_linear_q8(xp, rows, k, q.ctypes.data_as(_i8p), sp, b.ctypes.data_as(_fp) if b is not None else None,
                             n, FLOW_EPILOGUES[epilogue], o.ctypes.data_as(_fp), n,
                             a.ctypes.data_as(_fp) if a is not None else None,
                             a.shape[-1] if a is not None and a.ndim > 1 else 0, alpha)
    return o


def layer_norm_mod(x, w=None, b=None, shift=None, scale=None, eps=1e-6):
    """LayerNorm of rows rounded to bf16, then the AdaLN modulation in bf16 steps (oracle.h)."""
    x, xp = _f32(x)
    rows, dim = x.shape
    out = np.zeros_like(x)
    P = lambda a: np.ascontiguousarray(a, np.float32).ctypes.data_as(_fp) if a is not None else None
    keep = [np.ascontiguousarray(a, np.float32) if a is not None else None for a in (w, b, shift, scale)]
    lib().orc_layer_norm_mod(xp, rows, dim, *[k.ctypes.data_as(_fp) if k is not None else None for k in keep[:2]], eps,
                             *[k.ctypes.data_as(_fp) if k is not None else None for k in keep[2:]],
                             keep[2].shape[-1] if keep[2] is not None else 0, out.ctypes.data_as(_fp))
    return out


# ---- the flow LM around the transformer (flow_lm.rs, mlp.rs, conditioners.rs), f32 -------------------
class _FlowDescC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("d_model", "num_heads", "num_layers", "ff", "ldim", "n_bins",
                                            "flow_dim", "flow_depth", "lsd_steps", "gelu", "time_norm", "z_dim",
                                            "flow_type", "precision", "num_kv_heads", "attn_dim")]


FLOW_TYPES = {"lsd": 0, "drifting": 1, "pointwise": 2}
PRECISIONS = {"f32": 0, "q8": 1}


class FlowLM:
    """The oracle's single-stream flow LM over a flat f32 weight blob (layout: oracle.h), in the
    config's precision: f32, or q8 (int8 weights quantized here, bf16 activations)."""

    def __init__(self, cfg, blob):
        self.cfg = cfg
        self.q8 = getattr(cfg, "precision", "f32") == "q8"
        self.d = _FlowDescC(cfg.d_model, cfg.num_heads, cfg.num_layers, cfg.dim_feedforward, cfg.ldim, cfg.n_bins,
                            cfg.flow_dim, cfg.flow_depth, cfg.lsd_decode_steps, 0 if cfg.gelu == "erf" else 1,
                            0 if cfg.time_rms_norm == "rms" else 1, getattr(cfg, "z_dim", 0),
                            FLOW_TYPES[getattr(cfg, "flow_type", "lsd")], PRECISIONS[getattr(cfg, "precision", "f32")],
                            getattr(cfg, "num_kv_heads", 0), getattr(cfg, "attn_dim", 0))
        self.blob = np.ascontiguousarray(blob, np.float32)
        n = lib().orc_flow_lm_size(self._dp())
        if n != self.blob.size:
            raise OracleError(f"the blob holds {self.blob.size} floats, the layout {n}")
        self._bp = self.blob.ctypes.data_as(_fp)
        self._q = None
        if self.q8:
            self._q = lib().orc_flow_q8_prepare(self._dp(), self._bp)
            if not self._q:
                raise OracleError(lib().orc_last_error().decode())

    def __del__(self):
        if getattr(self, "_q", None):
            lib().orc_flow_q8_free(self._q)
            self._q = None

    def _dp(self):
        return ctypes.cast(ctypes.pointer(self.d), ctypes.c_void_p)

    def stream(self, capacity):
        c = self.cfg
        dt = "bf16" if self.q8 else "f32"
        a = getattr(c, "attn_dim", 0) or c.d_model
        return Stream(c.num_layers, c.num_heads, a // c.num_heads, capacity, cache=dt, act=dt,
                      kv_heads=getattr(c, "num_kv_heads", 0) or None, max_period=c.max_period)

    def time_embedding(self, s, t):
        out = np.zeros(self.cfg.flow_dim, np.float32)
        _ok(lib().orc_flow_time_embedding(self._dp(), self._bp, s, t, out.ctypes.data_as(_fp)))
        return out

    def flow_net(self, c, t_emb, x0):
        c, cp = _f32(c)
        t, tp = _f32(t_emb)
        x, xp = _f32(x0)
        out = np.zeros(self.cfg.ldim, np.float32)
        _ok(lib().orc_flow_net(self._dp(), self._bp, cp, tp, xp, out.ctypes.data_as(_fp)))
        return out

    def prompt_text(self, st, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        if self.q8:
            _ok(lib().orc_flow_q8_prompt_text(self._q, st.h, ids.ctypes.data_as(_ip), ids.size))
        else:
            _ok(lib().orc_flow_lm_prompt_text(self._dp(), self._bp, st.h, ids.ctypes.data_as(_ip), ids.size))

    def step(self, st, latent_in, noise, cond=None):
        """One frame: (latent [ldim], eos logit); cond [d_model]: the conditions added to the step
        input (flow_lm.rs:304-307), or None."""
        lat = None if latent_in is None else np.ascontiguousarray(latent_in, np.float32)
        latp = lat.ctypes.data_as(_fp) if lat is not None else None
        c = None if cond is None else np.ascontiguousarray(cond, np.float32)
        cp = c.ctypes.data_as(_fp) if c is not None else None
        nz, nzp = _f32(noise)
        out = np.zeros(self.cfg.ldim, np.float32)
        eos = np.zeros(1, np.float32)
        if self.q8:
            _ok(lib().orc_flow_q8_step(self._q, st.h, latp, cp, nzp, out.ctypes.data_as(_fp), eos.ctypes.data_as(_fp)))
        else:
            _ok(lib().orc_flow_lm_step(self._dp(), self._bp, st.h, latp, cp, nzp, out.ctypes.data_as(_fp),
                                       eos.ctypes.data_as(_fp)))
        return out, float(eos[0])
