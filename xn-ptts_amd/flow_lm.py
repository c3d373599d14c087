"""The flow LM around the paged transformer (ptts/src/flow_lm.rs, mlp.rs, conditioners.rs): the
tensor layout of its weights, and FlowLM, the binding of the xnp_flow_lm_* entry points of
include/xnp_kv.h.  Two precisions: f32 throughout (one stream at a time, the reference's own
case), or q8 -- int8 per-channel weights on MFMA with bf16 activations, for many streams a frame.

    TTSModel::prompt_text          tts_model.rs:297-307    FlowLM.prompt_text
    TTSModel::generate_step_parts  tts_model.rs:365-378    FlowLM.step
    SimpleMLPAdaLN (the flow net)  mlp.rs:159-238          inside FlowLM.step
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np

from .kv import _check, _ptr, _stream, load_library

FREQ_DIM = 256  # the time embedders' frequency embedding (mlp.rs:186-193)


FLOW_TYPES = {"lsd": 0, "drifting": 1, "pointwise": 2}  # FlowType (flow_lm.rs:372-381)
PRECISIONS = {"f32": 0, "q8": 1}


@dataclass
class FlowLMConfig:
    """FlowLMConfig (flow_lm.rs:114-146).  z_dim 0: no z_proj; attn_dim 0: d_model; num_kv_heads 0:
    num_heads.  (FlowLM's transformer has no layer scale, flow_lm.rs:239-249; conditions are given at
    run time, FlowLM.set_condition and the conditions of FlowLM.step.)"""
    d_model: int = 512
    num_heads: int = 8
    num_layers: int = 6
    dim_feedforward: int = 2048
    ldim: int = 32
    n_bins: int = 4000
    flow_dim: int = 512
    flow_depth: int = 6
    lsd_decode_steps: int = 1
    gelu: str = "erf"
    time_rms_norm: str = "rms"
    max_period: float = 10000.0
    z_dim: int = 0
    flow_type: str = "lsd"
    precision: str = "f32"
    attn_dim: int = 0
    num_kv_heads: int = 0


def layout(cfg: FlowLMConfig):
    """The weight blob's tensors in order: (name, shape).  Every tensor is f32, row-major
    [out][in] for linears."""
    d, F, ld, ff = cfg.d_model, cfg.flow_dim, cfg.ldim, cfg.dim_feedforward
    a = cfg.attn_dim or d  # StreamingMultiheadAttention::load (transformer.rs:155-166)
    kv = a // cfg.num_heads * (cfg.num_kv_heads or cfg.num_heads)
    out = [("conditioner.embed", (cfg.n_bins + 1, d)), ("input_linear", (d, ld)), ("bos_emb", (ld,))]
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        out += [(p + "norm1.w", (d,)), (p + "norm1.b", (d,)), (p + "in_proj", (a + 2 * kv, d)), (p + "out_proj", (d, a)),
                (p + "norm2.w", (d,)), (p + "norm2.b", (d,)), (p + "linear1", (ff, d)), (p + "linear2", (d, ff))]
    zd = cfg.z_dim or d
    out += [("out_norm.w", (d,)), ("out_norm.b", (d,))]
    if cfg.z_dim:
        out += [("z_proj", (cfg.z_dim, d))]
    out += [("out_eos.w", (1, zd)), ("out_eos.b", (1,))]
    for i in range(2 if cfg.flow_type == "lsd" else 0):  # num_time_conds (flow_lm.rs:225-228)
        p = f"time_embed.{i}."
        out += [(p + "freqs", (FREQ_DIM // 2,)), (p + "mlp0.w", (F, FREQ_DIM)), (p + "mlp0.b", (F,)),
                (p + "mlp2.w", (F, F)), (p + "mlp2.b", (F,)), (p + "alpha", (F,))]
    out += [("cond_embed.w", (F, zd)), ("cond_embed.b", (F,)), ("input_proj.w", (F, ld)), ("input_proj.b", (F,))]
    for j in range(cfg.flow_depth):
        p = f"res_blocks.{j}."
        out += [(p + "in_ln.w", (F,)), (p + "in_ln.b", (F,)), (p + "mlp0.w", (F, F)), (p + "mlp0.b", (F,)),
                (p + "mlp2.w", (F, F)), (p + "mlp2.b", (F,)), (p + "ada.w", (3 * F, F)), (p + "ada.b", (3 * F,))]
    out += [("final.ada.w", (2 * F, F)), ("final.ada.b", (2 * F,)), ("final.linear.w", (ld, F)),
            ("final.linear.b", (ld,))]
    return out


def blob_size(cfg: FlowLMConfig) -> int:
    return sum(int(np.prod(s)) for _, s in layout(cfg))


def split(cfg: FlowLMConfig, blob) -> dict:
    """Views of the blob by tensor name."""
    out, o = {}, 0
    for name, shape in layout(cfg):
        n = int(np.prod(shape))
        out[name] = blob[o:o + n].reshape(shape)
        o += n
    return out


def random_weights(cfg: FlowLMConfig, seed: int, std: float = 0.02, unit_norms: bool = True) -> np.ndarray:
    """A seeded random-init blob: linears and embeddings N(0, std), biases 0, norms 1 and 0 (or
    N(1, 0.1) and N(0, 0.1) with unit_norms False), alpha 1, and the time embedders'
    frequencies exp(-ln(max_period) j / 128), the usual timestep-embedding table."""
    rng = np.random.default_rng(seed)
    blob = np.zeros(blob_size(cfg), np.float32)
    for name, t in split(cfg, blob).items():
        leaf = name.rsplit(".", 1)[-1]
        if name.endswith("freqs"):
            t[:] = np.exp(-math.log(cfg.max_period) * np.arange(t.size) / t.size)
        elif name.endswith("alpha"):
            t[:] = 1.0
        elif t.ndim == 1 and ("norm" in name or "in_ln" in name):
            if leaf == "w":
                t[:] = 1.0 if unit_norms else 1 + 0.1 * rng.standard_normal(t.shape)
            else:
                t[:] = 0.0 if unit_norms else 0.1 * rng.standard_normal(t.shape)
        elif t.ndim == 1 and leaf == "b":
            t[:] = 0.0 if unit_norms else 0.02 * rng.standard_normal(t.shape)
        else:
            t[:] = std * rng.standard_normal(t.shape)
    return blob


class FlowLMDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "d_model", "num_heads", "num_layers", "ff", "ldim", "n_bins", "flow_dim", "flow_depth", "lsd_steps",
        "gelu", "time_norm", "max_rows", "z_dim", "flow_type", "precision", "num_kv_heads", "attn_dim")]


def desc_of(cfg: FlowLMConfig, max_rows: int = 1) -> FlowLMDesc:
    return FlowLMDesc(d_model=cfg.d_model, num_heads=cfg.num_heads, num_layers=cfg.num_layers,
                      ff=cfg.dim_feedforward, ldim=cfg.ldim, n_bins=cfg.n_bins, flow_dim=cfg.flow_dim,
                      flow_depth=cfg.flow_depth, lsd_steps=cfg.lsd_decode_steps,
                      gelu=0 if cfg.gelu == "erf" else 1, time_norm=0 if cfg.time_rms_norm == "rms" else 1,
                      max_rows=max_rows, z_dim=cfg.z_dim, flow_type=FLOW_TYPES[cfg.flow_type],
                      precision=PRECISIONS[cfg.precision], num_kv_heads=cfg.num_kv_heads, attn_dim=cfg.attn_dim)


class FlowLM:
    """The flow LM on one pool (f32 cache and activations for the f32 precision, bf16 for q8):
    weights uploaded once (quantized on the host for q8), then prompts and frames for batches of
    that pool's streams."""

    def __init__(self, pool, cfg: FlowLMConfig, blob: np.ndarray, max_rows: int = 1):
        self._lib = load_library()
        self.cfg = cfg
        self.pool = pool
        self.desc = desc_of(cfg, max_rows)
        blob = np.ascontiguousarray(blob, np.float32)
        h = ctypes.c_void_p()
        _check(self._lib.xnp_flow_lm_create(pool._h, ctypes.byref(self.desc), blob.ctypes.data, blob.size,
                                            ctypes.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            self._lib.xnp_flow_lm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prompt_text(self, ids, tokens, stream=None):
        """tokens [n][t] int: the LUT rows of each stream's tokens through the transformer."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        arr = (ctypes.c_int32 * len(ids))(*ids)
        _check(self._lib.xnp_flow_lm_prompt_text(self._h, arr, len(ids), tokens.ctypes.data, tokens.shape[1],
                                                 _stream(stream)))

    def set_condition(self, cond):
        """The model's summed conditions (condition_providers, flow_lm.rs:218-222): cond [d_model]
        host values, or None for none."""
        if cond is None:
            _check(self._lib.xnp_flow_lm_set_condition(self._h, None, 0))
            return
        c = np.ascontiguousarray(cond, np.float32)
        _check(self._lib.xnp_flow_lm_set_condition(self._h, c.ctypes.data, c.size))

    def step(self, ids, latent_in, noise, latent_out, eos_out, stream=None, graph: bool = False, conditions=None):
        """One frame for each stream: latent_in [n][ldim] (None: bos_emb), noise [n][ldim],
        latent_out [n][ldim], eos_out [n], conditions [n][d_model] (each stream's
        FlowLMState::conditions; None: the model's, if set) -- f32 device tensors.  graph: replay a
        recording of the frame's launches (xnp_flow_lm_step_graph; needs a non-null stream)."""
        arr = (ctypes.c_int32 * len(ids))(*ids)
        fn = self._lib.xnp_flow_lm_step_graph if graph else self._lib.xnp_flow_lm_step
        _check(fn(self._h, arr, len(ids), _ptr(latent_in), _ptr(conditions), _ptr(noise), _ptr(latent_out),
                  _ptr(eos_out), _stream(stream)))
