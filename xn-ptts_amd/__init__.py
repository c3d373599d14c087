"""xnp-kv: MI355X-native paged KV cache for the Phonon flow LM (gradium-ai/xn-ptts).

The compute lives in libxnp_kv.so (hand-written HIP kernels for gfx950 behind the C ABI of
include/xnp_kv.h); this package is the Python binding over it.  The directory name has a hyphen,
so load it by path, e.g. importlib.util.spec_from_file_location("xn_ptts_amd", <dir>/__init__.py).
"""
from .kv import (BF16, BLOCK, DTYPES, F32, I8, LIB_PATH, RING_ABSOLUTE, RING_SHIFT, KvPool, LayerWeights,
                 XnpError, flow_linear_q8, frame_budget, layer_norm, layer_norm_mod, linear_q8, load_library, quantize_rows, read_voice_file,
                 seq_budget, voice_kv_name, voice_layers)
from .flow_lm import FlowLM, FlowLMConfig

__all__ = ["KvPool", "FlowLM", "FlowLMConfig", "LayerWeights", "XnpError", "load_library", "frame_budget", "seq_budget", "layer_norm", "layer_norm_mod", "flow_linear_q8",
           "linear_q8", "quantize_rows", "read_voice_file", "voice_kv_name", "voice_layers", "LIB_PATH", "F32", "BF16", "I8", "BLOCK", "DTYPES", "RING_SHIFT",
           "RING_ABSOLUTE"]
