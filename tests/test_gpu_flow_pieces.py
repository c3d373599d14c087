"""GPU parity of the q8 flow net's pieces, through the C ABI (xnp_flow_linear_q8, xnp_layer_norm_mod),
against the oracle's (orc_flow_linear_q8, orc_layer_norm_mod) on the same bf16 inputs.

Bar: the same bf16 values, bit for bit, except where the GPU's summation order (MFMA for the
product, a wave reduction for the norm's moments) moves an f32 result across a bf16 rounding
boundary: then one bf16 step at most, and for at most 1 % of the elements.  These fix the rounding
points of the q8 frame one by one; the end-to-end frame is held to its own bar in
test_gpu_flow_lm.py.
"""
import numpy as np
import pytest
import torch

from conftest import oracle, xnp
from helpers import bf16_round, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ulps(got, want):
    want64 = np.abs(want.astype(np.float64))
    spacing = np.exp2(np.floor(np.log2(np.maximum(want64, 1e-30))) - 7)
    return np.abs(got.astype(np.float64) - want) / spacing


def _close(got, want, what):
    u = _ulps(got, want)
    assert (u <= 1).all(), (what, float(u.max()))
    assert (got != want).mean() <= 0.01, (what, float((got != want).mean()))


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(torch.bfloat16)


@pytest.mark.parametrize("rows,k,n", [(100, 48, 40), (130, 512, 600), (64, 1024, 1)])
@pytest.mark.parametrize("epilogue", ["store", "silu", "silu_add", "gated", "axpy_f32", "store_f32"])
def test_flow_linear_q8_matches_the_oracle(rows, k, n, epilogue):
    rng = np.random.default_rng(rows * 7 + k + n)
    x = bf16_round(rng.standard_normal((rows, k)).astype(np.float32))
    q, s = oracle.quantize_rows((0.05 * rng.standard_normal((n, k))).astype(np.float32))
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    aux = out0 = None
    alpha = 1.0
    if epilogue == "silu_add":
        aux = bf16_round(rng.standard_normal(n).astype(np.float32))
    elif epilogue == "gated":
        aux = bf16_round(rng.standard_normal((rows, n)).astype(np.float32))
        out0 = bf16_round(rng.standard_normal((rows, n)).astype(np.float32))
    elif epilogue == "axpy_f32":
        aux, alpha = rng.standard_normal((rows, n)).astype(np.float32), 0.5
    want = oracle.flow_linear_q8(x, q, s, epilogue, bias=b, aux=aux, out=out0, alpha=alpha)
    f32_out = epilogue in ("axpy_f32", "store_f32")
    y = (torch.zeros((rows, n), dtype=torch.float32, device=DEV) if f32_out
         else (_bf(out0) if out0 is not None else torch.zeros((rows, n), dtype=torch.bfloat16, device=DEV)))
    if aux is None:
        a = None
    elif epilogue == "gated":
        a = _bf(aux)
    else:
        a = torch.from_numpy(aux).to(DEV)
    xnp.flow_linear_q8(_bf(x), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), y, epilogue,
                       bias=torch.from_numpy(b).to(DEV), aux=a, alpha=alpha)
    torch.cuda.synchronize()
    _close(y.float().cpu().numpy(), want, epilogue)


# Long K: K >= 2048 runs the GEMM's two-half groups (alternate K chunks, summed in LDS); 2064 leaves
# the halves 17 and 16 chunks, the last one partial; 1024 x 2048 x 2048 takes 64-row tiles.  Over
# thousands of terms the f32 sum's order matters beyond one bf16 step for outputs near zero (the
# oracle's own sequential sum lies up to 4 steps from the exact one at K = 2064), so each element
# may also differ by the recursive-summation bound of both sums, 2 K 2^-24 s sum|x q|.
@pytest.mark.parametrize("rows,k,n", [(70, 2048, 96), (600, 2064, 520), (1024, 2048, 2048)])
@pytest.mark.parametrize("epilogue", ["store", "store_f32"])
def test_flow_linear_q8_long_k_within_the_summation_bound(rows, k, n, epilogue):
    rng = np.random.default_rng(rows + k + n)
    x = bf16_round(rng.standard_normal((rows, k)).astype(np.float32))
    q, s = oracle.quantize_rows((0.05 * rng.standard_normal((n, k))).astype(np.float32))
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    want = oracle.flow_linear_q8(x, q, s, epilogue, bias=b)
    y = torch.zeros((rows, n), dtype=torch.float32 if epilogue == "store_f32" else torch.bfloat16, device=DEV)
    xnp.flow_linear_q8(_bf(x), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), y, epilogue,
                       bias=torch.from_numpy(b).to(DEV))
    torch.cuda.synchronize()
    _close_within_sum(y.float().cpu().numpy(), want, x, q, s, epilogue)


def _close_within_sum(got, want, x, q, s, what):
    # one bf16 step, plus the recursive-summation bound of both f32 sums, 2 K 2^-24 s sum|x q|
    k = x.shape[-1]
    bound = 2.0 * k * 2.0 ** -24 * (np.abs(x) @ np.abs(q.astype(np.float32)).T) * s[None, :]
    want64 = np.abs(want.astype(np.float64))
    spacing = np.exp2(np.floor(np.log2(np.maximum(want64, 1e-30))) - 7)
    assert (np.abs(got.astype(np.float64) - want) <= spacing + bound).all(), what
    assert (got != want).mean() <= 0.01, (what, float((got != want).mean()))


# 128 x 64 tiles (wide projections that still make 512 work groups with them, such as the stacked
# adaLN projection at 2048 rows): 257 column tiles by 2 row tiles, the last of one row or of 72; N
# 8 columns past a multiple of 64 with K of exactly 8 chunks (the staged epilogue, rounds unrolled),
# or 4 past with K of 8.25 chunks (the per-element epilogue, the looped rounds' past-K masks).  Over
# 2-3M outputs some lie near zero, where the order of the f32 sum moves them by more than one bf16
# step; so the bar is the long-K one (a dropped or doubled chunk fails it almost everywhere).
@pytest.mark.parametrize("rows,k,n", [(129, 512, 16392), (200, 528, 16388)])
@pytest.mark.parametrize("epilogue", ["store", "store_f32"])
def test_flow_linear_q8_on_128_row_tiles_matches_the_oracle(rows, k, n, epilogue):
    rng = np.random.default_rng(rows + k + n)
    x = bf16_round(rng.standard_normal((rows, k)).astype(np.float32))
    q, s = oracle.quantize_rows((0.05 * rng.standard_normal((n, k))).astype(np.float32))
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    want = oracle.flow_linear_q8(x, q, s, epilogue, bias=b)
    y = torch.zeros((rows, n), dtype=torch.float32 if epilogue == "store_f32" else torch.bfloat16, device=DEV)
    xnp.flow_linear_q8(_bf(x), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), y, epilogue,
                       bias=torch.from_numpy(b).to(DEV))
    torch.cuda.synchronize()
    _close_within_sum(y.float().cpu().numpy(), want, x, q, s, epilogue)


def test_flow_linear_q8_reads_f32_rows_rounded():
    # input_linear / input_proj: K = 32 latents in f32, rounded to bf16 as they are staged
    rng = np.random.default_rng(89)
    x = rng.standard_normal((70, 32)).astype(np.float32)
    q, s = oracle.quantize_rows((0.05 * rng.standard_normal((512, 32))).astype(np.float32))
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    want = oracle.flow_linear_q8(x, q, s, "store", bias=b)
    y = torch.zeros((70, 512), dtype=torch.bfloat16, device=DEV)
    xnp.flow_linear_q8(torch.from_numpy(x).to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), y,
                       bias=torch.from_numpy(b).to(DEV))
    torch.cuda.synchronize()
    _close(y.float().cpu().numpy(), want, "f32 x")
    with pytest.raises(xnp.XnpError, match="store or add epilogue"):
        xnp.flow_linear_q8(torch.from_numpy(x).to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), y,
                           "silu")


@pytest.mark.parametrize("rows_of_cond", [True, False])
def test_the_condition_add_on_f32_rows_matches_the_oracle(rows_of_cond):
    # input_linear plus the conditions (flow_lm.rs:304-307): y[m][j] = bf16(bf16(c[m][j]) + bf16(y)),
    # with a condition row per row, or one row for every row (ld_aux 0: the model's summed conditions)
    rng = np.random.default_rng(91 + rows_of_cond)
    x = rng.standard_normal((70, 32)).astype(np.float32)
    q, s = oracle.quantize_rows((0.05 * rng.standard_normal((512, 32))).astype(np.float32))
    c = (0.5 * rng.standard_normal((70, 512) if rows_of_cond else 512)).astype(np.float32)
    want = oracle.flow_linear_q8(x, q, s, "add_f32", aux=c)
    y = torch.zeros((70, 512), dtype=torch.bfloat16, device=DEV)
    xnp.flow_linear_q8(torch.from_numpy(x).to(DEV), torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), y,
                       "add_f32", aux=torch.from_numpy(c).to(DEV))
    torch.cuda.synchronize()
    _close(y.float().cpu().numpy(), want, "add_f32")
    plain = oracle.flow_linear_q8(x, q, s, "store")
    assert rel_err(want, plain) > 0.1  # the condition is there


@pytest.mark.parametrize("affine,mod", [(True, True), (False, True), (True, False)])
def test_layer_norm_mod_matches_the_oracle(affine, mod):
    rng = np.random.default_rng(90 + 2 * affine + mod)
    rows, dim = 75, 512
    x = bf16_round((1 + 2 * rng.standard_normal((rows, dim))).astype(np.float32))
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32) if affine else None
    b = (0.1 * rng.standard_normal(dim)).astype(np.float32) if affine else None
    ada = bf16_round(rng.standard_normal((rows, 3 * dim)).astype(np.float32))  # (shift, scale, gate) rows
    shift, scale = (ada[:, :dim], ada[:, dim:2 * dim]) if mod else (None, None)
    want = oracle.layer_norm_mod(x, w, b, shift, scale)
    out = torch.zeros((rows, dim), dtype=torch.bfloat16, device=DEV)
    ada_d = _bf(ada)
    T = lambda a: torch.from_numpy(a).to(DEV) if a is not None else None
    xnp.layer_norm_mod(_bf(x), out, T(w), T(b), ada_d[:, :dim] if mod else None, ada_d[:, dim:2 * dim] if mod else None)
    torch.cuda.synchronize()
    _close(out.float().cpu().numpy(), want, (affine, mod))
