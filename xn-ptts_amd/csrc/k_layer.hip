// The rest of the flow-LM layer and the flow LM around it: LayerNorm, the q8 projection GEMM on
// MFMA with its epilogues, the f32 linears of batch-1 frames, and the row gathers.
#include "kernels_common.h"

namespace xnp {

// ---------------------------------------------------------------------------------------------
// the rest of the flow-LM layer (transformer.rs:591-634): LayerNorm, and the q8 projections as
// MFMA GEMMs with per-channel int8 weights

// LayerNorm over rows of `dim` bf16 values (norm1, norm2: transformer.rs:547-548): one wave per
// row, each lane holding dim / 64 values; mean and biased variance in f32 (two passes over the
// registers), y = (x - mean) * (1 / sqrt(var + eps)) (* w + b when MODE has kLnAffine), rounded
// to bf16.  With kLnMod, then the AdaLN modulation (mlp.rs:4-11) as bf16 tensor operations round
// it: bf16(bf16(y * bf16(scale + 1)) + shift), with shift and scale bf16 rows of stride ld_mod.
constexpr int kLnAffine = 1, kLnMod = 2;

template <int CH, int MODE>
__global__ __launch_bounds__(256) void k_layer_norm(const uint16_t *x, int rows, int dim, const float *w,
                                                    const float *b, float eps, const uint16_t *shift,
                                                    const uint16_t *scale, int ld_mod, uint16_t *out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const uint16_t *xr = x + (size_t)row * dim;
    float v[CH][8];
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const uint4 raw = *(const uint4 *)(xr + (c * 64 + lane) * 8);
        const uint32_t *u = (const uint32_t *)&raw;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[c][2 * i] = bf16_value(u[i] & 0xffffu);
            v[c][2 * i + 1] = bf16_value(u[i] >> 16);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += v[c][i];
    }
    uint4 rsh[CH], rsc[CH]; // the modulation's rows, loaded with x
    if constexpr ((MODE & kLnMod) != 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            rsh[c] = *(const uint4 *)(shift + (size_t)row * ld_mod + (c * 64 + lane) * 8);
            rsc[c] = *(const uint4 *)(scale + (size_t)row * ld_mod + (c * 64 + lane) * 8);
        }
    }
    float4 aw[CH][2], ab[CH][2]; // the affine's weights and biases, loaded with x too
    if constexpr ((MODE & kLnAffine) != 0) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int e0 = (c * 64 + lane) * 8;
            aw[c][0] = *(const float4 *)(w + e0);
            aw[c][1] = *(const float4 *)(w + e0 + 4);
            ab[c][0] = *(const float4 *)(b + e0);
            ab[c][1] = *(const float4 *)(b + e0 + 4);
        }
    }
    // a scheduling barrier: keeps the loads above here, issued together with x's, rather than
    // sunk to their uses after the row's reductions (a second round trip)
    __builtin_amdgcn_sched_barrier(0);
    sum = wave_sum(sum);
    const float mean = sum / (float)dim;
    float sq = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = v[c][i] - mean;
            sq = __builtin_fmaf(d, d, sq);
        }
    sq = wave_sum(sq);
    const float rstd = 1.0f / __builtin_sqrtf(sq / (float)dim + eps);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int e0 = (c * 64 + lane) * 8;
        float ww[8], bb[8];
        if constexpr ((MODE & kLnAffine) != 0) {
            const float4 w0 = aw[c][0], w1 = aw[c][1], b0 = ab[c][0], b1 = ab[c][1];
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) ww[i] = wv[i], bb[i] = bv[i];
        }
        uint32_t o4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float y[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int e = 2 * i + j;
                y[j] = (v[c][e] - mean) * rstd;
                if constexpr ((MODE & kLnAffine) != 0) y[j] = y[j] * ww[e] + bb[e];
                if constexpr ((MODE & kLnMod) != 0) {
                    const uint32_t us = ((const uint32_t *)&rsc[c])[i], uh = ((const uint32_t *)&rsh[c])[i];
                    const float sc1 = bf16_value(bf16_bits(bf16_value(j ? us >> 16 : us & 0xffffu) + 1.0f));
                    const float p = bf16_value(bf16_bits(bf16_value(bf16_bits(y[j])) * sc1));
                    y[j] = p + bf16_value(j ? uh >> 16 : uh & 0xffffu);
                }
            }
            o4[i] = pack_bf16(y[0], y[1]);
        }
        st_stream(out + (size_t)row * dim + e0, make_uint4(o4[0], o4[1], o4[2], o4[3]));
    }
}

template <int MODE>
static hipError_t layer_norm_mode(const void *x, int rows, int dim, const float *w, const float *b, float eps,
                                  const void *shift, const void *scale, int ld_mod, void *out, hipStream_t stream) {
    const dim3 grid((rows + 3) / 4), block(256);
    const uint16_t *xs = (const uint16_t *)x, *sh = (const uint16_t *)shift, *sc = (const uint16_t *)scale;
    uint16_t *o = (uint16_t *)out;
#define XNP_LN(C) hipLaunchKernelGGL((k_layer_norm<C, MODE>), grid, block, 0, stream, xs, rows, dim, w, b, eps, sh, sc, ld_mod, o)
    switch (dim / 512) {
    case 1: XNP_LN(1); break;
    case 2: XNP_LN(2); break;
    case 3: XNP_LN(3); break;
    case 4: XNP_LN(4); break;
    default: return hipErrorInvalidValue;
    }
#undef XNP_LN
    return hipGetLastError();
}

hipError_t launch_layer_norm_mod(const void *x, int rows, int dim, const float *w, const float *b, float eps,
                                 const void *shift, const void *scale, int ld_mod, void *out, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (dim % 512 || (w == nullptr) != (b == nullptr) || (shift == nullptr) != (scale == nullptr) ||
        (shift && ld_mod % 8))
        return hipErrorInvalidValue;
    if (w && shift) return layer_norm_mode<kLnAffine | kLnMod>(x, rows, dim, w, b, eps, shift, scale, ld_mod, out, stream);
    if (w) return layer_norm_mode<kLnAffine>(x, rows, dim, w, b, eps, shift, scale, ld_mod, out, stream);
    if (shift) return layer_norm_mode<kLnMod>(x, rows, dim, w, b, eps, shift, scale, ld_mod, out, stream);
    return layer_norm_mode<0>(x, rows, dim, w, b, eps, shift, scale, ld_mod, out, stream);
}

hipError_t launch_layer_norm(const void *x, int rows, int dim, const float *w, const float *b, float eps, void *out,
                             hipStream_t stream) {
    return launch_layer_norm_mod(x, rows, dim, w, b, eps, nullptr, nullptr, 0, out, stream);
}

// y = epilogue(s[n] * sum_k A[m][k] W[n][k]): A [M][K] bf16, W [N][K] int8 with one f32 scale per
// output channel (row of W), the sum on v_mfma_f32_16x16x32_bf16 with W widened to bf16 exactly
// (|q| <= 127).  One work group of 4 waves per 64 x 64 tile of y, each wave 32 x 32 (2 x 2 MFMA
// tiles); K in chunks of 64 staged through LDS, double-buffered, with the loads of the next three
// chunks in flight while one is multiplied.  The product, plus the bias when given, is rounded to bf16 (the
// projection's output tensor), then: kStore writes it (column ranges may go to separate outputs:
// q, k and v), kGelu* write gelu(y) rounded, kResidual adds y (times the layer scale, rounded,
// when given) into X and rounds: X + layer_scale(linear(..)) as transformer.rs:612-633 does; the
// flow net's epilogues are listed with their enum.  N may be any width (columns past N are
// neither loaded nor stored) and K any multiple of 16 (the last chunk's loads past K read zeros).
constexpr int kGmT = 64;  // tile rows and columns
constexpr int kGmK = 64;  // K chunk
constexpr int kGmLd = 72; // LDS row length in bf16
constexpr int kGmPD = 3;  // K chunks of loads in flight

// MI: 16-row MFMA tiles per wave in M, so tiles of 32 MI rows.  MI = 1 doubles the work groups of a
// narrow projection (N = 512 at 2048 rows gives 256 groups of 64 rows: one wave per SIMD).  MI = 4
// (128 x 64 tiles, each wave 64 x 32) for wide ones that still give two groups per CU: a wave's
// MFMAs per LDS byte read, and per staged byte, rise by a third.
//
// KS: groups of KS x 256 threads.  Half h (256 threads, the tile's 4 waves) takes K chunks h, h + KS,
// .. into its own LDS buffers; at the end half 1 hands its sums to half 0 through LDS, which adds
// them and runs the epilogue.  For long K (linear2: K = 2048), where a group's chunks run one
// after another.
// STG: the epilogue goes through LDS (N % 8 == 0, the outputs and their rows 16-byte aligned in
// 8-column steps): y, rounded to bf16, as [row][col], then a thread takes 8 consecutive columns of
// a row, so that its accesses to the output (and to x, the gate, aux) are 16 bytes (32 for f32
// rows) instead of 2, with its operands loaded before the K loop.  Measured in the layer step at
// 2048 rows: the epilogue took 2.4-3.1 us of each projection with 2-byte stores.
// NKC: K is exactly NKC x KS chunks (8 or 16 per half: the flow LM's 512-2048 wide projections),
// so the rounds run unrolled whole and without the past-K clamps and masks; 0: any K, in a loop.
// Tiles go to the XCDs in contiguous runs (xcd_tile), so each XCD's L2 holds about an eighth of A.
constexpr int kGsLd = 72; // the staged epilogue's LDS row in bf16

template <int EPI, bool AF32, int MI, int KS, bool STG, int NKC>
__global__ __launch_bounds__(256 * KS) void k_gemm_q8(const uint16_t *A, int M, int K, const int8_t *W, const float *s,
                                                      int N, GemmOut go) {
    constexpr int BM = 32 * MI;
    static_assert(KS == 1 || KS == 2, "one or two halves");
    __shared__ __attribute__((aligned(16))) uint16_t As[KS][2][BM][kGmLd];
    __shared__ __attribute__((aligned(16))) uint16_t Ws[KS][2][kGmT][kGmLd];
    const int ntn = (N + kGmT - 1) / kGmT, tile = xcd_tile(blockIdx.x, gridDim.x);
    const int m0 = (tile / ntn) * BM, n0 = (tile % ntn) * kGmT;
    const int tid = threadIdx.x & 255, h = KS > 1 ? (int)(threadIdx.x >> 8) : 0;
    const int w = tid >> 6, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
    const int wm = w & 1, wn = w >> 1;

    // staging: A rows a_r + 32 i, i < MI (the tile's 32 MI rows), 8 values at k 8 a_k; W row w_r, 16
    // int8 at k 16 w_k.
    // kGmPD chunks of loads are in flight: set c % kGmPD holds chunk c from its load until it is
    // written to LDS.  The words stay as loaded until then -- zeroing past K, rounding f32 A rows
    // and widening W happen at the LDS store, since any use at the load would make the wave wait
    // for it there.
    constexpr int NA = MI; // A rows a thread stages
    const int a_r = tid >> 3, a_k = tid & 7, w_r = tid >> 2, w_k = tid & 3;
    int ar[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) ar[i] = min(m0 + a_r + 32 * i, M - 1);
    const int wr = min(n0 + w_r, N - 1);
    constexpr int AW = AF32 ? 2 : 1; // uint4 per 8 A values
    uint4 ra[NA][kGmPD][AW], rw[kGmPD];
    // NKC > 0: K is a whole number of chunks, so nothing reaches past it and the clamps and masks
    // below drop out (they were 14-18 of a round's 47-51 VALU instructions)
    constexpr bool kWhole = NKC > 0;
    auto load = [&](int kc, int set) {
        // past K (K % 16 == 0, so no 16-byte load straddles it): an in-bounds address, zeroed at
        // the store
        const int k0 = kc * kGmK;
        const int ka = kWhole || k0 + 8 * a_k < K ? k0 + 8 * a_k : 0, kw = kWhole || k0 + 16 * w_k < K ? k0 + 16 * w_k : 0;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            if constexpr (AF32) {
                const float *af = (const float *)A;
                ra[i][set][0] = *(const uint4 *)(af + (size_t)ar[i] * K + ka);
                ra[i][set][AW - 1] = *(const uint4 *)(af + (size_t)ar[i] * K + ka + 4);
            } else {
                ra[i][set][0] = *(const uint4 *)(A + (size_t)ar[i] * K + ka);
            }
        }
        rw[set] = *(const uint4 *)(W + (size_t)wr * K + kw);
    };
    auto masked = [](const uint4 &u, uint32_t m) { return make_uint4(u.x & m, u.y & m, u.z & m, u.w & m); };
    auto bf16_row = [&](const uint4 (&u)[AW]) { // 8 A values as bf16 pairs
        if constexpr (AF32) {
            return make_uint4(pack_bf16(__uint_as_float(u[0].x), __uint_as_float(u[0].y)),
                              pack_bf16(__uint_as_float(u[0].z), __uint_as_float(u[0].w)),
                              pack_bf16(__uint_as_float(u[AW - 1].x), __uint_as_float(u[AW - 1].y)),
                              pack_bf16(__uint_as_float(u[AW - 1].z), __uint_as_float(u[AW - 1].w)));
        } else {
            return u[0];
        }
    };
    auto widen2 = [](uint32_t u, int sh) { // two int8 -> a bf16 pair (exact: |q| <= 127)
        return pack_bf16((float)(int8_t)((u >> sh) & 0xffu), (float)(int8_t)((u >> (sh + 8)) & 0xffu));
    };
    auto store = [&](int buf, int set, int kc) {
        uint4 av[NA], wq = rw[set];
#pragma unroll
        for (int i = 0; i < NA; ++i) av[i] = bf16_row(ra[i][set]);
        // words past K zeroed with masks rather than under a branch: a branch here splits the
        // loop, and past the join the compiler no longer knows which loads are still in flight
        // (it then waits for all of them before the next load)
        if constexpr (!kWhole) {
            const int k0 = kc * kGmK;
            const uint32_t ma = k0 + 8 * a_k < K ? ~0u : 0u, mw = k0 + 16 * w_k < K ? ~0u : 0u;
#pragma unroll
            for (int i = 0; i < NA; ++i) av[i] = masked(av[i], ma);
            wq = masked(wq, mw);
        }
#pragma unroll
        for (int i = 0; i < NA; ++i) *(uint4 *)&As[h][buf][a_r + 32 * i][8 * a_k] = av[i];
        *(uint4 *)&Ws[h][buf][w_r][16 * w_k] = make_uint4(widen2(wq.x, 0), widen2(wq.x, 16), widen2(wq.y, 0), widen2(wq.y, 16));
        *(uint4 *)&Ws[h][buf][w_r][16 * w_k + 8] =
            make_uint4(widen2(wq.z, 0), widen2(wq.z, 16), widen2(wq.w, 0), widen2(wq.w, 16));
    };

    // the epilogue's per-column operands, loaded before the loop so that they arrive with it
    float sc[2], bn[2], lsn[2];
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
        const int n = min(n0 + 32 * wn + 16 * ni + l16, N - 1);
        sc[ni] = s[n];
        bn[ni] = go.bias ? go.bias[n] : 0.f;
        lsn[ni] = (EPI == kResidual && go.ls) ? go.ls[n] : 1.f;
    }

    // the staged epilogue's pieces (rows er + 32 e, columns n0 + ec ..) and their operands
    const int er = tid >> 3, ec = 8 * (tid & 7), ne = n0 + ec;
    uint4 xo[MI], gt[MI];
    float4 ax[MI][2], lv[2];
    if constexpr (STG) {
        if (h == 0) {
#pragma unroll
            for (int e = 0; e < MI; ++e) {
                const int mm = min(m0 + er + 32 * e, M - 1), nn = ne < N ? ne : 0;
                if constexpr (EPI == kResidual || EPI == kGated)
                    xo[e] = *(const uint4 *)((const uint16_t *)go.out[0] + (size_t)mm * go.ld[0] + nn);
                if constexpr (EPI == kGated)
                    gt[e] = *(const uint4 *)((const uint16_t *)go.aux + (size_t)mm * go.ld_aux + nn);
                if constexpr (EPI == kAxpyF32 || EPI == kAddF32) {
                    ax[e][0] = *(const float4 *)((const float *)go.aux + (size_t)mm * go.ld_aux + nn);
                    ax[e][1] = *(const float4 *)((const float *)go.aux + (size_t)mm * go.ld_aux + nn + 4);
                }
            }
            if constexpr (EPI == kResidual) {
                lv[0] = lv[1] = make_float4(1.f, 1.f, 1.f, 1.f);
                if (go.ls && ne < N) {
                    lv[0] = *(const float4 *)(go.ls + ne);
                    lv[1] = *(const float4 *)(go.ls + ne + 4);
                }
            }
            if constexpr (EPI == kSiluAddVec) {
                lv[0] = *(const float4 *)((const float *)go.aux + (ne < N ? ne : 0));
                lv[1] = *(const float4 *)((const float *)go.aux + (ne < N ? ne : 0) + 4);
            }
        }
    }

    f32x4_t acc[MI][2];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // this half's chunks: c = 0 .. nkh - 1 is chunk h + KS c.  Both halves run nkmax rounds, one
    // barrier each, whatever their own count (the launcher takes KS = 2 only when nk >= 2 KS).
    // Every round loads and stores unconditionally, past this half's last chunk its last chunk
    // again (a duplicate nobody reads): loads under a branch leave the compiler unsure which loads
    // are in flight after it, and it then drains them all before the next one.  NKC > 0: K is
    // NKC x KS chunks exactly, and the rounds are unrolled whole -- the back edge of a loop makes
    // the compiler copy load registers still in flight, which waits for them.
    const int nk = NKC > 0 ? NKC * KS : (K + kGmK - 1) / kGmK;
    const int nkh = NKC > 0 ? NKC : (nk - h + KS - 1) / KS, nkmax = NKC > 0 ? NKC : (nk + KS - 1) / KS;
    auto chunk = [&](int c) { return h + KS * min(c, nkh - 1); };
    auto round = [&](int c, int u) { // u = c % kGmPD: set indices stay constants
        const int buf = c & 1;
        load(chunk(c + kGmPD), u); // set u held chunk c, already in LDS
        if (c < nkh) {
#pragma unroll
            for (int ks = 0; ks < kGmK / 32; ++ks) {
                bf16x8_t a[MI], bw[2];
#pragma unroll
                for (int i = 0; i < MI; ++i)
                    a[i] = as_bf16x8(*(const uint4 *)&As[h][buf][16 * MI * wm + 16 * i + l16][32 * ks + 8 * g]);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    bw[i] = as_bf16x8(*(const uint4 *)&Ws[h][buf][32 * wn + 16 * i + l16][32 * ks + 8 * g]);
#pragma unroll
                for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                    for (int ni = 0; ni < 2; ++ni)
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mi], bw[ni], acc[mi][ni], 0, 0, 0);
            }
        }
        // buffer buf ^ 1's last readers finished before the previous barrier
        store(buf ^ 1, (u + 1) % kGmPD, chunk(c + 1));
        __syncthreads();
    };
#pragma unroll
    for (int c = 0; c < kGmPD; ++c) load(chunk(c), c);
    store(0, 0, h);
    __syncthreads();
    if constexpr (NKC > 0) {
#pragma unroll
        for (int c = 0; c < NKC; ++c) round(c, c % kGmPD);
    } else {
        for (int cb = 0; cb < nkmax; cb += kGmPD) {
#pragma unroll
            for (int u = 0; u < kGmPD; ++u) {
                if (cb + u >= nkmax) break; // uniform over the group
                round(cb + u, u);
            }
        }
    }
    if constexpr (KS > 1) {
        // half 1's sums to half 0 through LDS (the tiles are free: every half passed the loop's
        // last barrier after its last read); half 0 adds them, in the same order in every group
        static_assert(sizeof(As) >= 256 * MI * 8 * sizeof(float), "room for half 1's sums");
        float *red = (float *)&As[0][0][0][0];
        if (h == 1) {
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                    for (int r = 0; r < 4; ++r) red[((mi * 2 + ni) * 4 + r) * 256 + tid] = acc[mi][ni][r];
        }
        __syncthreads();
        if (!STG && h == 1) return;
        if (h == 0) {
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[mi][ni][r] += red[((mi * 2 + ni) * 4 + r) * 256 + tid];
        }
    }

    if constexpr (STG) {
        // y into LDS (lane: column 32 wn + 16 ni + l16, rows 16 MI wm + 16 mi + 4 g + r); both halves
        // meet at the barriers, half 1 with nothing to store
        static_assert(sizeof(As) >= 32 * MI * kGsLd * sizeof(uint16_t), "room for the tile");
        uint16_t(*st)[kGsLd] = (uint16_t(*)[kGsLd]) & As[0][0][0][0];
        if constexpr (KS > 1) __syncthreads(); // half 0 has read half 1's sums
        if (h == 0) {
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float v = go.bias ? acc[mi][ni][r] * sc[ni] + bn[ni] : acc[mi][ni][r] * sc[ni];
                        st[16 * MI * wm + 16 * mi + 4 * g + r][32 * wn + 16 * ni + l16] = (uint16_t)bf16_bits(v);
                    }
        }
        __syncthreads();
        if (h != 0) return;
#pragma unroll
        for (int e = 0; e < MI; ++e) {
            const int m = m0 + er + 32 * e;
            if (m >= M || ne >= N) continue;
            const uint4 yv = *(const uint4 *)&st[er + 32 * e][ec];
            const uint32_t *yw = (const uint32_t *)&yv;
            float y[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                y[2 * i] = bf16_value(yw[i] & 0xffffu);
                y[2 * i + 1] = bf16_value(yw[i] >> 16);
            }
            if constexpr (EPI == kStore) {
                int seg = 0;
                if (go.nseg > 1 && ne >= go.col0[1]) seg = (go.nseg > 2 && ne >= go.col0[2]) ? 2 : 1;
                st_stream((uint16_t *)go.out[seg] + (size_t)m * go.ld[seg] + (ne - go.col0[seg]), yv);
            } else if constexpr (EPI == kStoreF32) {
                float *o = (float *)go.out[0] + (size_t)m * go.ld[0] + ne;
                *(float4 *)o = make_float4(y[0], y[1], y[2], y[3]);
                *(float4 *)(o + 4) = make_float4(y[4], y[5], y[6], y[7]);
            } else if constexpr (EPI == kAxpyF32) {
                const float cu[8] = {ax[e][0].x, ax[e][0].y, ax[e][0].z, ax[e][0].w,
                                     ax[e][1].x, ax[e][1].y, ax[e][1].z, ax[e][1].w};
                float r8[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    r8[i] = bf16_value(bf16_bits(bf16_value(bf16_bits(cu[i])) + bf16_value(bf16_bits(y[i] * go.alpha))));
                float *o = (float *)go.out[0] + (size_t)m * go.ld[0] + ne;
                *(float4 *)o = make_float4(r8[0], r8[1], r8[2], r8[3]);
                *(float4 *)(o + 4) = make_float4(r8[4], r8[5], r8[6], r8[7]);
            } else if constexpr (EPI == kAddF32) {
                const float cu[8] = {ax[e][0].x, ax[e][0].y, ax[e][0].z, ax[e][0].w,
                                     ax[e][1].x, ax[e][1].y, ax[e][1].z, ax[e][1].w};
                float r8[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) r8[i] = bf16_value(bf16_bits(cu[i])) + y[i];
                st_stream((uint16_t *)go.out[0] + (size_t)m * go.ld[0] + ne,
                          make_uint4(pack_bf16(r8[0], r8[1]), pack_bf16(r8[2], r8[3]), pack_bf16(r8[4], r8[5]), pack_bf16(r8[6], r8[7])));
            } else {
                float r8[8];
                const uint32_t *xw = (const uint32_t *)&xo[e], *gw = (const uint32_t *)&gt[e];
                const float l8[8] = {lv[0].x, lv[0].y, lv[0].z, lv[0].w, lv[1].x, lv[1].y, lv[1].z, lv[1].w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float yi = y[i];
                    if constexpr (EPI == kGeluErf) {
                        r8[i] = 0.5f * yi * (1.0f + erff(yi * 0.7071067811865476f));
                    } else if constexpr (EPI == kGeluTanh) {
                        const float cc = 0.7978845608028654f;
                        r8[i] = 0.5f * yi * (1.0f + tanhf(cc * (yi + 0.044715f * yi * yi * yi)));
                    } else if constexpr (EPI == kResidual) {
                        const float a = go.ls ? bf16_value(bf16_bits(yi * l8[i])) : yi;
                        r8[i] = bf16_value((i & 1) ? xw[i >> 1] >> 16 : xw[i >> 1] & 0xffffu) + a;
                    } else if constexpr (EPI == kSilu) {
                        r8[i] = yi / (1.0f + expf(-yi));
                    } else if constexpr (EPI == kSiluAddVec) {
                        const float z = bf16_value(bf16_bits(yi + l8[i]));
                        r8[i] = z / (1.0f + expf(-z));
                    } else { // kGated
                        const float gate = bf16_value((i & 1) ? gw[i >> 1] >> 16 : gw[i >> 1] & 0xffffu);
                        r8[i] = bf16_value((i & 1) ? xw[i >> 1] >> 16 : xw[i >> 1] & 0xffffu) +
                                bf16_value(bf16_bits(gate * yi));
                    }
                }
                st_stream((uint16_t *)go.out[0] + (size_t)m * go.ld[0] + ne,
                          make_uint4(pack_bf16(r8[0], r8[1]), pack_bf16(r8[2], r8[3]), pack_bf16(r8[4], r8[5]), pack_bf16(r8[6], r8[7])));
            }
        }
        return;
    }

    // lane: column n0 + 32 wn + 16 ni + l16, rows m0 + 16 MI wm + 16 mi + 4 g + r
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
        const int n = n0 + 32 * wn + 16 * ni + l16;
        if (n >= N) continue;
        int seg = 0;
        if constexpr (EPI == kStore) {
            if (go.nseg > 1 && n >= go.col0[1]) seg = (go.nseg > 2 && n >= go.col0[2]) ? 2 : 1;
        }
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 16 * MI * wm + 16 * mi + 4 * g + r;
                if (m >= M) continue;
                const float y = bf16_value(bf16_bits(go.bias ? acc[mi][ni][r] * sc[ni] + bn[ni] : acc[mi][ni][r] * sc[ni]));
                if constexpr (EPI == kStore) {
                    ((uint16_t *)go.out[seg])[(size_t)m * go.ld[seg] + (n - go.col0[seg])] = (uint16_t)bf16_bits(y);
                } else if constexpr (EPI == kGeluErf || EPI == kGeluTanh) {
                    float gv;
                    if constexpr (EPI == kGeluErf) {
                        gv = 0.5f * y * (1.0f + erff(y * 0.7071067811865476f));
                    } else {
                        const float c = 0.7978845608028654f;
                        gv = 0.5f * y * (1.0f + tanhf(c * (y + 0.044715f * y * y * y)));
                    }
                    ((uint16_t *)go.out[0])[(size_t)m * go.ld[0] + n] = (uint16_t)bf16_bits(gv);
                } else if constexpr (EPI == kResidual) {
                    const float a = go.ls ? bf16_value(bf16_bits(y * lsn[ni])) : y;
                    uint16_t *xp = (uint16_t *)go.out[0] + (size_t)m * go.ld[0] + n;
                    *xp = (uint16_t)bf16_bits(bf16_value(*xp) + a);
                } else if constexpr (EPI == kSilu) {
                    ((uint16_t *)go.out[0])[(size_t)m * go.ld[0] + n] = (uint16_t)bf16_bits(y / (1.0f + expf(-y)));
                } else if constexpr (EPI == kSiluAddVec) {
                    const float z = bf16_value(bf16_bits(y + ((const float *)go.aux)[n]));
                    ((uint16_t *)go.out[0])[(size_t)m * go.ld[0] + n] = (uint16_t)bf16_bits(z / (1.0f + expf(-z)));
                } else if constexpr (EPI == kGated) {
                    const float gate = bf16_value(((const uint16_t *)go.aux)[(size_t)m * go.ld_aux + n]);
                    uint16_t *xp = (uint16_t *)go.out[0] + (size_t)m * go.ld[0] + n;
                    *xp = (uint16_t)bf16_bits(bf16_value(*xp) + bf16_value(bf16_bits(gate * y)));
                } else if constexpr (EPI == kAxpyF32) {
                    const float cur = bf16_value(bf16_bits(((const float *)go.aux)[(size_t)m * go.ld_aux + n]));
                    ((float *)go.out[0])[(size_t)m * go.ld[0] + n] =
                        bf16_value(bf16_bits(cur + bf16_value(bf16_bits(y * go.alpha))));
                } else if constexpr (EPI == kAddF32) {
                    const float c = bf16_value(bf16_bits(((const float *)go.aux)[(size_t)m * go.ld_aux + n]));
                    ((uint16_t *)go.out[0])[(size_t)m * go.ld[0] + n] = (uint16_t)bf16_bits(c + y);
                } else { // kStoreF32
                    ((float *)go.out[0])[(size_t)m * go.ld[0] + n] = y;
                }
            }
    }
}

// The staged epilogue's conditions: 8-column pieces that stay inside N and inside one kStore segment,
// and 16-byte aligned accesses to every output and operand row.
static bool gemm_staged(int N, int epi, const GemmOut &go) {
    if (N % 8) return false;
    const int nout = epi == kStore ? go.nseg : 1;
    for (int j = 0; j < nout; ++j)
        if (!go.out[j] || go.ld[j] % 8 || (uintptr_t)go.out[j] % 16 || (epi == kStore && go.col0[j] % 8)) return false;
    if ((epi == kGated || epi == kAxpyF32 || epi == kAddF32) && (go.ld_aux % 8 || (uintptr_t)go.aux % 16)) return false;
    if (epi == kSiluAddVec && (uintptr_t)go.aux % 16) return false;
    if (epi == kResidual && go.ls && (uintptr_t)go.ls % 16) return false;
    return true;
}

template <int MI, int KS, bool STG, int NKC>
static hipError_t gemm_q8_stg(const void *A, int M, int K, const int8_t *W, const float *s, int N, int epi,
                              const GemmOut &go, hipStream_t stream) {
    const dim3 grid(((N + kGmT - 1) / kGmT) * ((M + 32 * MI - 1) / (32 * MI))), block(256 * KS);
    const uint16_t *a = (const uint16_t *)A;
#define XNP_GEMM(E) hipLaunchKernelGGL((k_gemm_q8<E, false, MI, KS, STG, NKC>), grid, block, 0, stream, a, M, K, W, s, N, go)
    if (go.a_f32) {
        if ((epi != kStore && epi != kAddF32) || NKC != 0) return hipErrorInvalidValue;
        if (epi == kStore)
            hipLaunchKernelGGL((k_gemm_q8<kStore, true, MI, KS, STG, 0>), grid, block, 0, stream, a, M, K, W, s, N, go);
        else
            hipLaunchKernelGGL((k_gemm_q8<kAddF32, true, MI, KS, STG, 0>), grid, block, 0, stream, a, M, K, W, s, N, go);
        return hipGetLastError();
    }
    switch (epi) {
    case kStore: XNP_GEMM(kStore); break;
    case kGeluErf: XNP_GEMM(kGeluErf); break;
    case kGeluTanh: XNP_GEMM(kGeluTanh); break;
    case kResidual: XNP_GEMM(kResidual); break;
    case kSilu: XNP_GEMM(kSilu); break;
    case kSiluAddVec: XNP_GEMM(kSiluAddVec); break;
    case kGated: XNP_GEMM(kGated); break;
    case kAxpyF32: XNP_GEMM(kAxpyF32); break;
    case kStoreF32: XNP_GEMM(kStoreF32); break;
    case kAddF32: XNP_GEMM(kAddF32); break;
    default: return hipErrorInvalidValue;
    }
#undef XNP_GEMM
    return hipGetLastError();
}

// The staged epilogue's kernels come unrolled whole for K of 8 or 16 chunks per half (the flow
// LM's 512-2048 wide projections); others run the rounds in a loop.
template <int MI, int KS>
static hipError_t gemm_q8_mi(const void *A, int M, int K, const int8_t *W, const float *s, int N, int epi,
                             const GemmOut &go, hipStream_t stream) {
    if (!gemm_staged(N, epi, go)) return gemm_q8_stg<MI, KS, false, 0>(A, M, K, W, s, N, epi, go, stream);
    if (!go.a_f32 && K == 8 * KS * kGmK) return gemm_q8_stg<MI, KS, true, 8>(A, M, K, W, s, N, epi, go, stream);
    if (!go.a_f32 && K == 16 * KS * kGmK) return gemm_q8_stg<MI, KS, true, 16>(A, M, K, W, s, N, epi, go, stream);
    return gemm_q8_stg<MI, KS, true, 0>(A, M, K, W, s, N, epi, go, stream);
}

hipError_t launch_gemm_q8(const void *A, int M, int K, const int8_t *W, const float *s, int N, int epi,
                          const GemmOut &go, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    if (N <= 0 || K <= 0 || K % 16) return hipErrorInvalidValue;
    // 32-row tiles when 64-row ones would leave the chip's 1024 SIMDs under two waves each; 128-row
    // tiles when those still give 512 groups (two per CU)
    const int64_t ntn = (N + kGmT - 1) / kGmT;
    const int64_t groups64 = ntn * ((M + kGmT - 1) / kGmT), groups128 = ntn * ((M + 127) / 128);
    const bool mi1 = groups64 < 512;
    // two halves per group on alternate K chunks when K is long (32 chunks and more)
    if (K >= 32 * kGmK)
        return mi1 ? gemm_q8_mi<1, 2>(A, M, K, W, s, N, epi, go, stream) : gemm_q8_mi<2, 2>(A, M, K, W, s, N, epi, go, stream);
    if (groups128 >= 512 && !go.a_f32) return gemm_q8_mi<4, 1>(A, M, K, W, s, N, epi, go, stream);
    return mi1 ? gemm_q8_mi<1, 1>(A, M, K, W, s, N, epi, go, stream) : gemm_q8_mi<2, 1>(A, M, K, W, s, N, epi, go, stream);
}

// ---------------------------------------------------------------------------------------------
// f32 pieces of the flow LM around the transformer (flow_lm.rs, mlp.rs, conditioners.rs):
// linears with bias and fused epilogues, LayerNorm with the AdaLN modulation, the LUT gather.
// Batch-1 frames make these matrix-vector products: one wave per output channel, the weight
// row held in registers, each row of x reduced across the wave.

// NORM: a bit set of kNormLn (LayerNorm the row of x over K), kNormAffine (then * w + b) and
// kNormMod (then the AdaLN modulation y * (1 + scale) + shift, mlp.rs:4-11).  Compile-time, so
// that the norm's operands load together with x instead of behind a branch after the reductions.
constexpr int kNormLn = 1, kNormAffine = 2, kNormMod = 4;

template <int KC, int EPI, int NORM>
__global__ __launch_bounds__(256) void k_linear_f32(const float *x, int ldx, int M, int K, const float *W,
                                                    const float *bias, int N, LinOut lo, LinNorm ln) {
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (n >= N) return;
    // every load is issued unconditionally (the index clamped), so that all of them are in flight
    // together rather than each behind a branch and a wait.  Columns past K are zeroed on the x side,
    // inside the row loop: a select on w would be hoisted out of the loop, and every w load would
    // then be waited for before any x load is issued.
    float w[KC], nw[KC], nb[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const int kk = min(c * 64 + lane, K - 1);
        w[c] = W[(size_t)n * K + kk];
        if constexpr ((NORM & kNormAffine) != 0) {
            nw[c] = ln.w[kk];
            nb[c] = ln.b[kk];
        }
    }
    const float b = bias ? bias[n] : 0.f;
    for (int m = 0; m < M; ++m) {
        const float *xr = x + (size_t)m * ldx;
        float xv[KC], sh[KC], sc[KC];
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int kk = min(c * 64 + lane, K - 1);
            xv[c] = xr[kk];
            if constexpr ((NORM & kNormMod) != 0) {
                sh[c] = ln.shift[(size_t)m * ln.ld_mod + kk];
                sc[c] = ln.scale[(size_t)m * ln.ld_mod + kk];
            }
        }
        // the output's address (segments picked with constant indices, so the kernel arguments are
        // read as scalars), and the epilogue's operand loaded with x (every lane, the same word)
        float *o = lo.out[0] + (size_t)m * lo.ld[0] + (n - lo.col0[0]);
        if (lo.nseg > 1 && n >= lo.col0[1]) {
            if (lo.nseg > 2 && n >= lo.col0[2])
                o = lo.out[2] + (size_t)m * lo.ld[2] + (n - lo.col0[2]);
            else
                o = lo.out[1] + (size_t)m * lo.ld[1] + (n - lo.col0[1]);
        }
        float eo = 0.f, er = 0.f; // the auxiliary operand; the residual (the output's old value)
        if constexpr (EPI == kLinResidual || EPI == kLinGated) er = *o;
        if constexpr (EPI == kLinSiluAddVec)
            eo = lo.aux[n];
        else if constexpr (EPI == kLinGated || EPI == kLinAxpy)
            eo = lo.aux[(size_t)m * lo.ld_aux + n];
        // a scheduling barrier: the loads above stay here, issued together, rather than sunk to
        // their uses after the reductions (a round trip each)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr ((NORM & kNormLn) != 0) {
            // mean, then the centred sum of squares: the two passes of a textbook LayerNorm
            float sum = 0.f;
#pragma unroll
            for (int c = 0; c < KC; ++c) sum += c * 64 + lane < K ? xv[c] : 0.f;
            sum = wave_sum(sum);
            const float mean = sum / (float)K;
            float sq = 0.f;
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                const float d = c * 64 + lane < K ? xv[c] - mean : 0.f;
                sq = __builtin_fmaf(d, d, sq);
            }
            sq = wave_sum(sq);
            const float rstd = 1.0f / __builtin_sqrtf(sq / (float)K + ln.eps);
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                float y = (xv[c] - mean) * rstd;
                if constexpr ((NORM & kNormAffine) != 0) y = y * nw[c] + nb[c];
                if constexpr ((NORM & kNormMod) != 0) y = y * (sc[c] + 1.0f) + sh[c];
                xv[c] = y;
            }
        }
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < KC; ++c) acc = __builtin_fmaf(w[c], c * 64 + lane < K ? xv[c] : 0.f, acc);
        acc = wave_sum(acc);
        if (lane != 0) continue;
        const float y = acc + b;
        if constexpr (EPI == kLinStore) {
            *o = y;
        } else if constexpr (EPI == kLinGeluErf) {
            *o = 0.5f * y * (1.0f + erff(y * 0.7071067811865476f));
        } else if constexpr (EPI == kLinGeluTanh) {
            const float c = 0.7978845608028654f;
            *o = 0.5f * y * (1.0f + tanhf(c * (y + 0.044715f * y * y * y)));
        } else if constexpr (EPI == kLinSilu) {
            *o = y / (1.0f + expf(-y));
        } else if constexpr (EPI == kLinSiluAddVec) {
            const float z = y + eo;
            *o = z / (1.0f + expf(-z));
        } else if constexpr (EPI == kLinResidual) {
            *o = er + y;
        } else if constexpr (EPI == kLinGated) {
            *o = er + eo * y;
        } else { // kLinAxpy
            *o = eo + y * lo.alpha;
        }
    }
}

template <int KC, int NORM>
static hipError_t linear_f32_kc(const float *x, int ldx, int M, int K, const float *W, const float *b, int N, int epi,
                                const LinOut &lo, const LinNorm &ln, hipStream_t stream) {
    const dim3 grid((N + 3) / 4), block(256);
#define XNP_LIN(E) hipLaunchKernelGGL((k_linear_f32<KC, E, NORM>), grid, block, 0, stream, x, ldx, M, K, W, b, N, lo, ln)
    switch (epi) {
    case kLinStore: XNP_LIN(kLinStore); break;
    case kLinGeluErf: XNP_LIN(kLinGeluErf); break;
    case kLinGeluTanh: XNP_LIN(kLinGeluTanh); break;
    case kLinSilu: XNP_LIN(kLinSilu); break;
    case kLinSiluAddVec: XNP_LIN(kLinSiluAddVec); break;
    case kLinResidual: XNP_LIN(kLinResidual); break;
    case kLinGated: XNP_LIN(kLinGated); break;
    case kLinAxpy: XNP_LIN(kLinAxpy); break;
    default: return hipErrorInvalidValue;
    }
#undef XNP_LIN
    return hipGetLastError();
}

template <int NORM>
static hipError_t linear_f32_norm(const float *x, int ldx, int M, int K, const float *W, const float *b, int N, int epi,
                                  const LinOut &lo, const LinNorm &ln, hipStream_t stream) {
    const int kc = (K + 63) / 64;
    if (kc <= 1) return linear_f32_kc<1, NORM>(x, ldx, M, K, W, b, N, epi, lo, ln, stream);
    if (kc <= 4) return linear_f32_kc<4, NORM>(x, ldx, M, K, W, b, N, epi, lo, ln, stream);
    if (kc <= 8) return linear_f32_kc<8, NORM>(x, ldx, M, K, W, b, N, epi, lo, ln, stream);
    if (kc <= 16) return linear_f32_kc<16, NORM>(x, ldx, M, K, W, b, N, epi, lo, ln, stream);
    if (kc <= 32) return linear_f32_kc<32, NORM>(x, ldx, M, K, W, b, N, epi, lo, ln, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_linear_f32(const float *x, int ldx, int M, int K, const float *W, const float *b, int N, int epi,
                             const LinOut &lo, hipStream_t stream, const LinNorm *ln) {
    if (M <= 0 || N <= 0) return hipSuccess;
    if (!ln) return linear_f32_norm<0>(x, ldx, M, K, W, b, N, epi, lo, LinNorm(), stream);
    if ((ln->w == nullptr) != (ln->b == nullptr) || (ln->shift == nullptr) != (ln->scale == nullptr))
        return hipErrorInvalidValue;
    if (ln->w && ln->shift) return linear_f32_norm<kNormLn | kNormAffine | kNormMod>(x, ldx, M, K, W, b, N, epi, lo, *ln, stream);
    if (ln->w) return linear_f32_norm<kNormLn | kNormAffine>(x, ldx, M, K, W, b, N, epi, lo, *ln, stream);
    if (ln->shift) return linear_f32_norm<kNormLn | kNormMod>(x, ldx, M, K, W, b, N, epi, lo, *ln, stream);
    return linear_f32_norm<kNormLn>(x, ldx, M, K, W, b, N, epi, lo, *ln, stream);
}

// LUTConditioner::embed_tokens (conditioners.rs:239-262): out[r] = table[ids[r]], rows of dim f32.
__global__ void k_embed_f32(const float *table, const int32_t *ids, int rows, int dim, float *out) {
    const int r = blockIdx.x;
    const float *src = table + (size_t)ids[r] * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[(size_t)r * dim + i] = src[i];
}

__global__ void k_gather_rows(const uint4 *table, const int32_t *ids, int row_u4, uint4 *out) {
    const int r = blockIdx.x;
    const uint4 *src = table + (size_t)ids[r] * row_u4;
    for (int i = threadIdx.x; i < row_u4; i += blockDim.x) out[(size_t)r * row_u4 + i] = src[i];
}

hipError_t launch_gather_rows(const void *table, const int32_t *ids, int rows, int row_bytes, void *out,
                              hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (row_bytes % 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gather_rows, dim3(rows), dim3(256), 0, stream, (const uint4 *)table, ids, row_bytes / 16,
                       (uint4 *)out);
    return hipGetLastError();
}

hipError_t launch_embed_f32(const float *table, const int32_t *ids, int rows, int dim, float *out, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_embed_f32, dim3(rows), dim3(256), 0, stream, table, ids, rows, dim, out);
    return hipGetLastError();
}


} // namespace xnp
