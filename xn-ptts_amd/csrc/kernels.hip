// HIP kernels of the paged flow-LM KV cache, written for gfx950 (CDNA4, wave64).
//
// Bit-exactness contract with the CPU restatement: the library is built with
// -ffp-contract=off, RoPE rotates with host-computed cos/sin tables, bf16 rounding is
// round-to-nearest-even on the f32 bits, int8 quantization is rint(y / s) clamped to +-127 with
// IEEE division.  The attention arithmetic (dots, softmax, weighted sums) is f32 in an order of
// its own and is checked to a tolerance, not bit for bit.
#include "xnp_internal.h"

#include <hip/hip_ext.h>

#include <algorithm>


namespace xnp {

// Launch a kernel; with timing events, through hipExtLaunchKernel so that the events bracket the
// kernel alone.  Without them, a plain launch: the form a stream capture (hipGraph) records.
#define XNP_LAUNCH(kernel, grid, block, stream, tm, ...)                                            \
    do {                                                                                           \
        if ((tm).start || (tm).stop)                                                               \
            hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, (tm).start, (tm).stop, 0, __VA_ARGS__); \
        else                                                                                       \
            hipLaunchKernelGGL(kernel, grid, block, 0, stream, __VA_ARGS__);                       \
    } while (0)

// ---------------------------------------------------------------------------------------------
// element helpers

__device__ __forceinline__ float bf16_value(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Round to bf16 with v_cvt_pk_bf16_f32: round to nearest even, NaN kept quiet.  The same bits as
// the CPU restatement's software rounding (checked on this hardware over 4M inputs: random
// bits, exact ties, denormals, NaN and infinities).
typedef float f32x2v_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef __fp16 f16x2v_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    const bf16x2v_t h = __builtin_convertvector((f32x2v_t){a, b}, bf16x2v_t);
    uint32_t u;
    __builtin_memcpy(&u, &h, 4);
    return u;
}

__device__ __forceinline__ uint32_t bf16_bits(float x) { return pack_bf16(x, 0.f) & 0xffffu; }

template <bool ABF> __device__ __forceinline__ float round_act(float x) {
    if constexpr (ABF) return bf16_value(bf16_bits(x));
    return x;
}

__device__ __forceinline__ int quant(float y, float s) {
    if (!(s > 0.0f)) return 0;
    float r = __builtin_rintf(y / s);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int)r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 16 bytes with the non-temporal hint.  A decode launch reads each K/V tile once: streamed, the
// tiles stop displacing what the launch does reuse in L2 and the memory-side cache (records,
// tables, queries).  Measured on attend_core's page loads: bf16 decode at 1024 streams 192 ->
// 171 us, int8 window 104.4 -> 95.0 us; on the prefill's key/value staging 32.8 -> 32.2 us.  Only
// where one load instruction covers whole 128-byte lines (attend_core: 1 KB contiguous per wave).
__device__ __forceinline__ uint4 ld_stream(const void *p) {
    typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
    const u32x4_nt a = __builtin_nontemporal_load((const u32x4_nt *)p);
    return make_uint4(a.x, a.y, a.z, a.w);
}

template <int CDT> constexpr int esize() { return CDT == DT_F32 ? 4 : CDT == DT_BF16 ? 2 : 1; }

// Element offset of row 0 of tile (layer, kv, page, head).
// The (page, kv head) tile: pages hold the KVH heads a layer stores (query heads h share kv head
// h / (H / KVH), transformer.rs:199-211), not the H repeated ones.
__device__ __forceinline__ size_t tile_index(const PoolView &pv, int layer, int kv, int page, int j) {
    return (((size_t)layer * 2 + kv) * pv.NB + page) * pv.KVH + j;
}

// Two activation values (dims 2i, 2i+1) of a head row.
template <bool ABF> __device__ __forceinline__ float2 load_pair(const void *row, int i) {
    if constexpr (ABF) {
        uint32_t w = ((const uint32_t *)row)[i];
        return make_float2(bf16_value(w & 0xffffu), bf16_value(w >> 16));
    } else {
        return ((const float2 *)row)[i];
    }
}

// ---------------------------------------------------------------------------------------------
// append: one wave writes one new row of one head, keys (lanes 0-31, RoPE'd) and values
// (lanes 32-63), each lane one pair of dims.  complete_kv, transformer.rs:61-92, with the k
// rotation of rope.rs:74-95 fused in.

template <int CDT, bool ABF>
__device__ void append_row_wave(const PoolView &pv, int layer, int page, int row, int h, int key_pos,
                                const void *krow, const void *vrow, bool fresh) {
    const int lane = threadIdx.x & 63;
    const int kv = lane >> 5;
    const int pr = lane & 31;
    float2 x = load_pair<ABF>(kv ? vrow : krow, pr);
    if (kv == 0) {
        float2 cs = pv.rope[(size_t)key_pos * (pv.D / 2) + pr];
        float a = x.x * cs.x, b = x.y * cs.y, e = x.x * cs.y, f = x.y * cs.x;
        x.x = round_act<ABF>(a - b);
        x.y = round_act<ABF>(e + f);
    }
    const size_t tile = tile_index(pv, layer, kv, page, h);
    if constexpr (CDT == DT_F32) {
        ((float2 *)pv.pages)[tile * (kBlock * kHeadDim / 2) + row * (kHeadDim / 2) + pr] = x;
    } else if constexpr (CDT == DT_BF16) {
        ((uint32_t *)pv.pages)[tile * (kBlock * kHeadDim / 2) + row * (kHeadDim / 2) + pr] =
            bf16_bits(x.x) | (bf16_bits(x.y) << 16);
    } else {
        // int8: per-(page, head) scale amax / 127.  A page holding another live row keeps its
        // scale unless this row needs a larger one; then its other rows are requantized.
        float amax = fmaxf(fabsf(x.x), fabsf(x.y));
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
        const float s_row = amax / 127.0f;
        float *sp = pv.scales + tile;
        const float s_old = *sp;
        const float s_new = fresh ? s_row : fmaxf(s_old, s_row);
        const int req = (!fresh && s_new > s_old) ? 1 : 0;
        int8_t *pages8 = (int8_t *)pv.pages;
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            const int rq = __shfl(req, which * 32);
            if (rq) {
                const float so = __shfl(s_old, which * 32), sn = __shfl(s_new, which * 32);
                const size_t wt = tile_index(pv, layer, which, page, h);
                uint4 *tp = (uint4 *)(pages8 + wt * (kBlock * kHeadDim)) + lane;
                if ((lane >> 2) != row) { // 4 lanes per 64-byte row
                    uint4 w = *tp;
                    uint32_t *wv = (uint32_t *)&w;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        uint32_t o = 0;
#pragma unroll
                        for (int bt = 0; bt < 4; ++bt) {
                            int qv = (int)(int8_t)((wv[j] >> (8 * bt)) & 0xffu);
                            int nq = quant((float)qv * so, sn);
                            o |= ((uint32_t)(nq & 0xff)) << (8 * bt);
                        }
                        wv[j] = o;
                    }
                    *tp = w;
                }
            }
        }
        const uint32_t q0 = (uint32_t)(quant(x.x, s_new) & 0xff), q1 = (uint32_t)(quant(x.y, s_new) & 0xff);
        ((uint16_t *)(pages8 + tile * (kBlock * kHeadDim)))[row * (kHeadDim / 2) + pr] =
            (uint16_t)(q0 | (q1 << 8));
        if (pr == 0) *sp = s_new;
    }
}

// ---------------------------------------------------------------------------------------------
// block-table patches (pages taken since the previous batch)

__global__ void k_patch_tables(int32_t *tables, const TablePatch *patches, int n, int mbps) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) tables[(size_t)patches[i].sid * mbps + patches[i].blk] = patches[i].page;
}

hipError_t launch_patch_tables(const PoolView &pv, const TablePatch *patches, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_patch_tables, dim3((n + 255) / 256), dim3(256), 0, stream, pv.tables, patches, n,
                       pv.mbps);
    return hipGetLastError();
}

// The batch plan, read straight from the pinned staging buffer the host composed it in, and the
// block-table patches staged behind it: one launch, where copies would take a copy engine per
// part plus a patch kernel, with a hand-off between engines before each.  The launch boundary
// makes the host's writes to the buffer visible.
__global__ __launch_bounds__(256) void k_pull_plan(const uint4 *src, uint4 *dst, int n16, const TablePatch *patches,
                                                   int np, int32_t *tables, int mbps) {
    const int stride = gridDim.x * blockDim.x, i0 = blockIdx.x * blockDim.x + threadIdx.x;
    for (int i = i0; i < n16; i += stride) dst[i] = src[i];
    for (int i = i0; i < np; i += stride) {
        const TablePatch t = patches[i];
        tables[(size_t)t.sid * mbps + t.blk] = t.page;
    }
}

hipError_t launch_pull_plan(const PoolView &pv, const void *src, void *dst, size_t bytes, const TablePatch *patches,
                            int np, hipStream_t stream) {
    const int n16 = (int)((bytes + 15) / 16), work = std::max(n16, np);
    if (work <= 0) return hipSuccess;
    const int blocks = std::min((work + 255) / 256, 1024);
    hipLaunchKernelGGL(k_pull_plan, dim3(blocks), dim3(256), 0, stream, (const uint4 *)src, (uint4 *)dst, n16, patches,
                       np, pv.tables, pv.mbps);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// standalone append of t rows per stream.  Work item = (stream, page the rows touch); one wave
// per head walks the page's rows in order, since int8 rows of one page depend on each other.

template <int CDT, bool ABF>
__global__ __launch_bounds__(1024) void k_append(PoolView pv, BatchView bv, int layer, const void *k,
                                                 const void *v, int nseg) {
    const int b = blockIdx.x / nseg, seg = blockIdx.x % nseg;
    const StreamPlan P = bv.plans[b];
    const int j = threadIdx.x >> 6; // kv head
    const int t = bv.t;
    const int ws = P.write_slot;
    const int blk = (ws >> 4) + seg;
    const int i0 = max(0, blk * kBlock - ws), i1 = min(t, (blk + 1) * kBlock - ws);
    if (i0 >= i1) return;
    const int page = pv.tables[(size_t)P.sid * pv.mbps + blk];
    if (page < 0 || page >= pv.NB) return; // begin took this page; never index the pool without one
    constexpr int AE = ABF ? 2 : 4;
    for (int i = i0; i < i1; ++i) {
        const int slot = ws + i;
        const size_t arow = ((size_t)P.out_row * t + i) * pv.KVH + j;
        const bool fresh = P.ring ? (P.fresh != 0) : ((slot & 15) == 0);
        append_row_wave<CDT, ABF>(pv, layer, page, slot & 15, j, P.key_pos + i,
                                  (const char *)k + arow * kHeadDim * AE, (const char *)v + arow * kHeadDim * AE,
                                  fresh);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------
// decode: one work group per (stream, head).  Its SPLIT waves interleave the stream's pages (wave w
// takes pages w, w + SPLIT, ...), each keeping an online softmax over the rows it reads, and
// merge through LDS at the end: no partial ever leaves the CU.
//
// Lane layout over a 16 x 64 tile of one head: every lane loads 16 contiguous bytes per pass,
// DPL dims of one row (DPL = 4 f32, 8 bf16, 16 int8), so a pass is one coalesced 1 KB read per
// wave.  The LPR lanes of a row reduce the row's dot product with xor shuffles; each lane keeps
// an online softmax over the rows it saw and the lanes of one dim slice merge at the end.
// Scores are kept in log2 units (the query is prescaled by scale * log2(e)).

template <int CDT> struct Lanes {
    static constexpr int DPL = 16 / esize<CDT>();
    static constexpr int LPR = kHeadDim / DPL;
    static constexpr int RPP = 64 / LPR;
    static constexpr int NP = kBlock / RPP;
    // blocks in flight per wave: 4 KB (f32), 8 KB (bf16), 4 KB (int8) of K and V
    static constexpr int DEPTH = CDT == DT_F32 ? 1 : 2;
    // waves per SIMD the register budget is sized for (512 VGPRs / waves)
    static constexpr int WAVES = CDT == DT_F32 ? 3 : 4;
};

template <int CDT>
__device__ __forceinline__ void unpack(const uint4 &w, float (&x)[Lanes<CDT>::DPL]) {
    const uint32_t *u = (const uint32_t *)&w;
    if constexpr (CDT == DT_F32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(u[i]);
    } else if constexpr (CDT == DT_BF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = bf16_value(u[i] & 0xffffu);
            x[2 * i + 1] = bf16_value(u[i] >> 16);
        }
    } else {
        // int8 codes q as q + 128: flipping the top bit of each byte makes it unsigned, and an
        // unsigned byte converts to f32 in one instruction (v_cvt_f32_ubyte0..3).  The callers
        // take the 128 back out once per dot product / per accumulator.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t b = u[i] ^ 0x80808080u;
#pragma unroll
            for (int bt = 0; bt < 4; ++bt) x[4 * i + bt] = (float)((b >> (8 * bt)) & 0xffu);
        }
    }
}

// Rotated query slice (dims DPL*c .. DPL*c+DPL-1) at `pos`, rounded to the activation dtype and
// prescaled.
template <int DPL, bool ABF>
__device__ __forceinline__ void rotated_q(const PoolView &pv, const void *qrow, int c, int pos, float mul,
                                          float (&out)[DPL]) {
#pragma unroll
    for (int i = 0; i < DPL / 2; ++i) {
        const int pr = c * (DPL / 2) + i;
        float2 x = load_pair<ABF>(qrow, pr);
        float2 cs = pv.rope[(size_t)pos * (pv.D / 2) + pr];
        float a = x.x * cs.x, b = x.y * cs.y, e = x.x * cs.y, f = x.y * cs.x;
        out[2 * i] = round_act<ABF>(a - b) * mul;
        out[2 * i + 1] = round_act<ABF>(e + f) * mul;
    }
}

// One query row of GQ query heads h .. h + GQ - 1 (all of one kv head) against pages
// [0, R.nblk) of its stream, by a group of SPLIT waves: the body of the decode kernel and of the
// prompt-row kernel.  `pages` lists the stream's page ids by logical block (a decode record's
// copy, or the block table).  With GQ > 1 each page is read once for the GQ heads: K is unpacked
// (or taken by dot2) once per row, V once, and each head keeps its own online softmax.
template <int CDT, bool ABF, int SPLIT, bool PREFIX, int GQ = 1>
__device__ __forceinline__ void attend_core(const PoolView &pv, const BatchView &bv, int layer, const StreamRec &R,
                                            const int32_t *rec_pages, int h, const void *q, const void *knew,
                                            const void *vnew, void *out, float qmul, int fused) {
    using LN = Lanes<CDT>;
    constexpr int DPL = LN::DPL, LPR = LN::LPR, RPP = LN::RPP, NP = LN::NP, DEPTH = LN::DEPTH;
    constexpr int AE = ABF ? 2 : 4;
    __shared__ float part[SPLIT][GQ][kPartStride];

    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nb = R.nblk > w ? (R.nblk - w + SPLIT - 1) / SPLIT : 0; // this wave's pages
    const int kvh = h / (pv.H / pv.KVH);                               // the tiles the heads read

    // Per-page metadata, lane j holding page w + j * SPLIT: page id, seen rows, int8 scales.
    // Past the wave's last page the lanes hold page 0 with no row seen.
    int my_page = 0;
    uint32_t my_seen = 0;
    float my_sk = 0.f, my_sv = 0.f;
    // issued with the header load: record slots past nblk hold stale ids and are masked below
    const int pg_raw = w + lane * SPLIT < pv.mbps ? rec_pages[w + lane * SPLIT] : -1;
    if (lane < nb) {
        const int blk = w + lane * SPLIT;
        const int base = blk * kBlock;
        uint32_t seen = 0xffffu;
        if (R.mask_off >= 0) seen = (bv.masks[R.mask_off + (base >> 5)] >> (base & 16)) & 0xffffu;
        const int nvalid = R.span - base;
        if (nvalid < kBlock) seen &= (1u << max(nvalid, 0)) - 1u;
        const int pg = pg_raw;
        const bool ok = pg >= 0 && pg < pv.NB;
        if (!ok) seen = 0;
        my_page = ok ? pg : 0;
        my_seen = seen;
        if constexpr (CDT == DT_I8) {
            my_sk = pv.scales[tile_index(pv, layer, 0, my_page, kvh)];
            my_sv = pv.scales[tile_index(pv, layer, 1, my_page, kvh)];
        }
    }

    const int c = lane % LPR, g = lane / LPR;
    // bf16 pages and queries: scores by v_dot2_f32_bf16 on packed bf16 pairs (the page words as
    // they are, no unpacking), with the query's scale applied to each row's sum
    constexpr bool DOT2 = CDT == DT_BF16 && ABF;
    // int8 pages and bf16 queries: the query as f16 pairs (a bf16 value converts exactly), each
    // code byte b (q + 128) under the f16 exponent of 1024 by one byte permute, so that
    // v_dot2_f32_f16 sums q (1024 + b) = q (1152 + code) exactly per product; 1152 sum(q) comes
    // back out once per row
    constexpr bool H16 = CDT == DT_I8 && ABF;
    const bool two_q = PREFIX && R.prefix > 0; // PREFIX: some stream of the batch keeps a prefix
    float qw[GQ][DPL], qp[GQ][DPL];
    uint32_t qh[GQ][DPL / 2], ph[GQ][DPL / 2]; // DOT2, H16: the rotated queries' bf16 / f16 pairs
    // int8: unpack hands out q + 128, so a dot product is sum(qw (q + 128)) - 128 sum(qw) and a
    // value accumulator carries -128 sum(e sv) on every dim (vbias, taken out after the loop)
    float qwsum[GQ], qpsum[GQ], vbias[GQ];
#pragma unroll
    for (int e = 0; e < GQ; ++e) {
        const char *qrow = (const char *)q + ((size_t)R.b * pv.H + h + e) * kHeadDim * AE;
        rotated_q<DPL, ABF>(pv, qrow, c, R.pos, DOT2 || H16 ? 1.f : qmul, qw[e]);
        if (two_q) rotated_q<DPL, ABF>(pv, qrow, c, R.pos_pre, DOT2 || H16 ? 1.f : qmul, qp[e]);
        if constexpr (DOT2) {
#pragma unroll
            for (int i = 0; i < DPL / 2; ++i) {
                qh[e][i] = (__float_as_uint(qw[e][2 * i]) >> 16) | (__float_as_uint(qw[e][2 * i + 1]) & 0xffff0000u);
                ph[e][i] = (__float_as_uint(qp[e][2 * i]) >> 16) | (__float_as_uint(qp[e][2 * i + 1]) & 0xffff0000u);
            }
        }
        if constexpr (H16) {
#pragma unroll
            for (int i = 0; i < DPL / 2; ++i) {
                qh[e][i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(qw[e][2 * i], qw[e][2 * i + 1]));
                ph[e][i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(qp[e][2 * i], qp[e][2 * i + 1]));
            }
        }
        qwsum[e] = qpsum[e] = vbias[e] = 0.f;
        if constexpr (CDT == DT_I8) {
#pragma unroll
            for (int i = 0; i < DPL; ++i) qwsum[e] += qw[e][i];
            if (two_q) {
#pragma unroll
                for (int i = 0; i < DPL; ++i) qpsum[e] += qp[e][i];
            }
        }
    }

    const uint4 *kbase = (const uint4 *)((const char *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim * esize<CDT>()));
    const uint4 *vbase = (const uint4 *)((const char *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim * esize<CDT>()));
    const size_t page_u4 = (size_t)pv.KVH * (kBlock * kHeadDim * esize<CDT>() / 16);

    float m[GQ], l[GQ], acc[GQ][DPL];
#pragma unroll
    for (int e = 0; e < GQ; ++e) {
        m[e] = -1e30f;
        l[e] = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[e][i] = 0.f;
    }

    // One page's scores and softmax/accumulator update from its K and V registers.
    auto process = [&](const uint4 (&kr)[NP], const uint4 (&vr)[NP], int j) {
        const uint32_t seen = __builtin_amdgcn_readlane(my_seen, j);
        const int base = (w + j * SPLIT) * kBlock;
        float sk = 1.f, sv = 1.f;
        if constexpr (CDT == DT_I8) {
            sk = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(my_sk), j));
            sv = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(my_sv), j));
        }
        float s[GQ][NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int r = g + RPP * p;
            const bool pre = two_q && base + r < R.prefix; // a prefix row: the queries at pos_pre
            float dw[GQ];
            if constexpr (DOT2) {
                const uint32_t *u = (const uint32_t *)&kr[p];
#pragma unroll
                for (int e = 0; e < GQ; ++e) {
                    dw[e] = 0.f;
#pragma unroll
                    for (int i = 0; i < DPL / 2; ++i)
                        dw[e] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v_t, pre ? ph[e][i] : qh[e][i]),
                                                                __builtin_bit_cast(bf16x2v_t, u[i]), dw[e], false);
                }
            } else if constexpr (H16) {
                const uint32_t *u = (const uint32_t *)&kr[p];
#pragma unroll
                for (int e = 0; e < GQ; ++e) dw[e] = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t x = u[i] ^ 0x80808080u;
                    // bytes 0, 1 (then 2, 3) of x as the low bytes of two f16 whose high bytes are 0x64
                    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
                    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
#pragma unroll
                    for (int e = 0; e < GQ; ++e) {
                        dw[e] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2v_t, pre ? ph[e][2 * i] : qh[e][2 * i]),
                                                       __builtin_bit_cast(f16x2v_t, lo), dw[e], false);
                        dw[e] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2v_t, pre ? ph[e][2 * i + 1] : qh[e][2 * i + 1]),
                                                       __builtin_bit_cast(f16x2v_t, hi), dw[e], false);
                    }
                }
#pragma unroll
                for (int e = 0; e < GQ; ++e) dw[e] = __builtin_fmaf(-1152.f, pre ? qpsum[e] : qwsum[e], dw[e]);
            } else {
                float x[DPL];
                unpack<CDT>(kr[p], x);
#pragma unroll
                for (int e = 0; e < GQ; ++e) {
                    dw[e] = 0.f;
#pragma unroll
                    for (int i = 0; i < DPL; ++i) dw[e] = __builtin_fmaf(qw[e][i], x[i], dw[e]);
                    if constexpr (CDT == DT_I8) dw[e] = __builtin_fmaf(-128.f, qwsum[e], dw[e]);
                    if (pre) {
                        float dp = 0.f;
#pragma unroll
                        for (int i = 0; i < DPL; ++i) dp = __builtin_fmaf(qp[e][i], x[i], dp);
                        if constexpr (CDT == DT_I8) dp = __builtin_fmaf(-128.f, qpsum[e], dp);
                        dw[e] = dp;
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < GQ; ++e) {
#pragma unroll
                for (int o = 1; o < LPR; o <<= 1) dw[e] += __shfl_xor(dw[e], o);
                if constexpr (CDT == DT_I8) dw[e] *= sk;
                if constexpr (DOT2 || H16) dw[e] *= qmul;
                s[e][p] = ((seen >> r) & 1u) ? dw[e] : -INFINITY;
            }
        }
        // Lazy rescaling: the accumulators move to a new max only when some lane's max grew by
        // more than 8 (log2 units).  Until then exponents are taken against the older max and
        // stay below 2^8, and the final l and acc keep the same ratio.  Most pages skip the
        // rescale, the branch being uniform over the wave.
        float m_new[GQ];
        bool grow = false;
#pragma unroll
        for (int e = 0; e < GQ; ++e) {
            float smax = s[e][0];
#pragma unroll
            for (int p = 1; p < NP; ++p) smax = fmaxf(smax, s[e][p]);
            m_new[e] = fmaxf(m[e], smax);
            grow |= m_new[e] > m[e] + 8.f;
        }
        if (__any(grow)) {
#pragma unroll
            for (int e = 0; e < GQ; ++e) {
                const float alpha = fast_exp2(m[e] - m_new[e]);
                l[e] *= alpha;
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[e][i] *= alpha;
                if constexpr (CDT == DT_I8) vbias[e] *= alpha;
                m[e] = m_new[e];
            }
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            // an unseen row weighs 0, but its bytes may be anything (a page's unwritten rows
            // hold what the memory held before): zero them, since 0 * NaN would still be NaN.
            // int8 bytes always convert to finite values (scales start at 0 and are amax / 127),
            // so int8 rows need no zeroing.
            const bool rs = (seen >> (g + RPP * p)) & 1u;
            const uint4 vv = (CDT == DT_I8 || rs) ? vr[p] : make_uint4(0, 0, 0, 0);
            float x[DPL];
            unpack<CDT>(vv, x);
#pragma unroll
            for (int e = 0; e < GQ; ++e) {
                const float pe = fast_exp2(s[e][p] - m[e]);
                l[e] += pe;
                const float ev = (CDT == DT_I8) ? pe * sv : pe;
                if constexpr (CDT == DT_I8) vbias[e] += ev;
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[e][i] = __builtin_fmaf(ev, x[i], acc[e][i]);
            }
        }
    };
    auto load = [&](uint4 (&kr)[NP], uint4 (&vr)[NP], int j) {
        const int pg = __builtin_amdgcn_readlane(my_page, j);
        const size_t off = (size_t)pg * page_u4 + lane;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            kr[p] = ld_stream(kbase + off + 64 * p);
            vr[p] = ld_stream(vbase + off + 64 * p);
        }
    };

    // DEPTH pages in flight ahead of the one being reduced.  The loop body has no branch: past
    // the wave's last page the lanes' page is page 0, a tile every wave shares (so mostly a cache
    // hit), and its rows are unseen, so reducing it changes nothing.  Each wait then only covers
    // the oldest page's loads.
    uint4 kb[DEPTH + 1][NP], vb[DEPTH + 1][NP];

    // complete_kv: the wave that owns the write page appends this head's new row, then reads it
    // back with the rest of its pages (its own lanes' stores; no other wave touches the page).
    // A workgroup-scope fence orders the stores before the later loads on the same CU; nothing
    // waits for the stores to reach memory.  When the write page is not among the wave's first
    // DEPTH pages, those are loaded before the append, so the append's round trips overlap them.
    const int wblk = R.write_slot >> 4, wj = wblk / SPLIT;
    const bool owner = fused && w == wblk % SPLIT;
    const bool early = !owner || wj >= DEPTH;
    if (early) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(kb[d], vb[d], d);
    }
    if (owner) {
        const int slot = R.write_slot;
        const size_t arow = (size_t)R.b * pv.KVH + kvh;
        const bool fresh = (R.flags & 1) ? (R.flags & 2) != 0 : ((slot & 15) == 0);
        // with grouped heads every work group of the kv head writes the same row (the same bytes);
        // int8 pools append in a kernel of their own first, since their append rewrites the page
        append_row_wave<CDT, ABF>(pv, layer, __builtin_amdgcn_readlane(my_page, wj), slot & 15, kvh, R.key_pos,
                                  (const char *)knew + arow * kHeadDim * AE, (const char *)vnew + arow * kHeadDim * AE,
                                  fresh);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
        if constexpr (CDT == DT_I8) {
            if (lane == wj) { // the append may have raised this page's scales
                my_sk = pv.scales[tile_index(pv, layer, 0, my_page, kvh)];
                my_sv = pv.scales[tile_index(pv, layer, 1, my_page, kvh)];
            }
        }
    }
    if (!early) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(kb[d], vb[d], d);
    }
    for (int j = 0; j < nb; j += DEPTH + 1) {
#pragma unroll
        for (int u = 0; u <= DEPTH; ++u) {
            load(kb[(u + DEPTH) % (DEPTH + 1)], vb[(u + DEPTH) % (DEPTH + 1)], j + u + DEPTH);
            process(kb[u], vb[u], j + u);
        }
    }

#pragma unroll
    for (int e = 0; e < GQ; ++e) {
        if constexpr (CDT == DT_I8) {
#pragma unroll
            for (int i = 0; i < DPL; ++i) acc[e][i] = __builtin_fmaf(-128.f, vbias[e], acc[e][i]);
        }
        // Merge the row groups: lanes c, c + LPR, c + 2 LPR, ... hold the same dims.
#pragma unroll
        for (int o = LPR; o < 64; o <<= 1) {
            const float mo = __shfl_xor(m[e], o), lo = __shfl_xor(l[e], o);
            const float mn = fmaxf(m[e], mo);
            const float a = fast_exp2(m[e] - mn), bb = fast_exp2(mo - mn);
            l[e] = l[e] * a + lo * bb;
#pragma unroll
            for (int i = 0; i < DPL; ++i) {
                const float ao = __shfl_xor(acc[e][i], o);
                acc[e][i] = acc[e][i] * a + ao * bb;
            }
            m[e] = mn;
        }
        // the waves' shares of head h + e go through LDS
        if (g == 0) {
#pragma unroll
            for (int i = 0; i < DPL; ++i) part[w][e][c * DPL + i] = acc[e][i];
            if (lane == 0) {
                part[w][e][64] = m[e];
                part[w][e][65] = l[e];
            }
        }
    }
    __syncthreads();
    if (w != 0) return;
    // wave 0 writes the heads' outputs, lane d owning dim d
#pragma unroll
    for (int e = 0; e < GQ; ++e) {
        float M = -1e30f;
#pragma unroll
        for (int k = 0; k < SPLIT; ++k) M = fmaxf(M, part[k][e][64]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int k = 0; k < SPLIT; ++k) {
            const float a = fast_exp2(part[k][e][64] - M);
            L = __builtin_fmaf(part[k][e][65], a, L);
            A = __builtin_fmaf(part[k][e][lane], a, A);
        }
        const float r = A / L;
        const size_t o = ((size_t)R.b * pv.H + h + e) * kHeadDim + lane;
        if constexpr (ABF)
            ((uint16_t *)out)[o] = (uint16_t)bf16_bits(r);
        else
            ((float *)out)[o] = r;
    }
}

// Decode: one work group per (stream, GQ query heads of one kv head), streams longest first.  The
// stream record carries everything the group needs, its page ids included.
template <int CDT, bool ABF, int SPLIT, bool PREFIX, int GQ>
__global__ __launch_bounds__(64 * SPLIT) __attribute__((amdgpu_waves_per_eu(Lanes<CDT>::WAVES))) void k_decode(
    PoolView pv, BatchView bv, int layer, const void *q, const void *knew, const void *vnew, void *out, float qmul,
    int fused) {
    // Work groups go to the 8 XCDs in turn (group b to XCD b % 8).  A stream has P = H / GQ groups
    // (slot s: query heads GQ s ..).  In runs of 8 P groups, XCD x takes the P groups of stream x of
    // the run, one after another: the heads of one page block (adjacent tiles in HBM) are read from
    // one XCD at about the same time, and the groups that share a kv head (consecutive slots) meet
    // in its L2.  Measured against one head per XCD: int8 window 107.5 -> 105.6 us, bf16 decode
    // 192.2 -> 191.8 us.
    const int P = pv.H / GQ, b = blockIdx.x;
    const int full = bv.n / 8 * 8; // streams in whole runs
    int sidx, slot;
    if (b < full * P) {
        sidx = b / (8 * P) * 8 + b % 8;
        slot = b % (8 * P) / 8;
    } else {
        sidx = full + (b - full * P) / P;
        slot = (b - full * P) % P;
    }
    const char *rec = bv.recs + (size_t)sidx * bv.rec_stride;
    const StreamRec R = *(const StreamRec *)rec;
    attend_core<CDT, ABF, SPLIT, PREFIX, GQ>(pv, bv, layer, R, (const int32_t *)(rec + sizeof(StreamRec)), slot * GQ,
                                             q, knew, vnew, out, qmul, fused);
}

// Prompt rows (transformer.rs:231-248), after k_append has written all t rows: row i of a stream
// attends causally to slots [0, current_end + i], its query rotated at position current_end + i.
// One work group per (stream, row, head), latest rows (the most keys) first.
template <int CDT, bool ABF, int SPLIT>
__global__ __launch_bounds__(64 * SPLIT) __attribute__((amdgpu_waves_per_eu(Lanes<CDT>::WAVES))) void k_prefill_rows(
    PoolView pv, BatchView bv, int layer, const void *q, void *out, float qmul) {
    const int t = bv.t;
    const int h = blockIdx.x % pv.H, rest = blockIdx.x / pv.H;
    const int i = t - 1 - rest % t, b = rest / t;
    const StreamPlan P = bv.plans[b];
    StreamRec R;
    R.b = P.out_row * t + i;
    R.span = P.write_slot + i + 1;
    R.nblk = (R.span + kBlock - 1) / kBlock;
    R.pos = P.pos + i;
    R.pos_pre = P.pos_pre + i;
    R.prefix = P.prefix;
    R.write_slot = P.write_slot + i;
    R.key_pos = P.key_pos + i;
    R.mask_off = -1;
    R.flags = 0;
    attend_core<CDT, ABF, SPLIT, false>(pv, bv, layer, R, pv.tables + (size_t)P.sid * pv.mbps, h, q, nullptr, nullptr,
                                        out, qmul, 0); // prompts never run on a ring
}

// ---------------------------------------------------------------------------------------------
// launchers

template <int CDT, bool ABF>
static hipError_t append_impl(const PoolView &pv, const BatchView &bv, int layer, const void *k,
                              const void *v, hipStream_t stream) {
    const int nseg = (bv.t + kBlock - 1) / kBlock + 1;
    hipLaunchKernelGGL((k_append<CDT, ABF>), dim3(bv.n * nseg), dim3(64 * pv.KVH), 0, stream, pv, bv, layer, k,
                       v, nseg);
    return hipGetLastError();
}

hipError_t launch_append(const PoolView &pv, const BatchView &bv, int layer, const void *k, const void *v,
                         hipStream_t stream) {
    if (bv.n == 0) return hipSuccess;
    switch (pv.cache_dt * 2 + pv.act_dt) {
    case DT_F32 * 2 + DT_F32: return append_impl<DT_F32, false>(pv, bv, layer, k, v, stream);
    case DT_BF16 * 2 + DT_BF16: return append_impl<DT_BF16, true>(pv, bv, layer, k, v, stream);
    case DT_I8 * 2 + DT_BF16: return append_impl<DT_I8, true>(pv, bv, layer, k, v, stream);
    case DT_I8 * 2 + DT_F32: return append_impl<DT_I8, false>(pv, bv, layer, k, v, stream);
    default: return hipErrorInvalidValue;
    }
}

// bf16 pools with 2 to 16 query heads per kv head decode a whole kv head per work group on MFMA
// (k_decode_gqa), unless a stream of the batch keeps a ring prefix (a second query position)
static bool decode_on_mfma(const PoolView &pv, bool prefix) {
    const int G = pv.H / pv.KVH;
    return pv.cache_dt == DT_BF16 && pv.act_dt == DT_BF16 && G >= 2 && G <= 16 && !prefix;
}

static hipError_t decode_gqa_impl(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                                  const void *v, void *out, float scale, bool fused, hipStream_t stream,
                                  const LaunchTiming &tm);

int decode_heads_per_group(const PoolView &pv, bool prefix) {
    // query heads of one kv head share a group's page reads: all of them on MFMA; else four when
    // four divide the group and no stream of the batch keeps a ring prefix (whose second query
    // would spill them), else two; int8 keeps one (its registers hold no second head at four
    // waves per SIMD)
    const int G = pv.H / pv.KVH;
    if (pv.cache_dt == DT_I8) return 1;
    if (decode_on_mfma(pv, prefix)) return G;
    return G % 4 == 0 && !prefix ? 4 : G % 2 == 0 ? 2 : 1;
}

template <int CDT, bool ABF, int GQ>
static hipError_t decode_impl(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                              const void *v, void *out, float scale, bool fused, hipStream_t stream,
                              const LaunchTiming &tm) {
    const float qmul = scale * 1.4426950408889634f;
    const dim3 grid(bv.n * pv.H / GQ);
    const int f = fused ? 1 : 0;
#define XNP_DECODE(S, PFX)                                                                                          \
    XNP_LAUNCH((k_decode<CDT, ABF, S, PFX, GQ>), grid, dim3(64 * S), stream, tm, pv, bv, layer, q, k, v, out, qmul, f)
    if (bv.prefix) {
        if constexpr (GQ >= 4) {
            return hipErrorInvalidValue; // four heads per group are built without a prefix
        } else {
            switch (bv.split) {
            case 1: XNP_DECODE(1, true); break;
            case 2: XNP_DECODE(2, true); break;
            case 4: XNP_DECODE(4, true); break;
            case 8: XNP_DECODE(8, true); break;
            default: return hipErrorInvalidValue;
            }
        }
    } else {
        switch (bv.split) {
        case 1: XNP_DECODE(1, false); break;
        case 2: XNP_DECODE(2, false); break;
        case 4: XNP_DECODE(4, false); break;
        case 8: XNP_DECODE(8, false); break;
        default: return hipErrorInvalidValue;
        }
    }
#undef XNP_DECODE
    return hipGetLastError();
}

hipError_t launch_decode(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                         const void *v, void *out, float scale, bool fused, hipStream_t stream,
                         const LaunchTiming &tm) {
    if (bv.n == 0) return hipSuccess;
    switch (pv.cache_dt * 2 + pv.act_dt) {
    case DT_F32 * 2 + DT_F32:
        switch (decode_heads_per_group(pv, bv.prefix != 0)) {
        case 4: return decode_impl<DT_F32, false, 4>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        case 2: return decode_impl<DT_F32, false, 2>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        default: return decode_impl<DT_F32, false, 1>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        }
    case DT_BF16 * 2 + DT_BF16:
        if (decode_on_mfma(pv, bv.prefix != 0))
            return decode_gqa_impl(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        switch (decode_heads_per_group(pv, bv.prefix != 0)) {
        case 4: return decode_impl<DT_BF16, true, 4>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        case 2: return decode_impl<DT_BF16, true, 2>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        default: return decode_impl<DT_BF16, true, 1>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        }
    case DT_I8 * 2 + DT_BF16: return decode_impl<DT_I8, true, 1>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
    case DT_I8 * 2 + DT_F32: return decode_impl<DT_I8, false, 1>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
    default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------------------------
// eviction on a shifting ring: rotate one kept key row by -count in place (transformer.rs:905-926)

template <int CDT, bool ABF>
__global__ void k_evict_rotate(PoolView pv, const EvictRow *rows, const float2 *cs_row) {
    const EvictRow R = rows[blockIdx.x / pv.L];
    const int layer = blockIdx.x % pv.L;
    const int j = threadIdx.x >> 5, pr = threadIdx.x & 31; // kv head, dim pair
    const int page = pv.tables[(size_t)R.sid * pv.mbps + (R.slot >> 4)];
    if (page < 0 || page >= pv.NB) return;
    const size_t e = tile_index(pv, layer, 0, page, j) * (kBlock * kHeadDim) + (R.slot & 15) * kHeadDim + 2 * pr;
    float2 x;
    if constexpr (CDT == DT_F32) {
        x = *(const float2 *)((const float *)pv.pages + e);
    } else {
        uint32_t w = *(const uint32_t *)((const uint16_t *)pv.pages + e);
        x = make_float2(bf16_value(w & 0xffffu), bf16_value(w >> 16));
    }
    const float2 cs = cs_row[pr];
    float a = x.x * cs.x, b = x.y * cs.y, ee = x.x * cs.y, f = x.y * cs.x;
    x.x = round_act<ABF>(a - b);
    x.y = round_act<ABF>(ee + f);
    if constexpr (CDT == DT_F32)
        *(float2 *)((float *)pv.pages + e) = x;
    else
        *(uint32_t *)((uint16_t *)pv.pages + e) = bf16_bits(x.x) | (bf16_bits(x.y) << 16);
}

hipError_t launch_evict_rotate(const PoolView &pv, const EvictRow *rows, int n, const float *cs,
                               const float *, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const dim3 grid(n * pv.L), block(32 * pv.KVH);
    const float2 *csr = (const float2 *)cs;
    switch (pv.cache_dt * 2 + pv.act_dt) {
    case DT_F32 * 2 + DT_F32: hipLaunchKernelGGL((k_evict_rotate<DT_F32, false>), grid, block, 0, stream, pv, rows, csr); break;
    case DT_BF16 * 2 + DT_BF16: hipLaunchKernelGGL((k_evict_rotate<DT_BF16, true>), grid, block, 0, stream, pv, rows, csr); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// page copy (fork of a partial last page, unsharing before a ring): every layer, K and V, scales

__global__ void k_copy_page(PoolView pv, int src, int dst, int tile_u4) {
    const int layer = blockIdx.x >> 1, kv = blockIdx.x & 1;
    const uint4 *s = (const uint4 *)pv.pages + tile_index(pv, layer, kv, src, 0) * tile_u4;
    uint4 *d = (uint4 *)pv.pages + tile_index(pv, layer, kv, dst, 0) * tile_u4;
    const int n = tile_u4 * pv.KVH;
    for (int i = threadIdx.x; i < n; i += blockDim.x) d[i] = s[i];
    if (pv.scales && threadIdx.x < pv.KVH)
        pv.scales[tile_index(pv, layer, kv, dst, threadIdx.x)] = pv.scales[tile_index(pv, layer, kv, src, threadIdx.x)];
}

hipError_t launch_copy_page(const PoolView &pv, int src_page, int dst_page, hipStream_t stream) {
    const int es = pv.cache_dt == DT_F32 ? 4 : pv.cache_dt == DT_BF16 ? 2 : 1;
    const int tile_u4 = kBlock * kHeadDim * es / 16;
    hipLaunchKernelGGL(k_copy_page, dim3(pv.L * 2), dim3(256), 0, stream, pv, src_page, dst_page, tile_u4);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// raw row I/O: rows [n][H][D] in the cache dtype <-> the stream's pages; int8 scales per page

__global__ void k_rows_io(PoolView pv, int sid, int layer, int kv, int slot0, void *rows, float *scales,
                          int write, int row_u4) {
    const int s = blockIdx.x;
    const int slot = slot0 + s;
    const int page = pv.tables[(size_t)sid * pv.mbps + (slot >> 4)];
    if (page < 0 || page >= pv.NB) return;
    const int per_head = row_u4 / pv.KVH;
    for (int i = threadIdx.x; i < row_u4; i += blockDim.x) {
        const int h = i / per_head, w = i % per_head;
        uint4 *pg = (uint4 *)pv.pages + tile_index(pv, layer, kv, page, h) * (kBlock * per_head) + (slot & 15) * per_head + w;
        uint4 *rw = (uint4 *)rows + (size_t)s * row_u4 + i;
        if (write)
            *pg = *rw;
        else
            *rw = *pg;
    }
    if (scales && ((slot & 15) == 0 || s == 0) && threadIdx.x < pv.KVH) {
        const int bi = (slot >> 4) - (slot0 >> 4);
        float *ps = pv.scales + tile_index(pv, layer, kv, page, threadIdx.x);
        float *us = scales + (size_t)bi * pv.KVH + threadIdx.x;
        if (write)
            *ps = *us;
        else
            *us = *ps;
    }
}

hipError_t launch_rows_io(const PoolView &pv, int sid, int layer, int kv, int slot0, int n, void *rows,
                          float *scales, bool write, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int es = pv.cache_dt == DT_F32 ? 4 : pv.cache_dt == DT_BF16 ? 2 : 1;
    const int row_u4 = pv.KVH * kHeadDim * es / 16;
    hipLaunchKernelGGL(k_rows_io, dim3(n), dim3(256), 0, stream, pv, sid, layer, kv, slot0, rows,
                       pv.cache_dt == DT_I8 ? scales : nullptr, write ? 1 : 0, row_u4);
    return hipGetLastError();
}

// A voice stored as the KV cache (voice_from_kv_cache, ptts-wasm/src/lib.rs:291-325): rows
// [0, n) of one layer from an f32 [2][n][H][D] tensor (keys, already rotated, then values),
// converted to the cache dtype: f32 as is, bf16 rounded to nearest even, int8 with one scale per
// (page, head), amax / 127 over the rows the page receives, and codes rint(x / s).  One wave per
// (page, head, keys or values); lane d holds dimension d of each of the page's 16 rows, so every
// row is one coalesced 256 B read.  Rows past n in the last page are left as they are.
template <int CDT>
__global__ __launch_bounds__(64) void k_load_kv(PoolView pv, int sid, int layer, const float *kv, int n) {
    const int b = blockIdx.x, j = blockIdx.y, which = blockIdx.z, lane = threadIdx.x;
    const int h = j * (pv.H / pv.KVH); // the voice repeats kv head j over its group's query heads
    const int page = pv.tables[(size_t)sid * pv.mbps + b];
    if (page < 0 || page >= pv.NB) return;
    const int rows = min(kBlock, n - b * kBlock);
    float x[kBlock];
#pragma unroll
    for (int r = 0; r < kBlock; ++r) { // all 16 loads in flight; rows past n re-read the last one
        const int slot = b * kBlock + min(r, rows - 1);
        x[r] = kv[(((size_t)which * n + slot) * pv.H + h) * kHeadDim + lane];
    }
    const size_t tile = tile_index(pv, layer, which, page, j);
    if constexpr (CDT == DT_F32) {
        float *pg = (float *)pv.pages + tile * (kBlock * kHeadDim);
#pragma unroll
        for (int r = 0; r < kBlock; ++r)
            if (r < rows) pg[r * kHeadDim + lane] = x[r];
    } else if constexpr (CDT == DT_BF16) {
        uint16_t *pg = (uint16_t *)pv.pages + tile * (kBlock * kHeadDim);
#pragma unroll
        for (int r = 0; r < kBlock; ++r)
            if (r < rows) pg[r * kHeadDim + lane] = (uint16_t)bf16_bits(x[r]);
    } else {
        float amax = 0.f;
#pragma unroll
        for (int r = 0; r < kBlock; ++r)
            if (r < rows) amax = fmaxf(amax, fabsf(x[r]));
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
        const float sc = amax / 127.0f;
        int8_t *pg = (int8_t *)pv.pages + tile * (kBlock * kHeadDim);
#pragma unroll
        for (int r = 0; r < kBlock; ++r)
            if (r < rows) pg[r * kHeadDim + lane] = (int8_t)quant(x[r], sc);
        if (lane == 0) pv.scales[tile] = sc;
    }
}

hipError_t launch_load_kv(const PoolView &pv, int sid, int layer, const float *kv, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const dim3 grid((n + kBlock - 1) / kBlock, pv.KVH, 2);
    switch (pv.cache_dt) {
    case DT_F32: hipLaunchKernelGGL(k_load_kv<DT_F32>, grid, dim3(64), 0, stream, pv, sid, layer, kv, n); break;
    case DT_BF16: hipLaunchKernelGGL(k_load_kv<DT_BF16>, grid, dim3(64), 0, stream, pv, sid, layer, kv, n); break;
    case DT_I8: hipLaunchKernelGGL(k_load_kv<DT_I8>, grid, dim3(64), 0, stream, pv, sid, layer, kv, n); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// prompt prefill on MFMA (bf16 cache and activations), transformer.rs:231-248 batched, with the
// append of the prompt's K/V rows (complete_kv, transformer.rs:84-91) fused in.
//
// One work group of 8 waves per (stream, head).  Query rows are taken in rounds of 256: 16 tiles
// of 16 rows, wave w owning tiles w and 15 - w of the round, so that every wave sees about the
// same number of causal keys.  Keys are staged through LDS in chunks of 64 (four pages), K and
// V both as [key][dim], double-buffered, with the next chunk's loads in flight while one is
// attended over.  Keys before the prompt come from the pages; the prompt's own keys come
// from the k/v inputs, rotated at their position and rounded to bf16, and are written into
// their pages during the last round, so that each is written exactly once and never read back
// from HBM.
//
// Both contractions are computed transposed so that P never leaves registers:
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16, A = K rows from LDS (lane: key lane%16, 8 dims),
//                 B = the wave's rotated query rows (registers; lane: query lane%16, 8 dims);
//                 the result holds, per lane, query row lane%16 against keys 4(lane/16) .. +3;
//   softmax       online per query row; its max and sum reduce over the 4 lanes of a row;
//   O^T += V^T P^T  B = P^T straight from the S^T registers (lane: query lane%16, 8 keys),
//                 A = V^T by transposed LDS reads of the same 8 keys (ds_read_b64_tr_b16).
// A and B always hold the same key (or dim) in the same (lane / 16, element) slot, so each
// contraction is right whatever order the instruction walks k in.

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4 &u) {
    bf16x8_t r;
    __builtin_memcpy(&r, &u, 16);
    return r;
}

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;

// ds_read_b64_tr_b16 (gfx950).  Within each group of 16 lanes, lane j supplies the address of
// four consecutive b16 values D[j][0..3], and lane i receives D[4 s + i / 4][i % 4] as element
// s.  Pointing lane j at row r0 + j / 4, columns c0 + 4 (j % 4) of a row-major b16 matrix thus
// hands lane i column c0 + i of rows r0 .. r0 + 3: a transposed read.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t *p) {
    const v4s_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(__attribute__((address_space(3))) uint16_t *)p);
    uint2 u;
    __builtin_memcpy(&u, &r, 8);
    return u;
}

constexpr int kPfKeys = 64;      // keys per chunk (four pages)
constexpr int kPfLd = 72;        // LDS row length in bf16: 64 + 8 of padding, rows 16-byte aligned
constexpr int kPfWaves = 8;      // waves per work group
constexpr int kPfRound = 256;    // query rows per round: 8 waves x 2 tiles x 16 rows
constexpr int kPfMaxPages = 512; // page ids a work group keeps in LDS
static_assert(kPfMaxPages >= kLaneBlocks * 8, "every page of a stream fits (a pool refuses more than 60 x 8)");
static_assert(64 * kPfWaves == kPfKeys * 8, "one thread stages 16 bytes of one key per chunk");

__global__ __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(4))) void k_prefill_mfma(
    PoolView pv, BatchView bv, int layer, const void *q, const void *knew, const void *vnew, void *out, float qmul,
    int fused) {
    __shared__ __attribute__((aligned(16))) uint16_t ks[2 * kPfKeys][kPfLd]; // K of two chunks, [key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t vs[2 * kPfKeys][kPfLd]; // V of two chunks, [key][dim]
    __shared__ int32_t spages[kPfMaxPages];
    const int t = bv.t;
    const int h = blockIdx.x % pv.H, b = blockIdx.x / pv.H;
    const StreamPlan P = bv.plans[b];
    const int32_t *tab = pv.tables + (size_t)P.sid * pv.mbps;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
    const int c0 = P.write_slot; // slot (= position) of prompt row 0
    const int kvh = h / (pv.H / pv.KVH);
    const size_t page_elems = (size_t)pv.KVH * kBlock * kHeadDim;
    uint16_t *kpages = (uint16_t *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim);
    uint16_t *vpages = (uint16_t *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim);
    // the stream's page ids for every key any round sees, read once
    for (int i = tid; i < min((c0 + t + kBlock - 1) / kBlock, kPfMaxPages); i += 64 * kPfWaves) spages[i] = tab[i];
    // this thread's share of a chunk: 16 bytes (8 dims) of one key's K and V
    const int skey = tid >> 3, spart = tid & 7;

    const int nqt = (t + 15) / 16;
    for (int tq0 = 0; tq0 < nqt; tq0 += kPfRound / 16) {
        const int nq = min(kPfRound / 16, nqt - tq0);
        const bool last = tq0 + nq == nqt;
        // this wave's tiles: (w, nq-1-w) for w < nq/2; the middle one alone when nq is odd
        int tile[2] = {-1, -1};
        if (w < nq / 2) {
            tile[0] = tq0 + w;
            tile[1] = tq0 + nq - 1 - w;
        } else if (w == nq / 2 && (nq & 1)) {
            tile[0] = tq0 + w;
        }
        const int kend = c0 + min(t, 16 * (tq0 + nq)); // the round's rows see keys [0, kend)
        const int nch = (kend + kPfKeys - 1) / kPfKeys;

        // B operands of S^T: query row 16 tile + l16, dims 32 kc + 8 g .. +7, rotated at its
        // position and rounded to bf16 as the reference's bf16 q is.  Every load is issued
        // before any is used (rows past the prompt read row t - 1 and are zeroed after).
        bf16x8_t qb[2][2];
        float m[2], lsum[2]; // running max (scaled, log2 units) and this lane's share of the sum
        f32x4_t o[2][4];
        {
            uint4 qraw[2][2];
            float4 qcs[2][2][2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int qr = min(16 * max(tile[j], 0) + l16, t - 1);
                const uint16_t *qp = (const uint16_t *)q + (((size_t)P.out_row * t + qr) * pv.H + h) * kHeadDim;
                const float4 *cs = (const float4 *)(pv.rope + (size_t)(P.pos + qr) * (kHeadDim / 2));
#pragma unroll
                for (int kc = 0; kc < 2; ++kc) {
                    qraw[j][kc] = *(const uint4 *)(qp + 32 * kc + 8 * g);
                    qcs[j][kc][0] = cs[(32 * kc + 8 * g) / 4];
                    qcs[j][kc][1] = cs[(32 * kc + 8 * g) / 4 + 1];
                }
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                m[j] = -1e30f;
                lsum[j] = 0.f;
#pragma unroll
                for (int dg = 0; dg < 4; ++dg) o[j][dg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                const bool live = tile[j] >= 0 && 16 * tile[j] + l16 < t;
#pragma unroll
                for (int kc = 0; kc < 2; ++kc) {
                    const uint32_t *u = (const uint32_t *)&qraw[j][kc];
                    const float4 ca = qcs[j][kc][0], cb = qcs[j][kc][1];
                    const float cf[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w}; // cos, sin of 4 pairs
                    uint32_t o4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float x0 = bf16_value(u[i] & 0xffffu), x1 = bf16_value(u[i] >> 16);
                        const float c = cf[2 * i], s = cf[2 * i + 1];
                        const float a = x0 * c, bb = x1 * s, e = x0 * s, f = x1 * c;
                        o4[i] = live ? pack_bf16(a - bb, e + f) : 0u;
                    }
                    qb[j][kc] = as_bf16x8(make_uint4(o4[0], o4[1], o4[2], o4[3]));
                }
            }
        }
        __syncthreads(); // spages written

        // Loads run one chunk ahead: chunk c's registers are consumed (rotated, stored to LDS
        // buffer c & 1) at step c, which then issues chunk c + 1's loads into them.
        struct Stage {
            uint4 k, v, rope; // the key's K and V pieces, 4 (cos, sin) pairs as packed bf16
            int info;         // bit 0: a prompt key, bit 1: write it to its page; page id above
        };
        auto issue = [&](int c, Stage &st) {
            const int slot = c * kPfKeys + skey;
            const bool in = c < nch && slot < kend;
            const bool fresh = fused && slot >= c0; // a prompt key: from the inputs, rotated here
            const int page = in ? spages[min(slot >> 4, kPfMaxPages - 1)] : -1;
            const bool ok = page >= 0 && page < pv.NB;
            const size_t poff = (size_t)(ok ? page : 0) * page_elems + (slot & 15) * kHeadDim + 8 * spart;
            const int i = fresh ? min(slot - c0, t - 1) : 0;
            const size_t arow = (((size_t)P.out_row * t + i) * pv.KVH + kvh) * kHeadDim + 8 * spart;
            st.k = st.v = make_uint4(0, 0, 0, 0);
            if (in && fresh) {
                st.k = ld_stream((const uint16_t *)knew + arow);
                st.v = ld_stream((const uint16_t *)vnew + arow);
            } else if (in && ok) {
                st.k = ld_stream(kpages + poff);
                st.v = ld_stream(vpages + poff);
            }
            st.rope = *(const uint4 *)(pv.rope16 + (size_t)(P.key_pos + i) * (kHeadDim / 2) + 4 * spart);
            st.info = (in && fresh ? 1 : 0) | (in && fresh && ok && last ? 2 : 0) | ((ok ? page : 0) << 2);
        };
        auto step = [&](int c, Stage &st) {
            const int buf = c & 1, kbase = c * kPfKeys, lb = buf * kPfKeys;
            // rotate a prompt key at its position; store this thread's piece of the chunk
            {
                uint4 kk = st.k;
                if (st.info & 1) {
                    const uint32_t *r = (const uint32_t *)&st.rope;
                    const uint32_t *u = (const uint32_t *)&st.k;
                    uint32_t o4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x0 = bf16_value(u[e] & 0xffffu), x1 = bf16_value(u[e] >> 16);
                        const float cc = bf16_value(r[e] & 0xffffu), sn = bf16_value(r[e] >> 16);
                        const float a = x0 * cc, bb = x1 * sn, ee = x0 * sn, f = x1 * cc;
                        o4[e] = pack_bf16(a - bb, ee + f);
                    }
                    kk = make_uint4(o4[0], o4[1], o4[2], o4[3]);
                }
                if (st.info & 2) { // complete_kv: the prompt's rows go into their pages once
                    const size_t poff = (size_t)(st.info >> 2) * page_elems + ((kbase + skey) & 15) * kHeadDim + 8 * spart;
                    *(uint4 *)(kpages + poff) = kk;
                    *(uint4 *)(vpages + poff) = st.v;
                }
                *(uint4 *)&ks[lb + skey][8 * spart] = kk;
                *(uint4 *)&vs[lb + skey][8 * spart] = st.v;
            }
            issue(c + 1, st);
            __syncthreads(); // chunk c is in LDS; every reader of chunk c - 2 (same buffer) is done
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int r0 = c0 + 16 * tile[j]; // slot of the tile's first row
                // skip a tile when every key of the chunk comes after all of its rows
                if (tile[j] < 0 || kbase > r0 + 15) continue;
                f32x4_t s[4];
#pragma unroll
                for (int kg = 0; kg < 4; ++kg) {
                    s[kg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kc = 0; kc < 2; ++kc) {
                        const bf16x8_t a = as_bf16x8(*(const uint4 *)&ks[lb + 16 * kg + l16][32 * kc + 8 * g]);
                        s[kg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[j][kc], s[kg], 0, 0, 0);
                    }
                }
                // lane: query slot r0 + l16 against key slots kbase + 16 kg + 4 g + r
                if (kbase + kPfKeys - 1 > r0) { // the chunk reaches past the tile's first row: mask
                    const int qs = r0 + l16;
#pragma unroll
                    for (int kg = 0; kg < 4; ++kg)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (kbase + 16 * kg + 4 * g + r > qs) s[kg][r] = -INFINITY;
                }
                float mx = fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3]));
#pragma unroll
                for (int kg = 1; kg < 4; ++kg)
                    mx = fmaxf(mx, fmaxf(fmaxf(s[kg][0], s[kg][1]), fmaxf(s[kg][2], s[kg][3])));
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                // lazy rescaling, as in decode: the row's sum and accumulators move to a new max only
                // when some row of the wave saw its max grow by more than 8 (log2 units); until then
                // exponents are taken against the older max and stay below 2^8
                const float mn = fmaxf(m[j], mx * qmul);
                if (__any(mn > m[j] + 8.f)) {
                    const float alpha = fast_exp2(m[j] - mn);
                    lsum[j] *= alpha;
#pragma unroll
                    for (int dg = 0; dg < 4; ++dg)
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[j][dg][r] *= alpha;
                    m[j] = mn;
                }
                const float mref = m[j];
                float psum = 0.f;
                uint32_t pk[4][2];
#pragma unroll
                for (int kg = 0; kg < 4; ++kg) {
                    float p[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        p[r] = fast_exp2(__builtin_fmaf(s[kg][r], qmul, -mref));
                        psum += p[r];
                    }
                    pk[kg][0] = pack_bf16(p[0], p[1]);
                    pk[kg][1] = pack_bf16(p[2], p[3]);
                }
                lsum[j] += psum;
#pragma unroll
                for (int kp = 0; kp < 2; ++kp) {
                    // k slots: keys 32 kp + 4 g .. +3 (elements 0-3) and 32 kp + 16 + 4 g .. +3 (4-7)
                    const bf16x8_t pb =
                        as_bf16x8(make_uint4(pk[2 * kp][0], pk[2 * kp][1], pk[2 * kp + 1][0], pk[2 * kp + 1][1]));
#pragma unroll
                    for (int dg = 0; dg < 4; ++dg) {
                        // V^T: lane gets dim 16 dg + l16 of the same eight keys, by two transposed reads
                        const uint16_t *vp = &vs[lb + 32 * kp + 4 * g + (l16 >> 2)][16 * dg + 4 * (l16 & 3)];
                        const uint2 lo = lds_read_tr16(vp), hi = lds_read_tr16(vp + 16 * kPfLd);
                        const bf16x8_t a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
                        o[j][dg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[j][dg], 0, 0, 0);
                    }
                }
            }
        };
        Stage st;
        issue(0, st);
        for (int c = 0; c < nch; ++c) step(c, st);
        __syncthreads(); // the next round's staging overwrites both buffers

        // out[row][h][16 dg + 4 g .. +3] = O / l, the row's sum reduced over its 4 lanes
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float l = lsum[j];
            l += __shfl_xor(l, 16);
            l += __shfl_xor(l, 32);
            const int qrow = 16 * tile[j] + l16;
            if (tile[j] < 0 || qrow >= t) continue;
            const float inv = 1.0f / l;
            uint16_t *orow = (uint16_t *)out + (((size_t)P.out_row * t + qrow) * pv.H + h) * kHeadDim;
#pragma unroll
            for (int dg = 0; dg < 4; ++dg)
                *(uint2 *)(orow + 16 * dg + 4 * g) = make_uint2(pack_bf16(o[j][dg][0] * inv, o[j][dg][1] * inv),
                                                                pack_bf16(o[j][dg][2] * inv, o[j][dg][3] * inv));
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Grouped-head decode on MFMA: bf16 pages and queries, 2 to 16 query heads per kv head, no ring
// prefix.  One work group per (stream, kv head), whose G query heads are the 16 columns of the
// MFMA tiles (columns past G hold zeros), so that each page is read once and its 16 keys meet all
// G heads in a few instructions.  The contractions are the prompt prefill's, transposed so that P
// never leaves registers:
//   S^T = K Q^T      v_mfma_f32_16x16x32_bf16, A = the page's K rows (lane: key l16, dims
//                    32 kc + 8 g .. +7) from a wave-private LDS tile that streamed whole-line loads
//                    fill, B = the rotated query rows; lane (l16, g) gets the scores of keys
//                    4 g .. 4 g + 3 for query head l16;
//   softmax          online per query column, its max and sum over the 4 lanes of the column;
//   O^T += V^T P^T   v_mfma_f32_16x16x16_bf16, B = P^T straight from the S^T registers, A = V^T by
//                    transposed reads (ds_read_b64_tr_b16) of the page's V, copied into a
//                    wave-private LDS tile.
// Pages, SPLIT waves per group, the fused append and the LDS merge are attend_core's.
typedef short s16x4_t __attribute__((ext_vector_type(4)));

template <int SPLIT>
__global__ __launch_bounds__(64 * SPLIT) __attribute__((amdgpu_waves_per_eu(4))) void k_decode_gqa(
    PoolView pv, BatchView bv, int layer, const void *q, const void *knew, const void *vnew, void *out, float qmul,
    int fused) {
    constexpr int DEPTH = 2; // pages in flight ahead of the one being reduced
    __shared__ __attribute__((aligned(16))) uint16_t vt[SPLIT][kBlock][kPfLd]; // each wave's V tile, [key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t kt[SPLIT][kBlock][kPfLd]; // each wave's K tile, [key][dim]
    __shared__ float part[SPLIT][16][kPartStride];
    const int G = pv.H / pv.KVH;
    // XCD runs as in k_decode: in runs of 8 KVH groups, XCD x takes the kv heads of stream x of the run
    const int b = blockIdx.x, full = bv.n / 8 * 8;
    const int sidx = b < full * pv.KVH ? b / (8 * pv.KVH) * 8 + b % 8 : full + (b - full * pv.KVH) / pv.KVH;
    const int kvh = b < full * pv.KVH ? b % (8 * pv.KVH) / 8 : (b - full * pv.KVH) % pv.KVH;
    const char *rec = bv.recs + (size_t)sidx * bv.rec_stride;
    const StreamRec R = *(const StreamRec *)rec;
    const int32_t *rec_pages = (const int32_t *)(rec + sizeof(StreamRec));
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, l16 = lane & 15;
    const int nb = R.nblk > w ? (R.nblk - w + SPLIT - 1) / SPLIT : 0; // this wave's pages

    // per-page metadata, lane j holding page w + j * SPLIT (as attend_core)
    int my_page = 0;
    uint32_t my_seen = 0;
    const int pg_raw = w + lane * SPLIT < pv.mbps ? rec_pages[w + lane * SPLIT] : -1;
    if (lane < nb) {
        const int base = (w + lane * SPLIT) * kBlock;
        uint32_t seen = 0xffffu;
        if (R.mask_off >= 0) seen = (bv.masks[R.mask_off + (base >> 5)] >> (base & 16)) & 0xffffu;
        const int nvalid = R.span - base;
        if (nvalid < kBlock) seen &= (1u << max(nvalid, 0)) - 1u;
        const bool ok = pg_raw >= 0 && pg_raw < pv.NB;
        my_page = ok ? pg_raw : 0;
        my_seen = ok ? seen : 0;
    }

    // B operands of S^T: query head kvh G + l16, dims 32 kc + 8 g .. +7, rotated at R.pos and
    // rounded to bf16 (zeros past G)
    bf16x8_t qb[2];
    {
        const bool live = l16 < G;
        const int hq = kvh * G + min(l16, G - 1);
        const uint16_t *qp = (const uint16_t *)q + ((size_t)R.b * pv.H + hq) * kHeadDim;
        const float4 *cs = (const float4 *)(pv.rope + (size_t)R.pos * (kHeadDim / 2));
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            const uint4 raw = *(const uint4 *)(qp + 32 * kc + 8 * g);
            const float4 ca = cs[(32 * kc + 8 * g) / 4], cb = cs[(32 * kc + 8 * g) / 4 + 1];
            const float cf[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w}; // cos, sin of 4 pairs
            const uint32_t *u = (const uint32_t *)&raw;
            uint32_t o4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x0 = bf16_value(u[i] & 0xffffu), x1 = bf16_value(u[i] >> 16);
                const float c = cf[2 * i], s = cf[2 * i + 1];
                const float a = x0 * c, bb = x1 * s, e = x0 * s, f = x1 * c;
                o4[i] = live ? pack_bf16(a - bb, e + f) : 0u;
            }
            qb[kc] = as_bf16x8(make_uint4(o4[0], o4[1], o4[2], o4[3]));
        }
    }

    const uint16_t *kbase = (const uint16_t *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim);
    const uint16_t *vbase = (const uint16_t *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim);
    const size_t page_elems = (size_t)pv.KVH * kBlock * kHeadDim;

    float m = -1e30f, lsum = 0.f; // running max (scaled, log2 units) and this lane's share of the sum
    f32x4_t o[4];                 // O^T: dims 16 dg + 4 g + r, query head l16
#pragma unroll
    for (int dg = 0; dg < 4; ++dg) o[dg] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // a page's K and V tiles, each in two streamed 1 KB loads (keys lane / 8 and 8 + lane / 8,
    // dims 8 (lane % 8) ..): every load covers whole 128-byte lines.  Loaded straight in the MFMA's
    // A layout, each load would take half of every line, and a streamed line is gone before the
    // other half is read (33 -> 36.6 us at 1 kv head); K therefore goes through an LDS tile too.
    // Measured against plain loads in A layout: 1 kv head 33.4 -> 28.8 us, 2: 56.5 -> 50.5, 4:
    // 101.5 -> 89 us.
    auto load = [&](uint4 (&kr)[2], uint4 (&vr)[2], int j) {
        const size_t pe = (size_t)__builtin_amdgcn_readlane(my_page, j) * page_elems;
        kr[0] = ld_stream(kbase + pe + 8 * lane);
        kr[1] = ld_stream(kbase + pe + 512 + 8 * lane);
        vr[0] = ld_stream(vbase + pe + 8 * lane);
        vr[1] = ld_stream(vbase + pe + 512 + 8 * lane);
    };
    auto process = [&](const uint4 (&kr)[2], const uint4 (&vr)[2], int j) {
        const uint32_t seen = __builtin_amdgcn_readlane(my_seen, j);
        f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
        // K through the wave's LDS tile into A layout (key l16, dims 32 kc + 8 g); a wave's LDS
        // accesses complete in order, so no barrier
        *(uint4 *)&kt[w][lane >> 3][8 * (lane & 7)] = kr[0];
        *(uint4 *)&kt[w][8 + (lane >> 3)][8 * (lane & 7)] = kr[1];
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(*(const uint4 *)&kt[w][l16][32 * kc + 8 * g]), qb[kc],
                                                       s, 0, 0, 0);
        // lane: query head l16 against keys 4 g + r of the page
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (!((seen >> (4 * g + r)) & 1u)) s[r] = -INFINITY;
        float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // lazy rescaling, as in attend_core
        const float mn = fmaxf(m, mx * qmul);
        if (__any(mn > m + 8.f)) {
            const float alpha = fast_exp2(m - mn);
            lsum *= alpha;
#pragma unroll
            for (int dg = 0; dg < 4; ++dg)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[dg][r] *= alpha;
            m = mn;
        }
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = fast_exp2(__builtin_fmaf(s[r], qmul, -m));
            lsum += p[r];
        }
        const s16x4_t pt = __builtin_bit_cast(s16x4_t, make_uint2(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3])));
        // the page's V into this wave's LDS tile (rows lane / 8 and 8 + lane / 8, dims 8 (lane % 8) ..);
        // an unseen row weighs 0 but its bytes may be anything, so it goes in as zeros (0 * NaN would
        // be NaN)
        const uint32_t keep0 = ((seen >> (lane >> 3)) & 1u) ? ~0u : 0u;
        const uint32_t keep1 = ((seen >> (8 + (lane >> 3))) & 1u) ? ~0u : 0u;
        *(uint4 *)&vt[w][lane >> 3][8 * (lane & 7)] =
            make_uint4(vr[0].x & keep0, vr[0].y & keep0, vr[0].z & keep0, vr[0].w & keep0);
        *(uint4 *)&vt[w][8 + (lane >> 3)][8 * (lane & 7)] =
            make_uint4(vr[1].x & keep1, vr[1].y & keep1, vr[1].z & keep1, vr[1].w & keep1);
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) {
            // V^T: lane gets dim 16 dg + l16 of keys 4 g .. 4 g + 3
            const uint2 a = lds_read_tr16(&vt[w][4 * g + (l16 >> 2)][16 * dg + 4 * (l16 & 3)]);
            o[dg] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), pt, o[dg], 0, 0, 0);
        }
    };

    uint4 kb[DEPTH + 1][2], vb[DEPTH + 1][2];
    // complete_kv: the wave that owns the write page appends the kv head's new row, as in attend_core
    const int wblk = R.write_slot >> 4, wj = wblk / SPLIT;
    const bool owner = fused && w == wblk % SPLIT;
    const bool early = !owner || wj >= DEPTH;
    if (early) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(kb[d], vb[d], d);
    }
    if (owner) {
        const int slot = R.write_slot;
        const size_t arow = (size_t)R.b * pv.KVH + kvh;
        const bool fresh = (R.flags & 1) ? (R.flags & 2) != 0 : ((slot & 15) == 0);
        append_row_wave<DT_BF16, true>(pv, layer, __builtin_amdgcn_readlane(my_page, wj), slot & 15, kvh, R.key_pos,
                                       (const char *)knew + arow * kHeadDim * 2, (const char *)vnew + arow * kHeadDim * 2,
                                       fresh);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    }
    if (!early) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(kb[d], vb[d], d);
    }
    for (int j = 0; j < nb; j += DEPTH + 1) {
#pragma unroll
        for (int u = 0; u <= DEPTH; ++u) {
            load(kb[(u + DEPTH) % (DEPTH + 1)], vb[(u + DEPTH) % (DEPTH + 1)], j + u + DEPTH);
            process(kb[u], vb[u], j + u);
        }
    }

    // the column's sum over its 4 lanes; the waves' shares through LDS; wave 0 writes the G heads
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
#pragma unroll
    for (int dg = 0; dg < 4; ++dg)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[w][l16][16 * dg + 4 * g + r] = o[dg][r];
    if (g == 0) {
        part[w][l16][64] = m;
        part[w][l16][65] = lsum;
    }
    __syncthreads();
    if (w != 0) return;
    for (int e = 0; e < G; ++e) {
        float M = -1e30f;
#pragma unroll
        for (int k = 0; k < SPLIT; ++k) M = fmaxf(M, part[k][e][64]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int k = 0; k < SPLIT; ++k) {
            const float a = fast_exp2(part[k][e][64] - M);
            L = __builtin_fmaf(part[k][e][65], a, L);
            A = __builtin_fmaf(part[k][e][lane], a, A);
        }
        ((uint16_t *)out)[((size_t)R.b * pv.H + kvh * G + e) * kHeadDim + lane] = (uint16_t)bf16_bits(A / L);
    }
}

static hipError_t decode_gqa_impl(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                                  const void *v, void *out, float scale, bool fused, hipStream_t stream,
                                  const LaunchTiming &tm) {
    const float qmul = scale * 1.4426950408889634f;
    const dim3 grid(bv.n * pv.KVH);
    const int f = fused ? 1 : 0;
    switch (bv.split) {
    case 1: XNP_LAUNCH((k_decode_gqa<1>), grid, dim3(64), stream, tm, pv, bv, layer, q, k, v, out, qmul, f); break;
    case 2: XNP_LAUNCH((k_decode_gqa<2>), grid, dim3(128), stream, tm, pv, bv, layer, q, k, v, out, qmul, f); break;
    case 4: XNP_LAUNCH((k_decode_gqa<4>), grid, dim3(256), stream, tm, pv, bv, layer, q, k, v, out, qmul, f); break;
    case 8: XNP_LAUNCH((k_decode_gqa<8>), grid, dim3(512), stream, tm, pv, bv, layer, q, k, v, out, qmul, f); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int CDT, bool ABF>
static hipError_t prefill_rows_impl(const PoolView &pv, const BatchView &bv, int layer, const void *q, void *out,
                                    float scale, hipStream_t stream, const LaunchTiming &tm) {
    const float qmul = scale * 1.4426950408889634f;
    const dim3 grid(bv.n * bv.t * pv.H);
    switch (bv.split) {
    case 1: XNP_LAUNCH((k_prefill_rows<CDT, ABF, 1>), grid, dim3(64), stream, tm, pv, bv, layer, q, out, qmul); break;
    case 2: XNP_LAUNCH((k_prefill_rows<CDT, ABF, 2>), grid, dim3(128), stream, tm, pv, bv, layer, q, out, qmul); break;
    case 4: XNP_LAUNCH((k_prefill_rows<CDT, ABF, 4>), grid, dim3(256), stream, tm, pv, bv, layer, q, out, qmul); break;
    case 8: XNP_LAUNCH((k_prefill_rows<CDT, ABF, 8>), grid, dim3(512), stream, tm, pv, bv, layer, q, out, qmul); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool prefill_fuses_append(const PoolView &pv) { return pv.cache_dt == DT_BF16 && pv.act_dt == DT_BF16; }

hipError_t launch_prefill(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                          const void *v, void *out, float scale, bool fused, hipStream_t stream,
                          const LaunchTiming &tm) {
    if (bv.n == 0) return hipSuccess;
    if (fused && !prefill_fuses_append(pv)) return hipErrorInvalidValue;
    switch (pv.cache_dt * 2 + pv.act_dt) {
    case DT_F32 * 2 + DT_F32: return prefill_rows_impl<DT_F32, false>(pv, bv, layer, q, out, scale, stream, tm);
    case DT_BF16 * 2 + DT_BF16:
        XNP_LAUNCH(k_prefill_mfma, dim3(bv.n * pv.H), dim3(64 * kPfWaves), stream, tm, pv, bv, layer, q, k, v, out,
                   scale * 1.4426950408889634f, fused ? 1 : 0);
        return hipGetLastError();
    case DT_I8 * 2 + DT_BF16: return prefill_rows_impl<DT_I8, true>(pv, bv, layer, q, out, scale, stream, tm);
    case DT_I8 * 2 + DT_F32: return prefill_rows_impl<DT_I8, false>(pv, bv, layer, q, out, scale, stream, tm);
    default: return hipErrorInvalidValue;
    }
}

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
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) sum += __shfl_xor(sum, o);
    const float mean = sum / (float)dim;
    float sq = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = v[c][i] - mean;
            sq = __builtin_fmaf(d, d, sq);
        }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) sq += __shfl_xor(sq, o);
    const float rstd = 1.0f / __builtin_sqrtf(sq / (float)dim + eps);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int e0 = (c * 64 + lane) * 8;
        float ww[8], bb[8];
        if constexpr ((MODE & kLnAffine) != 0) {
            const float4 w0 = *(const float4 *)(w + e0), w1 = *(const float4 *)(w + e0 + 4);
            const float4 b0 = *(const float4 *)(b + e0), b1 = *(const float4 *)(b + e0 + 4);
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
        *(uint4 *)(out + (size_t)row * dim + e0) = make_uint4(o4[0], o4[1], o4[2], o4[3]);
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
// narrow projection (N = 512 at 2048 rows gives 256 groups of 64 rows: one wave per SIMD).
//
// KS: groups of KS x 256 threads.  Half h (256 threads, the tile's 4 waves) takes K chunks h, h + KS,
// .. into its own LDS buffers; at the end half 1 hands its sums to half 0 through LDS, which adds
// them and runs the epilogue.  For long K (linear2: K = 2048), where a group's chunks run one
// after another.
template <int EPI, bool AF32, int MI, int KS>
__global__ __launch_bounds__(256 * KS) void k_gemm_q8(const uint16_t *A, int M, int K, const int8_t *W, const float *s,
                                                      int N, GemmOut go) {
    constexpr int BM = 32 * MI;
    static_assert(KS == 1 || KS == 2, "one or two halves");
    __shared__ __attribute__((aligned(16))) uint16_t As[KS][2][BM][kGmLd];
    __shared__ __attribute__((aligned(16))) uint16_t Ws[KS][2][kGmT][kGmLd];
    const int ntn = (N + kGmT - 1) / kGmT;
    const int m0 = (blockIdx.x / ntn) * BM, n0 = (blockIdx.x % ntn) * kGmT;
    const int tid = threadIdx.x & 255, h = KS > 1 ? (int)(threadIdx.x >> 8) : 0;
    const int w = tid >> 6, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
    const int wm = w & 1, wn = w >> 1;

    // staging: A rows a_r (and a_r + 32 when MI = 2), 8 values at k 8 a_k; W row w_r, 16 int8 at
    // k 16 w_k.
    // kGmPD chunks of loads are in flight: set c % kGmPD holds chunk c from its load until it is
    // written to LDS.  The words stay as loaded until then -- zeroing past K, rounding f32 A rows
    // and widening W happen at the LDS store, since any use at the load would make the wave wait
    // for it there.
    const int a_r = tid >> 3, a_k = tid & 7, w_r = tid >> 2, w_k = tid & 3;
    const int ar0 = min(m0 + a_r, M - 1), ar1 = min(m0 + a_r + 32 * (MI - 1), M - 1), wr = min(n0 + w_r, N - 1);
    constexpr int AW = AF32 ? 2 : 1; // uint4 per 8 A values
    uint4 ra0[kGmPD][AW], ra1[kGmPD][AW], rw[kGmPD];
    auto load = [&](int kc, int set) {
        // past K (K % 16 == 0, so no 16-byte load straddles it): an in-bounds address, zeroed at
        // the store
        const int k0 = kc * kGmK;
        const int ka = k0 + 8 * a_k < K ? k0 + 8 * a_k : 0, kw = k0 + 16 * w_k < K ? k0 + 16 * w_k : 0;
        if constexpr (AF32) {
            const float *af = (const float *)A;
            ra0[set][0] = *(const uint4 *)(af + (size_t)ar0 * K + ka);
            ra0[set][AW - 1] = *(const uint4 *)(af + (size_t)ar0 * K + ka + 4);
            if constexpr (MI == 2) {
                ra1[set][0] = *(const uint4 *)(af + (size_t)ar1 * K + ka);
                ra1[set][AW - 1] = *(const uint4 *)(af + (size_t)ar1 * K + ka + 4);
            }
        } else {
            ra0[set][0] = *(const uint4 *)(A + (size_t)ar0 * K + ka);
            if constexpr (MI == 2) ra1[set][0] = *(const uint4 *)(A + (size_t)ar1 * K + ka);
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
        uint4 a0 = bf16_row(ra0[set]), a1 = a0, wq = rw[set];
        if constexpr (MI == 2) a1 = bf16_row(ra1[set]);
        if ((kc + 1) * kGmK > K) { // the chunk reaches past K (uniform over the group)
            const int k0 = kc * kGmK;
            const uint32_t ma = k0 + 8 * a_k < K ? ~0u : 0u, mw = k0 + 16 * w_k < K ? ~0u : 0u;
            a0 = masked(a0, ma);
            a1 = masked(a1, ma);
            wq = masked(wq, mw);
        }
        *(uint4 *)&As[h][buf][a_r][8 * a_k] = a0;
        if constexpr (MI == 2) *(uint4 *)&As[h][buf][a_r + 32][8 * a_k] = a1;
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

    f32x4_t acc[MI][2];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // this half's chunks: c = 0 .. nkh - 1 is chunk h + KS c.  Both halves run nkmax rounds, one
    // barrier each, whatever their own count (the launcher takes KS = 2 only when nk >= 2 KS).
    const int nk = (K + kGmK - 1) / kGmK;
    const int nkh = (nk - h + KS - 1) / KS, nkmax = (nk + KS - 1) / KS;
    load(h, 0);
#pragma unroll
    for (int c = 1; c < kGmPD; ++c)
        if (c < nkh) load(h + KS * c, c);
    store(0, 0, h);
    __syncthreads();
    for (int cb = 0; cb < nkmax; cb += kGmPD) {
#pragma unroll
        for (int u = 0; u < kGmPD; ++u) { // set indices stay constants
            const int c = cb + u;
            if (c >= nkmax) break; // uniform over the group
            const int buf = c & 1;
            if (c + kGmPD < nkh) load(h + KS * (c + kGmPD), u); // set u held chunk c, already in LDS
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
            if (c + 1 < nkh) store(buf ^ 1, (u + 1) % kGmPD, h + KS * (c + 1));
            __syncthreads();
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
        if (h == 1) return;
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[mi][ni][r] += red[((mi * 2 + ni) * 4 + r) * 256 + tid];
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
                } else { // kStoreF32
                    ((float *)go.out[0])[(size_t)m * go.ld[0] + n] = y;
                }
            }
    }
}

template <int MI, int KS>
static hipError_t gemm_q8_mi(const void *A, int M, int K, const int8_t *W, const float *s, int N, int epi,
                             const GemmOut &go, hipStream_t stream) {
    const dim3 grid(((N + kGmT - 1) / kGmT) * ((M + 32 * MI - 1) / (32 * MI))), block(256 * KS);
    const uint16_t *a = (const uint16_t *)A;
#define XNP_GEMM(E) hipLaunchKernelGGL((k_gemm_q8<E, false, MI, KS>), grid, block, 0, stream, a, M, K, W, s, N, go)
    if (go.a_f32) {
        if (epi != kStore) return hipErrorInvalidValue;
        hipLaunchKernelGGL((k_gemm_q8<kStore, true, MI, KS>), grid, block, 0, stream, a, M, K, W, s, N, go);
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
    default: return hipErrorInvalidValue;
    }
#undef XNP_GEMM
    return hipGetLastError();
}

hipError_t launch_gemm_q8(const void *A, int M, int K, const int8_t *W, const float *s, int N, int epi,
                          const GemmOut &go, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    if (N <= 0 || K <= 0 || K % 16) return hipErrorInvalidValue;
    // 32-row tiles when 64-row ones would leave the chip's 1024 SIMDs under two waves each
    const int64_t groups64 = (int64_t)((N + kGmT - 1) / kGmT) * ((M + kGmT - 1) / kGmT);
    // two halves per group on alternate K chunks when K is long (32 chunks and more)
    if (K >= 32 * kGmK)
        return groups64 < 512 ? gemm_q8_mi<1, 2>(A, M, K, W, s, N, epi, go, stream)
                              : gemm_q8_mi<2, 2>(A, M, K, W, s, N, epi, go, stream);
    return groups64 < 512 ? gemm_q8_mi<1, 1>(A, M, K, W, s, N, epi, go, stream)
                          : gemm_q8_mi<2, 1>(A, M, K, W, s, N, epi, go, stream);
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
    // every load is issued unconditionally (the index clamped, the value then zeroed), so that all
    // of them are in flight together rather than each behind a branch and a wait
    float w[KC], nw[KC], nb[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const int k = c * 64 + lane, kk = min(k, K - 1);
        const float wv = W[(size_t)n * K + kk];
        w[c] = k < K ? wv : 0.f;
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
        if constexpr ((NORM & kNormLn) != 0) {
            // mean, then the centred sum of squares: the two passes of a textbook LayerNorm
            float sum = 0.f;
#pragma unroll
            for (int c = 0; c < KC; ++c) sum += c * 64 + lane < K ? xv[c] : 0.f;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
            const float mean = sum / (float)K;
            float sq = 0.f;
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                const float d = c * 64 + lane < K ? xv[c] - mean : 0.f;
                sq = __builtin_fmaf(d, d, sq);
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o);
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
        for (int c = 0; c < KC; ++c) acc = __builtin_fmaf(w[c], xv[c], acc); // w is 0 past K
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
        if (lane != 0) continue;
        const float y = acc + b;
        int seg = 0;
        if (lo.nseg > 1 && n >= lo.col0[1]) seg = (lo.nseg > 2 && n >= lo.col0[2]) ? 2 : 1;
        float *o = lo.out[seg] + (size_t)m * lo.ld[seg] + (n - lo.col0[seg]);
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
            const float z = y + lo.aux[n];
            *o = z / (1.0f + expf(-z));
        } else if constexpr (EPI == kLinResidual) {
            *o = *o + y;
        } else if constexpr (EPI == kLinGated) {
            *o = *o + lo.aux[(size_t)m * lo.ld_aux + n] * y;
        } else { // kLinAxpy
            *o = lo.aux[(size_t)m * lo.ld_aux + n] + y * lo.alpha;
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
