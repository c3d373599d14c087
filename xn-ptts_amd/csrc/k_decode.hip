// Decode attention on the VALU: fused append + RoPE + single-query attention over a stream's pages
// (k_decode), the prompt-row variant for f32 and int8 pools (k_prefill_rows), and the decode and
// prefill dispatch.
#include "kernels_common.h"

#include <type_traits>

namespace xnp {

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
    int my_page = 0, my_ok = 0;
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
        my_ok = ok ? 1 : 0;
        my_seen = seen;
    }

    const uint4 *kbase = (const uint4 *)((const char *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim * esize<CDT>()));
    const uint4 *vbase = (const uint4 *)((const char *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim * esize<CDT>()));
    const size_t page_u4 = (size_t)pv.KVH * (kBlock * kHeadDim * esize<CDT>() / 16);
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

    // The first DEPTH pages' loads go out before the queries are rotated, so that a group's first
    // K/V bytes are one round trip behind its page ids, not two (the rotation waits for the query
    // and RoPE rows).  The wave that owns the write page loads them after its append instead when
    // the write page is among them; otherwise before it, so the append's round trips overlap them.
    const int wblk = R.write_slot >> 4, wj = wblk / SPLIT;
    const bool owner = fused && w == wblk % SPLIT && __builtin_amdgcn_readlane(my_ok, wj) != 0;
    const bool early = !owner || wj >= DEPTH;
    if (early) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(kb[d], vb[d], d);
    }
    // int8: the pages' scales, after the first pages' loads (a wait for the page ids before those
    // would otherwise wait for these too)
    if constexpr (CDT == DT_I8) {
        if (lane < nb) {
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
    float qpow[GQ], ppow[GQ]; // H16: the power of two each query was scaled down by (f16_fit_exponent)
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
        qpow[e] = ppow[e] = 1.f;
        if constexpr (H16) {
            const int xq = f16_fit_exponent<DPL, 1, 2>(qw[e]); // the row's 4 lanes: c = lane % 4
            const int xp = two_q ? f16_fit_exponent<DPL, 1, 2>(qp[e]) : 0;
            qpow[e] = pow2i(xq);
            ppow[e] = pow2i(xp);
#pragma unroll
            for (int i = 0; i < DPL; ++i) qw[e][i] *= pow2i(-xq);
            if (two_q) {
#pragma unroll
                for (int i = 0; i < DPL; ++i) qp[e][i] *= pow2i(-xp);
            }
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
                dw[e] = group_sum<LPR>(dw[e]);
                if constexpr (CDT == DT_I8) dw[e] *= sk;
                if constexpr (H16) dw[e] *= pre ? ppow[e] : qpow[e];
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

    // complete_kv: the wave that owns the write page (above) appends this head's new row, then
    // reads it back with the rest of its pages (its own lanes' stores; no other wave touches the
    // page).  A workgroup-scope fence orders the stores before the later loads on the same CU;
    // nothing waits for the stores to reach memory.  An invalid write page id (never handed out by
    // the host, which checks it) appends nothing, as k_append skips it: the row would otherwise
    // land in page 0, another stream's tile.
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
        auto merge = [&](auto O) {
            constexpr int o = decltype(O)::value;
            if constexpr (o >= LPR) {
                const float mo = xor_lane<o>(m[e]), lo = xor_lane<o>(l[e]);
                const float mn = fmaxf(m[e], mo);
                const float a = fast_exp2(m[e] - mn), bb = fast_exp2(mo - mn);
                l[e] = l[e] * a + lo * bb;
#pragma unroll
                for (int i = 0; i < DPL; ++i) {
                    const float ao = xor_lane<o>(acc[e][i]);
                    acc[e][i] = acc[e][i] * a + ao * bb;
                }
                m[e] = mn;
            }
        };
        merge(std::integral_constant<int, 4>{});
        merge(std::integral_constant<int, 8>{});
        merge(std::integral_constant<int, 16>{});
        merge(std::integral_constant<int, 32>{});
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
    StreamRec R = *(const StreamRec *)rec;
    if (bv.wrow >= 0) window_row(R, bv.wrow);
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

// The MFMA decode (k_decode_gqa): bf16 activations over bf16 or int8 pages with 2 to 16 query heads
// per kv head decode a whole kv head per work group, a ring prefix (a second query position)
// included.  One head per kv head stays on the VALU: on MFMA each lane would carry four scores of
// which one is live, and the int8 window measured 108.6 us there against 99.5 us (at 4 and 8 heads
// per kv head: 34 and 23.7 us against 70 and 68).
static bool decode_on_mfma(const PoolView &pv, bool prefix) {
    (void)prefix;
    const int G = pv.H / pv.KVH;
    if (pv.act_dt != DT_BF16 || G < 2 || G > 16) return false;
    return pv.cache_dt == DT_BF16 || pv.cache_dt == DT_I8;
}

int decode_min_split(const PoolView &pv, bool prefix) {
    // one wave per (stream, kv head) on MFMA measured slower than two: one kv head of 8 query
    // heads, caches of 512 rows, 17.0 -> 19.3 us; the int8 window at 2 kv heads 30.0 -> 30.6 us
    return decode_on_mfma(pv, prefix) ? 2 : 1;
}

int decode_heads_per_group(const PoolView &pv, bool prefix) {
    // query heads of one kv head share a group's page reads: all of them on MFMA; else four when
    // four divide the group and no stream of the batch keeps a ring prefix (whose second query
    // would spill them), else two; int8 on the VALU keeps one (its registers hold no second head
    // at four waves per SIMD)
    const int G = pv.H / pv.KVH;
    if (decode_on_mfma(pv, prefix)) return G;
    if (pv.cache_dt == DT_I8) return 1;
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
            return launch_decode_gqa(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        switch (decode_heads_per_group(pv, bv.prefix != 0)) {
        case 4: return decode_impl<DT_BF16, true, 4>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        case 2: return decode_impl<DT_BF16, true, 2>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        default: return decode_impl<DT_BF16, true, 1>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        }
    case DT_I8 * 2 + DT_BF16:
        if (decode_on_mfma(pv, bv.prefix != 0))
            return launch_decode_gqa(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
        return decode_impl<DT_I8, true, 1>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
    case DT_I8 * 2 + DT_F32: return decode_impl<DT_I8, false, 1>(pv, bv, layer, q, k, v, out, scale, fused, stream, tm);
    default: return hipErrorInvalidValue;
    }
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

hipError_t launch_window_prefill(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                                 const void *v, void *out, float scale, hipStream_t stream, const LaunchTiming &tm) {
    if (bv.n == 0) return hipSuccess;
    if (pv.cache_dt != DT_BF16 || pv.act_dt != DT_BF16) return hipErrorInvalidValue;
    return launch_prefill_mfma(pv, bv, layer, q, k, v, out, scale, false, true, stream, tm);
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
        return launch_prefill_mfma(pv, bv, layer, q, k, v, out, scale, fused, false, stream, tm);
    case DT_I8 * 2 + DT_BF16: return launch_prefill_mfma_i8(pv, bv, layer, q, out, scale, stream, tm);
    case DT_I8 * 2 + DT_F32: return prefill_rows_impl<DT_I8, false>(pv, bv, layer, q, out, scale, stream, tm);
    default: return hipErrorInvalidValue;
    }
}

} // namespace xnp
