// Attention on MFMA (bf16): the causal prompt prefill with its fused append (k_prefill_mfma), the
// windowed attention of a Mimi chunk (k_prefill_window) and the grouped-head decode (k_decode_gqa).
#include "kernels_common.h"

#include <type_traits>

namespace xnp {

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


typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// Scores against int8 pages on MFMA take the rotated bf16 queries as f16.  Each query column (query
// l16 of a tile: 8 dims in each of its 4 lanes g, at 32 kc + 8 g) is scaled by the power of two 2^-x
// that fits it into f16 (f16_fit_exponent: exact for every bf16 value the column holds), and summed
// over its 64 dims: a code c enters the product as the f16 value 1152 + c (c ^ 0x80 under the f16
// exponent of 1024), so the score is 2^x s_k (sum - 1152 qsum).
__device__ __forceinline__ void queries_f16(const bf16x8_t (&qq)[2], f16x8_t (&qh)[2], float &qsum, float &qpow) {
    float xv[16];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
        uint4 u;
        __builtin_memcpy(&u, &qq[kc], 16);
        const uint32_t *w4 = (const uint32_t *)&u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xv[8 * kc + 2 * i] = bf16_value(w4[i] & 0xffffu);
            xv[8 * kc + 2 * i + 1] = bf16_value(w4[i] >> 16);
        }
    }
    const int xq = f16_fit_exponent<16, 16, 2>(xv); // the column's 4 lanes: g = lane / 16
    qpow = pow2i(xq);
    qsum = 0.f;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
        uint32_t h4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x0 = xv[8 * kc + 2 * i] * pow2i(-xq), x1 = xv[8 * kc + 2 * i + 1] * pow2i(-xq);
            h4[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
            qsum += x0;
            qsum += x1;
        }
        qh[kc] = __builtin_bit_cast(f16x8_t, make_uint4(h4[0], h4[1], h4[2], h4[3]));
    }
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
}

constexpr int kPfKeys = 64;      // keys per chunk (four pages)
constexpr int kPfLd = 72;        // LDS row length in bf16: 64 + 8 of padding, rows 16-byte aligned
constexpr int kPfWaves = 8;      // waves per work group
constexpr int kPfRound = 256;    // query rows per round: 8 waves x 2 tiles x 16 rows
constexpr int kPfMaxPages = 512; // page ids a work group keeps in LDS
static_assert(kPfMaxPages >= kLaneBlocks * 8, "every page of a stream fits (a pool refuses more than 60 x 8)");
static_assert(64 * kPfWaves == kPfKeys * 8, "one thread stages 16 bytes of one key per chunk");

template <int CDT>
__global__ __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(4))) void k_prefill_mfma(
    PoolView pv, BatchView bv, int layer, const void *q, const void *knew, const void *vnew, void *out, float qmul,
    int fused) {
    static_assert(CDT == DT_BF16 || CDT == DT_I8, "bf16 or int8 pages");
    constexpr bool I8 = CDT == DT_I8;
    __shared__ __attribute__((aligned(16))) uint16_t ks[2 * kPfKeys][kPfLd]; // K of two chunks, [key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t vs[2 * kPfKeys][kPfLd]; // V of two chunks, [key][dim]
    __shared__ int32_t spages[kPfMaxPages];
    __shared__ float ssc[2][kPfKeys / kBlock][2]; // int8: each chunk's pages' K and V scales
    const int t = bv.t;
    // plan b is the batch's row b (its out_row): the inputs' and the output's rows are b's, so their
    // addresses do not wait for the plan
    const int h = blockIdx.x % pv.H, b = blockIdx.x / pv.H;
    const StreamPlan P = bv.plans[b];
    const int32_t *tab = pv.tables + (size_t)P.sid * pv.mbps;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
    const int c0 = P.write_slot; // slot (= position) of prompt row 0
    const int kvh = h / (pv.H / pv.KVH);
    const size_t page_elems = (size_t)pv.KVH * kBlock * kHeadDim;
    uint16_t *kpages = (uint16_t *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim);
    uint16_t *vpages = (uint16_t *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim);
    const int8_t *kpages8 = (const int8_t *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim);
    const int8_t *vpages8 = (const int8_t *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim);
    // the stream's page ids for every key any round sees, at most one per thread, loaded straight
    // into LDS (lane l of wave w: id 64 w + l): no register holds them, and nothing waits for them
    // before the first round's queries and first chunk go out.  Loads complete in the order
    // issued, so the waits for those (every wave's query loads come after these) cover them, and
    // the first round's barrier follows those waits; no earlier read of spages exists.
    const int npg = min((c0 + t + kBlock - 1) / kBlock, kPfMaxPages);
    static_assert(kPfMaxPages <= 64 * kPfWaves, "one page id per thread");
    if (64 * w < npg) dma4_at(tab + min(tid, npg - 1), lds_addr(&spages[0]) + 256 * w);
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

        // Loads run one chunk ahead: chunk c's registers are consumed (rotated, stored to LDS
        // buffer c & 1) at step c, which then issues chunk c + 1's loads into them.
        struct Stage {
            uint4 k, v, rope; // the key's K and V pieces (int8: 8 codes each in x, y), 4 (cos, sin) pairs as packed bf16
            int info;         // bit 0: a prompt key, bit 1: write it to its page
            float sk, sv;     // int8, the first thread of each page's keys: the page's scales
        };
        // LDS: the page ids are in LDS (all but the first round's first chunk, which reads the
        // table itself); a compile-time choice, so that no pointer is selected between the two
        auto issue = [&](int c, Stage &st, auto LDS) {
            const int slot = c * kPfKeys + skey;
            const bool in = c < nch && slot < kend;
            const bool fresh = !I8 && fused && slot >= c0; // a prompt key: from the inputs, rotated here
            const int i = fresh ? min(slot - c0, t - 1) : 0;
            const size_t arow = (((size_t)b * t + i) * pv.KVH + kvh) * kHeadDim + 8 * spart;
            st.k = st.v = make_uint4(0, 0, 0, 0);
            st.sk = st.sv = 0.f;
            if constexpr (I8) {
                // int8 pages (the prompt's rows appended before): 8 codes of K and of V; the first
                // thread of each page's keys also takes its scales (0 for a page outside the pool,
                // as the bf16 path's zero rows: score 0, no value)
                if (in) {
                    const int blk = min(slot >> 4, kPfMaxPages - 1);
                    int page;
                    if constexpr (decltype(LDS)::value)
                        page = spages[blk];
                    else
                        page = tab[blk];
                    if (page >= 0 && page < pv.NB) {
                        const size_t poff = (size_t)page * page_elems + (slot & 15) * kHeadDim + 8 * spart;
                        const uint2 kk = *(const uint2 *)(kpages8 + poff), vv = *(const uint2 *)(vpages8 + poff);
                        st.k = make_uint4(kk.x, kk.y, 0, 0);
                        st.v = make_uint4(vv.x, vv.y, 0, 0);
                        if ((skey & 15) == 0 && spart == 0) {
                            st.sk = pv.scales[tile_index(pv, layer, 0, page, kvh)];
                            st.sv = pv.scales[tile_index(pv, layer, 1, page, kvh)];
                        }
                    }
                }
                st.info = 0;
                return;
            }
            if (in && fresh) {
                st.k = ld_stream((const uint16_t *)knew + arow);
                st.v = ld_stream((const uint16_t *)vnew + arow);
            } else if (in) {
                const int blk = min(slot >> 4, kPfMaxPages - 1);
                int page;
                if constexpr (decltype(LDS)::value)
                    page = spages[blk];
                else
                    page = tab[blk];
                if (page >= 0 && page < pv.NB) {
                    const size_t poff = (size_t)page * page_elems + (slot & 15) * kHeadDim + 8 * spart;
                    st.k = ld_stream(kpages + poff);
                    st.v = ld_stream(vpages + poff);
                }
            }
            st.rope = *(const uint4 *)(pv.rope16 + (size_t)(P.key_pos + i) * (kHeadDim / 2) + 4 * spart);
            st.info = (in && fresh ? 1 : 0) | (in && fresh && last ? 2 : 0);
        };

        // B operands of S^T: query row 16 tile + l16, dims 32 kc + 8 g .. +7, rotated at its
        // position and rounded to bf16 as the reference's bf16 q is.  The queries' loads and the
        // first chunk's go out before any is used (rows past the prompt read row t - 1 and are
        // zeroed after).
        bf16x8_t qb[2][2];
        f16x8_t qh[2][2];                // int8: the queries as f16, scaled by 2^-x per column
        float qsum[2] = {0.f, 0.f}, qpow[2] = {1.f, 1.f}; // int8: their sums, 2^x
        float m[2], lsum[2]; // running max (scaled, log2 units) and this lane's share of the sum
        f32x4_t o[2][4];
        Stage st;
        {
            uint4 qraw[2][2], qcs[2][2]; // q pieces; their 4 (cos, sin) pairs as packed bf16
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int qr = min(16 * max(tile[j], 0) + l16, t - 1);
                const uint16_t *qp = (const uint16_t *)q + (((size_t)b * t + qr) * pv.H + h) * kHeadDim;
                const uint32_t *cs = pv.rope16 + (size_t)(P.pos + qr) * (kHeadDim / 2);
#pragma unroll
                for (int kc = 0; kc < 2; ++kc) {
                    qraw[j][kc] = *(const uint4 *)(qp + 32 * kc + 8 * g);
                    qcs[j][kc] = *(const uint4 *)(cs + 16 * kc + 4 * g);
                }
            }
            if (tq0 > 0)
                issue(0, st, std::true_type{});
            else
                issue(0, st, std::false_type{});
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                m[j] = -1e30f;
                lsum[j] = 0.f;
#pragma unroll
                for (int dg = 0; dg < 4; ++dg) o[j][dg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                const bool live = tile[j] >= 0 && 16 * tile[j] + l16 < t;
#pragma unroll
                for (int kc = 0; kc < 2; ++kc) {
                    const uint4 r = rotate8(qraw[j][kc], qcs[j][kc]);
                    qb[j][kc] = as_bf16x8(live ? r : make_uint4(0, 0, 0, 0));
                }
                if constexpr (I8) queries_f16(qb[j], qh[j], qsum[j], qpow[j]);
            }
        }
        __syncthreads(); // spages written

        auto step = [&](int c, Stage &st) {
            const int buf = c & 1, kbase = c * kPfKeys, lb = buf * kPfKeys;
            if constexpr (I8) {
                // K codes as f16 1152 + c (one byte permute each: c ^ 0x80 under the f16 exponent of
                // 1024), V codes as bf16 (exact); the pages' scales beside them
                uint32_t hk[4], bv2[4];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t kx = (i ? st.k.y : st.k.x) ^ 0x80808080u, vx = i ? st.v.y : st.v.x;
                    hk[2 * i] = __builtin_amdgcn_perm(0x64646464u, kx, 0x04010400u);
                    hk[2 * i + 1] = __builtin_amdgcn_perm(0x64646464u, kx, 0x04030402u);
                    bv2[2 * i] = pack_bf16((float)(int8_t)(vx & 0xffu), (float)(int8_t)((vx >> 8) & 0xffu));
                    bv2[2 * i + 1] = pack_bf16((float)(int8_t)((vx >> 16) & 0xffu), (float)(int8_t)(vx >> 24));
                }
                *(uint4 *)&ks[lb + skey][8 * spart] = make_uint4(hk[0], hk[1], hk[2], hk[3]);
                *(uint4 *)&vs[lb + skey][8 * spart] = make_uint4(bv2[0], bv2[1], bv2[2], bv2[3]);
                if ((skey & 15) == 0 && spart == 0) {
                    ssc[buf][skey >> 4][0] = st.sk;
                    ssc[buf][skey >> 4][1] = st.sv;
                }
            } else {
            // rotate a prompt key at its position; store this thread's piece of the chunk
            {
                const uint4 kk = st.info & 1 ? rotate8(st.k, st.rope) : st.k;
                if (st.info & 2) { // complete_kv: the prompt's rows go into their pages once
                    const int slot = kbase + skey;
                    const int page = spages[min(slot >> 4, kPfMaxPages - 1)];
                    if (page >= 0 && page < pv.NB) {
                        const size_t poff = (size_t)page * page_elems + (slot & 15) * kHeadDim + 8 * spart;
                        st_stream(kpages + poff, kk);
                        st_stream(vpages + poff, st.v);
                    }
                }
                *(uint4 *)&ks[lb + skey][8 * spart] = kk;
                *(uint4 *)&vs[lb + skey][8 * spart] = st.v;
            }
            }
            issue(c + 1, st, std::true_type{});
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
                        const uint4 a = *(const uint4 *)&ks[lb + 16 * kg + l16][32 * kc + 8 * g];
                        if constexpr (I8)
                            s[kg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), qh[j][kc],
                                                                          s[kg], 0, 0, 0);
                        else
                            s[kg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), qb[j][kc], s[kg], 0, 0, 0);
                    }
                    if constexpr (I8) { // the 16 keys of group kg are one page: its K scale, the bias out
                        const float f = ssc[buf][kg][0] * qpow[j];
#pragma unroll
                        for (int r = 0; r < 4; ++r) s[kg][r] = __builtin_fmaf(-1152.f, qsum[j], s[kg][r]) * f;
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
                // the row's max: a chain of pairs (v_max3), then over the row's 4 lanes by row swaps
                float mx = fmax_fin(s[0][0], s[0][1]);
#pragma unroll
                for (int e = 2; e < 16; e += 2) mx = fmaxf(fmaxf(mx, s[e >> 2][e & 3]), s[e >> 2][(e & 3) + 1]);
                mx = swap_max<32>(swap_max<16>(mx));
                // lazy rescaling, as in decode: the row's sum and accumulators move to a new max only
                // when some row of the wave saw its max grow by more than 8 (log2 units); until then
                // exponents are taken against the older max and stay below 2^8
                const float mn = fmax_fin(m[j], mx * qmul);
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
                    if constexpr (I8) { // P^T carries p sv (the page's V scale), so O needs none
                        const float sv = ssc[buf][kg][1];
#pragma unroll
                        for (int r = 0; r < 4; ++r) p[r] *= sv;
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
        for (int c = 0; c < nch; ++c) step(c, st);
        __syncthreads(); // the next round's staging overwrites both buffers

        // out[row][h][..] = O / l, the row's sum reduced over its 4 lanes.  The lane holds dims
        // 16 dg + 4 g .. +3 of row l16; through rows 16 w .. 16 w + 15 of ks (free after the barrier
        // above), each store instruction writes 8 whole 128-byte rows, so the non-temporal stores go
        // out as full lines.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (tile[j] < 0) continue;
            const float l = swap_sum<32>(swap_sum<16>(lsum[j]));
            const float inv = 1.0f / l;
            uint16_t(*st)[kPfLd] = &ks[16 * w];
#pragma unroll
            for (int dg = 0; dg < 4; ++dg)
                *(uint2 *)&st[l16][16 * dg + 4 * g] = make_uint2(pack_bf16(o[j][dg][0] * inv, o[j][dg][1] * inv),
                                                                 pack_bf16(o[j][dg][2] * inv, o[j][dg][3] * inv));
            // the lane index recomputed here (lane_here): hoisted out of the rounds, the output's
            // address pieces were held across them and spilled
            const int ln = lane_here(lane);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = (ln >> 3) + 8 * i, unit = ln & 7, qrow = 16 * tile[j] + r;
                const uint4 v = *(const uint4 *)&st[r][8 * unit];
                if (qrow < t) st_stream((uint16_t *)out + (((size_t)b * t + qrow) * pv.H + h) * kHeadDim + 8 * unit, v);
            }
        }
        if (!last) __syncthreads(); // the next round's staging overwrites ks
    }
}

// ---------------------------------------------------------------------------------------------
// prompt prefill for streams whose keys fit 256 slots (write_slot + t <= 256): the same
// contractions and tiles as k_prefill_mfma, but every key of the prompt is held in LDS at once, so
// each thread issues all of its loads (its queries, the prompt's 4 chunks of K and V and their RoPE
// rows) before it uses any.  The loads are unconditional (addresses clamped to real rows) and issued
// in the order they are consumed, so the compiler's waits take them one by one as they land
// (vector-memory loads complete in issue order) instead of draining the queue at every chunk, and a
// group never waits on a chain of per-chunk round trips.  Then each thread rotates its keys, writes
// its K and V pieces into LDS and, for the prompt's own rows, into their pages; one barrier; then
// the chunks' S^T, softmax and O^T on MFMA from LDS alone.
//
// K's and V's LDS rows are 128 bytes, their 16-byte units placed at unit ^ pf_swz(key).  Every read
// instruction of both contractions and the staging writes fall in distinct banks: the reads of K (16
// keys at one unit: lanes l16 of each group of 16), the transposed reads of V (4 keys at two adjacent
// units), and the staging writes (8 keys at all 8 units), whether the LDS serves 128 or 256 bytes a
// clock.  (The padded 144-byte rows of k_prefill_mfma leave the transposed reads 2-way conflicted.)
//
// Work groups are numbered so that each XCD takes a contiguous run of (stream, head) groups: the H
// groups of one stream read the H 128-byte pieces of the same 1 KB input rows through one L2 and
// at about the same time.
constexpr int kPfFastKeys = 256; // key slots a group holds: 4 chunks of 64

__device__ __forceinline__ int pf_swz(int r) {
    return ((r ^ (r >> 3)) & 1) | (r & 2) | (((r ^ (r >> 2)) & 1) << 2);
}

// PAGES: some keys of the stream come from its pages (keys before the prompt, or every key when the
// append ran separately), so their loads wait for the page ids; otherwise every key is a prompt row
// of the inputs and nothing waits before the loads go out.  DEPTH: chunks whose K/V loads go out
// before the first is used; the others go out as the first ones are consumed.
template <bool FUSED, bool PAGES, int DEPTH>
__device__ __forceinline__ void prefill_fast_group(const PoolView &pv, const BatchView &bv, int layer, const void *q,
                                                   const void *knew, const void *vnew, void *out, float qmul,
                                                   int b, int h, uint16_t (*ks)[kPfKeys][kHeadDim],
                                                   uint16_t (*vs)[kPfKeys][kHeadDim], uint4 *rp, int32_t *spages) {
    constexpr int NC = kPfFastKeys / kPfKeys;
    static_assert(DEPTH >= 1 && DEPTH <= NC, "chunks in flight");
    const int t = bv.t;
    const StreamPlan P = bv.plans[b];
    const int32_t *tab = pv.tables + (size_t)P.sid * pv.mbps;
    // the wave index through readfirstlane: the compiler then knows it (and the tiles, masks and
    // branches derived from it) to be uniform over the wave, and branches on the scalar unit
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
              l16 = lane & 15;
    const int c0 = PAGES ? P.write_slot : 0; // slot (= position) of prompt row 0
    const int kend = c0 + t;                 // keys [0, kend): at most kPfFastKeys
    const int nch = (kend + kPfKeys - 1) / kPfKeys;
    const int kvh = h / (pv.H / pv.KVH);
    const size_t page_elems = (size_t)pv.KVH * kBlock * kHeadDim;
    uint16_t *kpages = (uint16_t *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim);
    uint16_t *vpages = (uint16_t *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim);
    // this thread's share of each chunk: 16 bytes (8 dims, unit spart) of key skey
    const int skey = tid >> 3, spart = tid & 7;

    // Loads, all unconditional (addresses clamped to real rows) and in the order they are used:
    // the page of each chunk's key (for its page store, or its load), the RoPE rows of the chunks'
    // keys (parked in LDS below, so that no register holds them through the loop), this wave's
    // queries and their RoPE rows, then the chunks' K and V.
    // The RoPE rows of the chunks' keys go straight into this thread's own LDS pieces (no other thread
    // reads them; lane l of a wave's 1 KB load lands at 16 l), first of all: loads complete in issue
    // order, so every wait the compiler places for a later load covers them too.
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int slot = min(c * kPfKeys + skey, kend - 1), i = max(slot - c0, 0);
        dma16(pv.rope16 + (size_t)(P.key_pos + i) * (kHeadDim / 2) + 4 * spart, &rp[c * 64 * kPfWaves + 64 * w]);
    }
    // page ids: thread i < 16 holds block i's (the page stores and page loads read them from LDS)
    const int my_pg = tab[min(tid, (kend - 1) >> 4)];
    // this wave's query tiles: (w, nq-1-w) for w < nq/2; the middle one alone when nq is odd
    const int nq = (t + 15) / 16;
    int tile[2] = {-1, -1};
    if (w < nq / 2) {
        tile[0] = w;
        tile[1] = nq - 1 - w;
    } else if (w == nq / 2 && (nq & 1)) {
        tile[0] = w;
    }
    // B operands of S^T: query row 16 tile + l16, dims 32 kc + 8 g .. +7, with their (cos, sin) rows
    uint4 qraw[2][2], qcs[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int qr = min(16 * max(tile[j], 0) + l16, t - 1);
        const uint16_t *qp = (const uint16_t *)q + (((size_t)b * t + qr) * pv.H + h) * kHeadDim;
        const uint32_t *cs = pv.rope16 + (size_t)(P.pos + qr) * (kHeadDim / 2);
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            qraw[j][kc] = *(const uint4 *)(qp + 32 * kc + 8 * g);
            qcs[j][kc] = *(const uint4 *)(cs + 16 * kc + 4 * g);
        }
    }
    uint4 kr[NC], vr[NC];
    auto issue = [&](auto C) {
        constexpr int c = decltype(C)::value;
        const int slot = min(c * kPfKeys + skey, kend - 1);
        const bool fresh = FUSED && slot >= c0;
        const int i = fresh ? slot - c0 : 0;
        const size_t arow = (((size_t)b * t + i) * pv.KVH + kvh) * kHeadDim + 8 * spart;
        const uint16_t *ksrc = (const uint16_t *)knew + arow, *vsrc = (const uint16_t *)vnew + arow;
        if constexpr (PAGES) {
            const int pgc = spages[slot >> 4];
            const int page = pgc >= 0 && pgc < pv.NB ? pgc : 0;
            const size_t poff = (size_t)page * page_elems + (slot & 15) * kHeadDim + 8 * spart;
            ksrc = fresh ? ksrc : kpages + poff;
            vsrc = fresh ? vsrc : vpages + poff;
        }
        kr[c] = ld_stream(ksrc);
        vr[c] = ld_stream(vsrc);
    };
    if constexpr (PAGES) { // the page loads need the page ids: a round trip before any chunk goes out
        if (tid < kPfFastKeys / kBlock) spages[tid] = my_pg;
        __syncthreads();
    }
    issue(std::integral_constant<int, 0>{});
    if constexpr (DEPTH > 1) issue(std::integral_constant<int, 1>{});
    if constexpr (DEPTH > 2) issue(std::integral_constant<int, 2>{});
    if constexpr (DEPTH > 3) issue(std::integral_constant<int, 3>{});
    // nothing below moves above the loads: an LDS store hoisted above them would wait for the loads
    // its data comes from before they go out
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!PAGES)
        if (tid < kPfFastKeys / kBlock) spages[tid] = my_pg;

    // the queries, rotated at their positions and rounded to bf16 as the reference's bf16 q is
    bf16x8_t qb[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const bool live = tile[j] >= 0 && 16 * tile[j] + l16 < t;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            const uint4 r = rotate8(qraw[j][kc], qcs[j][kc]);
            qb[j][kc] = as_bf16x8(live ? r : make_uint4(0, 0, 0, 0));
        }
    }

    float m[2], lsum[2]; // running max (scaled, log2 units) and this lane's share of the sum
    f32x4_t o[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        m[j] = -1e30f;
        lsum[j] = 0.f;
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) o[j][dg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    // out[row][h][..] = O / l of tile j, the row's sum reduced over its 4 lanes.  The lane holds dims
    // 16 dg + 4 g .. +3 of row l16; through this wave's 2 KB of LDS (chunk slot 0, which no wave reads
    // after the last chunk's barrier), each store instruction writes 8 whole 128-byte rows, so the
    // non-temporal stores go out as full lines (8-byte pieces went out as partial ones: 1.3x the
    // written bytes).  Unit u of row r sits at unit u ^ (r & 7).
    auto store_tile = [&](int j) {
        const float l = swap_sum<32>(swap_sum<16>(lsum[j]));
        const float inv = 1.0f / l;
        uint16_t *st = (w < 4 ? &ks[0][0][0] : &vs[0][0][0]) + (w & 3) * 16 * kHeadDim;
#pragma unroll
        for (int dg = 0; dg < 4; ++dg)
            *(uint2 *)(st + l16 * kHeadDim + 8 * ((2 * dg + (g >> 1)) ^ (l16 & 7)) + 4 * (g & 1)) =
                make_uint2(pack_bf16(o[j][dg][0] * inv, o[j][dg][1] * inv),
                           pack_bf16(o[j][dg][2] * inv, o[j][dg][3] * inv));
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = (lane >> 3) + 8 * i, unit = lane & 7, qrow = 16 * tile[j] + r;
            const uint4 v = *(const uint4 *)(st + r * kHeadDim + 8 * (unit ^ (r & 7)));
            if (qrow < t) st_stream((uint16_t *)out + (((size_t)b * t + qrow) * pv.H + h) * kHeadDim + 8 * unit, v);
        }
    };
    // The lane's LDS read offsets within a chunk slot, computed once: the swizzle of a row depends
    // on its low 4 bits only, so the slot, the 16-key group, the 32-key half and the second
    // transposed read are constant offsets from these.
    //   K (A of S^T):  row l16 (+ 16 kg), unit 4 kc + g
    //   V (A of O^T):  row 4 g + l16 / 4 (+ 32 kp, + 16), unit 2 dg + (l16 % 4) / 2, half l16 % 2
    constexpr int kRowB = kHeadDim * 2, kSlotB = kPfKeys * kRowB;
    const char *ksb = (const char *)&ks[0][0][0], *vsb = (const char *)&vs[0][0][0];
    int kofs[2], vofs[4];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) kofs[kc] = l16 * kRowB + 16 * ((4 * kc + g) ^ pf_swz(l16));
    {
        const int vrow = 4 * g + (l16 >> 2), vf = pf_swz(vrow), vu = (l16 & 3) >> 1;
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) vofs[dg] = vrow * kRowB + 16 * ((2 * dg + vu) ^ vf) + 8 * (l16 & 1);
    }
    auto step = [&](auto C) {
        constexpr int c = decltype(C)::value;
        const int kbase = c * kPfKeys, u = c & 1;
        // stage chunk c: a prompt key rotated at its position (rotated whatever the key, then chosen:
        // a use under a branch lets the compiler sink a load behind the others, and its wait would
        // then drain them all); the piece into LDS slot c & 1, the prompt's rows into their pages
        // (complete_kv, transformer.rs:84-91; a page id outside the pool writes nothing)
        {
            const int slot = kbase + skey, cl = min(slot, kend - 1);
            const bool fresh = FUSED && cl >= c0;
            // kr[c] has landed, and with it the RoPE pieces loaded before it; their LDS read stays below
            asm volatile("" ::"v"(kr[c].x) : "memory");
            const uint4 rot = rotate8(kr[c], rp[c * 64 * kPfWaves + tid]);
            const uint4 kk = fresh ? rot : kr[c];
            const int pu = 8 * (spart ^ pf_swz(skey));
            *(uint4 *)&ks[u][skey][pu] = kk;
            *(uint4 *)&vs[u][skey][pu] = vr[c];
            // chunk c is in slot c & 1; every reader of chunk c - 2 (same slot) is done; the page ids
            // are in LDS.  An LDS-only barrier: __syncthreads would also wait for earlier chunks' page
            // stores, which nothing here reads back.
            lds_barrier();
            const int pgc = spages[min(slot, kend - 1) >> 4];
            if (FUSED && fresh && slot < kend && pgc >= 0 && pgc < pv.NB) {
                const size_t poff = (size_t)pgc * page_elems + (slot & 15) * kHeadDim + 8 * spart;
                st_stream(kpages + poff, kk);
                st_stream(vpages + poff, vr[c]);
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r0 = c0 + 16 * tile[j]; // slot of the tile's first row
            // skip a tile when every key of the chunk comes after all of its rows (and every chunk
            // past the keys)
            if (c >= nch || tile[j] < 0 || kbase > r0 + 15) continue;
            // key kbase + 16 kg + 4 g + r is seen by row r0 + l16 when 16 kg + 4 g + r <= rel + l16: a
            // group of 16 keys is seen whole (16 kg + 15 <= rel), not at all (16 kg > rel + 15: its
            // products and exponentials are skipped, P = 0), or in part (masked key by key)
            const int rel = r0 - kbase;
            f32x4_t s[4];
#pragma unroll
            for (int kg = 0; kg < 4; ++kg) {
                s[kg] = f32x4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
                if (16 * kg > rel + 15) continue;
                s[kg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kc = 0; kc < 2; ++kc) {
                    const bf16x8_t a = as_bf16x8(*(const uint4 *)(ksb + u * kSlotB + kg * 16 * kRowB + kofs[kc]));
                    s[kg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[j][kc], s[kg], 0, 0, 0);
                }
                if (16 * kg + 15 > rel) {
                    const int lim = rel + l16 - 16 * kg - 4 * g; // the lane's keys r <= lim are seen
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (r > lim) s[kg][r] = -INFINITY;
                }
            }
            // the row's max: a chain of pairs (v_max3), then over the row's 4 lanes by row swaps
            float mx = fmax_fin(s[0][0], s[0][1]);
#pragma unroll
            for (int e = 2; e < 16; e += 2) mx = fmaxf(fmaxf(mx, s[e >> 2][e & 3]), s[e >> 2][(e & 3) + 1]);
            mx = swap_max<32>(swap_max<16>(mx));
            // lazy rescaling, as in decode: the row's sum and accumulators move to a new max only
            // when some row of the wave saw its max grow by more than 8 (log2 units)
            const float mn = fmax_fin(m[j], mx * qmul);
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
                pk[kg][0] = pk[kg][1] = 0u;
                if (16 * kg > rel + 15) continue;
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
                if (32 * kp > rel + 15) continue; // both groups unseen: P is 0
                // k slots: keys 32 kp + 4 g .. +3 (elements 0-3) and 32 kp + 16 + 4 g .. +3 (4-7)
                const bf16x8_t pb =
                    as_bf16x8(make_uint4(pk[2 * kp][0], pk[2 * kp][1], pk[2 * kp + 1][0], pk[2 * kp + 1][1]));
#pragma unroll
                for (int dg = 0; dg < 4; ++dg) {
                    // V^T: lane gets dim 16 dg + l16 of the same eight keys, by two transposed reads
                    const char *vp = vsb + u * kSlotB + kp * 32 * kRowB + vofs[dg];
                    const uint2 lo = lds_read_tr16((const uint16_t *)vp);
                    const uint2 hi = lds_read_tr16((const uint16_t *)(vp + 16 * kRowB));
                    const bf16x8_t a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
                    o[j][dg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[j][dg], 0, 0, 0);
                }
            }
        }
        // the registers of chunk c take chunk c + DEPTH: issued after this chunk's products, so that
        // they are not held through them
        if constexpr (c + DEPTH < NC) issue(std::integral_constant<int, c + DEPTH>{});
    };
    // every chunk is staged, those past the keys too (clamped copies of the last key, never seen):
    // then no load is still in flight into a register the code after the steps takes over
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
    step(std::integral_constant<int, 3>{});
    static_assert(NC == 4, "the steps above");
    // the output after every chunk: a store issued between the chunks would make each later wait for
    // a chunk's loads wait for it too (the wait counts every access issued after the load it needs)
    if (tile[0] >= 0) store_tile(0);
    if (tile[1] >= 0) store_tile(1);
}

#ifndef XNP_PF_DEPTH
#define XNP_PF_DEPTH 4
#endif

template <bool FUSED>
__global__ __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(4))) void k_prefill_fast(
    PoolView pv, BatchView bv, int layer, const void *q, const void *knew, const void *vnew, void *out, float qmul) {
    __shared__ __attribute__((aligned(16))) uint16_t ks[2][kPfKeys][kHeadDim]; // K of two chunks, [key][unit ^ pf_swz(key)]
    __shared__ __attribute__((aligned(16))) uint16_t vs[2][kPfKeys][kHeadDim]; // V, likewise
    __shared__ uint4 rp[kPfFastKeys / kPfKeys * 64 * kPfWaves];                // each thread's keys' RoPE rows
    __shared__ int32_t spages[kPfFastKeys / kBlock];                            // the page of each block of keys
    const int tl = xcd_tile(blockIdx.x, bv.n * pv.H);
    const int h = tl % pv.H, b = tl / pv.H;
    if (!FUSED || bv.plans[b].write_slot > 0)
        prefill_fast_group<FUSED, true, XNP_PF_DEPTH>(pv, bv, layer, q, knew, vnew, out, qmul, b, h, ks, vs, rp, spages);
    else
        prefill_fast_group<FUSED, false, XNP_PF_DEPTH>(pv, bv, layer, q, knew, vnew, out, qmul, b, h, ks, vs, rp, spages);
}

// ---------------------------------------------------------------------------------------------
// Windowed attention of a Mimi chunk on MFMA (bf16 window cache and activations),
// transformer.rs:764-781: t query rows over a window cache of W rows (slot p mod W holds position
// p) and the chunk's own rows, each row seeing the W keys up to itself, for chunks of any length.
//
// One work group of 8 waves per (stream, head), two work groups per CU.  Keys are indexed
// virtually: the window's held rows first (j < ncache, oldest first, at slot (wbase + j) mod W),
// then the chunk's rows (j = ncache + i: input row i, rotated at its position and rounded to bf16).
// Query row i has virtual index ncache + i and sees key j when ncache + i - W < j <= ncache + i.
// The chunk's rows reach the window by their own append (k_window_append); this kernel only reads.
//
// Query rows are taken in rounds of 256: 8 pairs of 16-row tiles, pair i rows 32 i .. 32 i + 31 of
// the round, wave w owning pair w.  A round's keys (from the window of its first row to
// its last row) stream through a ring of 3 LDS slots in chunks of 64 (K and V as
// [key][unit ^ swz(key)], K's rope pieces beside them), loaded straight into LDS
// (global_load_lds_dwordx4) 2 chunks ahead of the one attended, so that no register holds them.
// At each chunk a lane waits for its own loads of it, rotates the chunk's own keys among them in
// place, and one barrier hands the chunk to every wave.
//
// The two tiles of a pair are the 32 columns of v_mfma_f32_32x32x16_bf16.  A wave holds one pair's
// queries and accumulators in 128 registers, so four waves share a SIMD (the chunk and block loops
// stay rolled: unrolled, the compiler hoists operand reads across them and spills; a few setup values
// still spill once per group).  With two pairs a wave (4 waves a group, 253 registers, two waves a
// SIMD) each K and V piece served 64 queries, but the waves waited 44 % of their cycles and the
// launch took 6 % longer.  Both contractions are computed transposed so that P never leaves
// registers:
//   S^T = K Q^T      A = 32 keys of K from LDS (lane: key lane % 32, dims 16 kk + 8 (lane / 32)),
//                    B = the pair's rotated queries (lane: query column lane % 32, same dims);
//                    lane l holds column l % 32 against keys 8 (r / 4) + 4 (l / 32) + r % 4;
//   softmax          online per column; its max and sum pair lanes l and l ^ 32 (permlane32_swap);
//   O^T += V^T P^T   B = P^T straight from the S^T registers (16 keys a step), A = V^T by
//                    transposed LDS reads (ds_read_b64_tr_b16) of the same keys.
// A and B always hold the same key (or dim) in the same (lane / 32, element) slot, so each
// contraction is right whatever order the instruction walks k in.

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

constexpr int kWpChunk = 64;  // keys of a chunk
constexpr int kWpSlots = 3;   // chunk slots of the LDS ring: 2 chunks load while one is attended
constexpr int kWpWaves = 8;   // waves per work group
constexpr int kWpPairs = 1;   // tile pairs per wave
constexpr int kWpRound = 256; // query rows per round: 8 waves x 1 pair x 32 rows
// A chunk is 24 direct loads of 1 KB (8 keys each), 3 a wave: one each of K, V and K's rope pieces.
constexpr int kWpLoadsC = kWpChunk / 8 / kWpWaves; // loads of K (of V, of rope pieces) per wave per chunk
constexpr int kWpKeysW = kWpChunk / kWpWaves;      // keys of a chunk each wave loads
static_assert(kWpRound == kWpWaves * kWpPairs * 32, "a round is the waves' pairs");
static_assert(kWpLoadsC == 1 && kWpSlots == 3, "the waits below count 3 loads a chunk, 2 chunks ahead");

// K's and V's LDS rows are 128 bytes, their 16-byte units placed at unit ^ swz(key): for 16 keys in
// a row (the reads of K's pieces) and for keys 4a .. 4a + 3 with two adjacent units each (the
// transposed reads of V), every unit of a read falls in its own banks.
__device__ __forceinline__ int swz(int key) {
    const int x = (key >> 1) & 7;
    return ((x & 1) << 1) | (((x >> 1) & 1) << 2) | ((x >> 2) & 1);
}

// the pair of a lane's value: lanes l and l ^ 32 exchange (both halves of the result hold both)
__device__ __forceinline__ float pair_max(float x) { return swap_max<32>(x); }
__device__ __forceinline__ float pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Vector-memory loads of a wave complete in the order issued (one counter, vmcnt), so a wave waits
// for chunk c by letting only the `ahead` chunks it issued after it (3 loads each) stay in flight.
// The loads land in LDS, which the compiler does not track: this wait is the only one they get.
__device__ __forceinline__ void wait_chunks(int ahead) {
    if (ahead <= 0)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (ahead == 1)
        asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
}

__global__ __launch_bounds__(64 * kWpWaves) __attribute__((amdgpu_waves_per_eu(4))) void k_prefill_window(
    PoolView pv, BatchView bv, int layer, const void *q, const void *knew, const void *vnew, void *out, float qmul) {
    __shared__ __attribute__((aligned(16))) uint16_t ks[kWpSlots][kWpChunk][kHeadDim]; // K, [key][unit ^ swz]
    __shared__ __attribute__((aligned(16))) uint16_t vs[kWpSlots][kWpChunk][kHeadDim]; // V, [key][unit ^ swz]
    __shared__ __attribute__((aligned(16))) uint4 rs[kWpSlots][kWpWaves][kWpLoadsC][64]; // the lanes' rope pieces
    __shared__ int32_t spages[kPfMaxPages];
    const int t = bv.t;
    const int h = blockIdx.x % pv.H, b = blockIdx.x / pv.H;
    const StreamPlan P = bv.plans[b];
    const int32_t *tab = pv.tables + (size_t)P.sid * pv.mbps;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, hi = lane >> 5, col = lane & 31;
    const int W = P.window;
    const int ncache = P.pos_pre; // the window's held rows; keys from the pages are these
    const int nfrom = ncache;
    const int kvh = h / (pv.H / pv.KVH);
    const size_t page_elems = (size_t)pv.KVH * kBlock * kHeadDim;
    uint16_t *kpages = (uint16_t *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim);
    uint16_t *vpages = (uint16_t *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim);

    // the K and V rings' LDS addresses, taken once (see lds_addr)
    const uint32_t ks_at = lds_addr(&ks[0][0][0]), vs_at = lds_addr(&vs[0][0][0]);
    // the stream's page ids, read once: the pages of cached keys and of the rows written (before the
    // rounds, so that no register holds their addresses through them; the first round's barrier
    // precedes every read of them)
    for (int i = tid; i < min(pv.mbps, kPfMaxPages); i += 64 * kWpWaves) spages[i] = tab[i];

    // A chunk's keys j0 + key go straight into LDS slot `slot` by 1 KB loads: lane l of load i of
    // wave w takes key 16 w + 8 i + l / 8 and holds its unit (l % 8) ^ swz(key), and the rope piece
    // of a step's own key to its own place (every load is issued, so that each chunk is 6 loads of
    // the lane, and nothing of it sits in registers).  Keys past the round (j >= khi) read the
    // round's last key, so that LDS only ever holds finite values where P is 0.
    auto issue = [&](int j0, int khi, int slot) {
        const int ln = lane_here(lane);
#pragma unroll
        for (int i = 0; i < kWpLoadsC; ++i) {
            const int row = kWpKeysW * w + 8 * i, key = row + (ln >> 3), j = min(j0 + key, khi - 1);
            const int unit = (ln & 7) ^ swz(key);
            const uint16_t *ksrc, *vsrc;
            if (j >= nfrom) {
                const size_t arow = (((size_t)P.out_row * t + (j - ncache)) * pv.KVH + kvh) * kHeadDim + 8 * unit;
                ksrc = (const uint16_t *)knew + arow;
                vsrc = (const uint16_t *)vnew + arow;
            } else {
                int s = P.wbase + j;
                if (s >= W) s -= W;
                const int pg = spages[s >> 4];
                const size_t poff = (size_t)(pg >= 0 && pg < pv.NB ? pg : 0) * page_elems + (s & 15) * kHeadDim + 8 * unit;
                ksrc = kpages + poff;
                vsrc = vpages + poff;
            }
            const uint32_t kv_off = (uint32_t)((slot * kWpChunk + row) * kHeadDim) * 2;
            if (j0 + row >= nfrom) { // every key of this load is a row of the step: read once, streamed
                dma16_at_nt(ksrc, ks_at + kv_off);
                dma16_at_nt(vsrc, vs_at + kv_off);
            } else {
                dma16_at(ksrc, ks_at + kv_off);
                dma16_at(vsrc, vs_at + kv_off);
            }
            const int r = max(j - ncache, 0);
            dma16(pv.rope16 + (size_t)(P.key_pos + r) * (kHeadDim / 2) + 4 * unit, &rs[slot][w][i][0]);
        }
    };
    // ...then, once they have landed, the step's own keys rotated in place by the lane that loaded
    // them
    auto settle = [&](int j0, int khi, int slot) {
        const int ln = lane_here(lane);
#pragma unroll
        for (int i = 0; i < kWpLoadsC; ++i) {
            const int key = kWpKeysW * w + 8 * i + (ln >> 3), j = j0 + key;
            if (j >= khi || j < nfrom) continue;
            uint4 *kp = (uint4 *)&ks[slot][key][8 * (ln & 7)]; // this lane's own pieces
            *kp = rotate8(*kp, rs[slot][w][i][ln]);
        }
    };
    const int nqt = (t + 15) / 16;
    for (int tq0 = 0; tq0 < nqt; tq0 += kWpRound / 16) {
        const int nq = min(kWpRound / 16, nqt - tq0);
        // the round's keys: from the window of its first row to its last row
        const int khi = ncache + min(t, 16 * (tq0 + nq));
        const int klo = max(0, (ncache + 16 * tq0 - W + 1) / kWpChunk * kWpChunk);
        const int nch = (khi - klo + kWpChunk - 1) / kWpChunk;

        // the wave's pairs: pair i = w (p = 0) and 7 - w (p = 1) hold the round's tiles 2 i and 2 i + 1,
        // rows 32 i .. 32 i + 31 (a tile past the round's last is not stored)
        int vq[kWpPairs], vq_min[kWpPairs], vq_max[kWpPairs], qr[kWpPairs];
        bool act[kWpPairs];
        bf16x8_t qb[kWpPairs][4];
        // chunk loads write LDS, so a later round's wait until every reader of the previous round is
        // done.  The round's first chunk goes out ahead of the queries when it reads no page (keys of
        // the step itself), the rest of the ring once the queries are in.
        if (tq0 > 0) __syncthreads();
        const bool early = klo >= nfrom;
        if (early) issue(klo, khi, 0);
        {
            uint4 qraw[kWpPairs][4], qcs[kWpPairs][4];
#pragma unroll
            for (int p = 0; p < kWpPairs; ++p) {
                const int i = p == 0 ? w : kWpRound / 32 - 1 - w, r0 = 16 * tq0 + 32 * i;
                act[p] = 32 * i < 16 * nq;
                // column col: query row r0 + col, dims 16 kk + 8 hi .. +7, rotated at its position and
                // rounded to bf16 as the reference's bf16 q is; rows past the step read row t - 1 and
                // are never stored
                qr[p] = min(r0 + col, t - 1);
                vq[p] = ncache + qr[p];
                vq_min[p] = ncache + r0;
                vq_max[p] = ncache + min(r0 + 31, t - 1);
                const uint16_t *qp = (const uint16_t *)q + (((size_t)P.out_row * t + qr[p]) * pv.H + h) * kHeadDim;
                const uint32_t *cs = pv.rope16 + (size_t)(P.pos + qr[p]) * (kHeadDim / 2);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    qraw[p][kk] = *(const uint4 *)(qp + 16 * kk + 8 * hi);
                    qcs[p][kk] = *(const uint4 *)(cs + 8 * kk + 4 * hi);
                }
            }
#pragma unroll
            for (int p = 0; p < kWpPairs; ++p)
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    qb[p][kk] = as_bf16x8(rotate8(qraw[p][kk], qcs[p][kk]));
                    // rotated here: the compiler's waits for these loads, placed after the chunk loads
                    // below, would count those too and wait for them
                    asm volatile("" ::"v"(qb[p][kk]));
                }
            wait_chunks(0); // this lane's loads so far (the first chunk, the page ids) have landed
            __syncthreads(); // ...and every lane's: the page ids and the first chunk are in LDS
#pragma unroll
            for (int c = early ? 1 : 0; c < kWpSlots; ++c)
                if (c < nch) issue(klo + kWpChunk * c, khi, c);
        }
        // the last key any query of the wave sees (pair 1 holds the later rows)
        int wq_max = -1;
#pragma unroll
        for (int p = 0; p < kWpPairs; ++p)
            if (act[p]) wq_max = max(wq_max, vq_max[p]);

        float m[kWpPairs], lsum[kWpPairs]; // running max (scaled, log2 units), this lane's share of the sum
        f32x16_t o[kWpPairs][2];           // O^T: dims 32 hh + 8 (r / 4) + 4 hi + r % 4, column col
#pragma unroll
        for (int p = 0; p < kWpPairs; ++p) {
            m[p] = -1e30f;
            lsum[p] = 0.f;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[p][hh][r] = 0.f;
        }

        for (int cb = 0; cb < nch; cb += kWpSlots) {
#pragma unroll 1
            for (int u = 0; u < kWpSlots; ++u) { // rolled: see above
                const int c = cb + u;
                if (c >= nch) break;
                const int j0 = klo + kWpChunk * c;
                // this lane's loads of chunk c have landed: after them it issued chunk c + 1 (chunks
                // 0 .. 2 went out first, then one a step)
                wait_chunks(min(c == 0 ? kWpSlots - 1 : kWpSlots - 2, nch - 1 - c));
                settle(j0, khi, u);
                lds_barrier(); // chunk c is in LDS; every wave is done with chunk c - 1's slot
                if (c > 0 && c + kWpSlots - 1 < nch)
                    issue(j0 + kWpChunk * (kWpSlots - 1), khi, (u + kWpSlots - 1) % kWpSlots);
#pragma unroll 1
                for (int kb = 0; kb < kWpChunk; kb += 32) {
                    const int jb = j0 + kb; // the block's first key
                    if (jb > wq_max) break; // after every query of the wave
                    // S^T for each pair that sees some key of the block; the K pieces serve both
                    bf16x8_t ka[4];
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk)
                        ka[kk] = as_bf16x8(*(const uint4 *)&ks[u][kb + col][8 * ((2 * kk + hi) ^ swz(kb + col))]);
                    bool need[kWpPairs];
                    uint32_t pk[kWpPairs][8];
#pragma unroll
                    for (int p = 0; p < kWpPairs; ++p) {
                        // uniform: a pair skips a block after its last row or before its first row's window
                        need[p] = act[p] && jb <= vq_max[p] && !(jb + 31 <= vq_min[p] - W);
                        if (!need[p]) continue;
                        f32x16_t s;
#pragma unroll
                        for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[kk], qb[p][kk], s, 0, 0, 0);
                        // mask unless every key of the block is visible to every query of the pair: key
                        // jb + 4 hi + kr(r) (kr = 8 (r / 4) + r % 4) is seen when kr(r) <= lim, and on a
                        // window when kr(r) > lim - W
                        if (jb + 31 > vq_min[p] || jb <= vq_max[p] - W) {
                            const int lim = vq[p] - jb - 4 * hi;
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                const int kr = 8 * (r >> 2) + (r & 3);
                                if (kr > lim || kr <= lim - W) s[r] = -INFINITY;
                            }
                        }
                        float mx = fmax_fin(s[0], s[1]);
#pragma unroll
                        for (int r = 2; r < 16; ++r) mx = fmaxf(mx, s[r]);
                        mx = pair_max(mx);
                        // lazy rescaling, as in decode: the column's sum and accumulators move to a new
                        // max only when some column of the pair saw its max grow by more than 8 (log2
                        // units); until then exponents are taken against the older max
                        const float mn = fmax_fin(m[p], mx * qmul);
                        if (__any(mn > m[p] + 8.f)) {
                            const float alpha = fast_exp2(m[p] - mn);
                            lsum[p] *= alpha;
#pragma unroll
                            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                                for (int r = 0; r < 16; ++r) o[p][hh][r] *= alpha;
                            m[p] = mn;
                        }
                        float psum = 0.f;
#pragma unroll
                        for (int r = 0; r < 16; r += 2) {
                            const float p0 = fast_exp2(__builtin_fmaf(s[r], qmul, -m[p]));
                            const float p1 = fast_exp2(__builtin_fmaf(s[r + 1], qmul, -m[p]));
                            psum += p0 + p1;
                            pk[p][r >> 1] = pack_bf16(p0, p1);
                        }
                        lsum[p] += psum;
                    }
#pragma unroll
                    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            // V^T: lane gets dim 32 hh + col of keys 16 kh + 4 hi .. +3 and 16 kh + 8 + 4 hi ..
                            // +3, by two transposed reads; B = P^T of the same k slots
                            const int vr = kb + 16 * kh + 4 * hi + ((lane & 15) >> 2);
                            const int vu = 4 * hh + 2 * (col >> 4) + ((lane & 3) >> 1), vo = 4 * (lane & 1);
                            const uint2 lo = lds_read_tr16(&vs[u][vr][8 * (vu ^ swz(vr)) + vo]);
                            const uint2 up = lds_read_tr16(&vs[u][vr + 8][8 * (vu ^ swz(vr + 8)) + vo]);
                            const bf16x8_t va = as_bf16x8(make_uint4(lo.x, lo.y, up.x, up.y));
#pragma unroll
                            for (int p = 0; p < kWpPairs; ++p) {
                                if (!need[p]) continue;
                                const bf16x8_t pb = as_bf16x8(make_uint4(pk[p][4 * kh], pk[p][4 * kh + 1], pk[p][4 * kh + 2],
                                                                         pk[p][4 * kh + 3]));
                                o[p][hh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, o[p][hh], 0, 0, 0);
                            }
                        }
                }
            }
        }
        // The output leaves as whole 128-byte rows: once every wave is done attending, each wave
        // writes its pair's O / l (l: the column's sum over its lane pair), rounded to bf16, into 4 KB
        // of the K and V rings of its own, as [row 32 p + col][unit ^ (row & 7)], and stores 8 rows at a
        // time.
        lds_barrier();
        constexpr int kStageRows = 32 * kWpPairs, kRingRows = kWpSlots * kWpChunk;
        static_assert(kWpWaves * kStageRows <= 2 * kRingRows, "the waves' output tiles fit the K and V rings");
        uint16_t *stage = kStageRows * w < kRingRows ? &ks[0][0][0] + kStageRows * w * kHeadDim
                                                     : &vs[0][0][0] + (kStageRows * w - kRingRows) * kHeadDim;
#pragma unroll
        for (int p = 0; p < kWpPairs; ++p) {
            const float inv = 1.0f / pair_sum(lsum[p]); // not stored for a pair past the round
            const int row = 32 * p + col;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    *(uint2 *)(stage + row * kHeadDim + 8 * ((4 * hh + rr) ^ (row & 7)) + 4 * hi) =
                        make_uint2(pack_bf16(o[p][hh][4 * rr] * inv, o[p][hh][4 * rr + 1] * inv),
                                   pack_bf16(o[p][hh][4 * rr + 2] * inv, o[p][hh][4 * rr + 3] * inv));
        }
        lds_barrier();
#pragma unroll
        for (int k = 0; k < 2 * kWpPairs * 32 / 16; ++k) {
            const int row = 8 * k + (lane >> 3), unit = lane & 7, p = row >> 5;
            const int qrow = 16 * tq0 + 32 * (p == 0 ? w : kWpRound / 32 - 1 - w) + (row & 31);
            if (act[p] && qrow < t)
                st_stream((uint16_t *)out + (((size_t)P.out_row * t + qrow) * pv.H + h) * kHeadDim + 8 * unit,
                          *(const uint4 *)(stage + row * kHeadDim + 8 * (unit ^ (row & 7))));
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Grouped-head decode on MFMA: bf16 or int8 pages, bf16 queries, 2 to 16 query heads per kv head
// (the kernel takes any G from 1; the launcher sends G = 1 to the VALU decode).  One work
// group per (stream, kv head), whose G query heads are the 16 columns of the
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
// Pages, SPLIT waves per group, the fused append and the LDS merge are attend_core's.  PREFIX (some
// stream of the batch keeps an absolute ring's prefix): the keys before the prefix are scored
// against the queries rotated at pos_pre (attend_core's second query position), a second S^T of
// the same K operand on the pages that hold prefix rows, taken row by row in the same lanes.
//
// CDT = DT_I8 (int8 pages with f32 scales per (page, kv head); the fused append is attend_core's,
// re-reading the write page's scales after it): the VALU decode's arithmetic moved onto the MFMA.
// With PREFIX, the queries at pos_pre get an f16 copy, power of two and sum of their own.  A code
// byte c goes
// to f16 as 1024 + (c + 128) = 1152 + c by one byte permute (c ^ 0x80 under the f16 exponent of
// 1024), the rotated bf16 queries convert to f16 exactly, so v_mfma_f32_16x16x32_f16 sums
// q (1152 + c) and the score is sk (that sum - 1152 sum(q)).  V codes widen to bf16 exactly
// (|c| <= 127) and P^T carries p sv rounded to bf16, so O needs no bias; the softmax sum keeps p.
template <int SPLIT, bool PREFIX, int CDT>
__global__ __launch_bounds__(64 * SPLIT) __attribute__((amdgpu_waves_per_eu(4))) void k_decode_gqa(
    PoolView pv, BatchView bv, int layer, const void *q, const void *knew, const void *vnew, void *out, float qmul,
    int fused) {
    static_assert(CDT == DT_BF16 || CDT == DT_I8, "bf16 or int8 pages");
    constexpr bool I8 = CDT == DT_I8;
    constexpr int NL = I8 ? 1 : 2; // 1 KB loads per K or V tile of a page
    constexpr int DEPTH = 2;       // pages in flight ahead of the one being reduced
    __shared__ __attribute__((aligned(16))) uint16_t vt[SPLIT][kBlock][kPfLd]; // each wave's V tile, [key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t kt[SPLIT][kBlock][kPfLd]; // each wave's K tile, [key][dim]
    __shared__ float part[SPLIT][16][kPartStride];
    const int G = pv.H / pv.KVH;
    // XCD runs as in k_decode: in runs of 8 KVH groups, XCD x takes the kv heads of stream x of the run
    const int b = blockIdx.x, full = bv.n / 8 * 8;
    const int sidx = b < full * pv.KVH ? b / (8 * pv.KVH) * 8 + b % 8 : full + (b - full * pv.KVH) / pv.KVH;
    const int kvh = b < full * pv.KVH ? b % (8 * pv.KVH) / 8 : (b - full * pv.KVH) % pv.KVH;
    const char *rec = bv.recs + (size_t)sidx * bv.rec_stride;
    StreamRec R = *(const StreamRec *)rec;
    if (bv.wrow >= 0) window_row(R, bv.wrow);
    const int32_t *rec_pages = (const int32_t *)(rec + sizeof(StreamRec));
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, l16 = lane & 15;
    const int nb = R.nblk > w ? (R.nblk - w + SPLIT - 1) / SPLIT : 0; // this wave's pages

    // per-page metadata, lane j holding page w + j * SPLIT (as attend_core)
    int my_page = 0, my_ok = 0;
    uint32_t my_seen = 0;
    float my_sk = 0.f, my_sv = 0.f; // int8: the page's K and V scales
    const int pg_raw = w + lane * SPLIT < pv.mbps ? rec_pages[w + lane * SPLIT] : -1;
    if (lane < nb) {
        const int base = (w + lane * SPLIT) * kBlock;
        uint32_t seen = 0xffffu;
        if (R.mask_off >= 0) seen = (bv.masks[R.mask_off + (base >> 5)] >> (base & 16)) & 0xffffu;
        const int nvalid = R.span - base;
        if (nvalid < kBlock) seen &= (1u << max(nvalid, 0)) - 1u;
        const bool ok = pg_raw >= 0 && pg_raw < pv.NB;
        my_page = ok ? pg_raw : 0;
        my_ok = ok ? 1 : 0;
        my_seen = ok ? seen : 0;
    }

    // B operands of S^T: query head kvh G + l16, dims 32 kc + 8 g .. +7, rotated at R.pos (PREFIX:
    // and at R.pos_pre) with the packed bf16 RoPE rows and rounded to bf16 (zeros past G).  The
    // query and RoPE pieces are loaded here, unconditionally (head clamped), and rotated once the
    // first pages' loads are out (below), so that those wait for nothing but the page ids.
    uint4 qraw[2], qcs[2], pcs[2];
    {
        const int hq = kvh * G + min(l16, G - 1);
        const uint16_t *qp = (const uint16_t *)q + ((size_t)R.b * pv.H + hq) * kHeadDim;
        const uint32_t *cs = pv.rope16 + (size_t)R.pos * (kHeadDim / 2);
        const uint32_t *ps = pv.rope16 + (size_t)(PREFIX && R.prefix > 0 ? R.pos_pre : R.pos) * (kHeadDim / 2);
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            qraw[kc] = *(const uint4 *)(qp + 32 * kc + 8 * g);
            qcs[kc] = *(const uint4 *)(cs + 16 * kc + 4 * g);
            if constexpr (PREFIX) pcs[kc] = *(const uint4 *)(ps + 16 * kc + 4 * g);
        }
    }

    constexpr int ES = I8 ? 1 : 2; // bytes per cached value
    const char *kbase = (const char *)pv.pages + tile_index(pv, layer, 0, 0, kvh) * (kBlock * kHeadDim * ES);
    const char *vbase = (const char *)pv.pages + tile_index(pv, layer, 1, 0, kvh) * (kBlock * kHeadDim * ES);
    const size_t page_bytes = (size_t)pv.KVH * kBlock * kHeadDim * ES;
    // a page's K and V tiles, each in two streamed 1 KB loads (keys lane / 8 and 8 + lane / 8,
    // dims 8 (lane % 8) ..): every load covers whole 128-byte lines.  Loaded straight in the MFMA's
    // A layout, each load would take half of every line, and a streamed line is gone before the
    // other half is read (33 -> 36.6 us at 1 kv head); K therefore goes through an LDS tile too.
    // Measured against plain loads in A layout: 1 kv head 33.4 -> 28.8 us, 2: 56.5 -> 50.5, 4:
    // 101.5 -> 89 us.
    // int8: a tile is 1 KB, lane l's 16 bytes being key l / 4, dims 16 (l % 4) ..
    auto load = [&](uint4 (&kr)[NL], uint4 (&vr)[NL], int j) {
        const size_t pe = (size_t)__builtin_amdgcn_readlane(my_page, j) * page_bytes;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            kr[i] = ld_stream(kbase + pe + 1024 * i + 16 * lane);
            vr[i] = ld_stream(vbase + pe + 1024 * i + 16 * lane);
        }
    };
    // The first DEPTH pages' loads go out before the queries are rotated; the wave that owns the
    // write page loads them after its append instead when the write page is among them (as in
    // attend_core).
    uint4 kb[DEPTH + 1][NL], vb[DEPTH + 1][NL];
    const int wblk = R.write_slot >> 4, wj = wblk / SPLIT;
    const bool owner = fused && w == wblk % SPLIT && __builtin_amdgcn_readlane(my_ok, wj) != 0;
    const bool early = !owner || wj >= DEPTH;
    if (early) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(kb[d], vb[d], d);
    }
    // int8: the pages' scales, after those loads (a wait for the page ids before them would
    // otherwise wait for these too)
    if constexpr (I8) {
        if (lane < nb) {
            my_sk = pv.scales[tile_index(pv, layer, 0, my_page, kvh)];
            my_sv = pv.scales[tile_index(pv, layer, 1, my_page, kvh)];
        }
    }

    bf16x8_t qb[2], qpre[2];
    {
        const bool live = l16 < G;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            qb[kc] = as_bf16x8(live ? rotate8(qraw[kc], qcs[kc]) : make_uint4(0, 0, 0, 0));
            if constexpr (PREFIX) qpre[kc] = as_bf16x8(live ? rotate8(qraw[kc], pcs[kc]) : make_uint4(0, 0, 0, 0));
        }
    }
    // int8: the same queries as f16 (PREFIX: those at pos_pre too, with a power of two and a sum
    // of their own)
    f16x8_t qh[2], qhp[2];
    float qsum = 0.f, qpow = 1.f, qsump = 0.f, qpowp = 1.f;
    if constexpr (I8) {
        queries_f16(qb, qh, qsum, qpow);
        if constexpr (PREFIX) queries_f16(qpre, qhp, qsump, qpowp);
    }

    float m = -1e30f, lsum = 0.f; // running max (scaled, log2 units) and this lane's share of the sum
    f32x4_t o[4];                 // O^T: dims 16 dg + 4 g + r, query head l16
#pragma unroll
    for (int dg = 0; dg < 4; ++dg) o[dg] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto process = [&](const uint4 (&kr)[NL], const uint4 (&vr)[NL], int j) {
        const uint32_t seen = __builtin_amdgcn_readlane(my_seen, j);
        f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
        // K through the wave's LDS tile into A layout (key l16, dims 32 kc + 8 g); a wave's LDS
        // accesses complete in order, so no barrier
        bf16x8_t ka[2];
        f16x8_t kh[2];
        if constexpr (I8) {
            const uint32_t *u = (const uint32_t *)&kr[0];
            uint32_t hv[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t x = u[i] ^ 0x80808080u;
                hv[2 * i] = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);     // dims 4i, 4i + 1
                hv[2 * i + 1] = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u); // dims 4i + 2, 4i + 3
            }
            *(uint4 *)&kt[w][lane >> 2][16 * (lane & 3)] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
            *(uint4 *)&kt[w][lane >> 2][16 * (lane & 3) + 8] = make_uint4(hv[4], hv[5], hv[6], hv[7]);
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                kh[kc] = __builtin_bit_cast(f16x8_t, *(const uint4 *)&kt[w][l16][32 * kc + 8 * g]);
                s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[kc], qh[kc], s, 0, 0, 0);
            }
            const float sk = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(my_sk), j));
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = __builtin_fmaf(-1152.f, qsum, s[r]) * sk * qpow;
        } else {
            *(uint4 *)&kt[w][lane >> 3][8 * (lane & 7)] = kr[0];
            *(uint4 *)&kt[w][8 + (lane >> 3)][8 * (lane & 7)] = kr[1];
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                ka[kc] = as_bf16x8(*(const uint4 *)&kt[w][l16][32 * kc + 8 * g]);
                s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[kc], qb[kc], s, 0, 0, 0);
            }
        }
        if constexpr (PREFIX) {
            // a page holding prefix rows (uniform): those rows take the scores of the queries at pos_pre
            const int base = (w + j * SPLIT) * kBlock;
            if (base < R.prefix) {
                f32x4_t sp = f32x4_t{0.f, 0.f, 0.f, 0.f};
                if constexpr (I8) {
#pragma unroll
                    for (int kc = 0; kc < 2; ++kc) sp = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[kc], qhp[kc], sp, 0, 0, 0);
                    const float sk = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(my_sk), j));
#pragma unroll
                    for (int r = 0; r < 4; ++r) sp[r] = __builtin_fmaf(-1152.f, qsump, sp[r]) * sk * qpowp;
                } else {
#pragma unroll
                    for (int kc = 0; kc < 2; ++kc) sp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[kc], qpre[kc], sp, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (base + 4 * g + r < R.prefix) s[r] = sp[r];
            }
        }
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
        s16x4_t pt;
        if constexpr (I8) {
            // p sv in P^T; the V codes into this wave's LDS tile as bf16 (row lane / 4, dims
            // 16 (lane % 4) ..).  int8 codes are finite, so unseen rows (p = 0) need no zeroing.
            const float sv = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(my_sv), j));
            pt = __builtin_bit_cast(s16x4_t, make_uint2(pack_bf16(p[0] * sv, p[1] * sv), pack_bf16(p[2] * sv, p[3] * sv)));
            const uint32_t *u = (const uint32_t *)&vr[0];
            uint32_t bw[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                bw[2 * i] = pack_bf16((float)(int8_t)(u[i] & 0xffu), (float)(int8_t)((u[i] >> 8) & 0xffu));
                bw[2 * i + 1] = pack_bf16((float)(int8_t)((u[i] >> 16) & 0xffu), (float)(int8_t)(u[i] >> 24));
            }
            *(uint4 *)&vt[w][lane >> 2][16 * (lane & 3)] = make_uint4(bw[0], bw[1], bw[2], bw[3]);
            *(uint4 *)&vt[w][lane >> 2][16 * (lane & 3) + 8] = make_uint4(bw[4], bw[5], bw[6], bw[7]);
        } else {
            pt = __builtin_bit_cast(s16x4_t, make_uint2(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3])));
            // the page's V into this wave's LDS tile (rows lane / 8 and 8 + lane / 8, dims 8 (lane % 8) ..);
            // an unseen row weighs 0 but its bytes may be anything, so it goes in as zeros (0 * NaN would
            // be NaN)
            const uint32_t keep0 = ((seen >> (lane >> 3)) & 1u) ? ~0u : 0u;
            const uint32_t keep1 = ((seen >> (8 + (lane >> 3))) & 1u) ? ~0u : 0u;
            *(uint4 *)&vt[w][lane >> 3][8 * (lane & 7)] =
                make_uint4(vr[0].x & keep0, vr[0].y & keep0, vr[0].z & keep0, vr[0].w & keep0);
            *(uint4 *)&vt[w][8 + (lane >> 3)][8 * (lane & 7)] =
                make_uint4(vr[1].x & keep1, vr[1].y & keep1, vr[1].z & keep1, vr[1].w & keep1);
        }
#pragma unroll
        for (int dg = 0; dg < 4; ++dg) {
            // V^T: lane gets dim 16 dg + l16 of keys 4 g .. 4 g + 3
            const uint2 a = lds_read_tr16(&vt[w][4 * g + (l16 >> 2)][16 * dg + 4 * (l16 & 3)]);
            o[dg] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), pt, o[dg], 0, 0, 0);
        }
    };

    // complete_kv: the wave that owns the write page appends the kv head's new row, as in attend_core
    // an invalid write page id appends nothing, as in attend_core
    if (owner) {
        const int slot = R.write_slot;
        const size_t arow = (size_t)R.b * pv.KVH + kvh;
        const bool fresh = (R.flags & 1) ? (R.flags & 2) != 0 : ((slot & 15) == 0);
        append_row_wave<CDT, true>(pv, layer, __builtin_amdgcn_readlane(my_page, wj), slot & 15, kvh, R.key_pos,
                                   (const char *)knew + arow * kHeadDim * 2, (const char *)vnew + arow * kHeadDim * 2,
                                   fresh);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
        if constexpr (I8) {
            if (lane == wj) { // an int8 append may have raised this page's scales (and rewritten its codes)
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

hipError_t launch_decode_gqa(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                             const void *v, void *out, float scale, bool fused, hipStream_t stream,
                             const LaunchTiming &tm) {
    const float qmul = scale * 1.4426950408889634f;
    const dim3 grid(bv.n * pv.KVH);
    const int f = fused ? 1 : 0;
    if (pv.act_dt != DT_BF16 || (pv.cache_dt != DT_BF16 && pv.cache_dt != DT_I8)) return hipErrorInvalidValue;
#define XNP_GQA(S, PFX, C) XNP_LAUNCH((k_decode_gqa<S, PFX, C>), grid, dim3(64 * S), stream, tm, pv, bv, layer, q, k, v, out, qmul, f)
#define XNP_GQA_SPLIT(PFX, C)                                                                                       \
    switch (bv.split) {                                                                                            \
    case 1: XNP_GQA(1, PFX, C); break;                                                                             \
    case 2: XNP_GQA(2, PFX, C); break;                                                                             \
    case 4: XNP_GQA(4, PFX, C); break;                                                                             \
    case 8: XNP_GQA(8, PFX, C); break;                                                                             \
    default: return hipErrorInvalidValue;                                                                          \
    }
    if (pv.cache_dt == DT_I8 && bv.prefix) {
        XNP_GQA_SPLIT(true, DT_I8);
    } else if (pv.cache_dt == DT_I8) {
        XNP_GQA_SPLIT(false, DT_I8);
    } else if (bv.prefix) {
        XNP_GQA_SPLIT(true, DT_BF16);
    } else {
        XNP_GQA_SPLIT(false, DT_BF16);
    }
#undef XNP_GQA_SPLIT
#undef XNP_GQA
    return hipGetLastError();
}

hipError_t launch_prefill_mfma(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                               const void *v, void *out, float scale, bool fused, bool window, hipStream_t stream,
                               const LaunchTiming &tm) {
    if ((fused || window) && (!k || !v)) return hipErrorInvalidValue; // the step's own rows are read from k, v
    const float qmul = scale * 1.4426950408889634f;
    if (window)
        XNP_LAUNCH(k_prefill_window, dim3(bv.n * pv.H), dim3(64 * kWpWaves), stream, tm, pv, bv, layer, q, k, v, out,
                   qmul);
    else if (bv.kmax <= kPfFastKeys && fused)
        XNP_LAUNCH(k_prefill_fast<true>, dim3(bv.n * pv.H), dim3(64 * kPfWaves), stream, tm, pv, bv, layer, q, k, v,
                   out, qmul);
    else if (bv.kmax <= kPfFastKeys)
        XNP_LAUNCH(k_prefill_fast<false>, dim3(bv.n * pv.H), dim3(64 * kPfWaves), stream, tm, pv, bv, layer, q, k, v,
                   out, qmul);
    else
        XNP_LAUNCH(k_prefill_mfma<DT_BF16>, dim3(bv.n * pv.H), dim3(64 * kPfWaves), stream, tm, pv, bv, layer, q, k, v,
                   out, qmul, fused ? 1 : 0);
    return hipGetLastError();
}

// Prompt rows over int8 pages (bf16 activations), after k_append has written them: k_prefill_mfma
// reading every key from the pages, scores in f16 against the codes, values in bf16.
hipError_t launch_prefill_mfma_i8(const PoolView &pv, const BatchView &bv, int layer, const void *q, void *out,
                                  float scale, hipStream_t stream, const LaunchTiming &tm) {
    if (pv.cache_dt != DT_I8 || pv.act_dt != DT_BF16) return hipErrorInvalidValue;
    const float qmul = scale * 1.4426950408889634f;
    XNP_LAUNCH(k_prefill_mfma<DT_I8>, dim3(bv.n * pv.H), dim3(64 * kPfWaves), stream, tm, pv, bv, layer, q, nullptr,
               nullptr, out, qmul, 0);
    return hipGetLastError();
}

} // namespace xnp
