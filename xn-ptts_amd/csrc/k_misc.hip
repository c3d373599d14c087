// Small kernels of the paged flow-LM KV cache: block-table patches and plan pulls, the standalone
// append of t rows, shifting-ring eviction, page copies, raw row I/O and voice loading.
#include "kernels_common.h"

namespace xnp {

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

// ---------------------------------------------------------------------------------------------
// A window step's rows into the window after its attention (Mimi's chunk, bf16 and f32 pools):
// slot s takes the step's last row i with (p + i) % window == s; a row that a later row of the
// step overwrites is never written.  One work group per (stream, page of the window), one wave per
// kv head for the page's 16 slots.
//   bf16: lane l takes 16-byte unit l % 8 of the K and V rows of slots l / 8 and l / 8 + 8, and
//         each slot's row comes from the lane's own arithmetic: four 16-byte loads and the RoPE
//         pieces of its two keys, all issued unconditionally (a slot the step leaves alone loads
//         row 0, never stored), then rotate8 on the keys (the packed bf16 table the prefill
//         kernels rotate with: the same products and roundings as append_row_wave) and four
//         16-byte stores.
//   f32:  each lane one pair of dims (keys in lanes 0-31, values in 32-63, as append_row_wave),
//         every slot's loads first, then the rotations and stores.
// A loop of append_row_wave calls took 96 us per layer at 256 streams x 250 rows (each slot's loads
// waited for the previous slot's stores), and one slot per step of a scalar loop 68 us (two
// integer divisions per slot on the scalar unit).

template <int CDT, bool ABF>
__global__ __launch_bounds__(1024) void k_window_append(PoolView pv, BatchView bv, int layer, const void *k,
                                                        const void *v) {
    static_assert((CDT == DT_BF16 && ABF) || (CDT == DT_F32 && !ABF), "bf16 and f32 windows; int8 ones append row by row");
    const int b = blockIdx.x / pv.mbps, blk = blockIdx.x % pv.mbps;
    const StreamPlan P = bv.plans[b];
    const int W = P.window, t = bv.t, j = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (W <= 0 || kBlock * blk >= W) return;
    const int page = pv.tables[(size_t)P.sid * pv.mbps + blk];
    if (page < 0 || page >= pv.NB) return; // begin took this page; never index the pool without one
    const int rb = ((kBlock * blk - P.pos) % W + W) % W; // the first row of the step in the page's slot 0
    // the last row of the step in slot kBlock * blk + n, or -1
    auto last_row = [&](int n) {
        const int s = kBlock * blk + n, r = (rb + n) % W;
        return s < W && r < t ? (t <= W ? r : r + W * ((t - 1 - r) / W)) : -1;
    };
    if constexpr (CDT == DT_BF16) {
        const int unit = lane & 7;
        int row[2];
        uint4 kx[2], vx[2], cs[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            row[hf] = last_row((lane >> 3) + 8 * hf);
            const int i = max(row[hf], 0);
            const size_t arow = (((size_t)P.out_row * t + i) * pv.KVH + j) * kHeadDim + 8 * unit;
            kx[hf] = ld_stream((const uint16_t *)k + arow); // read once: streamed past the caches
            vx[hf] = ld_stream((const uint16_t *)v + arow);
            cs[hf] = *(const uint4 *)(pv.rope16 + (size_t)(P.key_pos + i) * (kHeadDim / 2) + 4 * unit);
        }
        uint16_t *kt = (uint16_t *)pv.pages + tile_index(pv, layer, 0, page, j) * (kBlock * kHeadDim);
        uint16_t *vt = (uint16_t *)pv.pages + tile_index(pv, layer, 1, page, j) * (kBlock * kHeadDim);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            if (row[hf] < 0) continue;
            const int o = ((lane >> 3) + 8 * hf) * kHeadDim + 8 * unit;
            *(uint4 *)(kt + o) = rotate8(kx[hf], cs[hf]);
            *(uint4 *)(vt + o) = vx[hf];
        }
    } else {
        const int kv = lane >> 5, pr = lane & 31;
        const char *src = (const char *)(kv ? v : k);
        int row[kBlock];
        float2 x[kBlock], cs[kBlock];
#pragma unroll
        for (int n = 0; n < kBlock; ++n) {
            row[n] = last_row(n);
            const int i = max(row[n], 0);
            x[n] = load_pair<false>(src + (((size_t)P.out_row * t + i) * pv.KVH + j) * kHeadDim * 4, pr);
            cs[n] = pv.rope[(size_t)(P.key_pos + i) * (pv.D / 2) + pr];
        }
        const size_t tile = tile_index(pv, layer, kv, page, j);
#pragma unroll
        for (int n = 0; n < kBlock; ++n) {
            if (row[n] < 0) continue;
            float2 y = x[n];
            if (kv == 0) { // the key rotated at its position (rope.rs:74-95), as append_row_wave rotates it
                const float a = y.x * cs[n].x, bb = y.y * cs[n].y, e = y.x * cs[n].y, f = y.y * cs[n].x;
                y.x = a - bb;
                y.y = e + f;
            }
            ((float2 *)pv.pages)[tile * (kBlock * kHeadDim / 2) + n * (kHeadDim / 2) + pr] = y;
        }
    }
}

hipError_t launch_window_append(const PoolView &pv, const BatchView &bv, int layer, const void *k, const void *v,
                                hipStream_t stream) {
    if (bv.n == 0) return hipSuccess;
    const dim3 grid(bv.n * pv.mbps), block(64 * pv.KVH);
    switch (pv.cache_dt * 2 + pv.act_dt) {
    case DT_F32 * 2 + DT_F32: hipLaunchKernelGGL((k_window_append<DT_F32, false>), grid, block, 0, stream, pv, bv, layer, k, v); break;
    case DT_BF16 * 2 + DT_BF16: hipLaunchKernelGGL((k_window_append<DT_BF16, true>), grid, block, 0, stream, pv, bv, layer, k, v); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
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

} // namespace xnp
