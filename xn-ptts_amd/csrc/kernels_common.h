// Device helpers shared by the HIP kernel files of the paged flow-LM KV cache (gfx950, wave64).
//
// Bit-exactness contract with the CPU restatement: the library is built with
// -ffp-contract=off, RoPE rotates with host-computed cos/sin tables, bf16 rounding is
// round-to-nearest-even on the f32 bits, int8 quantization is rint(y / s) clamped to +-127 with
// IEEE division.  The attention arithmetic (dots, softmax, weighted sums) is f32 in an order of
// its own and is checked to a tolerance, not bit for bit.
#pragma once

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

// The sum of x over the wave's 64 lanes, in every lane, without the LDS pipe: two DPP quad
// permutes (lanes i ^ 1, i ^ 2), the half-row and row mirrors (i <-> 7 - i in each 8, i <-> 15 - i
// in each 16), then gfx950's row swaps (i <-> i ^ 16, i <-> i ^ 32).  Each step adds a lane whose
// partial covers a disjoint set of lanes, so every lane ends with the whole sum; the order of the
// additions differs from an xor butterfly's (ds_bpermute shuffles, about 100 cycles each).
template <int CTRL> __device__ __forceinline__ float dpp_move(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
// The sum of x over each aligned group of N lanes (N = 1, 2, 4, 8 or 16), in every lane of the
// group: the first N's steps of wave_sum.
template <int N> __device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "groups within a 16-lane row");
    if constexpr (N >= 2) x += dpp_move<0xB1>(x);
    if constexpr (N >= 4) x += dpp_move<0x4E>(x);
    if constexpr (N >= 8) x += dpp_move<0x141>(x);
    if constexpr (N >= 16) x += dpp_move<0x140>(x);
    return x;
}
// The value x holds in lane (this lane) ^ O: a DPP row rotation for O = 8 (by 8 within a 16-lane
// row), gfx950's row swaps for 16 and 32 (each returns both halves; this lane takes its partner's),
// an LDS-pipe shuffle otherwise.
template <int O> __device__ __forceinline__ float xor_lane(float x) {
    if constexpr (O == 8) {
        return dpp_move<0x128>(x); // row_ror:8
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
    } else if constexpr (O == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
    } else {
        return __shfl_xor(x, O);
    }
}
// max(a, b) for finite or -inf values: the median of a, b and the largest finite float, one
// v_med3_f32.  fmaxf quiets each operand the compiler cannot prove quiet first (the results of
// lane swaps, selects, loads), one more instruction each.  Callers pass attention scores (finite,
// or -inf where masked) and their running maxima.
__device__ __forceinline__ float fmax_fin(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, 3.40282347e38f); }

// The max (sum) of x over lanes l and l ^ O, O = 16 or 32, in both: gfx950's row swaps return the
// partner's value beside the lane's own, so the two results combine without a lane-index select.
template <int O> __device__ __forceinline__ float swap_max(float x) {
    static_assert(O == 16 || O == 32, "row swaps");
    const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                           : __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmax_fin(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <int O> __device__ __forceinline__ float swap_sum(float x) {
    static_assert(O == 16 || O == 32, "row swaps");
    const auto r = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                           : __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The max of x over each 32-lane half of the wave, in every lane of the half: DPP steps within each
// 16-lane row (quad permutes, the half-row and row mirrors), then the row swap with lane l ^ 16.
// IEEE maxima throughout (fmaxf, not fmax_fin): it takes the int8 rows' amax, whose scale and codes
// stay the oracle's for any input, infinities included.
__device__ __forceinline__ float half_max(float x) {
    x = fmaxf(x, dpp_move<0xB1>(x));  // quad_perm [1, 0, 3, 2]
    x = fmaxf(x, dpp_move<0x4E>(x));  // quad_perm [2, 3, 0, 1]
    x = fmaxf(x, dpp_move<0x141>(x)); // row_half_mirror
    x = fmaxf(x, dpp_move<0x140>(x)); // row_mirror
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_move<0xB1>(x);  // quad_perm [1, 0, 3, 2]
    x += dpp_move<0x4E>(x);  // quad_perm [2, 3, 0, 1]
    x += dpp_move<0x141>(x); // row_half_mirror
    x += dpp_move<0x140>(x); // row_mirror
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// 16 bytes with the non-temporal hint.  A decode launch reads each K/V tile once: streamed, the
// tiles stop displacing what the launch does reuse in L2 and the memory-side cache (records,
// tables, queries).  Measured on attend_core's page loads: bf16 decode at 1024 streams 192 ->
// 171 us, int8 window 104.4 -> 95.0 us; on the prefill's key/value staging 32.8 -> 32.2 us.  Only
// where one load instruction covers whole 128-byte lines (attend_core: 1 KB contiguous per wave):
// the prefill's query loads, two instructions of 64 bytes a row, took the launch 25.4 -> 30.1 us.
__device__ __forceinline__ uint4 ld_stream(const void *p) {
    typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
    const u32x4_nt a = __builtin_nontemporal_load((const u32x4_nt *)p);
    return make_uint4(a.x, a.y, a.z, a.w);
}

// Stores with the non-temporal hint, for rows that nothing in the launch reads back: they go out to
// memory as they are written, while the launch still computes, instead of staying dirty in L2 until
// the launch's end writes L2 back.  Each store instruction should cover whole 128-byte lines (8
// lanes x 16 bytes per row): hinted 8-byte pieces go out as partial lines (the prefill's output
// written that way read 1.3x its bytes in WRITE_SIZE).  Measured: the prefill's page and output
// stores at 64 streams x 256 positions 29.4 -> 26.5-26.9 us per launch (32 x 512 on k_prefill_mfma
// 50.8 -> 42.4-43.3 us with whole-line output stores); the projections' and LayerNorm's outputs in
// the 2048-stream layer step 5.23 -> 5.16 ms per step.  The decode's own stores (2 bytes a lane for
// its output, 4 for the append) stay plain: hinted, they cost 1.5 us of 171 at 1024 streams and
// 1.3 of 28.6 at one kv head.
__device__ __forceinline__ void st_stream(void *p, const uint4 &v) {
    typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(u32x4_nt{v.x, v.y, v.z, v.w}, (u32x4_nt *)p);
}
__device__ __forceinline__ void st_stream(void *p, const uint2 &v) {
    typedef unsigned u32x2_nt __attribute__((ext_vector_type(2)));
    __builtin_nontemporal_store(u32x2_nt{v.x, v.y}, (u32x2_nt *)p);
}

// Rotate 8 bf16 values (4 pairs) with 4 packed bf16 (cos, sin) pairs, rounded to bf16 (rope.rs:74-95):
// x0 c - x1 s and x0 s + x1 c, each product rounded to f32, then the sum, then bf16.  A product of
// two bf16 values has at most 16 significant bits, so it is exact in f32 (outside the subnormal
// range, below 2^-126), and an fma taking one product unrounded gives the same two roundings with
// one instruction fewer per output.  (v_dot2_f32_bf16 does not: its sums differ by an f32 ulp now
// and then, either way, and a zero sum comes out +0 where the separate products give -0.)
__device__ __forceinline__ uint4 rotate8(const uint4 &x, const uint4 &cs) {
    const uint32_t *u = (const uint32_t *)&x, *r = (const uint32_t *)&cs;
    uint32_t o4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float x0 = bf16_value(u[e] & 0xffffu), x1 = bf16_value(u[e] >> 16);
        const float c = bf16_value(r[e] & 0xffffu), s = bf16_value(r[e] >> 16);
        o4[e] = pack_bf16(__builtin_fmaf(x0, c, -(x1 * s)), __builtin_fmaf(x0, s, x1 * c));
    }
    return make_uint4(o4[0], o4[1], o4[2], o4[3]);
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
        const float amax = half_max(fmaxf(fabsf(x.x), fabsf(x.y))); // over this row's 32 lanes
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

// The dispatcher hands work group b of a grid to XCD b % 8, and each XCD has its own L2.  A tile
// grid numbered row-major would give every XCD every eighth tile, so each XCD would read nearly
// all of the tiles' shared operand rows.  xcd_tile renumbers group b of G so that XCD x takes one
// contiguous run of about G / 8 tiles (XCDs below G % 8 one more), which share their rows.
__device__ __forceinline__ int xcd_tile(int b, int G) {
    const int q = G >> 3, r = G & 7, x = b & 7, i = b >> 3;
    return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
}

// ---------------------------------------------------------------------------------------------
// direct-to-LDS loads with hand-placed waits (the window prefill's ring, the q8 GEMM's ring)

// The lane index, recomputed where it is used: the address pieces of a chunk's loads would
// otherwise be kept in registers across the whole loop, which the loop's own work needs.
__device__ __forceinline__ int lane_here(int lane) {
    int x;
    asm volatile("v_mov_b32 %0, %1" : "=v"(x) : "v"(lane));
    return x;
}

// A work-group barrier for LDS alone: __syncthreads also waits for every global access of the wave
// in flight, which would drain the chunk loads issued ahead.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// A 1 KB load of the wave straight into LDS: lane l's 16 bytes at src go to lds + 16 l
// (global_load_lds_dwordx4, LDS base in M0).  Written out here because the compiler makes every LDS
// access after its own form of this load wait for all loads in flight (vmcnt(0)), which would drain
// the chunks issued ahead; the caller's own `s_waitcnt vmcnt(n)` is the wait these loads get.  Every
// wait the compiler places for its own loads stays correct, as vector-memory accesses complete in
// the order issued (they can only wait longer).
// The LDS byte address of a pointer into a __shared__ array.  The cast of a generic pointer carries
// a null check that needs the pointer's high half (the LDS aperture), a register pair kept live
// from the prologue; taken once of an array's first element, it folds to the array's address, and
// dma16_at then takes uniform offsets from it.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}
__device__ __forceinline__ void dma16_at(const void *src, uint32_t lds) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base) : "memory", "m0");
}
__device__ __forceinline__ void dma16(const void *src, void *lds) { dma16_at(src, lds_addr(lds)); }
// dma16_at with the non-temporal hint, for data read once (a step's own rows)
__device__ __forceinline__ void dma16_at_nt(const void *src, uint32_t lds) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(base) : "memory", "m0");
}
// The same with 4 bytes a lane: lane l's word at src goes to lds + 4 l (global_load_lds_dword).
__device__ __forceinline__ void dma4_at(const void *src, uint32_t lds) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(base) : "memory", "m0");
}

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

// A query taken as f16 (int8 pages with bf16 activations) is first scaled by a power of two 2^-x
// that puts the row's largest |value| into [2^14, 2^15): every bf16 value then fits f16 (whose
// largest is 65504, while bf16 reaches 3.4e38) with the largest at full precision.  Scaling by a
// power of two is exact, the products of f16 values are exact in f32, and f32 sums round alike at
// any power-of-two scale, so scores taken with the scaled query and multiplied by 2^x are those of
// the unscaled query wherever that one fits f16.  The row's DPL values of this lane are reduced
// over the N lanes XOR-distant by O0, 2 O0, ..; returns x.
template <int DPL, int O0, int N>
__device__ __forceinline__ int f16_fit_exponent(const float (&x)[DPL]) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) m = fmaxf(m, fabsf(x[i]));
#pragma unroll
    for (int k = 0, o = O0; k < N; ++k, o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    const int ex = (int)((__float_as_uint(m) >> 23) & 0xffu) - 127; // floor(log2 m) for a normal m
    return m > 0.f ? min(max(ex - 14, -100), 100) : 0;
}
// 2^x for |x| <= 126
__device__ __forceinline__ float pow2i(int x) { return __uint_as_float((uint32_t)(127 + x) << 23); }

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

// Row r of a window step run row by row, from the step's record (row 0's, every page of the window
// listed): position p + r in slot (p + r) % window; it sees slots [0, min(p + r + 1, window)) (the
// slot it takes held position p + r - window, which left its window), and an int8 page starts
// afresh when no other slot of it holds a row yet.
__device__ __forceinline__ void window_row(StreamRec &R, int r) {
    const int W = R.window, p = R.pos + r;
    R.b += r;
    R.pos = R.pos_pre = R.key_pos = p;
    R.write_slot = p % W;
    R.span = min(p + 1, W);
    R.nblk = (R.span + kBlock - 1) / kBlock;
    const int filled = min(p, W), b0 = R.write_slot & ~(kBlock - 1), e = min(b0 + kBlock, filled);
    const int others = max(0, e - b0) - (R.write_slot < e ? 1 : 0);
    R.flags = 1 | (others > 0 ? 0 : 2);
}

// Launchers one kernel file provides to another.
hipError_t launch_decode_gqa(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                             const void *v, void *out, float scale, bool fused, hipStream_t stream,
                             const LaunchTiming &tm);
// window: the windowed attention of a Mimi chunk over a window cache (no rows written)
hipError_t launch_prefill_mfma(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                               const void *v, void *out, float scale, bool fused, bool window, hipStream_t stream,
                               const LaunchTiming &tm);
// prompt rows over int8 pages (bf16 activations) on MFMA, after the append wrote them
hipError_t launch_prefill_mfma_i8(const PoolView &pv, const BatchView &bv, int layer, const void *q, void *out,
                                  float scale, hipStream_t stream, const LaunchTiming &tm);

} // namespace xnp
