// Structures shared by the host library (pool.cpp, flow_lm.cpp) and the HIP kernel files (k_*.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/xnp_kv.h"

namespace xnp {

constexpr int kBlock = 16;   // positions per page
constexpr int kHeadDim = 64; // the kernels' head dimension
constexpr int kMaxHeads = 16;
constexpr int kPartStride = 68; // floats per wave partial: acc[64], m, l, pad
constexpr int kLaneBlocks = 60;  // pages one wave's lanes index: 64 minus the prefetch overrun
constexpr int32_t kMaxRopeRows = XNP_MAX_ROPE_ROWS; // positions the RoPE tables may grow to

enum : int32_t { DT_F32 = 0, DT_BF16 = 1, DT_I8 = 2 };
enum : int32_t { RING_NONE = 0, RING_SHIFT = 1, RING_ABSOLUTE = 2 };

// Where one pool's device memory lives and how it is strided.
struct PoolView {
    void *pages;          // [L][2][NB][H][16][D], cache dtype
    float *scales;        // [L][2][NB][H] (int8 only)
    int32_t *tables;      // [max_streams][mbps] page ids, -1 where none
    const float2 *rope;   // [max_pos][D/2] (cos, sin), rounded to the activation dtype; max_pos: its rows now
    const uint32_t *rope16; // bf16 activations only: the same table as packed bf16 (cos | sin << 16)
    int32_t L, H, KVH, D, NB, mbps, max_pos;
    int32_t cache_dt, act_dt;
};

// One stream of an open batch.  64 bytes.
struct StreamPlan {
    int32_t sid;        // stream id: row of the block tables
    int32_t pos;        // RoPE position of query row 0 for keys at or past `prefix`
    int32_t pos_pre;    // RoPE position of query row 0 for keys before `prefix`
    int32_t prefix;     // 0 unless an absolute ring keeps a prefix
    int32_t write_slot; // slot of new row 0 (rows go to write_slot + i)
    int32_t key_pos;    // RoPE position of new key row 0
    int32_t span;       // decode attends slots [0, span) (t == 1)
    int32_t mask_off;   // word offset of the seen bitmap in masks[], -1: every slot is seen
    int32_t ring;       // 1 on a ring: int8 freshness comes from `fresh`, not from the slot
    int32_t fresh;      // ring + int8: the write slot's page holds no other live row
    int32_t out_row;    // row of q/k/v/out (= index in the batch)
    int32_t window;     // a window cache: its slots (rows at slot position % window), else 0
    int32_t wbase;      // a window cache: the slot of its oldest held row
    int32_t pad[3];
};

// One stream of a decode batch, as its work groups read it: 64 bytes, followed in the record by
// the page ids of its nblk blocks.
struct StreamRec {
    int32_t b;          // batch row: row of q/k/v/out
    int32_t nblk;       // blocks [0, nblk) the decode reads
    int32_t pos, pos_pre, prefix; // as StreamPlan
    int32_t write_slot, key_pos, span, mask_off;
    int32_t flags;      // 1: ring (int8 freshness from bit 2), 2: the write page starts afresh
    int32_t window;     // a window step's base record: the window's slots (row r derives its own)
    int32_t pad[5];
};

// Everything a batch's kernels read, in one device buffer.
struct BatchView {
    const StreamPlan *plans;
    const char *recs; // stream records in decode order (longest first), rec_stride bytes apart
    const uint32_t *masks;
    int32_t n, t, rec_stride;
    int32_t split;  // waves per (stream, head) work group
    int32_t prefix; // 1 if some stream of the batch is an absolute ring keeping a prefix
    int32_t wrow;   // a window step run row by row: the row this launch attends (-1 otherwise)
    int32_t kmax;   // a prompt step (t > 1): the most key slots a stream of it attends, write_slot + t
};

// A table entry to set before the batch's kernels run.
struct TablePatch {
    int32_t sid, blk, page, pad;
};

// One row to rotate in place on eviction (XNP_RING_SHIFT).
struct EvictRow {
    int32_t sid, slot;
};

// Events a launch records around its kernel (both null: none).
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
};

// The library's static scratch (k_scratch.hip), one array per device: xnp_layer_step_static's
// workspace.  static_scratch_init takes the array's address on `device`, which must be current;
// pool creation calls it.  static_scratch returns that address (null before the init).
constexpr uint64_t kStaticScratchBytes = XNP_STATIC_SCRATCH_BYTES;
hipError_t static_scratch_init(int device);
void *static_scratch(int device);
// Calls on one device's array must not overlap.  claim: kBusy while another call holds the array
// (between its claim and its release: its launches are being issued, from any host thread) or
// while a call on another stream may still be running on the device; otherwise the array is held
// and kOk (the last call on `stream` itself is ordered before this one by the stream; a call being
// captured runs only when its graph is launched, in the graph's order).  release: after the call's
// launches, on every path once claimed, let go of the array and record its completion on `stream`
// (nothing recorded when capturing).
enum class ScratchClaim { kOk, kBusy, kError };
ScratchClaim static_scratch_claim(int device, hipStream_t stream, bool capturing);
hipError_t static_scratch_release(int device, hipStream_t stream, bool capturing);

// What the open batch's kernel launches are chosen by beyond its size and the caller's buffers: the
// decode template (a ring prefix in the batch), the waves per work group, and the RoPE tables the
// kernels read.  A recording of the launches (a hipGraph) replays right only for a batch with the
// same key.
struct BatchLaunchKey {
    int32_t prefix = -1, split = 0;
    const void *rope = nullptr, *rope16 = nullptr;
    bool operator==(const BatchLaunchKey &o) const {
        return prefix == o.prefix && split == o.split && rope == o.rope && rope16 == o.rope16;
    }
};
BatchLaunchKey batch_launch_key(const xnp_pool *p);

// The pool's description and the library's error reporting (pool.cpp), for the other host files.
xnp_status pool_fail(xnp_status code, const char *fmt, ...);
const xnp_pool_desc *pool_desc(const xnp_pool *p);
bool pool_host_only(const xnp_pool *p);

// Launchers (k_*.hip).  All asynchronous on `stream`; return the launch status.
hipError_t launch_patch_tables(const PoolView &pv, const TablePatch *patches, int n,
                               hipStream_t stream);
// Copies `bytes` (rounded up to 16) from src, a device view of pinned host memory, to dst, and
// applies np table patches read from host memory too: a batch plan's upload in one launch.
hipError_t launch_pull_plan(const PoolView &pv, const void *src, void *dst, size_t bytes, const TablePatch *patches,
                            int np, hipStream_t stream);
hipError_t launch_append(const PoolView &pv, const BatchView &bv, int layer, const void *k,
                         const void *v, hipStream_t stream);
// Query heads one decode work group covers (all of one kv head), for a pool that stores grouped
// heads in a bf16 or f32 cache: the whole group on MFMA for bf16 with 2 to 16 of them and no ring
// prefix in the batch; else 4 when 4 divide the group and no prefix, 2 when 2 do, else 1 (always
// 1 for int8).
int decode_heads_per_group(const PoolView &pv, bool prefix);
// The fewest waves per work group a one-row decode of this pool and batch takes by default: 2 on
// MFMA (grouped heads), else 1.
int decode_min_split(const PoolView &pv, bool prefix);
hipError_t launch_decode(const PoolView &pv, const BatchView &bv, int layer, const void *q,
                         const void *k, const void *v, void *out, float scale, bool fused,
                         hipStream_t stream, const LaunchTiming &timing);
// Prompt attention over the pages.  fused: the prompt's K/V rows come from k and v and the
// kernel writes them into the pages itself (only where prefill_fuses_append holds); otherwise
// launch_append has written them already and k, v are unused.
bool prefill_fuses_append(const PoolView &pv);
hipError_t launch_prefill(const PoolView &pv, const BatchView &bv, int layer, const void *q,
                          const void *k, const void *v, void *out, float scale, bool fused,
                          hipStream_t stream, const LaunchTiming &timing);
// A window step of t rows on a bf16 pool (Mimi's chunk, transformer.rs:764-781): the windowed
// attention of every row on MFMA over the held rows (pages) and the step's own (k, v), then the
// append of the last min(t, window) rows into their slots, (p + i) % window.
hipError_t launch_window_prefill(const PoolView &pv, const BatchView &bv, int layer, const void *q, const void *k,
                                 const void *v, void *out, float scale, hipStream_t stream, const LaunchTiming &timing);
hipError_t launch_window_append(const PoolView &pv, const BatchView &bv, int layer, const void *k, const void *v,
                                hipStream_t stream);
hipError_t launch_evict_rotate(const PoolView &pv, const EvictRow *rows, int n,
                               const float *cos_row, const float *sin_row, hipStream_t stream);
hipError_t launch_copy_page(const PoolView &pv, int src_page, int dst_page, hipStream_t stream);
// Epilogues of the q8 projection GEMM (launch_gemm_q8).
// Epilogues of the q8 projection (launch_gemm_q8), y = bf16(s[n] * acc (+ bias[n])):
//   kStore out = y; kGelu* out = bf16(gelu(y)); kResidual out = bf16(out + y (* ls[n], rounded));
//   kSilu out = bf16(silu(y)); kSiluAddVec z = bf16(y + aux[n]) (f32), out = bf16(silu(z));
//   kGated out = bf16(out + bf16(aux[m][n] * y)) (aux bf16, the AdaLN gate); kAxpyF32 out (f32) =
//   bf16(bf16(aux[m][n]) + bf16(y * alpha)) (aux f32); kStoreF32 out (f32) = y; kAddF32 out (bf16) =
//   bf16(bf16(aux[m][n]) + y) (aux f32, ld_aux 0 for one row: a condition broadcast-added).
enum : int32_t {
    kStore = 0, kGeluErf = 1, kGeluTanh = 2, kResidual = 3, kSilu = 4, kSiluAddVec = 5, kGated = 6, kAxpyF32 = 7,
    kStoreF32 = 8, kAddF32 = 9
};

// Where a q8 projection writes.  kStore: columns [col0[j], col0[j+1]) go to out[j] (row stride
// ld[j], column n - col0[j]), j < nseg; the others: out[0] with stride ld[0] (kResidual reads and
// writes it, with the layer scale ls when not null).
struct GemmOut {
    void *out[3] = {nullptr, nullptr, nullptr};
    int32_t ld[3] = {0, 0, 0};
    int32_t col0[3] = {0, 0, 0};
    int32_t nseg = 1;
    const float *ls = nullptr;
    const float *bias = nullptr; // per output channel, added before the rounding to bf16
    const void *aux = nullptr;   // the epilogue's operand (see above)
    int32_t ld_aux = 0;
    float alpha = 1.f;
    bool a_f32 = false;          // A holds f32, rounded to bf16 as it is staged (kStore and kAddF32 only)
};

hipError_t launch_layer_norm(const void *x, int rows, int dim, const float *w, const float *b, float eps, void *out,
                             hipStream_t stream);
// LayerNorm of bf16 rows (w, b: the affine, both null for none), rounded, then when shift is
// given the AdaLN modulation of mlp.rs:4-11 in bf16 steps: bf16(bf16(y * bf16(scale + 1)) + shift),
// shift and scale bf16 rows of stride ld_mod.
hipError_t launch_layer_norm_mod(const void *x, int rows, int dim, const float *w, const float *b, float eps,
                                 const void *shift, const void *scale, int ld_mod, void *out, hipStream_t stream);
hipError_t launch_gemm_q8(const void *A, int M, int K, const int8_t *W, const float *s, int N, int epi,
                          const GemmOut &go, hipStream_t stream);
// Epilogues of the f32 linear (launch_linear_f32), y = x W^T + b:
//   kLinStore out = y; kLinGelu* out = gelu(y); kLinSilu out = silu(y); kLinSiluAddVec
//   out = silu(y + aux[n]); kLinResidual out += y; kLinGated out += aux[m][n] * y; kLinAxpy
//   out = aux[m][n] + alpha * y (aux may be out itself).
enum : int32_t {
    kLinStore = 0, kLinGeluErf = 1, kLinGeluTanh = 2, kLinSilu = 3, kLinSiluAddVec = 4, kLinResidual = 5,
    kLinGated = 6, kLinAxpy = 7
};

// Where an f32 linear writes: columns [col0[j], col0[j+1]) to out[j] (row stride ld[j]).
struct LinOut {
    float *out[3] = {nullptr, nullptr, nullptr};
    int32_t ld[3] = {0, 0, 0};
    int32_t col0[3] = {0, 0, 0};
    int32_t nseg = 1;
    const float *aux = nullptr;
    int32_t ld_aux = 0;
    float alpha = 1.f;
};

// A LayerNorm over each row of x applied as the linear reads it (mean, then the centred sum of
// squares, rstd = 1 / sqrt(var + eps)): eps; the
// affine w, b (both null: none); the AdaLN modulation y * (1 + scale) + shift with per-row
// shift/scale of row stride ld_mod (shift null: none).
struct LinNorm {
    const float *w = nullptr, *b = nullptr;
    float eps = 1e-5f;
    const float *shift = nullptr, *scale = nullptr;
    int32_t ld_mod = 0;
};

hipError_t launch_linear_f32(const float *x, int ldx, int M, int K, const float *W, const float *b, int N, int epi,
                             const LinOut &lo, hipStream_t stream, const LinNorm *ln = nullptr);
hipError_t launch_embed_f32(const float *table, const int32_t *ids, int rows, int dim, float *out, hipStream_t stream);
// out[r] = table[ids[r]] for rows of row_bytes bytes (a multiple of 16)
hipError_t launch_gather_rows(const void *table, const int32_t *ids, int rows, int row_bytes, void *out,
                              hipStream_t stream);
float bf16_round_host(float x); // to nearest even, NaN kept quiet: the kernels' rounding on the host
hipError_t launch_load_kv(const PoolView &pv, int sid, int layer, const float *kv, int n, hipStream_t stream);
hipError_t launch_rows_io(const PoolView &pv, int sid, int layer, int kv, int slot0, int n,
                          void *rows, float *scales, bool write, hipStream_t stream);

} // namespace xnp
