/*
 * xnp_kv.h -- C ABI of the MI355X (gfx950) flow-LM KV cache: a block-paged K/V store shared by
 * many concurrent utterance streams, with per-frame append + RoPE, ring slots and eviction,
 * single-query decode attention and causal prompt prefill, all as hand-written HIP kernels.
 *
 * It replaces, batched across streams, the op surface that the reference's
 * StreamingMultiheadAttention::forward (ptts/src/transformer.rs:183-251) drives through the
 * `xn` tensor crate, plus the state API above it:
 *   StreamingMHAState / init_state            transformer.rs:14-25, 169-180   xnp_stream_open
 *   complete_kv (slice_set / scatter_set)     transformer.rs:61-92, 216-218   xnp_append
 *   RotaryEmbedding::forward (rope_i)         rope.rs:37-95                   inside append/decode
 *   sdpa_decode                               transformer.rs:223, 230         xnp_decode
 *   matmul_t / softmax / matmul (t > 1)       transformer.rs:231-248          xnp_prefill
 *   RingSlots::decode_mask                    transformer.rs:42-52            per-stream seen bitmap
 *   start_ring / set_ring_slot / evict        transformer.rs:842-929          xnp_ring_*
 *   with_seq_budget                           transformer.rs:350-392          xnp_stream_fork
 *   advance                                   transformer.rs:337-344          xnp_stream_advance
 *   Session::step eviction policy             s2s.rs:318-333                  xnp_ring_slide
 *   plan::frame_budget / seq_budget           plan.rs:43-54                   xnp_frame_budget, ...
 *
 * Conventions (after ptts-ffi, ptts-ffi/src/lib.rs:56-77 and ptts-ffi/include/ptts.h:50-51):
 *   - Every call returns an xnp_status; XNP_OK is 0.  On failure, xnp_last_error() returns a
 *     thread-local message saying why, valid until the next failing call on that thread.
 *   - A refused call changes nothing (as evict does, transformer.rs:896-904).
 *   - The pool owns the device pages, the scales and the block tables.  The caller owns every
 *     q/k/v/out buffer (device memory) and the hipStream_t, passed as void*.  Calls that touch
 *     the device are asynchronous on that stream and never synchronize it.  All of one pool's
 *     device work must go to one stream (or the caller orders the streams).
 *   - One host thread at a time per pool.  No allocation happens between xnp_batch_begin and
 *     xnp_batch_end, so the per-layer calls of a batch can be captured in a hipGraph.
 *
 * Layouts (row-major, D = head_dim, H = num_heads, KVH = num_kv_heads):
 *   q, out          [n][t][H][D]     activation dtype (f32 or bf16)
 *   k, v            [n][t][KVH][D]   activation dtype; KV head j serves query heads
 *                                    j*H/KVH .. (j+1)*H/KVH-1 (transformer.rs:199-211)
 *   pages           [L][2][num_blocks][KVH][16][D] cache dtype; one (page, kv head) is a
 *                                    contiguous 16 x D tile.  The cache stores the KVH heads,
 *                                    not the H repeated ones the reference's cache holds
 *                                    (transformer.rs:199-211): the query heads of a group read
 *                                    the same tiles
 *   int8 scales     [L][2][num_blocks][KVH]        f32, one per (page, kv head), K and V apart
 */
#ifndef XNP_KV_H
#define XNP_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XNP_BLOCK 16 /* positions per page */

typedef enum xnp_dtype { XNP_F32 = 0, XNP_BF16 = 1, XNP_I8 = 2 } xnp_dtype;

typedef enum xnp_status {
    XNP_OK = 0,
    XNP_E_INVALID = 1,       /* bad argument, shape or dtype */
    XNP_E_STREAM = 2,        /* no such open stream */
    XNP_E_NO_ROOM = 3,       /* the stream's capacity is full (step_graph.rs:245-247) */
    XNP_E_OUT_OF_BLOCKS = 4, /* the pool has no free page left */
    XNP_E_RING = 5,          /* ring misuse: not a ring, slot range, t != 1, slot still holds a row
                                (transformer.rs:68-73, 855-867) */
    XNP_E_EVICT = 6,         /* evict refused (transformer.rs:885-901) */
    XNP_E_BUDGET = 7,        /* fork into a budget smaller than the filled prefix, or of a ring
                                (transformer.rs:356-364) */
    XNP_E_HEADS = 8,         /* heads do not divide (transformer.rs:703-711) */
    XNP_E_STATE = 9,         /* call out of order: batch open or not open, host-only pool */
    XNP_E_HIP = 10           /* the HIP runtime failed */
} xnp_status;

/* Ring eviction modes.  XNP_RING_SHIFT is the reference: evict rotates every kept key past the
 * prefix back by the number of evicted rows, in place (transformer.rs:905-926).  XNP_RING_ABSOLUTE
 * keeps each key at the rotation it was written with and rotates the query instead, once for
 * keys before the prefix and once for those past it; attention depends only on the difference
 * of the two positions, so outputs equal the shifting ring's up to rounding, and no key is ever
 * rewritten (int8 caches need it). */
typedef enum xnp_ring_mode { XNP_RING_SHIFT = 1, XNP_RING_ABSOLUTE = 2 } xnp_ring_mode;

#define XNP_POOL_HOST_ONLY 1 /* metadata only: no device memory; device calls return XNP_E_STATE */
#define XNP_MAX_ROPE_ROWS (1 << 24) /* positions a pool's RoPE tables may grow to */

typedef struct xnp_pool xnp_pool;

typedef struct xnp_pool_desc {
    int32_t num_layers;   /* L */
    int32_t num_heads;    /* H, heads of q, out and the cache */
    int32_t num_kv_heads; /* KVH, heads of the k and v handed to append; divides H */
    int32_t head_dim;     /* D; the kernels take 64 */
    int32_t num_blocks;   /* pages of XNP_BLOCK positions, shared by all streams and layers */
    int32_t max_streams;
    int32_t max_blocks_per_stream;
    int32_t cache_dtype;  /* xnp_dtype of the cached K/V */
    int32_t act_dtype;    /* xnp_dtype of q/k/v/out: XNP_F32 or XNP_BF16 */
    float max_period;     /* RoPE theta (rope.rs:47) */
    int32_t max_pos;      /* RoPE table rows to start with; a batch whose positions reach past the
                             table's rows grows it (doubling, up to XNP_MAX_ROPE_ROWS) */
    int32_t flags;        /* XNP_POOL_* */
    uint64_t page_seed;   /* 0: pages are handed out in order; else a Fisher-Yates shuffle of the
                             free list seeded with it (shuffled block tables) */
    int32_t device;       /* HIP device ordinal */
    int32_t decode_split; /* waves sharing one (stream, head) in decode: 1, 2, 4 or 8; a stream
                             holds at most 60 * decode_split pages; 0: the fewest that fit (one only
                             while a head's K and V tiles of a stream hold at most 128 KB), at least
                             two on the MFMA decode of grouped heads, raised per batch (up to 8)
                             while the batch has under 1024 waves (xnp_pool_stats.decode_waves) */
} xnp_pool_desc;

typedef struct xnp_stream_info {
    int32_t current_end; /* position of the next row (StreamingMHAState::current_end) */
    int32_t capacity;    /* positions the stream may hold (S_cap) */
    int32_t ring_mode;   /* 0 without a ring, else xnp_ring_mode */
    int32_t ring_write;  /* RingSlots::write */
    int32_t ring_filled; /* RingSlots::filled */
    int32_t ring_prefix; /* absolute ring: the prefix its evictions keep */
    int32_t ring_shift;  /* absolute ring: rows evicted so far */
    int32_t in_view;     /* valid ring slots */
    int32_t blocks;      /* pages the stream holds */
    int32_t shared;      /* of which shared with another stream */
    int32_t window;      /* a window cache (xnp_window_open): its rows, else 0 */
} xnp_stream_info;

typedef struct xnp_pool_stats {
    int32_t free_blocks;
    int32_t open_streams;
    int32_t batch_open; /* streams in the open batch, 0 if none */
    int32_t work_items; /* decode work groups of the open batch: one per (stream, head) */
    int64_t device_bytes;
    int32_t rope_rows;  /* rows of the RoPE tables now (positions 0 .. rope_rows - 1) */
    int32_t decode_waves; /* waves per decode work group of the open one-row batch, 0 if none */
} xnp_pool_stats;

/* ---- pool ------------------------------------------------------------------------------ */
xnp_status xnp_pool_create(const xnp_pool_desc *desc, xnp_pool **out);
xnp_status xnp_pool_destroy(xnp_pool *pool);
xnp_status xnp_pool_stats_get(const xnp_pool *pool, xnp_pool_stats *out);
/* Rows pos0 .. pos0+n-1 of the pool's RoPE table as [n][D/2] (cos, sin) pairs: the values the
 * kernels rotate with, built on the host as rope.rs:44-58 does (RotaryEmbedding::new).  Rows past
 * the table's current size (xnp_pool_stats.rope_rows) are refused.
 *
 * The tables grow in xnp_batch_begin when a step's positions reach their end (absolute rings and
 * window caches count positions on after their evictions, as the reference builds RoPE rows at any
 * offset, transformer.rs:794-803): the device tables are reallocated and the old ones freed, which
 * waits for the device.  Launches recorded before (a hipGraph of xnp_attend) read the old tables
 * and must be recorded again; xnp_flow_lm_step_graph does so itself.  Angles are pos * inv_freq in
 * f32, as the reference computes them, so large positions carry the same f32 rounding there. */
xnp_status xnp_pool_rope_rows(const xnp_pool *pool, int32_t pos0, int32_t n, float *cos_sin);

/* ---- streams ---------------------------------------------------------------------------- */
/* StreamingMultiheadAttention::init_state(1, capacity), transformer.rs:169-180.  Pages are taken
 * as rows arrive, not up front. */
xnp_status xnp_stream_open(xnp_pool *pool, int32_t capacity, int32_t *id);
xnp_status xnp_stream_close(xnp_pool *pool, int32_t id);
/* with_seq_budget, transformer.rs:350-392: a new stream of `capacity` positions holding src's
 * filled prefix.  Full pages are shared (no later write can reach them); the partial last page
 * is copied on hip_stream.  Refused for a ring and for capacity < current_end. */
xnp_status xnp_stream_fork(xnp_pool *pool, int32_t src, int32_t capacity, int32_t *id,
                           void *hip_stream);
xnp_status xnp_stream_info_get(const xnp_pool *pool, int32_t id, xnp_stream_info *out);
/* StreamingTransformerState::advance, transformer.rs:337-344: count n more filled positions,
 * taking pages for them; their contents are what xnp_write_rows puts there. */
xnp_status xnp_stream_advance(xnp_pool *pool, int32_t id, int32_t n);
/* The stream's page ids, logical block order, -1 where none is held (at most `cap` entries). */
xnp_status xnp_stream_blocks(const xnp_pool *pool, int32_t id, int32_t *pages, int32_t cap,
                             int32_t *count);
/* The seen map attention uses at the next step: valid[slot] for slot < capacity. */
xnp_status xnp_ring_valid(const xnp_pool *pool, int32_t id, uint8_t *valid, int32_t cap);

/* Raw rows [slot0, slot0 + n) of one layer, kv 0 = keys, 1 = values: rows [n][KVH][D] in the
 * cache dtype (device memory); for int8 also scales [nb][KVH] for the nb pages the rows touch.
 * No RoPE, no quantization: a voice cache loaded as is, or a cache read back. */
xnp_status xnp_write_rows(xnp_pool *pool, int32_t id, int32_t layer, int32_t kv, int32_t slot0,
                          int32_t n, const void *rows, const float *scales, void *hip_stream);
xnp_status xnp_read_rows(const xnp_pool *pool, int32_t id, int32_t layer, int32_t kv,
                         int32_t slot0, int32_t n, void *rows, float *scales, void *hip_stream);
/* voice_from_kv_cache, ptts-wasm/src/lib.rs:291-325: a voice stored as the flow LM's KV cache
 * (`transformer.layers.{i}.self_attn/cache`, f32 [2, 1, n, H, D]: keys, already rotated, then
 * values) becomes rows [0, n) of one layer of stream id, converted to the cache dtype on the
 * device: bf16 rounded to nearest even; int8 with one scale per (page, head), amax / 127 over the
 * page's rows, codes rint(x / s) clamped to +-127.  kv is device memory, [2][n][H][D] f32.  The
 * stream must hold exactly n rows and no ring: open it, xnp_stream_advance(n), then load every
 * layer.  Forks of it (xnp_stream_fork, with_seq_budget) then share its full pages. */
xnp_status xnp_stream_load_kv(xnp_pool *pool, int32_t id, int32_t layer, const float *kv, int32_t n,
                              void *hip_stream);

/* ---- Mimi's window cache (transformer.rs:257-318,398-468) -------------------------------- */
/* KvCache::new(context): a stream whose steps attend the last `window` positions, the causal
 * window of Mimi's attention (delta < context, transformer.rs:764-781), keys rotated at their
 * absolute position (KvCache::absolute_offset).  Its rows place themselves, row p in slot
 * p % window over the row leaving the window, so no eviction call is needed.  A step takes any
 * number of rows t, more than the window included (Mimi's encoder over a whole voice clip,
 * tts_model.rs:509-515; its decoder takes 2 a frame): with t > 1 every stream of the batch must be
 * a window cache, and xnp_attend is the only per-layer call such a batch takes.  On a bf16 pool a
 * step of more than 4 rows runs every row's windowed attention in one MFMA launch, then writes the
 * last min(t, window) rows into their slots; shorter steps, and every step on f32 and int8 pools,
 * run row by row.  xnp_stream_fork clones a window as it is, every page copied
 * (transformer.rs:348-354). */
xnp_status xnp_window_open(xnp_pool *pool, int32_t window, int32_t *id);

/* ---- ring (transformer.rs:842-929) ------------------------------------------------------ */
/* start_ring: valid[s] = s < current_end; write = filled = current_end.  `prefix` is used by
 * XNP_RING_ABSOLUTE only.  Shared pages are copied first (on hip_stream). */
xnp_status xnp_ring_start(xnp_pool *pool, int32_t id, int32_t mode, int32_t prefix,
                          void *hip_stream);
xnp_status xnp_ring_set_slot(xnp_pool *pool, int32_t id, int32_t slot);
/* evict: all slots checked before any change; count > current_end, a slot below the prefix or
 * holding no row is refused.  XNP_RING_SHIFT rotates the kept keys on hip_stream. */
xnp_status xnp_ring_evict(xnp_pool *pool, int32_t id, int32_t prefix, const int32_t *slots,
                          int32_t count, void *hip_stream);
/* Session::step's policy, s2s.rs:324-333: when `window` slots past the prefix are in view, evict
 * the oldest `drop`, then set the write slot to prefix + step % span.  s2s runs it with
 * span = window = context and drop = context / 3; a sliding window uses drop = 1 and
 * span = window + XNP_BLOCK, so a page is never shared by the oldest and the newest rows. */
xnp_status xnp_ring_slide(xnp_pool *pool, int32_t id, int32_t prefix, int32_t span,
                          int32_t window, int32_t drop, int64_t step, void *hip_stream);

/* xnp_ring_slide over n streams, stream i at step steps[i]: one call per batched step.  Stops at
 * the first stream refused (its index in *failed, -1 if none); the streams before it have slid. */
xnp_status xnp_ring_slide_batch(xnp_pool *pool, const int32_t *ids, int32_t n, int32_t prefix,
                                int32_t span, int32_t window, int32_t drop, const int64_t *steps,
                                int32_t *failed, void *hip_stream);

/* ---- a batched step ---------------------------------------------------------------------- */
/* Open a step over streams ids[0..n), t new rows each (t > 1: prompt prefill, no ring).  Checks
 * every stream (capacity, ring slot) and takes the pages the new rows need, all or nothing;
 * uploads the step's plan (positions, block tables, masks, decode work list) on hip_stream. */
xnp_status xnp_batch_begin(xnp_pool *pool, const int32_t *ids, int32_t n, int32_t t,
                           void *hip_stream);
/* complete_kv for one layer: rotate k at each row's position, write k and v into the pages
 * (int8: quantize), at current_end (+ row) or the ring's write slot. */
xnp_status xnp_append(xnp_pool *pool, int32_t layer, const void *k, const void *v,
                      void *hip_stream);
/* sdpa_decode for one layer (t == 1): rotate q, attend over the stream's cache including the
 * appended row, under the ring's mask; out = softmax(q K^T * scale) V. */
xnp_status xnp_decode(xnp_pool *pool, int32_t layer, const void *q, void *out, float scale,
                      void *hip_stream);
/* causal prompt attention for one layer (t > 1, transformer.rs:231-248): row i of a stream sees
 * positions 0 .. current_end + i. */
xnp_status xnp_prefill(xnp_pool *pool, int32_t layer, const void *q, void *out, float scale,
                       void *hip_stream);
/* xnp_append then xnp_decode (t == 1, one fused kernel) or xnp_prefill (t > 1). */
xnp_status xnp_attend(xnp_pool *pool, int32_t layer, const void *q, const void *k,
                      const void *v, void *out, float scale, void *hip_stream);
/* Close the step: current_end += t; a ring marks the written slot valid. */
xnp_status xnp_batch_end(xnp_pool *pool);
/* Drop the step: give back the pages it took; nothing else changes. */
xnp_status xnp_batch_abort(xnp_pool *pool);

/* Consistency check (no counterpart in the reference): apply the pending block-table changes,
 * read the device tables back (synchronizes hip_stream) and count the entries of open streams
 * that differ from the host's page map.  0 is the only right answer. */
xnp_status xnp_pool_check_tables(xnp_pool *pool, int32_t *mismatches, void *hip_stream);

/* Test hook (no counterpart in the reference): on a host-only pool, set stream id's page map
 * entry for logical block blk to `page` as given, without the allocator's bookkeeping, so that tests
 * can plant the broken maps xnp_batch_begin refuses.  Device pools refuse it (XNP_E_STATE).  Put the
 * entry back before closing the stream. */
xnp_status xnp_debug_set_block(xnp_pool *pool, int32_t id, int32_t blk, int32_t page);

/* Measurement hook (no counterpart in the reference): the pool's next decode or prefill launch
 * records HIP events `start` and `stop` (hipEvent_t, created by the caller) as the kernel starts
 * and ends (hipExtLaunchKernel), so that the kernel alone is timed.  Either may be null: a start
 * recorded by one launch and a stop by a later one time the launches between them.  Applies to
 * one launch. */
xnp_status xnp_pool_time_next(xnp_pool *pool, void *start_event, void *stop_event);

/* ---- the rest of a flow-LM layer (transformer.rs:591-634) --------------------------------- */
/* The layer around the attention: norm1 -> in_proj -> attention -> out_proj -> residual, norm2 ->
 * linear1 -> gelu -> linear2 -> residual (StreamingTransformerLayer::forward, transformer.rs:591-634),
 * for every row of an open batch at once.  Activations are bf16; the projections are linears
 * without bias (Q::linear_load, transformer.rs:163-164, 549-550) whose weights are int8 with one
 * f32 scale per output channel, multiplied on MFMA.  All pointers are device memory. */
typedef enum xnp_gelu { XNP_GELU_ERF = 0, XNP_GELU_TANH = 1 } xnp_gelu; /* Gelu, transformer.rs:615-618 */

typedef struct xnp_layer_weights {
    int32_t d_model;      /* a multiple of 512, at most 2048 */
    int32_t ff;           /* dim_feedforward, a multiple of 64 */
    int32_t gelu;         /* xnp_gelu */
    const int8_t *wqkv;   /* in_proj  [(H + 2 KVH) D][d_model]: q rows, then k, then v */
    const float *sqkv;    /*          [(H + 2 KVH) D] */
    const int8_t *wout;   /* out_proj [d_model][H D] */
    const float *sout;
    const int8_t *w1;     /* linear1  [ff][d_model] */
    const float *s1;
    const int8_t *w2;     /* linear2  [d_model][ff] */
    const float *s2;
    const float *ln1_w, *ln1_b, *ln2_w, *ln2_b; /* norm1, norm2 [d_model], eps 1e-5 */
    const float *ls1, *ls2;                     /* layer_scale_1/2 [d_model] (layer_scale.rs), or NULL */
} xnp_layer_weights;

/* Device bytes of scratch xnp_layer_step needs for `rows` rows (n streams x t rows of a batch). */
xnp_status xnp_layer_workspace(const xnp_pool *pool, int32_t rows, int32_t d_model, int32_t ff,
                               uint64_t *bytes);
/* One layer for the open batch: x [n][t][d_model] bf16 (the residual stream, updated in place),
 * appending each row's k and v into the pages and attending as xnp_attend does (decode for
 * t == 1, prompt prefill for t > 1).  `workspace` holds at least xnp_layer_workspace bytes; the
 * call allocates nothing. */
xnp_status xnp_layer_step(xnp_pool *pool, int32_t layer, const xnp_layer_weights *w, void *x,
                          void *workspace, uint64_t workspace_bytes, void *hip_stream);

/* xnp_layer_step without a workspace argument (no counterpart in the reference): for callers that
 * cannot allocate device memory -- code under hipGraph capture, tight serving loops, hosts that
 * forbid hipMalloc.  The scratch is a fixed array of XNP_STATIC_SCRATCH_BYTES inside the library,
 * one per device, held until the process ends; a step needing more (xnp_layer_workspace) is refused
 * with XNP_E_INVALID.  The call allocates nothing, host or device.  Every call on one device shares
 * that device's array, so calls must not overlap: a call is refused with XNP_E_STATE, running
 * nothing, while another call is issuing its launches (another host thread, any pool or stream) or
 * while the last call's work on another HIP stream may still be running (it waits for nothing).
 * Calls ordered on one stream from one thread, or synchronized between, always proceed; a call being
 * captured into a hipGraph is not checked against others, and the caller orders the graph's launches
 * with the other users of the array.  Nothing in the array needs to start at zero (every byte a step
 * reads it wrote first in the same call), so the previous call's contents do not matter. */
#define XNP_STATIC_SCRATCH_BYTES (24u << 20) /* the 2048-row step of a 512-wide, FF 2048 layer takes 18 MiB */
xnp_status xnp_layer_step_static(xnp_pool *pool, int32_t layer, const xnp_layer_weights *w, void *x,
                                 void *hip_stream);

/* The pieces, on caller buffers (the current HIP device):
 * LayerNorm of rows of `dim` bf16 values (dim a multiple of 512, at most 2048). */
xnp_status xnp_layer_norm(const void *x, int32_t rows, int32_t dim, const float *w, const float *b,
                          float eps, void *out, void *hip_stream);
/* y = epilogue(s[j] * sum_k x[m][k] w[j][k]) for x [rows][k] bf16, w [n][k] int8, s [n] f32; n a
 * multiple of 64, k of 64.  The product is rounded to bf16, then XNP_EPI_STORE writes it to
 * y [rows][n], XNP_EPI_GELU_ERF / _TANH write gelu of it, XNP_EPI_RESIDUAL adds it (times ls[j],
 * rounded, when ls is not NULL) into y and rounds. */
typedef enum xnp_epilogue {
    XNP_EPI_STORE = 0, XNP_EPI_GELU_ERF = 1, XNP_EPI_GELU_TANH = 2, XNP_EPI_RESIDUAL = 3,
    /* the flow net's (xnp_flow_linear_q8 only) */
    XNP_EPI_SILU = 4, XNP_EPI_SILU_ADD = 5, XNP_EPI_GATED = 6, XNP_EPI_AXPY_F32 = 7, XNP_EPI_STORE_F32 = 8,
    XNP_EPI_ADD_F32 = 9
} xnp_epilogue;
xnp_status xnp_linear_q8(const void *x, int32_t rows, int32_t k, const int8_t *w, const float *s,
                         int32_t n, int32_t epilogue, void *y, const float *ls, void *hip_stream);
/* The flow net's pieces (SimpleMLPAdaLN, mlp.rs:4-11,113-163), as the q8 flow LM runs them:
 * y = bf16(s[j] * sum_k x[m][k] w[j][k] (+ bias[j])) for x [rows][k] bf16 (x_f32: f32, rounded to
 * bf16 as it is read; XNP_EPI_STORE and _ADD_F32 only), w [n][k] int8, any n, k a multiple of 16,
 * then XNP_EPI_STORE y; _GELU_* gelu(y); _RESIDUAL y += y; _SILU silu(y); _SILU_ADD silu(bf16(y +
 * aux[j])) (aux f32 [n], the time embedding); _GATED y[m][j] = bf16(y[m][j] + bf16(aux[m][j] *
 * y)) (aux bf16, the AdaLN gate); _AXPY_F32 y[m][j] = bf16(bf16(aux[m][j]) + bf16(y * alpha)) (aux
 * and y f32: the solver step); _STORE_F32 y (f32); _ADD_F32 y[m][j] = bf16(bf16(aux[m][j]) + y)
 * (aux f32, ld_aux 0 for one row for every m: the flow LM's conditions, flow_lm.rs:304-307).  Every
 * result rounded to bf16 once; y rows of stride ldy, aux rows of stride ld_aux. */
xnp_status xnp_flow_linear_q8(const void *x, int32_t x_f32, int32_t rows, int32_t k, const int8_t *w,
                              const float *s, const float *bias, int32_t n, int32_t epilogue, void *y,
                              int32_t ldy, const void *aux, int32_t ld_aux, float alpha, void *hip_stream);
/* LayerNorm of bf16 rows (dim a multiple of 512; w, b both NULL for no affine) rounded to bf16,
 * then when shift is given the AdaLN modulation in bf16 steps, bf16(bf16(y * bf16(scale + 1)) +
 * shift), shift and scale bf16 rows of stride ld_mod (a multiple of 8). */
xnp_status xnp_layer_norm_mod(const void *x, int32_t rows, int32_t dim, const float *w, const float *b,
                              float eps, const void *shift, const void *scale, int32_t ld_mod, void *out,
                              void *hip_stream);
/* Per-row int8 weights on the host: s[r] = max |w[r][.]| / 127, q = rint(w / s) clamped to
 * +-127 (an all-zero row gets s = 0, q = 0). */
xnp_status xnp_quantize_rows(const float *w, int32_t rows, int32_t cols, int8_t *q, float *scales);

/* ---- the flow LM around the transformer (flow_lm.rs, mlp.rs, conditioners.rs) ----------- */
/* FlowLM's text prompt and frame steps (TTSModel::prompt_text and generate_step_parts,
 * tts_model.rs:297-378) on f32 kernels, for batches of an f32 pool's streams: the LUT gather,
 * input_linear, the transformer (norms, linears, GELU, residuals around the pool's attention),
 * out_norm, z_proj, the EOS head and the flow net (SimpleMLPAdaLN, mlp.rs:159-238).  FlowLMConfig
 * (flow_lm.rs:114-146) whole: z_dim, attn_dim, num_kv_heads, the flow types and time norms, and the
 * conditions broadcast-added to the step input (flow_lm.rs:304-307).  (FlowLM's transformer has no
 * layer scale: flow_lm.rs:239-249 loads it with None; xnp_layer_step takes one for other callers.)
 * Text sinks (tts_model.rs:299-301) stay with the caller: the sink row is one more prompt row. */
typedef enum xnp_time_norm { XNP_TIME_RMS = 0, XNP_TIME_RMS_VAR = 1 } xnp_time_norm; /* mlp.rs:17-28 */
/* FlowType (flow_lm.rs:372-381): the LSD solver over lsd_steps, or one flow-net call without time
 * conditions (Drifting: the latent is its output; Pointwise: noise plus it). */
typedef enum xnp_flow_type { XNP_FLOW_LSD = 0, XNP_FLOW_DRIFTING = 1, XNP_FLOW_POINTWISE = 2 } xnp_flow_type;
/* XNP_FLOW_F32: f32 weights and activations on an f32 pool (one stream a frame, the reference's
 * case).  XNP_FLOW_Q8: every linear's weights quantized at create as xnp_quantize_rows does
 * (biases, norms f32), bf16 activations on a bf16 pool, the projections on MFMA (many streams a
 * frame); each operation rounds its bf16 output once, as a bf16 tensor op does. */
typedef enum xnp_flow_precision { XNP_FLOW_F32 = 0, XNP_FLOW_Q8 = 1 } xnp_flow_precision;

typedef struct xnp_flow_lm_desc {
    int32_t d_model, num_heads, num_layers, ff; /* the transformer; the pool must match it */
    int32_t ldim, n_bins, flow_dim, flow_depth; /* latent width, LUT rows - 1, flow net width, blocks */
    int32_t lsd_steps;                          /* lsd_decode_steps */
    int32_t gelu;                               /* xnp_gelu */
    int32_t time_norm;                          /* xnp_time_norm */
    int32_t max_rows;                           /* rows one call may hold: streams x prompt tokens */
    int32_t z_dim;                              /* 0: no z_proj; else its width (flow_lm.rs:239-240) */
    int32_t flow_type;                          /* xnp_flow_type */
    int32_t precision;                          /* xnp_flow_precision */
    int32_t num_kv_heads;                       /* 0: num_heads; else grouped-query kv heads (flow_lm.rs:143-145, 253) */
    int32_t attn_dim;                           /* 0: d_model; else the attention's query and output width,
                                                   num_heads x the pool's head_dim (flow_lm.rs:139-141, 252) */
} xnp_flow_lm_desc;

typedef struct xnp_flow_lm xnp_flow_lm;

/* Floats of the weight blob: every tensor f32, row-major [out][in] for linears, in this order (zd:
 * z_dim when set, else d; a: attn_dim when set, else d; kv: a / num_heads x num_kv_heads) --
 * conditioner.embed [n_bins+1][d]; input_linear [d][ldim]; bos_emb [ldim];
 * per layer: norm1 w, b [d]; in_proj [a + 2 kv][d] (q rows, then k, then v); out_proj [d][a];
 *   norm2 w, b [d]; linear1 [ff][d]; linear2 [d][ff];
 * out_norm w, b [d]; z_proj [z][d] when z_dim; out_eos w [1][zd], b [1];
 * per time embedder (2, XNP_FLOW_LSD only): freqs [128]; mlp.0 w [F][256], b [F]; mlp.2 w [F][F],
 *   b [F]; alpha [F];
 * cond_embed w [F][zd], b [F]; input_proj w [F][ldim], b [F];
 * per res block: in_ln w, b [F]; mlp.0 w [F][F], b [F]; mlp.2 w [F][F], b [F];
 *   adaLN_modulation.1 w [3F][F], b [3F];
 * final_layer: adaLN_modulation.1 w [2F][F], b [2F]; linear w [ldim][F], b [ldim]. */
xnp_status xnp_flow_lm_weights_size(const xnp_flow_lm_desc *desc, int64_t *nfloats);
/* Upload the weights (host memory; quantized here for XNP_FLOW_Q8) for a pool whose layers and
 * heads match, with f32 cache and activations (XNP_FLOW_F32) or bf16 ones (XNP_FLOW_Q8: d_model
 * and flow_dim multiples of 512, every linear's input width a multiple of 16); the time embeddings
 * of the solver steps are computed once here, as lsd_time_embeddings does at load
 * (flow_lm.rs:82-95). */
xnp_status xnp_flow_lm_create(xnp_pool *pool, const xnp_flow_lm_desc *desc, const float *weights,
                              int64_t nfloats, xnp_flow_lm **out);
xnp_status xnp_flow_lm_destroy(xnp_flow_lm *lm);
/* prompt_text for streams ids[0..n), tokens [n][t] (host int32): their LUT rows through the
 * transformer, committed.  Token ids past the table are refused (conditioners.rs:248-256). */
xnp_status xnp_flow_lm_prompt_text(xnp_flow_lm *lm, const int32_t *ids, int32_t n,
                                   const int32_t *tokens, int32_t t, void *hip_stream);
/* The model's summed conditions (FlowLM::condition_providers, flow_lm.rs:218-222, the sum of
 * conditioners.rs:57-63): cond [dim] host f32, dim == d_model, or NULL for none.  Broadcast-added to
 * every frame's input_linear output (flow_lm.rs:304-307) whose step passes no conditions of its own.
 * Copied to the device before the call returns; a recorded frame graph is recorded again. */
xnp_status xnp_flow_lm_set_condition(xnp_flow_lm *lm, const float *cond, int32_t dim);
/* One frame for streams ids[0..n): latent_in [n][ldim] (NULL: bos_emb for every row), conditions
 * [n][d_model] (each stream's FlowLMState::conditions, flow_lm.rs:200, 304-307, as the s2s session
 * sets per frame, s2s.rs:334; NULL: the model's condition when set, else none), noise [n][ldim] (the
 * solver's start; zeros at temperature 0), latent_out [n][ldim], eos_logit [n], all f32 device
 * memory.  The condition row is added to input_linear's output (f32: y + c; q8: bf16(bf16(c) + y)).
 * The streams advance by one position. */
xnp_status xnp_flow_lm_step(xnp_flow_lm *lm, const int32_t *ids, int32_t n, const float *latent_in,
                            const float *conditions, const float *noise, float *latent_out, float *eos_logit,
                            void *hip_stream);
/* xnp_flow_lm_step with the frame's launches recorded once in a hipGraph and replayed, as
 * StepGraph records one step and replays it per frame (step_graph.rs:111-122, 234-267).  The plan
 * (positions, pages) is uploaded eagerly each call and read by the recorded kernels from the pool's
 * device buffers, as DeviceStep keeps the position on the device (transformer.rs:111-140).  A new
 * recording is made when n, a buffer or the stream changes, or when the batch's plan picks other
 * kernels than the recorded ones (a stream of the batch took up a ring prefix, another split, a
 * regrown RoPE table, another condition source); hip_stream must not be the null stream.  Results
 * are those of xnp_flow_lm_step. */
xnp_status xnp_flow_lm_step_graph(xnp_flow_lm *lm, const int32_t *ids, int32_t n, const float *latent_in,
                                  const float *conditions, const float *noise, float *latent_out,
                                  float *eos_logit, void *hip_stream);

/* ---- budgets (plan.rs:25, 43-54) --------------------------------------------------------- */
int32_t xnp_frame_budget(int32_t num_tokens, double frame_rate);
int32_t xnp_seq_budget(int32_t num_tokens, int32_t frame_budget);

const char *xnp_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
