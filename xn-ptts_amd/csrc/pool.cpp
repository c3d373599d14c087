// Host side of the paged flow-LM KV cache: the page allocator, per-stream state (current_end,
// ring slots), batch plans and the C ABI of include/xnp_kv.h.  Kernels are in k_*.hip.
#include "../../include/xnp_kv.h"
#include "xnp_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <utility>
#include <vector>

using namespace xnp;

namespace {

thread_local std::string g_err;

xnp_status fail(xnp_status code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

xnp_status hip_fail(hipError_t e, const char *what) {
    return fail(XNP_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                                                                        \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess) return hip_fail(e_, what);                                           \
    } while (0)

uint64_t splitmix64(uint64_t &s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// RotaryEmbedding::at_positions (rope.rs:37-63) for one position: cos/sin of pos * inv_freq[i],
// inv_freq[i] = 1 / theta^(i / half), each rounded to the activation dtype (rope.rs:55-56).
void rope_row(int D, float theta, float pos, bool act_bf16, float2 *out) {
    const int half = D / 2;
    for (int i = 0; i < half; i++) {
        float inv_freq = 1.0f / powf(theta, (float)i / (float)half);
        float angle = pos * inv_freq;
        float c = cosf(angle), s = sinf(angle);
        if (act_bf16) {
            c = bf16_round_host(c);
            s = bf16_round_host(s);
        }
        out[i] = make_float2(c, s);
    }
}

struct Stream {
    bool open = false;
    int32_t capacity = 0;
    int32_t current_end = 0;
    std::vector<int32_t> blocks; // logical block -> page, -1 where none
    int32_t ring = RING_NONE, write = 0, filled = 0, prefix = 0, shift = 0;
    std::vector<uint8_t> valid;
    int32_t nvalid = 0; // valid slots of the ring
    // Mimi's KvCache (transformer.rs:257-318): an absolute ring of `window` slots that places its
    // rows itself, row p in slot p % window, each overwriting the row that just left the window
    int32_t window = 0;
};

// Window steps of more rows than this on a bf16 pool run as one windowed prefill on MFMA plus an
// append; shorter ones (Mimi's decoder takes 2 a frame), and every window step on f32 and int8 pools,
// run row by row through the decode kernel.
constexpr int32_t kWindowRowByRow = 4;

// The window's blocks a step of t rows from position p writes: those of the slots the last
// min(t, window) rows land in, (p + i) % window (an earlier row's slot is taken again by a later one).
template <class F> void window_blocks(const Stream &s, int64_t p, int32_t t, F &&each) {
    const int32_t nb = (s.window + kBlock - 1) / kBlock;
    std::vector<uint8_t> hit(nb, 0);
    for (int64_t r = std::max<int64_t>(0, t - s.window); r < t; r++) {
        const int32_t b = (int32_t)((p + r) % s.window) / kBlock;
        if (!hit[b]) {
            hit[b] = 1;
            each(b);
        }
    }
}

// A pinned host buffer an upload is composed in; reused once its copy has completed.
struct Staging {
    char *host = nullptr; // pinned
    char *dev = nullptr;  // the same bytes as the device sees them
    hipEvent_t done = nullptr;
    bool pending = false;
};

constexpr int kStaging = 4;

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

} // namespace

struct xnp_pool {
    xnp_pool_desc d{};
    bool host_only = false;
    int split = 4;
    int esz = 2;
    int mask_words = 0; // per stream
    int rec_stride = 0;

    // device
    void *pages = nullptr;
    float *scales = nullptr;
    int32_t *tables = nullptr;
    float2 *rope = nullptr;
    uint32_t *rope16 = nullptr; // bf16 pools: the table as packed bf16 pairs
    char *dbatch = nullptr; // batch plan upload
    char *daux = nullptr;   // table patches and eviction rows
    size_t batch_bytes = 0, aux_bytes = 0;
    Staging stage[kStaging];
    int stage_next = 0;
    LaunchTiming timing; // events the next decode or prefill launch records, then cleared
    int64_t device_bytes = 0;

    // host
    std::vector<float2> rope_host; // [rope_rows][D/2]
    int32_t rope_rows = 0;         // rows of the RoPE tables: desc.max_pos at first, grown as positions reach it
    std::vector<Stream> streams;
    std::vector<int32_t> free_ids;
    std::vector<int32_t> free_pages;
    std::vector<int32_t> refcnt;
    std::vector<TablePatch> patches;
    std::vector<uint32_t> patch_mark; // [max_streams * mbps]: generation an entry was last coalesced in
    uint32_t patch_gen = 0;
    std::vector<int32_t> shadow_tables; // host-only pools: what the device tables would hold
    std::vector<int32_t> writer;        // [num_blocks] during xnp_batch_begin's check: the stream writing each page, -1 none

    struct Batch {
        bool open = false;
        int n = 0, t = 0;
        hipStream_t stream = nullptr;
        std::vector<int32_t> ids;
        std::vector<std::pair<int32_t, int32_t>> taken; // (stream, block) pages taken by begin
        BatchView bv{};
        bool wsteps = false; // a step of several rows on window caches: one decode per row
    } batch;

    PoolView view() const {
        PoolView pv;
        pv.pages = pages;
        pv.scales = scales;
        pv.tables = tables;
        pv.rope = rope;
        pv.rope16 = rope16;
        pv.L = d.num_layers;
        pv.H = d.num_heads;
        pv.KVH = d.num_kv_heads;
        pv.D = d.head_dim;
        pv.NB = d.num_blocks;
        pv.mbps = d.max_blocks_per_stream;
        pv.max_pos = rope_rows;
        pv.cache_dt = d.cache_dtype;
        pv.act_dt = d.act_dtype;
        return pv;
    }

    Stream *get(int32_t id) {
        if (id < 0 || id >= (int32_t)streams.size() || !streams[id].open) return nullptr;
        return &streams[id];
    }
    const Stream *get(int32_t id) const {
        if (id < 0 || id >= (int32_t)streams.size() || !streams[id].open) return nullptr;
        return &streams[id];
    }

    int32_t take_page(int32_t sid, int32_t blk) {
        int32_t p = free_pages.back();
        free_pages.pop_back();
        refcnt[p] = 1;
        streams[sid].blocks[blk] = p;
        patches.push_back({sid, blk, p, 0});
        return p;
    }

    // Holders of page p; 0 for no page (-1) or an id outside the pool (only xnp_debug_set_block,
    // on a host-only pool, can plant one): no path indexes the page counts with such an id.
    int32_t refs(int32_t p) const { return p >= 0 && p < d.num_blocks ? refcnt[p] : 0; }

    void drop_page(int32_t sid, int32_t blk) {
        int32_t p = streams[sid].blocks[blk];
        if (p < 0) return;
        // an id outside the pool (only xnp_debug_set_block can plant one) is cleared without
        // touching the page counts
        if (p < d.num_blocks && --refcnt[p] == 0) free_pages.push_back(p);
        streams[sid].blocks[blk] = -1;
        patches.push_back({sid, blk, -1, 0});
    }

    // A staging buffer free for composing an upload.
    xnp_status stage_acquire(Staging **out) {
        Staging &s = stage[stage_next];
        stage_next = (stage_next + 1) % kStaging;
        if (s.pending) {
            HIP_TRY(hipEventSynchronize(s.done), "waiting for a staging buffer");
            s.pending = false;
        }
        *out = &s;
        return XNP_OK;
    }

    // A batch plan (bytes at the start of s) into dst, with np table patches staged at o_patch:
    // one kernel reads both from the pinned buffer.
    xnp_status pull(Staging *s, char *dst, size_t bytes, size_t o_patch, int np, hipStream_t stream) {
        HIP_TRY(launch_pull_plan(view(), s->dev, dst, bytes, (const TablePatch *)(s->dev + o_patch), np, stream),
                "plan pull");
        HIP_TRY(hipEventRecord(s->done, stream), "recording a plan pull");
        s->pending = true;
        return XNP_OK;
    }

    xnp_status upload(Staging *s, char *dst, size_t bytes, hipStream_t stream) {
        HIP_TRY(hipMemcpyAsync(dst, s->host, bytes, hipMemcpyHostToDevice, stream), "plan upload");
        HIP_TRY(hipEventRecord(s->done, stream), "recording an upload");
        s->pending = true;
        return XNP_OK;
    }

    // One patch per touched table entry, carrying the entry's value now.  The patch kernel applies
    // its list in no particular order, so an entry touched twice since the last flush (a stream
    // closed and reopened, a page dropped and taken again) must appear once, or a stale -1 could
    // land after the live page id.
    void coalesce_patches() {
        if (++patch_gen == 0) {
            std::fill(patch_mark.begin(), patch_mark.end(), 0u);
            patch_gen = 1;
        }
        std::vector<TablePatch> out;
        out.reserve(patches.size());
        for (auto it = patches.rbegin(); it != patches.rend(); ++it) {
            const size_t key = (size_t)it->sid * d.max_blocks_per_stream + it->blk;
            if (patch_mark[key] == patch_gen) continue;
            patch_mark[key] = patch_gen;
            const Stream &s = streams[it->sid];
            const int32_t v = s.open && it->blk < (int32_t)s.blocks.size() ? s.blocks[it->blk] : -1;
            out.push_back({it->sid, it->blk, v, 0});
        }
        patches.swap(out);
    }

    // Apply the queued block-table changes on the device before anything reads the tables.
    xnp_status flush_patches(hipStream_t stream) {
        coalesce_patches();
        if (host_only) {
            // the host-only pool keeps a shadow of the device tables, patched in reverse order:
            // any order the kernel could take gives the same tables only if entries are unique
            for (auto it = patches.rbegin(); it != patches.rend(); ++it)
                shadow_tables[(size_t)it->sid * d.max_blocks_per_stream + it->blk] = it->page;
            patches.clear();
            return XNP_OK;
        }
        size_t cap = aux_bytes / sizeof(TablePatch);
        size_t done = 0;
        while (done < patches.size()) {
            size_t n = std::min(cap, patches.size() - done);
            Staging *s;
            if (xnp_status st = stage_acquire(&s)) return st;
            std::memcpy(s->host, patches.data() + done, n * sizeof(TablePatch));
            if (xnp_status st = upload(s, daux, n * sizeof(TablePatch), stream)) return st;
            HIP_TRY(launch_patch_tables(view(), (const TablePatch *)daux, (int)n, stream), "table patch");
            done += n;
        }
        patches.clear();
        return XNP_OK;
    }

    // The device RoPE tables from rope_host: the f32 (cos, sin) pairs and, for bf16 activations, the
    // same values packed as bf16 pairs (they are bf16 already: no rounding here).
    xnp_status upload_rope(float2 *dst, uint32_t *dst16) {
        HIP_TRY(hipMemcpy(dst, rope_host.data(), sizeof(float2) * rope_host.size(), hipMemcpyHostToDevice),
                "rope table upload");
        if (dst16) {
            std::vector<uint32_t> packed(rope_host.size());
            for (size_t i = 0; i < packed.size(); i++) {
                uint32_t c, sn;
                std::memcpy(&c, &rope_host[i].x, 4);
                std::memcpy(&sn, &rope_host[i].y, 4);
                packed[i] = (c >> 16) | (sn & 0xffff0000u);
            }
            HIP_TRY(hipMemcpy(dst16, packed.data(), sizeof(uint32_t) * packed.size(), hipMemcpyHostToDevice),
                    "bf16 rope table upload");
        }
        return XNP_OK;
    }

    // Positions below `need` get RoPE rows.  The reference builds its rows at any offset on every
    // call (transformer.rs:794-803), and an absolute ring or a window cache keeps counting positions
    // after its evictions, so the tables grow (doubling) when a batch reaches their end: new rows are
    // built on the host as at creation, the device tables reallocated and the old ones freed (which
    // waits for the device).  Recordings of earlier launches read the old tables: the pool's launch
    // key changes (batch_launch_key), so they are recorded again.
    xnp_status grow_rope(int64_t need) {
        if (need <= rope_rows) return XNP_OK;
        if (need > kMaxRopeRows)
            return fail(XNP_E_INVALID, "position %lld is beyond the largest RoPE table (%d rows)", (long long)need - 1,
                        kMaxRopeRows);
        const int64_t rows = std::max<int64_t>(need, std::min<int64_t>(2 * (int64_t)rope_rows, kMaxRopeRows));
        const int half = d.head_dim / 2;
        const size_t old = rope_host.size();
        rope_host.resize((size_t)rows * half);
        for (int64_t pos = rope_rows; pos < rows; pos++)
            rope_row(d.head_dim, d.max_period, (float)pos, d.act_dtype == XNP_BF16, &rope_host[(size_t)pos * half]);
        if (!host_only) {
            float2 *nr = nullptr;
            uint32_t *n16 = nullptr;
            hipError_t e = hipMalloc(&nr, sizeof(float2) * rope_host.size());
            if (e == hipSuccess && rope16) e = hipMalloc(&n16, sizeof(uint32_t) * rope_host.size());
            xnp_status st = e == hipSuccess ? upload_rope(nr, n16) : hip_fail(e, "rope table growth");
            if (st != XNP_OK) {
                if (nr) (void)hipFree(nr);
                if (n16) (void)hipFree(n16);
                rope_host.resize(old);
                return st;
            }
            // the pool takes the new tables whole before the old ones go: a failed free below then
            // leaves a consistent pool (the new tables in use) and reports the failure
            float2 *old_rope = rope;
            uint32_t *old_rope16 = rope16;
            device_bytes += (int64_t)((rope_host.size() - old) * (sizeof(float2) + (rope16 ? sizeof(uint32_t) : 0)));
            rope = nr;
            rope16 = n16;
            rope_rows = (int32_t)rows;
            const hipError_t e1 = hipFree(old_rope);
            const hipError_t e2 = old_rope16 ? hipFree(old_rope16) : hipSuccess;
            if (e1 != hipSuccess) return hip_fail(e1, "freeing the old rope table");
            if (e2 != hipSuccess) return hip_fail(e2, "freeing the old bf16 rope table");
            return XNP_OK;
        }
        rope_rows = (int32_t)rows;
        return XNP_OK;
    }

    // Give `sid` its own copy of every page it shares (before in-place writes).
    xnp_status unshare(int32_t sid, hipStream_t stream) {
        Stream &s = streams[sid];
        int need = 0;
        for (int32_t p : s.blocks)
            if (refs(p) > 1) need++;
        if (need > (int)free_pages.size())
            return fail(XNP_E_OUT_OF_BLOCKS, "out of blocks: %d needed to unshare, %d free", need,
                        (int)free_pages.size());
        std::vector<std::pair<int32_t, int32_t>> copies;
        for (size_t b = 0; b < s.blocks.size(); b++) {
            int32_t p = s.blocks[b];
            if (refs(p) <= 1) continue;
            refcnt[p]--;
            int32_t q = take_page(sid, (int32_t)b);
            copies.push_back({p, q});
        }
        if (!host_only)
            for (auto &c : copies) HIP_TRY(launch_copy_page(view(), c.first, c.second, stream), "page copy");
        return XNP_OK;
    }
};

// ---------------------------------------------------------------------------------------------
// pool

extern "C" const char *xnp_last_error(void) { return g_err.c_str(); }

namespace xnp {

// bf16 rounding on the host: to nearest even, NaN kept quiet (the kernels' rounding).
float bf16_round_host(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) {
        if (u & 0x007fffffu) u |= 0x00400000u;
        u &= 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    std::memcpy(&x, &u, 4);
    return x;
}

xnp_status pool_fail(xnp_status code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
const xnp_pool_desc *pool_desc(const xnp_pool *p) { return &p->d; }
BatchLaunchKey batch_launch_key(const xnp_pool *p) {
    BatchLaunchKey k;
    k.prefix = p->batch.bv.prefix;
    k.split = p->batch.bv.split;
    k.rope = p->rope;
    k.rope16 = p->rope16;
    return k;
}
bool pool_host_only(const xnp_pool *p) { return p->host_only; }
} // namespace xnp

extern "C" int32_t xnp_frame_budget(int32_t num_tokens, double frame_rate) {
    // plan.rs:43-45
    return (int32_t)std::ceil(((double)num_tokens / 3.0 + 2.0) * frame_rate);
}

extern "C" int32_t xnp_seq_budget(int32_t num_tokens, int32_t frame_budget) {
    // plan.rs:25, 52-54
    return num_tokens + 512 + frame_budget;
}

static void pool_free(xnp_pool *p) {
    if (!p->host_only) {
        for (auto &s : p->stage) {
            if (s.pending && s.done) (void)hipEventSynchronize(s.done);
            if (s.done) (void)hipEventDestroy(s.done);
            if (s.host) (void)hipHostFree(s.host);
        }
        void *bufs[] = {p->pages, p->scales, p->tables, p->rope, p->rope16, p->dbatch, p->daux};
        for (void *b : bufs)
            if (b) (void)hipFree(b);
    }
    delete p;
}

extern "C" xnp_status xnp_pool_create(const xnp_pool_desc *desc, xnp_pool **out) {
    if (!desc || !out) return fail(XNP_E_INVALID, "null argument");
    *out = nullptr;
    const xnp_pool_desc &d = *desc;
    if (d.num_layers <= 0 || d.num_blocks <= 0 || d.max_streams <= 0 || d.max_blocks_per_stream <= 0)
        return fail(XNP_E_INVALID, "layers, blocks, streams and blocks per stream must be positive");
    if (d.num_heads <= 0 || d.num_heads > kMaxHeads)
        return fail(XNP_E_HEADS, "the config's %d attention heads are not in 1..%d", d.num_heads, kMaxHeads);
    if (d.num_kv_heads <= 0 || d.num_heads % d.num_kv_heads)
        return fail(XNP_E_HEADS, "the config's %d key/value heads do not divide its %d attention heads",
                    d.num_kv_heads, d.num_heads);
    if (d.head_dim != kHeadDim) return fail(XNP_E_INVALID, "head_dim %d: the kernels take %d", d.head_dim, kHeadDim);
    const bool combo_ok = (d.cache_dtype == XNP_F32 && d.act_dtype == XNP_F32) ||
                          (d.cache_dtype == XNP_BF16 && d.act_dtype == XNP_BF16) ||
                          (d.cache_dtype == XNP_I8 && (d.act_dtype == XNP_BF16 || d.act_dtype == XNP_F32));
    if (!combo_ok)
        return fail(XNP_E_INVALID, "cache dtype %d with activation dtype %d is not supported", d.cache_dtype,
                    d.act_dtype);
    if (d.max_pos <= 0 || !(d.max_period > 0.0f)) return fail(XNP_E_INVALID, "max_pos and max_period must be positive");
    // default: the fewest waves per (stream, head) whose lanes can index a stream's pages, and one
    // wave only while a stream's K and V tiles of one head hold at most 128 KB.  Measured against
    // two waves: the int8 window (528 rows, 66 KB) 95.3-95.6 -> 91.9-92.2 us, bf16 caches of 256
    // rows (64 KB) 57 -> 53.6 us, of 512 rows (128 KB) equal, of 900 rows (225 KB) 150.4 -> 151.8
    // us.  The MFMA decode keeps two (batch_begin).
    const int cache_esz = d.cache_dtype == XNP_F32 ? 4 : d.cache_dtype == XNP_BF16 ? 2 : 1;
    const int one_wave_pages = std::min(kLaneBlocks, (128 << 10) / (2 * kBlock * d.head_dim * cache_esz));
    const int split = d.decode_split ? d.decode_split
                      : d.max_blocks_per_stream <= one_wave_pages ? 1
                      : d.max_blocks_per_stream <= kLaneBlocks * 2 ? 2
                      : d.max_blocks_per_stream <= kLaneBlocks * 4 ? 4 : 8;
    if (split != 1 && split != 2 && split != 4 && split != 8)
        return fail(XNP_E_INVALID, "decode_split %d is not 1, 2, 4 or 8", d.decode_split);
    if (d.max_blocks_per_stream > kLaneBlocks * split)
        return fail(XNP_E_INVALID, "%d pages per stream: decode with %d waves per head reads at most %d",
                    d.max_blocks_per_stream, split, kLaneBlocks * split);
    if ((int64_t)d.max_streams * d.max_blocks_per_stream > (int64_t)1 << 28)
        return fail(XNP_E_INVALID, "max_streams x max_blocks_per_stream too large");

    xnp_pool *p = new (std::nothrow) xnp_pool();
    if (!p) return fail(XNP_E_INVALID, "out of host memory");
    p->d = d;
    p->host_only = (d.flags & XNP_POOL_HOST_ONLY) != 0;
    p->split = split;
    p->esz = d.cache_dtype == XNP_F32 ? 4 : d.cache_dtype == XNP_BF16 ? 2 : 1;
    p->mask_words = (d.max_blocks_per_stream * kBlock + 31) / 32;

    p->streams.resize(d.max_streams);
    p->patch_mark.assign((size_t)d.max_streams * d.max_blocks_per_stream, 0u);
    if (p->host_only) p->shadow_tables.assign((size_t)d.max_streams * d.max_blocks_per_stream, -1);
    for (int32_t i = d.max_streams - 1; i >= 0; i--) p->free_ids.push_back(i);
    p->refcnt.assign(d.num_blocks, 0);
    std::vector<int32_t> order(d.num_blocks);
    for (int32_t i = 0; i < d.num_blocks; i++) order[i] = i;
    if (d.page_seed) {
        uint64_t s = d.page_seed;
        for (int32_t i = d.num_blocks - 1; i > 0; i--) {
            // Fisher-Yates with an unbiased draw in [0, i] by rejection
            uint64_t bound = (uint64_t)i + 1, lim = UINT64_MAX - UINT64_MAX % bound, r;
            do r = splitmix64(s); while (r >= lim);
            std::swap(order[i], order[(size_t)(r % bound)]);
        }
    }
    p->free_pages.assign(order.rbegin(), order.rend()); // pop_back hands out order[0] first

    if (d.max_pos > kMaxRopeRows) return fail(XNP_E_INVALID, "max_pos %d: the RoPE table holds at most %d rows", d.max_pos, kMaxRopeRows);
    const int half = d.head_dim / 2;
    p->rope_rows = d.max_pos;
    p->rope_host.resize((size_t)d.max_pos * half);
    for (int32_t pos = 0; pos < d.max_pos; pos++)
        rope_row(d.head_dim, d.max_period, (float)pos, d.act_dtype == XNP_BF16, &p->rope_host[(size_t)pos * half]);

    // plan upload layout: plans, work items, masks (each 256-byte aligned)
    p->rec_stride = (int)align_up(sizeof(StreamRec) + sizeof(int32_t) * d.max_blocks_per_stream, 64);
    p->batch_bytes = align_up(sizeof(StreamPlan) * d.max_streams, 256) +
                     align_up((size_t)p->rec_stride * d.max_streams, 256) +
                     align_up(sizeof(uint32_t) * (size_t)p->mask_words * d.max_streams, 256);
    p->aux_bytes = std::max<size_t>(sizeof(TablePatch) * 65536,
                                    align_up(sizeof(EvictRow) * d.max_blocks_per_stream * kBlock, 256) + 4096);

    if (p->host_only) {
        *out = p;
        return XNP_OK;
    }

    auto dev_fail = [&](hipError_t e, const char *what) {
        xnp_status st = hip_fail(e, what);
        pool_free(p);
        return st;
    };
    hipError_t e = hipSetDevice(d.device);
    if (e != hipSuccess) return dev_fail(e, "hipSetDevice");
    e = static_scratch_init(d.device); // the static scratch's address on this device, once per device
    if (e != hipSuccess) return dev_fail(e, "static scratch address");
    // a page holds the num_kv_heads heads a layer stores, not the repeated query heads
    const size_t page_elems = (size_t)d.num_kv_heads * kBlock * d.head_dim;
    const size_t page_bytes = page_elems * p->esz;
    const size_t pages_bytes = page_bytes * d.num_blocks * 2 * d.num_layers;
    struct {
        void **ptr;
        size_t bytes;
        const char *what;
    } allocs[] = {
        {&p->pages, pages_bytes, "pages"},
        {(void **)&p->scales, d.cache_dtype == XNP_I8 ? sizeof(float) * d.num_kv_heads * (size_t)d.num_blocks * 2 * d.num_layers : 0, "scales"},
        {(void **)&p->tables, sizeof(int32_t) * (size_t)d.max_streams * d.max_blocks_per_stream, "block tables"},
        {(void **)&p->rope, sizeof(float2) * p->rope_host.size(), "rope table"},
        {(void **)&p->rope16, d.act_dtype == XNP_BF16 ? sizeof(uint32_t) * p->rope_host.size() : 0, "bf16 rope table"},
        {(void **)&p->dbatch, p->batch_bytes, "batch plan"},
        {(void **)&p->daux, p->aux_bytes, "aux upload"},
    };
    for (auto &a : allocs) {
        if (!a.bytes) continue;
        e = hipMalloc(a.ptr, a.bytes);
        if (e != hipSuccess) return dev_fail(e, a.what);
        p->device_bytes += (int64_t)a.bytes;
    }
    e = hipMemset(p->tables, 0xff, sizeof(int32_t) * (size_t)d.max_streams * d.max_blocks_per_stream);
    if (e != hipSuccess) return dev_fail(e, "table init");
    if (p->scales) {
        e = hipMemset(p->scales, 0, sizeof(float) * d.num_kv_heads * (size_t)d.num_blocks * 2 * d.num_layers);
        if (e != hipSuccess) return dev_fail(e, "scale init");
    }
    if (xnp_status st = p->upload_rope(p->rope, p->rope16)) {
        pool_free(p);
        return st;
    }
    // a plan with the table patches behind it, or an aux upload
    const size_t stage_bytes = p->batch_bytes + p->aux_bytes;
    for (auto &s : p->stage) {
        e = hipHostMalloc((void **)&s.host, stage_bytes, hipHostMallocDefault);
        if (e != hipSuccess) return dev_fail(e, "pinned staging");
        e = hipHostGetDevicePointer((void **)&s.dev, s.host, 0);
        if (e != hipSuccess) return dev_fail(e, "pinned staging's device address");
        e = hipEventCreateWithFlags(&s.done, hipEventDisableTiming);
        if (e != hipSuccess) return dev_fail(e, "staging event");
    }
    e = hipDeviceSynchronize();
    if (e != hipSuccess) return dev_fail(e, "pool init");
    *out = p;
    return XNP_OK;
}

extern "C" xnp_status xnp_pool_destroy(xnp_pool *pool) {
    if (!pool) return XNP_OK;
    if (!pool->host_only) (void)hipSetDevice(pool->d.device);
    pool_free(pool);
    return XNP_OK;
}

extern "C" xnp_status xnp_pool_stats_get(const xnp_pool *pool, xnp_pool_stats *out) {
    if (!pool || !out) return fail(XNP_E_INVALID, "null argument");
    out->free_blocks = (int32_t)pool->free_pages.size();
    out->open_streams = (int32_t)(pool->streams.size() - pool->free_ids.size());
    out->batch_open = pool->batch.open ? std::max(pool->batch.n, 1) : 0;
    out->work_items = pool->batch.open && pool->batch.t == 1 ? pool->batch.n * pool->d.num_heads : 0;
    out->device_bytes = pool->device_bytes;
    out->rope_rows = pool->rope_rows;
    out->decode_waves = pool->batch.open && pool->batch.t == 1 ? pool->batch.bv.split : 0;
    return XNP_OK;
}

extern "C" xnp_status xnp_debug_set_block(xnp_pool *pool, int32_t id, int32_t blk, int32_t page) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (!pool->host_only) return fail(XNP_E_STATE, "only a host-only pool takes a planted page map");
    Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    if (blk < 0 || blk >= (int32_t)s->blocks.size()) return fail(XNP_E_INVALID, "block %d of %d", blk, (int)s->blocks.size());
    s->blocks[blk] = page;
    return XNP_OK;
}

extern "C" xnp_status xnp_pool_time_next(xnp_pool *pool, void *start_event, void *stop_event) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    pool->timing.start = (hipEvent_t)start_event;
    pool->timing.stop = (hipEvent_t)stop_event;
    return XNP_OK;
}

static xnp_status no_batch(const xnp_pool *p);

extern "C" xnp_status xnp_pool_check_tables(xnp_pool *pool, int32_t *mismatches, void *hip_stream) {
    if (!pool || !mismatches) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    hipStream_t hs = (hipStream_t)hip_stream;
    if (!pool->host_only) HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
    if (xnp_status st = pool->flush_patches(hs)) return st;
    const size_t n = (size_t)pool->d.max_streams * pool->d.max_blocks_per_stream;
    std::vector<int32_t> dev;
    const int32_t *tab = pool->shadow_tables.data();
    if (!pool->host_only) {
        dev.resize(n);
        HIP_TRY(hipMemcpyAsync(dev.data(), pool->tables, n * sizeof(int32_t), hipMemcpyDeviceToHost, hs), "table read");
        HIP_TRY(hipStreamSynchronize(hs), "table read");
        tab = dev.data();
    }
    int32_t bad = 0;
    for (size_t sid = 0; sid < pool->streams.size(); sid++) {
        const Stream &s = pool->streams[sid];
        if (!s.open) continue;
        for (size_t b = 0; b < s.blocks.size(); b++)
            bad += tab[sid * pool->d.max_blocks_per_stream + b] != s.blocks[b];
    }
    *mismatches = bad;
    return XNP_OK;
}

extern "C" xnp_status xnp_pool_rope_rows(const xnp_pool *pool, int32_t pos0, int32_t n, float *cos_sin) {
    if (!pool || !cos_sin) return fail(XNP_E_INVALID, "null argument");
    if (pos0 < 0 || n < 0 || (int64_t)pos0 + n > pool->rope_rows)
        return fail(XNP_E_INVALID, "rows %d..%d of a %d-row table", pos0, pos0 + n, pool->rope_rows);
    const size_t half = pool->d.head_dim / 2;
    std::memcpy(cos_sin, pool->rope_host.data() + (size_t)pos0 * half, sizeof(float2) * half * n);
    return XNP_OK;
}

// ---------------------------------------------------------------------------------------------
// streams

static xnp_status no_batch(const xnp_pool *p) {
    if (p->batch.open) return fail(XNP_E_STATE, "a batch is open: end or abort it first");
    return XNP_OK;
}

extern "C" xnp_status xnp_stream_open(xnp_pool *pool, int32_t capacity, int32_t *id) {
    if (!pool || !id) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    const int32_t maxcap = pool->d.max_blocks_per_stream * kBlock;
    if (capacity < 0 || capacity > maxcap)
        return fail(XNP_E_INVALID, "capacity %d: a stream holds at most %d positions", capacity, maxcap);
    if (pool->free_ids.empty()) return fail(XNP_E_STREAM, "all %d streams are open", pool->d.max_streams);
    int32_t sid = pool->free_ids.back();
    pool->free_ids.pop_back();
    Stream &s = pool->streams[sid];
    s = Stream();
    s.open = true;
    s.capacity = capacity;
    s.blocks.assign((capacity + kBlock - 1) / kBlock, -1);
    *id = sid;
    return XNP_OK;
}

extern "C" xnp_status xnp_stream_close(xnp_pool *pool, int32_t id) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    for (size_t b = 0; b < s->blocks.size(); b++) pool->drop_page(id, (int32_t)b);
    *s = Stream();
    pool->free_ids.push_back(id);
    return XNP_OK;
}

extern "C" xnp_status xnp_stream_fork(xnp_pool *pool, int32_t src, int32_t capacity, int32_t *id,
                                      void *hip_stream) {
    if (!pool || !id) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    Stream *s = pool->get(src);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", src);
    if (s->window) {
        // with_seq_budget clones a Mimi cache as it is (transformer.rs:348-354): a window rewrites
        // its pages in place, so every page is copied, and the budget does not apply
        int held = 0;
        for (int32_t p : s->blocks) held += p >= 0;
        if (held > (int)pool->free_pages.size())
            return fail(XNP_E_OUT_OF_BLOCKS, "out of blocks: %d needed, %d free", held, (int)pool->free_pages.size());
        int32_t dst;
        if (xnp_status st = xnp_stream_open(pool, s->capacity, &dst)) return st;
        s = pool->get(src);
        Stream &t = pool->streams[dst];
        t = *s;
        t.blocks.assign(s->blocks.size(), -1);
        if (!pool->host_only) HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
        for (size_t b = 0; b < s->blocks.size(); b++) {
            if (s->blocks[b] < 0) continue;
            const int32_t q = pool->take_page(dst, (int32_t)b);
            if (!pool->host_only)
                HIP_TRY(launch_copy_page(pool->view(), s->blocks[b], q, (hipStream_t)hip_stream), "page copy");
        }
        *id = dst;
        return XNP_OK;
    }
    if (s->ring != RING_NONE) return fail(XNP_E_BUDGET, "a ring cache cannot be resized");
    const int32_t used = s->current_end;
    if (used > capacity)
        return fail(XNP_E_BUDGET, "cannot fit %d filled KV positions into a budget of %d", used, capacity);
    const int32_t maxcap = pool->d.max_blocks_per_stream * kBlock;
    if (capacity > maxcap)
        return fail(XNP_E_INVALID, "capacity %d: a stream holds at most %d positions", capacity, maxcap);
    if (pool->free_ids.empty()) return fail(XNP_E_STREAM, "all %d streams are open", pool->d.max_streams);
    const bool tail = used % kBlock != 0;
    if (tail && pool->free_pages.empty()) return fail(XNP_E_OUT_OF_BLOCKS, "out of blocks: the pool has no free page");
    int32_t dst;
    xnp_status st = xnp_stream_open(pool, capacity, &dst);
    if (st) return st;
    s = pool->get(src); // streams may not move, but keep the reference fresh
    Stream &t = pool->streams[dst];
    t.current_end = used;
    const int32_t full = used / kBlock;
    for (int32_t b = 0; b < full; b++) {
        int32_t p = s->blocks[b];
        t.blocks[b] = p;
        if (pool->refs(p) > 0) pool->refcnt[p]++;
        pool->patches.push_back({dst, b, p, 0});
    }
    if (tail) {
        int32_t q = pool->take_page(dst, full);
        if (!pool->host_only) {
            hipStream_t hs = (hipStream_t)hip_stream;
            HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
            HIP_TRY(launch_copy_page(pool->view(), s->blocks[full], q, hs), "page copy");
        }
    }
    *id = dst;
    return XNP_OK;
}

extern "C" xnp_status xnp_stream_info_get(const xnp_pool *pool, int32_t id, xnp_stream_info *out) {
    if (!pool || !out) return fail(XNP_E_INVALID, "null argument");
    const Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    out->current_end = s->current_end;
    out->capacity = s->capacity;
    out->ring_mode = s->ring;
    out->ring_write = s->write;
    out->ring_filled = s->filled;
    out->ring_prefix = s->prefix;
    out->window = s->window;
    out->ring_shift = s->shift;
    int32_t in_view = 0, blocks = 0, shared = 0;
    for (uint8_t v : s->valid) in_view += v;
    for (int32_t p : s->blocks)
        if (p >= 0) {
            blocks++;
            shared += pool->refs(p) > 1;
        }
    out->in_view = in_view;
    out->blocks = blocks;
    out->shared = shared;
    return XNP_OK;
}

extern "C" xnp_status xnp_stream_blocks(const xnp_pool *pool, int32_t id, int32_t *pages, int32_t cap,
                                        int32_t *count) {
    if (!pool || !count) return fail(XNP_E_INVALID, "null argument");
    const Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    *count = (int32_t)s->blocks.size();
    if (pages)
        for (int32_t i = 0; i < std::min(cap, *count); i++) pages[i] = s->blocks[i];
    return XNP_OK;
}

extern "C" xnp_status xnp_ring_valid(const xnp_pool *pool, int32_t id, uint8_t *valid, int32_t cap) {
    if (!pool || !valid) return fail(XNP_E_INVALID, "null argument");
    const Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    for (int32_t i = 0; i < std::min(cap, s->capacity); i++)
        valid[i] = s->ring == RING_NONE ? (i < s->current_end) : s->valid[i];
    return XNP_OK;
}

// Pages for blocks [b0, b1) of stream sid, all or nothing.
static xnp_status take_range(xnp_pool *pool, int32_t sid, int32_t b0, int32_t b1,
                             std::vector<std::pair<int32_t, int32_t>> *taken) {
    Stream &s = pool->streams[sid];
    int need = 0;
    for (int32_t b = b0; b < b1; b++) need += s.blocks[b] < 0;
    if (need > (int)pool->free_pages.size())
        return fail(XNP_E_OUT_OF_BLOCKS, "out of blocks: %d needed, %d free", need, (int)pool->free_pages.size());
    for (int32_t b = b0; b < b1; b++)
        if (s.blocks[b] < 0) {
            pool->take_page(sid, b);
            if (taken) taken->push_back({sid, b});
        }
    return XNP_OK;
}

extern "C" xnp_status xnp_stream_advance(xnp_pool *pool, int32_t id, int32_t n) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    if (s->ring != RING_NONE) return fail(XNP_E_RING, "a ring cache steps one row at a time");
    if (n < 0 || s->current_end + n > s->capacity)
        return fail(XNP_E_NO_ROOM, "no room left: the stream holds %d positions", s->capacity);
    if (n == 0) return XNP_OK;
    const int32_t b0 = s->current_end / kBlock, b1 = (s->current_end + n - 1) / kBlock + 1;
    if (xnp_status st = take_range(pool, id, b0, b1, nullptr)) return st;
    s->current_end += n;
    return XNP_OK;
}

// Copy on write before rows [slot0, slot0 + n) of stream id are rewritten: a page shared with a
// fork gets a copy of its own first.  Then the table patches reach the device.
static xnp_status own_pages(xnp_pool *pool, int32_t id, int32_t slot0, int32_t n, hipStream_t hs) {
    Stream &s = pool->streams[id];
    const int32_t b0 = slot0 / kBlock, b1 = (slot0 + n - 1) / kBlock + 1;
    int need = 0;
    for (int32_t b = b0; b < b1; b++) need += pool->refs(s.blocks[b]) > 1;
    if (need > (int)pool->free_pages.size())
        return fail(XNP_E_OUT_OF_BLOCKS, "out of blocks: %d needed to copy shared pages", need);
    for (int32_t b = b0; b < b1; b++) {
        int32_t p = s.blocks[b];
        if (pool->refs(p) <= 1) continue;
        pool->refcnt[p]--;
        int32_t q = pool->take_page(id, b);
        HIP_TRY(launch_copy_page(pool->view(), p, q, hs), "page copy");
    }
    return pool->flush_patches(hs);
}

static xnp_status rows_check(const xnp_pool *pool, int32_t id, int32_t layer, int32_t kv, int32_t slot0,
                             int32_t n, const void *rows) {
    if (!pool || (!rows && n > 0)) return fail(XNP_E_INVALID, "null argument");
    if (pool->host_only) return fail(XNP_E_STATE, "a host-only pool has no device pages");
    const Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    if (layer < 0 || layer >= pool->d.num_layers) return fail(XNP_E_INVALID, "layer %d of %d", layer, pool->d.num_layers);
    if (kv != 0 && kv != 1) return fail(XNP_E_INVALID, "kv %d is neither keys (0) nor values (1)", kv);
    if (slot0 < 0 || n < 0 || slot0 + n > s->capacity)
        return fail(XNP_E_INVALID, "rows %d..%d of a %d-slot stream", slot0, slot0 + n, s->capacity);
    for (int32_t slot = slot0; slot < slot0 + n; slot += kBlock - slot % kBlock)
        if (s->blocks[slot / kBlock] < 0) return fail(XNP_E_INVALID, "slot %d has no page", slot);
    return XNP_OK;
}

extern "C" xnp_status xnp_write_rows(xnp_pool *pool, int32_t id, int32_t layer, int32_t kv, int32_t slot0,
                                     int32_t n, const void *rows, const float *scales, void *hip_stream) {
    if (xnp_status st = rows_check(pool, id, layer, kv, slot0, n, rows)) return st;
    if (pool->d.cache_dtype == XNP_I8 && !scales && n > 0) return fail(XNP_E_INVALID, "an int8 cache needs scales");
    if (n == 0) return XNP_OK;
    hipStream_t hs = (hipStream_t)hip_stream;
    HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
    if (xnp_status st = own_pages(pool, id, slot0, n, hs)) return st;
    HIP_TRY(launch_rows_io(pool->view(), id, layer, kv, slot0, n, const_cast<void *>(rows),
                           const_cast<float *>(scales), true, hs),
            "row write");
    return XNP_OK;
}

extern "C" xnp_status xnp_stream_load_kv(xnp_pool *pool, int32_t id, int32_t layer, const float *kv, int32_t n,
                                         void *hip_stream) {
    if (xnp_status st = rows_check(pool, id, layer, 0, 0, n, kv)) return st;
    if (xnp_status st = no_batch(pool)) return st;
    const Stream &s = pool->streams[id];
    if (s.ring != RING_NONE) return fail(XNP_E_RING, "a voice loads into a plain cache, not a ring");
    if (n != s.current_end)
        return fail(XNP_E_INVALID, "a %d-row voice loads into a stream holding exactly as many rows, not %d", n,
                    s.current_end);
    if (n == 0) return XNP_OK;
    hipStream_t hs = (hipStream_t)hip_stream;
    HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
    if (xnp_status st = own_pages(pool, id, 0, n, hs)) return st;
    HIP_TRY(launch_load_kv(pool->view(), id, layer, kv, n, hs), "voice load");
    return XNP_OK;
}

extern "C" xnp_status xnp_read_rows(const xnp_pool *cpool, int32_t id, int32_t layer, int32_t kv, int32_t slot0,
                                    int32_t n, void *rows, float *scales, void *hip_stream) {
    if (xnp_status st = rows_check(cpool, id, layer, kv, slot0, n, rows)) return st;
    if (n == 0) return XNP_OK;
    xnp_pool *pool = const_cast<xnp_pool *>(cpool); // pending table patches must reach the device
    hipStream_t hs = (hipStream_t)hip_stream;
    HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
    if (xnp_status st = pool->flush_patches(hs)) return st;
    HIP_TRY(launch_rows_io(pool->view(), id, layer, kv, slot0, n, rows, scales, false, hs), "row read");
    return XNP_OK;
}

// ---------------------------------------------------------------------------------------------
// ring: transformer.rs:842-929

extern "C" xnp_status xnp_ring_start(xnp_pool *pool, int32_t id, int32_t mode, int32_t prefix, void *hip_stream) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    if (mode != XNP_RING_SHIFT && mode != XNP_RING_ABSOLUTE) return fail(XNP_E_INVALID, "bad ring mode %d", mode);
    if (s->ring != RING_NONE) return fail(XNP_E_RING, "the cache is a ring already");
    if (prefix < 0 || prefix > s->capacity)
        return fail(XNP_E_INVALID, "prefix %d of a %d-slot cache", prefix, s->capacity);
    if (!pool->host_only) HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
    if (xnp_status st = pool->unshare(id, (hipStream_t)hip_stream)) return st;
    const int32_t used = s->current_end;
    s->valid.assign(s->capacity, 0);
    for (int32_t i = 0; i < used; i++) s->valid[i] = 1;
    s->nvalid = used;
    s->ring = mode;
    s->write = used;
    s->filled = used;
    s->prefix = mode == XNP_RING_ABSOLUTE ? prefix : 0;
    s->shift = 0;
    return XNP_OK;
}

extern "C" xnp_status xnp_ring_set_slot(xnp_pool *pool, int32_t id, int32_t slot) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    if (s->ring == RING_NONE) return fail(XNP_E_RING, "not a ring cache, see start_ring");
    if (s->window) return fail(XNP_E_RING, "a window cache places its rows itself");
    if (slot < 0 || slot >= s->capacity) return fail(XNP_E_RING, "slot %d of a %d-slot ring", slot, s->capacity);
    s->write = slot;
    return XNP_OK;
}

extern "C" xnp_status xnp_ring_evict(xnp_pool *pool, int32_t id, int32_t prefix, const int32_t *slots,
                                     int32_t count, void *hip_stream) {
    if (!pool || (count > 0 && !slots)) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    if (s->ring == RING_NONE) return fail(XNP_E_RING, "not a ring cache, see start_ring");
    if (s->window) return fail(XNP_E_RING, "a window cache places its rows itself");
    if (count < 0 || count > s->current_end)
        return fail(XNP_E_EVICT, "cannot evict %d of %d positions", count, s->current_end);
    if (s->ring == RING_ABSOLUTE && prefix != s->prefix)
        return fail(XNP_E_EVICT, "an absolute ring evicts past its prefix %d, not %d", s->prefix, prefix);
    if (s->ring == RING_SHIFT && pool->d.cache_dtype == XNP_I8)
        return fail(XNP_E_EVICT, "an int8 cache evicts on an absolute ring");
    // Every slot is checked before any change (transformer.rs:896-901).
    for (int32_t j = 0; j < count; j++) {
        const int32_t sl = slots[j];
        if (sl < prefix || sl < 0 || sl >= s->capacity || !s->valid[sl])
            return fail(XNP_E_EVICT, "slot %d holds no row past the prefix", sl);
    }
    std::vector<EvictRow> rows;
    if (s->ring == RING_SHIFT && count > 0) {
        for (int32_t sl = prefix; sl < s->filled; sl++) {
            bool evicted = false;
            for (int32_t j = 0; j < count && !evicted; j++) evicted = slots[j] == sl;
            if (s->valid[sl] && !evicted) rows.push_back({id, sl});
        }
        // The rows must fit one upload (max_blocks_per_stream * 16 of them always do).
        if (!pool->host_only && !rows.empty()) {
            hipStream_t hs = (hipStream_t)hip_stream;
            HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
            if (xnp_status st = pool->flush_patches(hs)) return st;
            Staging *sg;
            if (xnp_status st = pool->stage_acquire(&sg)) return st;
            const int half = pool->d.head_dim / 2;
            rope_row(pool->d.head_dim, pool->d.max_period, -(float)count, pool->d.act_dtype == XNP_BF16,
                     (float2 *)sg->host);
            const size_t roff = 4096;
            static_assert(sizeof(float2) * 32 <= 4096, "rope row fits the header");
            (void)half;
            std::memcpy(sg->host + roff, rows.data(), sizeof(EvictRow) * rows.size());
            if (xnp_status st = pool->upload(sg, pool->daux, roff + sizeof(EvictRow) * rows.size(), hs)) return st;
            HIP_TRY(launch_evict_rotate(pool->view(), (const EvictRow *)(pool->daux + roff), (int)rows.size(),
                                        (const float *)pool->daux, nullptr, hs),
                    "evict rotate");
        }
    }
    for (int32_t j = 0; j < count; j++)
        if (s->valid[slots[j]]) {
            s->valid[slots[j]] = 0;
            s->nvalid--;
        }
    if (s->ring == RING_ABSOLUTE) s->shift += count;
    s->current_end -= count;
    return XNP_OK;
}

extern "C" xnp_status xnp_ring_slide(xnp_pool *pool, int32_t id, int32_t prefix, int32_t span, int32_t window,
                                     int32_t drop, int64_t step, void *hip_stream) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    Stream *s = pool->get(id);
    if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
    if (s->ring == RING_NONE) return fail(XNP_E_RING, "not a ring cache, see start_ring");
    if (span <= 0 || window <= 0 || window > span || drop <= 0 || drop > window || prefix < 0 ||
        prefix + span > s->capacity || step < 0)
        return fail(XNP_E_INVALID, "slide over %d slots past %d with a window of %d, dropping %d, at step %lld",
                    span, prefix, window, drop, (long long)step);
    // valid slots in [prefix, prefix + span): the ring's count less those outside the window
    int32_t in_view = s->nvalid;
    for (int32_t sl = 0; sl < prefix; sl++) in_view -= s->valid[sl];
    for (int32_t sl = prefix + span; sl < s->capacity; sl++) in_view -= s->valid[sl];
    if (in_view == window) {
        // s2s.rs:324-332: frames take the slots after the prefix in turn, so the oldest are the
        // next ones round.
        const int64_t oldest = step - in_view;
        std::vector<int32_t> slots(drop);
        for (int32_t j = 0; j < drop; j++)
            slots[j] = prefix + (int32_t)((((oldest + j) % span) + span) % span);
        if (xnp_status st = xnp_ring_evict(pool, id, prefix, slots.data(), drop, hip_stream)) return st;
    }
    return xnp_ring_set_slot(pool, id, prefix + (int32_t)(step % span));
}

extern "C" xnp_status xnp_ring_slide_batch(xnp_pool *pool, const int32_t *ids, int32_t n, int32_t prefix,
                                           int32_t span, int32_t window, int32_t drop, const int64_t *steps,
                                           int32_t *failed, void *hip_stream) {
    if (!pool || (n > 0 && (!ids || !steps))) return fail(XNP_E_INVALID, "null argument");
    if (failed) *failed = -1;
    for (int32_t i = 0; i < n; i++) {
        xnp_status st = xnp_ring_slide(pool, ids[i], prefix, span, window, drop, steps[i], hip_stream);
        if (st) {
            if (failed) *failed = i;
            return st;
        }
    }
    return XNP_OK;
}

// KvCache::new(context) (transformer.rs:264-267) for Mimi's attention: an absolute ring of
// `window` slots whose rows the batch calls place themselves (row p in slot p % window), so that
// each step attends the last `window` positions, as KvCache::trim and the window mask of
// transformer.rs:300-316,764-781 keep them.
extern "C" xnp_status xnp_window_open(xnp_pool *pool, int32_t window, int32_t *id) {
    if (!pool || !id) return fail(XNP_E_INVALID, "null argument");
    if (window <= 0) return fail(XNP_E_INVALID, "a window of %d rows", window);
    int32_t sid;
    if (xnp_status st = xnp_stream_open(pool, window, &sid)) return st;
    if (xnp_status st = xnp_ring_start(pool, sid, XNP_RING_ABSOLUTE, 0, nullptr)) {
        (void)xnp_stream_close(pool, sid);
        return st;
    }
    pool->streams[sid].window = window;
    *id = sid;
    return XNP_OK;
}

// ---------------------------------------------------------------------------------------------
// batches

extern "C" xnp_status xnp_batch_begin(xnp_pool *pool, const int32_t *ids, int32_t n, int32_t t, void *hip_stream) {
    if (!pool || (n > 0 && !ids)) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = no_batch(pool)) return st;
    if (n < 0 || n > pool->d.max_streams) return fail(XNP_E_INVALID, "%d streams in a batch of at most %d", n, pool->d.max_streams);
    if (t <= 0) return fail(XNP_E_INVALID, "a step appends at least one row, not %d", t);
    // check everything first
    std::vector<uint8_t> seen(pool->streams.size(), 0);
    int need = 0, windows = 0;
    int64_t max_pos = -1; // the step's largest RoPE position
    for (int32_t i = 0; i < n; i++) {
        const int32_t id = ids[i];
        const Stream *s = pool->get(id);
        if (!s) return fail(XNP_E_STREAM, "no open stream %d", id);
        if (seen[id]) return fail(XNP_E_INVALID, "stream %d appears twice in the batch", id);
        seen[id] = 1;
        int64_t last_pos;
        if (s->window) {
            // row i of the step goes to slot (p + i) % window, over the row leaving the window
            const int64_t p = (int64_t)s->current_end + s->shift;
            window_blocks(*s, p, t, [&](int32_t b) { need += s->blocks[b] < 0; });
            last_pos = p + t - 1;
            windows++;
        } else if (s->ring != RING_NONE) {
            if (t != 1) return fail(XNP_E_RING, "a ring cache takes one row at a time, not %d", t);
            if (s->valid[s->write]) return fail(XNP_E_RING, "ring slot %d still holds a row, evict it first", s->write);
            need += s->blocks[s->write / kBlock] < 0;
            last_pos = s->current_end + (s->ring == RING_ABSOLUTE ? s->shift : 0);
        } else {
            if (s->current_end + t > s->capacity)
                return fail(XNP_E_NO_ROOM, "no room left: the stream holds %d positions", s->capacity);
            for (int32_t b = s->current_end / kBlock; b <= (s->current_end + t - 1) / kBlock; b++) need += s->blocks[b] < 0;
            last_pos = s->current_end + t - 1;
        }
        if (last_pos >= kMaxRopeRows)
            return fail(XNP_E_INVALID, "position %lld is beyond the largest RoPE table (%d rows)", (long long)last_pos,
                        kMaxRopeRows);
        max_pos = std::max(max_pos, last_pos);
    }
    if (t > 1 && windows && windows != n)
        return fail(XNP_E_INVALID, "a step of %d rows holds window caches only, or none", t);
    const bool wsteps = t > 1 && windows; // one decode per row, each over its own records
    if (wsteps && pool->d.cache_dtype == XNP_I8 && pool->d.num_kv_heads < pool->d.num_heads)
        return fail(XNP_E_INVALID, "an int8 window cache with grouped heads takes one row a step");
    if (need > (int)pool->free_pages.size())
        return fail(XNP_E_OUT_OF_BLOCKS, "out of blocks: %d needed, %d free", need, (int)pool->free_pages.size());
    if (!pool->host_only) HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
    if (xnp_status st = pool->grow_rope(max_pos + 1)) return st;

    auto &B = pool->batch;
    B.ids.assign(ids, ids + n);
    B.taken.clear();
    B.n = n;
    B.t = t;
    B.stream = (hipStream_t)hip_stream;
    for (int32_t i = 0; i < n; i++) {
        Stream &s = pool->streams[ids[i]];
        if (s.window) {
            window_blocks(s, (int64_t)s.current_end + s.shift, t,
                          [&](int32_t b) { take_range(pool, ids[i], b, b + 1, &B.taken); });
        } else if (s.ring != RING_NONE)
            take_range(pool, ids[i], s.write / kBlock, s.write / kBlock + 1, &B.taken);
        else
            take_range(pool, ids[i], s.current_end / kBlock, (s.current_end + t - 1) / kBlock + 1, &B.taken);
    }
    // Every block a row of the step goes into must hold a page of this stream's own: a live page
    // id, not shared with a fork (copy on write ran before).  The kernels would write a bad id's row
    // nowhere (or, were the check absent, into another stream's page), so a broken page map stops
    // here, before anything is uploaded.
    pool->writer.resize(pool->d.num_blocks, -1);
    std::vector<int32_t> written; // pages marked in pool->writer, unmarked below
    auto unmark = [&] {
        for (int32_t pg : written) pool->writer[pg] = -1;
    };
    for (int32_t i = 0; i < n; i++) {
        const Stream &s = pool->streams[ids[i]];
        int32_t bad = -1; // the first block written without a page of its own
        auto check = [&](int32_t b) {
            const int32_t pg = s.blocks[b];
            const bool ok = pg >= 0 && pg < pool->d.num_blocks && pool->refcnt[pg] == 1 &&
                            (pool->writer[pg] < 0 || pool->writer[pg] == ids[i]);
            if (ok && pool->writer[pg] < 0) {
                pool->writer[pg] = ids[i];
                written.push_back(pg);
            }
            if (bad < 0 && !ok) bad = b;
        };
        if (s.window) {
            window_blocks(s, (int64_t)s.current_end + s.shift, t, check);
        } else if (s.ring != RING_NONE) {
            check(s.write / kBlock);
        } else {
            for (int32_t b = s.current_end / kBlock; b <= (s.current_end + t - 1) / kBlock; b++) check(b);
        }
        if (bad >= 0) {
            const int32_t pg = s.blocks[bad];
            const bool live = pg >= 0 && pg < pool->d.num_blocks;
            const int32_t refs = live ? pool->refcnt[pg] : 0, other = live ? pool->writer[pg] : -1;
            unmark();
            for (auto it = B.taken.rbegin(); it != B.taken.rend(); ++it) pool->drop_page(it->first, it->second);
            B.taken.clear();
            return fail(XNP_E_STATE,
                        "stream %d writes block %d, whose page %d is not its own (%d holders, written by stream %d "
                        "of the batch too): the page map is broken", ids[i], bad, pg, refs, other);
        }
    }
    unmark();

    // the plan, composed in host memory laid out as the device buffer
    std::vector<StreamPlan> plans(n);
    std::vector<uint32_t> masks;
    for (int32_t i = 0; i < n; i++) {
        const Stream &s = pool->streams[ids[i]];
        StreamPlan &P = plans[i];
        std::memset(&P, 0, sizeof P);
        P.sid = ids[i];
        P.out_row = i;
        P.mask_off = -1;
        if (s.ring == RING_NONE) {
            P.pos = P.pos_pre = s.current_end;
            P.write_slot = s.current_end;
            P.key_pos = s.current_end;
            P.span = s.current_end + 1;
        } else {
            P.pos_pre = s.current_end;
            P.pos = s.current_end + (s.ring == RING_ABSOLUTE ? s.shift : 0);
            P.prefix = s.ring == RING_ABSOLUTE ? s.prefix : 0;
            P.write_slot = s.write;
            P.key_pos = (s.ring == RING_ABSOLUTE && s.write >= s.prefix) ? P.pos : P.pos_pre;
            P.span = std::max(s.filled, s.write + 1);
            P.ring = 1;
            // RingSlots::decode_mask (transformer.rs:42-52): valid slots and the write slot.
            P.mask_off = (int32_t)masks.size();
            const int words = (P.span + 31) / 32;
            masks.resize(masks.size() + words, 0u);
            for (int32_t sl = 0; sl < P.span; sl++)
                if (s.valid[sl] || sl == s.write) masks[P.mask_off + sl / 32] |= 1u << (sl % 32);
            const int32_t b0 = s.write / kBlock * kBlock, b1 = std::min(b0 + kBlock, s.capacity);
            int other = 0;
            for (int32_t sl = b0; sl < b1; sl++) other |= (sl != s.write && s.valid[sl]);
            P.fresh = !other;
            if (s.window) {
                // the held rows are positions p - held .. p - 1, the oldest in slot (p - held) % window
                P.window = s.window;
                P.wbase = s.shift % s.window;
            }
        }
    }
    // decode order: longest streams first, so the short ones fill the tail of the launch
    std::vector<int32_t> order(n);
    for (int32_t i = 0; i < n; i++) order[i] = i;
    if (t == 1)
        std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return plans[a].span > plans[b].span; });
    // waves per decode work group, unless the caller fixed them: the pool's default (the fewest
    // whose lanes index a stream's pages), at least two on MFMA; and a batch of few groups fills
    // few CUs, so give each group more waves (a larger split only raises the pages a group can
    // index) until the batch has about one wave per SIMD
    B.bv.prefix = 0;
    B.bv.kmax = 0;
    for (int32_t i = 0; i < n; i++) {
        B.bv.prefix |= plans[i].prefix > 0;
        B.bv.kmax = std::max(B.bv.kmax, plans[i].write_slot + t);
    }
    B.bv.split = pool->split;
    if (!pool->d.decode_split && t == 1)
        B.bv.split = std::max(B.bv.split, decode_min_split(pool->view(), B.bv.prefix != 0));
    {
        const int gq = t == 1 ? decode_heads_per_group(pool->view(), B.bv.prefix != 0) : 1;
        const int64_t groups = (int64_t)n * t * pool->d.num_heads / gq;
        while (!pool->d.decode_split && B.bv.split < 8 && groups * B.bv.split < 1024)
            B.bv.split *= 2;
    }
    if (pool->host_only) {
        B.open = true;
        return XNP_OK;
    }
    hipStream_t hs = B.stream;
    auto undo = [&](xnp_status st) {
        for (auto it = B.taken.rbegin(); it != B.taken.rend(); ++it) pool->drop_page(it->first, it->second);
        B.taken.clear();
        return st;
    };
    hipError_t he = hipSetDevice(pool->d.device);
    if (he != hipSuccess) return undo(hip_fail(he, "hipSetDevice"));
    // the table patches ride behind the plan when they fit (a step takes a few pages), so one
    // kernel pulls both; a longer list goes ahead by itself
    pool->coalesce_patches();
    if (pool->patches.size() * sizeof(TablePatch) > pool->aux_bytes)
        if (xnp_status st = pool->flush_patches(hs)) return undo(st);
    Staging *sg;
    if (xnp_status st = pool->stage_acquire(&sg)) return undo(st);
    const size_t o_plans = 0;
    const size_t o_recs = align_up(sizeof(StreamPlan) * n, 256);
    const int32_t sets = t == 1 || wsteps ? 1 : 0; // a window step's rows derive theirs from row 0's
    const size_t o_masks = o_recs + align_up((size_t)pool->rec_stride * n * sets, 256);
    const size_t total = o_masks + sizeof(uint32_t) * masks.size();
    std::memcpy(sg->host + o_plans, plans.data(), sizeof(StreamPlan) * n);
    if (t == 1)
        for (int32_t r = 0; r < n; r++) {
            const StreamPlan &P = plans[order[r]];
            StreamRec R;
            std::memset(&R, 0, sizeof R);
            R.b = P.out_row;
            R.nblk = (P.span + kBlock - 1) / kBlock;
            R.pos = P.pos;
            R.pos_pre = P.pos_pre;
            R.prefix = P.prefix;
            R.write_slot = P.write_slot;
            R.key_pos = P.key_pos;
            R.span = P.span;
            R.mask_off = P.mask_off;
            R.flags = (P.ring ? 1 : 0) | (P.fresh ? 2 : 0);
            char *dst = sg->host + o_recs + (size_t)r * pool->rec_stride;
            std::memcpy(dst, &R, sizeof R);
            std::memcpy(dst + sizeof R, pool->streams[P.sid].blocks.data(), sizeof(int32_t) * R.nblk);
        }
    if (wsteps)
        // Mimi's chunk (transformer.rs:764-781): row i attends positions (p + i - window, p + i], the
        // causal window.  Row by row, each row's key takes the slot of position p + i - window, which
        // no later row sees, and every filled slot holds a position inside row i's window, so row i
        // sees slots [0, min(p + i + 1, window)).  The record is row 0's, with every page of the
        // window; the decode kernel derives row i's from it (window_row).
        for (int32_t j = 0; j < n; j++) {
            const Stream &st = pool->streams[plans[order[j]].sid];
            const int64_t p = (int64_t)st.current_end + st.shift;
            StreamRec R;
            std::memset(&R, 0, sizeof R);
            R.b = plans[order[j]].out_row * t;
            R.pos = R.pos_pre = R.key_pos = (int32_t)p;
            R.write_slot = (int32_t)(p % st.window);
            R.span = (int32_t)std::min<int64_t>(p + 1, st.window);
            R.nblk = (st.window + kBlock - 1) / kBlock;
            R.mask_off = -1;
            R.flags = 1;
            R.window = st.window;
            char *dst = sg->host + o_recs + (size_t)j * pool->rec_stride;
            std::memcpy(dst, &R, sizeof R);
            std::memcpy(dst + sizeof R, st.blocks.data(), sizeof(int32_t) * R.nblk);
        }
    std::memcpy(sg->host + o_masks, masks.data(), sizeof(uint32_t) * masks.size());
    const size_t o_patch = pool->batch_bytes;
    const int np = (int)pool->patches.size();
    std::memcpy(sg->host + o_patch, pool->patches.data(), sizeof(TablePatch) * np);
    if (xnp_status st = pool->pull(sg, pool->dbatch, total, o_patch, np, hs)) return undo(st);
    pool->patches.clear();
    B.bv.plans = (const StreamPlan *)(pool->dbatch + o_plans);
    B.bv.recs = pool->dbatch + o_recs;
    B.bv.rec_stride = pool->rec_stride;
    B.bv.masks = (const uint32_t *)(pool->dbatch + o_masks);
    B.bv.wrow = -1;
    B.bv.n = n;
    B.bv.t = t;
    B.wsteps = wsteps;
    B.open = true;
    return XNP_OK;
}

// The checks of a per-layer call: `decode` for one row per stream, else several; `window_rows` for
// the row-by-row attention of a window step of several rows, the only call such a batch takes.
static xnp_status batch_call(xnp_pool *pool, int32_t layer, void *hip_stream, bool decode, bool window_rows = false) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (!pool->batch.open) return fail(XNP_E_STATE, "no batch is open");
    if (pool->host_only) return fail(XNP_E_STATE, "a host-only pool runs no kernels");
    if (layer < 0 || layer >= pool->d.num_layers) return fail(XNP_E_INVALID, "layer %d of %d", layer, pool->d.num_layers);
    if ((hipStream_t)hip_stream != pool->batch.stream)
        return fail(XNP_E_INVALID, "a batch's calls go to the stream it began on");
    if (pool->batch.wsteps != window_rows)
        return fail(XNP_E_INVALID, "a window step of several rows runs through xnp_attend alone");
    if (!window_rows && decode && pool->batch.t != 1)
        return fail(XNP_E_INVALID, "decode takes one row per stream, not %d", pool->batch.t);
    if (!window_rows && !decode && pool->batch.t == 1)
        return fail(XNP_E_INVALID, "prefill takes more than one row per stream");
    HIP_TRY(hipSetDevice(pool->d.device), "hipSetDevice");
    return XNP_OK;
}

extern "C" xnp_status xnp_append(xnp_pool *pool, int32_t layer, const void *k, const void *v, void *hip_stream) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = batch_call(pool, layer, hip_stream, pool->batch.t == 1)) return st;
    if (pool->batch.n > 0 && (!k || !v)) return fail(XNP_E_INVALID, "null k or v");
    HIP_TRY(launch_append(pool->view(), pool->batch.bv, layer, k, v, pool->batch.stream), "append");
    return XNP_OK;
}

extern "C" xnp_status xnp_decode(xnp_pool *pool, int32_t layer, const void *q, void *out, float scale,
                                 void *hip_stream) {
    if (xnp_status st = batch_call(pool, layer, hip_stream, true)) return st;
    if (pool->batch.n > 0 && (!q || !out)) return fail(XNP_E_INVALID, "null q or out");
    const LaunchTiming tm = pool->timing;
    pool->timing = LaunchTiming();
    HIP_TRY(launch_decode(pool->view(), pool->batch.bv, layer, q, nullptr, nullptr, out, scale, false,
                          pool->batch.stream, tm),
            "decode");
    return XNP_OK;
}

extern "C" xnp_status xnp_prefill(xnp_pool *pool, int32_t layer, const void *q, void *out, float scale,
                                  void *hip_stream) {
    if (xnp_status st = batch_call(pool, layer, hip_stream, false)) return st;
    if (pool->batch.n > 0 && (!q || !out)) return fail(XNP_E_INVALID, "null q or out");
    const LaunchTiming tm = pool->timing;
    pool->timing = LaunchTiming();
    HIP_TRY(launch_prefill(pool->view(), pool->batch.bv, layer, q, nullptr, nullptr, out, scale, false,
                           pool->batch.stream, tm),
            "prefill");
    return XNP_OK;
}

extern "C" xnp_status xnp_attend(xnp_pool *pool, int32_t layer, const void *q, const void *k, const void *v,
                                 void *out, float scale, void *hip_stream) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (pool->batch.open && pool->batch.wsteps) {
        // window caches, several rows: row by row, each a fused append + decode over its records
        auto &B = pool->batch;
        if (xnp_status st = batch_call(pool, layer, hip_stream, false, true)) return st;
        if (B.n > 0 && (!q || !k || !v || !out)) return fail(XNP_E_INVALID, "null q, k, v or out");
        const LaunchTiming tm = pool->timing;
        pool->timing = LaunchTiming();
        if (pool->d.cache_dtype == XNP_BF16 && B.t > kWindowRowByRow) {
            // every row's windowed attention in one MFMA launch (the held rows from the pages, the
            // step's own from k and v), then the rows that stay into their slots
            HIP_TRY(launch_window_prefill(pool->view(), B.bv, layer, q, k, v, out, scale, B.stream, tm), "window attend");
            HIP_TRY(launch_window_append(pool->view(), B.bv, layer, k, v, B.stream), "window append");
            return XNP_OK;
        }
        BatchView bv = B.bv;
        for (int32_t r = 0; r < B.t; r++) {
            bv.wrow = r; // the kernel derives row r's record from the step's
            HIP_TRY(launch_decode(pool->view(), bv, layer, q, k, v, out, scale, true, B.stream,
                                  r == 0 ? tm : LaunchTiming()),
                    "attend");
        }
        return XNP_OK;
    }
    if (pool->batch.open && pool->batch.t > 1) {
        if (!prefill_fuses_append(pool->view())) {
            if (xnp_status st = xnp_append(pool, layer, k, v, hip_stream)) return st;
            return xnp_prefill(pool, layer, q, out, scale, hip_stream);
        }
        // one kernel writes the prompt's K/V rows into the pages and attends over them
        if (xnp_status st = batch_call(pool, layer, hip_stream, false)) return st;
        if (pool->batch.n > 0 && (!q || !k || !v || !out)) return fail(XNP_E_INVALID, "null q, k, v or out");
        const LaunchTiming tm = pool->timing;
        pool->timing = LaunchTiming();
        HIP_TRY(launch_prefill(pool->view(), pool->batch.bv, layer, q, k, v, out, scale, true, pool->batch.stream, tm),
                "attend");
        return XNP_OK;
    }
    if (xnp_status st = batch_call(pool, layer, hip_stream, true)) return st;
    if (pool->batch.n > 0 && (!q || !k || !v || !out)) return fail(XNP_E_INVALID, "null q, k, v or out");
    const LaunchTiming tm = pool->timing;
    pool->timing = LaunchTiming();
    // grouped heads on the VALU decode: every query head's group would append its kv head's row; on
    // an int8 pool, whose append rewrites the page, one kernel appends first and the decode only
    // reads.  The MFMA decode takes a whole kv head per group, so it appends once itself.
    const int G = pool->d.num_heads / pool->d.num_kv_heads;
    const bool fuse = !(pool->d.cache_dtype == XNP_I8 && G > 1) ||
                      decode_heads_per_group(pool->view(), pool->batch.bv.prefix != 0) == G;
    if (!fuse) HIP_TRY(launch_append(pool->view(), pool->batch.bv, layer, k, v, pool->batch.stream), "append");
    HIP_TRY(launch_decode(pool->view(), pool->batch.bv, layer, q, k, v, out, scale, fuse, pool->batch.stream, tm),
            "attend");
    return XNP_OK;
}

extern "C" xnp_status xnp_batch_end(xnp_pool *pool) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    auto &B = pool->batch;
    if (!B.open) return fail(XNP_E_STATE, "no batch is open");
    for (int32_t id : B.ids) {
        Stream &s = pool->streams[id];
        if (s.window) {
            // KvCache::append then trim (transformer.rs:280-316): the last `window` rows stay, the
            // newest in slot p % window
            const int64_t p = (int64_t)s.current_end + s.shift + B.t;
            const int32_t held = (int32_t)std::min<int64_t>(p, s.window);
            for (int32_t sl = s.filled; sl < held; sl++) s.valid[sl] = 1;
            s.nvalid = s.filled = s.current_end = held;
            s.shift = (int32_t)(p - held);
            s.write = (int32_t)(p % s.window);
        } else if (s.ring != RING_NONE) {
            // complete_kv's ring branch, transformer.rs:74-79 (begin refused a valid write slot)
            s.valid[s.write] = 1;
            s.nvalid++;
            s.filled = std::max(s.filled, s.write + 1);
            s.current_end += 1;
        } else {
            s.current_end += B.t;
        }
    }
    B.open = false;
    B.taken.clear();
    return XNP_OK;
}

extern "C" xnp_status xnp_batch_abort(xnp_pool *pool) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    auto &B = pool->batch;
    if (!B.open) return fail(XNP_E_STATE, "no batch is open");
    for (auto it = B.taken.rbegin(); it != B.taken.rend(); ++it) pool->drop_page(it->first, it->second);
    B.taken.clear();
    B.open = false;
    return XNP_OK;
}

// ---------------------------------------------------------------------------------------------
// the rest of the layer: transformer.rs:591-634

extern "C" xnp_status xnp_quantize_rows(const float *w, int32_t rows, int32_t cols, int8_t *q, float *scales) {
    if ((!w || !q || !scales) && rows > 0 && cols > 0) return fail(XNP_E_INVALID, "null argument");
    if (rows < 0 || cols < 0) return fail(XNP_E_INVALID, "a %d x %d matrix", rows, cols);
    for (int32_t r = 0; r < rows; r++) {
        const float *wr = w + (size_t)r * cols;
        float amax = 0.f;
        for (int32_t i = 0; i < cols; i++) amax = std::fmax(amax, std::fabs(wr[i]));
        const float s = amax / 127.0f;
        scales[r] = s;
        for (int32_t i = 0; i < cols; i++) {
            int v = 0;
            if (s > 0.0f) v = (int)std::fmin(std::fmax(std::rint(wr[i] / s), -127.0f), 127.0f);
            q[(size_t)r * cols + i] = (int8_t)v;
        }
    }
    return XNP_OK;
}

extern "C" xnp_status xnp_layer_norm(const void *x, int32_t rows, int32_t dim, const float *w, const float *b,
                                     float eps, void *out, void *hip_stream) {
    if (rows < 0 || dim <= 0 || dim % 512 || dim > 2048)
        return fail(XNP_E_INVALID, "layer norm over %d rows of %d: rows of a multiple of 512 up to 2048", rows, dim);
    if (rows > 0 && (!x || !w || !b || !out)) return fail(XNP_E_INVALID, "null argument");
    HIP_TRY(launch_layer_norm(x, rows, dim, w, b, eps, out, (hipStream_t)hip_stream), "layer norm");
    return XNP_OK;
}

static xnp_status linear_check(int32_t rows, int32_t k, int32_t n) {
    if (rows < 0 || k <= 0 || n <= 0 || k % 64 || n % 64)
        return fail(XNP_E_INVALID, "a q8 linear of %d x %d by %d: k and n must be multiples of 64", rows, k, n);
    return XNP_OK;
}

extern "C" xnp_status xnp_linear_q8(const void *x, int32_t rows, int32_t k, const int8_t *w, const float *s,
                                    int32_t n, int32_t epilogue, void *y, const float *ls, void *hip_stream) {
    if (xnp_status st = linear_check(rows, k, n)) return st;
    if (epilogue < XNP_EPI_STORE || epilogue > XNP_EPI_RESIDUAL) return fail(XNP_E_INVALID, "epilogue %d", epilogue);
    if (rows > 0 && (!x || !w || !s || !y)) return fail(XNP_E_INVALID, "null argument");
    GemmOut go;
    go.out[0] = y;
    go.ld[0] = n;
    go.ls = epilogue == XNP_EPI_RESIDUAL ? ls : nullptr;
    HIP_TRY(launch_gemm_q8(x, rows, k, w, s, n, epilogue, go, (hipStream_t)hip_stream), "q8 linear");
    return XNP_OK;
}

extern "C" xnp_status xnp_flow_linear_q8(const void *x, int32_t x_f32, int32_t rows, int32_t k, const int8_t *w,
                                         const float *s, const float *bias, int32_t n, int32_t epilogue, void *y,
                                         int32_t ldy, const void *aux, int32_t ld_aux, float alpha,
                                         void *hip_stream) {
    if (rows < 0 || k <= 0 || n <= 0 || k % 16 || ldy < n)
        return fail(XNP_E_INVALID, "a q8 linear of %d x %d by %d into rows of %d: k a multiple of 16", rows, k, n, ldy);
    if (epilogue < XNP_EPI_STORE || epilogue > XNP_EPI_ADD_F32) return fail(XNP_E_INVALID, "epilogue %d", epilogue);
    if (x_f32 && epilogue != XNP_EPI_STORE && epilogue != XNP_EPI_ADD_F32)
        return fail(XNP_E_INVALID, "an f32 x takes the store or add epilogue");
    const bool needs_aux = epilogue == XNP_EPI_SILU_ADD || epilogue == XNP_EPI_GATED || epilogue == XNP_EPI_AXPY_F32 ||
                           epilogue == XNP_EPI_ADD_F32;
    if (rows > 0 && (!x || !w || !s || !y || (needs_aux && !aux))) return fail(XNP_E_INVALID, "null argument");
    if ((epilogue == XNP_EPI_GATED || epilogue == XNP_EPI_AXPY_F32) && ld_aux < n)
        return fail(XNP_E_INVALID, "aux rows of %d for %d columns", ld_aux, n);
    if (epilogue == XNP_EPI_ADD_F32 && ld_aux != 0 && ld_aux < n)
        return fail(XNP_E_INVALID, "aux rows of %d for %d columns (0: one row for every row)", ld_aux, n);
    GemmOut go;
    go.out[0] = y, go.ld[0] = ldy, go.bias = bias, go.aux = aux, go.ld_aux = ld_aux, go.alpha = alpha;
    go.a_f32 = x_f32 != 0;
    HIP_TRY(launch_gemm_q8(x, rows, k, w, s, n, epilogue, go, (hipStream_t)hip_stream), "q8 linear");
    return XNP_OK;
}

extern "C" xnp_status xnp_layer_norm_mod(const void *x, int32_t rows, int32_t dim, const float *w, const float *b,
                                         float eps, const void *shift, const void *scale, int32_t ld_mod, void *out,
                                         void *hip_stream) {
    if (rows < 0 || dim <= 0 || dim % 512 || dim > 2048)
        return fail(XNP_E_INVALID, "layer norm over %d rows of %d: rows of a multiple of 512 up to 2048", rows, dim);
    if ((w == nullptr) != (b == nullptr) || (shift == nullptr) != (scale == nullptr))
        return fail(XNP_E_INVALID, "the affine takes w and b, the modulation shift and scale");
    if (shift && (ld_mod < dim || ld_mod % 8)) return fail(XNP_E_INVALID, "modulation rows of %d", ld_mod);
    if (rows > 0 && (!x || !out)) return fail(XNP_E_INVALID, "null argument");
    HIP_TRY(launch_layer_norm_mod(x, rows, dim, w, b, eps, shift, scale, ld_mod, out, (hipStream_t)hip_stream),
            "layer norm");
    return XNP_OK;
}

namespace {
// The layer step's scratch, carved from the caller's workspace: 256-byte aligned bf16 arrays.
struct LayerScratch {
    char *h, *q, *k, *v, *att, *f;
    uint64_t bytes;
};

LayerScratch layer_scratch(char *base, int64_t rows, int64_t dm, int64_t qd, int64_t kd, int64_t ff) {
    LayerScratch L{};
    uint64_t off = 0;
    auto take = [&](int64_t elems) {
        char *p = base ? base + off : nullptr;
        off += align_up((size_t)(elems * 2), 256);
        return p;
    };
    L.h = take(rows * dm);
    L.q = take(rows * qd);
    L.k = take(rows * kd);
    L.v = take(rows * kd);
    L.att = take(rows * qd);
    L.f = take(rows * ff);
    L.bytes = off;
    return L;
}
} // namespace

extern "C" xnp_status xnp_layer_workspace(const xnp_pool *pool, int32_t rows, int32_t d_model, int32_t ff,
                                          uint64_t *bytes) {
    if (!pool || !bytes) return fail(XNP_E_INVALID, "null argument");
    if (rows < 0 || d_model <= 0 || ff <= 0) return fail(XNP_E_INVALID, "rows %d, d_model %d, ff %d", rows, d_model, ff);
    const int64_t qd = (int64_t)pool->d.num_heads * pool->d.head_dim, kd = (int64_t)pool->d.num_kv_heads * pool->d.head_dim;
    *bytes = layer_scratch(nullptr, rows, d_model, qd, kd, ff).bytes;
    return XNP_OK;
}

static xnp_status layer_step_impl(xnp_pool *pool, int32_t layer, const xnp_layer_weights *w, void *x, void *workspace,
                                  uint64_t workspace_bytes, void *hip_stream) {
    if (!pool || !w || !x) return fail(XNP_E_INVALID, "null argument");
    if (xnp_status st = batch_call(pool, layer, hip_stream, pool->batch.t == 1)) return st;
    if (pool->d.act_dtype != XNP_BF16) return fail(XNP_E_INVALID, "the layer step runs on bf16 activations");
    const int32_t dm = w->d_model, ff = w->ff;
    const int32_t H = pool->d.num_heads, KVH = pool->d.num_kv_heads, D = pool->d.head_dim;
    const int32_t qd = H * D, kd = KVH * D, nqkv = qd + 2 * kd;
    if (dm <= 0 || dm % 512 || dm > 2048) return fail(XNP_E_INVALID, "d_model %d: a multiple of 512 up to 2048", dm);
    if (ff <= 0 || ff % 64) return fail(XNP_E_INVALID, "dim_feedforward %d: a multiple of 64", ff);
    if (w->gelu != XNP_GELU_ERF && w->gelu != XNP_GELU_TANH) return fail(XNP_E_INVALID, "gelu %d", w->gelu);
    if (!w->wqkv || !w->sqkv || !w->wout || !w->sout || !w->w1 || !w->s1 || !w->w2 || !w->s2 || !w->ln1_w ||
        !w->ln1_b || !w->ln2_w || !w->ln2_b)
        return fail(XNP_E_INVALID, "a weight of the layer is null");
    const int64_t rows = (int64_t)pool->batch.n * pool->batch.t;
    const LayerScratch need = layer_scratch(nullptr, rows, dm, qd, kd, ff);
    if (!workspace || workspace_bytes < need.bytes)
        return fail(XNP_E_INVALID, "workspace of %llu bytes; the step needs %llu", (unsigned long long)workspace_bytes,
                    (unsigned long long)need.bytes);
    if (rows == 0) return XNP_OK;
    const LayerScratch S = layer_scratch((char *)workspace, rows, dm, qd, kd, ff);
    hipStream_t hs = pool->batch.stream;
    const int M = (int)rows;
    // self-attention block: x + layer_scale_1(out_proj(attn(in_proj(norm1(x)))))
    HIP_TRY(launch_layer_norm(x, M, dm, w->ln1_w, w->ln1_b, 1e-5f, S.h, hs), "norm1");
    GemmOut qkv;
    qkv.nseg = 3;
    qkv.out[0] = S.q, qkv.ld[0] = qd, qkv.col0[0] = 0;
    qkv.out[1] = S.k, qkv.ld[1] = kd, qkv.col0[1] = qd;
    qkv.out[2] = S.v, qkv.ld[2] = kd, qkv.col0[2] = qd + kd;
    HIP_TRY(launch_gemm_q8(S.h, M, dm, w->wqkv, w->sqkv, nqkv, kStore, qkv, hs), "in_proj");
    if (xnp_status st = xnp_attend(pool, layer, S.q, S.k, S.v, S.att, 1.0f / std::sqrt((float)D), hip_stream))
        return st;
    GemmOut res;
    res.out[0] = x, res.ld[0] = dm, res.ls = w->ls1;
    HIP_TRY(launch_gemm_q8(S.att, M, qd, w->wout, w->sout, dm, kResidual, res, hs), "out_proj");
    // feed-forward block: x + layer_scale_2(linear2(gelu(linear1(norm2(x)))))
    HIP_TRY(launch_layer_norm(x, M, dm, w->ln2_w, w->ln2_b, 1e-5f, S.h, hs), "norm2");
    GemmOut hid;
    hid.out[0] = S.f, hid.ld[0] = ff;
    HIP_TRY(launch_gemm_q8(S.h, M, dm, w->w1, w->s1, ff, w->gelu == XNP_GELU_ERF ? kGeluErf : kGeluTanh, hid, hs),
            "linear1");
    res.ls = w->ls2;
    HIP_TRY(launch_gemm_q8(S.f, M, ff, w->w2, w->s2, dm, kResidual, res, hs), "linear2");
    return XNP_OK;
}

extern "C" xnp_status xnp_layer_step(xnp_pool *pool, int32_t layer, const xnp_layer_weights *w, void *x,
                                     void *workspace, uint64_t workspace_bytes, void *hip_stream) {
    return layer_step_impl(pool, layer, w, x, workspace, workspace_bytes, hip_stream);
}

extern "C" xnp_status xnp_layer_step_static(xnp_pool *pool, int32_t layer, const xnp_layer_weights *w, void *x,
                                            void *hip_stream) {
    if (!pool) return fail(XNP_E_INVALID, "null argument");
    if (pool->host_only) return fail(XNP_E_STATE, "a host-only pool runs no kernels");
    void *scr = static_scratch(pool->d.device); // the array's address on the pool's device
    if (!scr) return fail(XNP_E_STATE, "the static scratch of device %d is not set up", pool->d.device);
    if (w && pool->batch.open) {
        const int64_t rows = (int64_t)pool->batch.n * pool->batch.t;
        const int64_t qd = (int64_t)pool->d.num_heads * pool->d.head_dim, kd = (int64_t)pool->d.num_kv_heads * pool->d.head_dim;
        const uint64_t need = layer_scratch(nullptr, rows, w->d_model, qd, kd, w->ff).bytes;
        if (need > kStaticScratchBytes)
            return fail(XNP_E_INVALID, "the step of %lld rows needs %llu bytes of scratch; the static scratch holds %llu",
                        (long long)rows, (unsigned long long)need, (unsigned long long)kStaticScratchBytes);
    }
    // one user of the device's array at a time: a call is refused while another call is issuing its
    // launches, or while the last call's work on another stream may still be running (it waits for
    // nothing)
    hipStream_t hs = (hipStream_t)hip_stream;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(hs, &cap), "hipStreamIsCapturing");
    const bool capturing = cap != hipStreamCaptureStatusNone;
    switch (static_scratch_claim(pool->d.device, hs, capturing)) {
    case ScratchClaim::kOk: break;
    case ScratchClaim::kBusy:
        return fail(XNP_E_STATE, "the static scratch of device %d is in use by another call (one still issuing its "
                                 "launches, or one on another HIP stream that has not finished); synchronize with it "
                                 "or order the calls on one stream from one thread", pool->d.device);
    default: return fail(XNP_E_STATE, "the static scratch of device %d cannot be claimed", pool->d.device);
    }
    const xnp_status st = layer_step_impl(pool, layer, w, x, scr, kStaticScratchBytes, hip_stream);
    const hipError_t rel = static_scratch_release(pool->d.device, hs, capturing); // on every path
    if (st) return st;
    HIP_TRY(rel, "recording the static scratch's last use");
    return XNP_OK;
}
