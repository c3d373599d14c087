/*
 * oracle.c -- CPU restatement of the reference's flow-LM KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP library is compared against (see oracle.h).
 * Built with -ffp-contract=off so that every f32 product and sum is rounded on its own, as the
 * reference's Rust code does (Rust never contracts a*b+c into an fma).
 */
#include "oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];

static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

const char *orc_last_error(void) { return g_err; }

/* ---------------------------------------------------------------------------------------- */
/* element helpers                                                                          */

float orc_bf16_round(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) {
        if (u & 0x007fffffu) u |= 0x00400000u; /* keep NaN a (quiet) NaN */
        u &= 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u); /* round to nearest, ties to even */
        u &= 0xffff0000u;
    }
    memcpy(&x, &u, 4);
    return x;
}

static inline uint16_t bf16_bits(float x) {
    float r = orc_bf16_round(x);
    uint32_t u;
    memcpy(&u, &r, 4);
    return (uint16_t)(u >> 16);
}

static inline float bf16_value(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float x;
    memcpy(&x, &u, 4);
    return x;
}

static inline float round_act(float x, int act_dtype) {
    return act_dtype == ORC_BF16 ? orc_bf16_round(x) : x;
}

int8_t orc_quant(float y, float s) {
    if (!(s > 0.0f)) return 0;
    float r = rintf(y / s);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int8_t)r;
}

/* ---------------------------------------------------------------------------------------- */
/* RoPE: rope.rs:37-63 (tables) and the rope_i rotation of rope.rs:74-95                   */

void orc_rope_row(int head_dim, float max_period, float pos, int act_dtype, float *cos_out,
                  float *sin_out) {
    int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        /* rope.rs:47: 1.0f32 / max_period.powf(i as f32 / half_dim as f32) */
        float inv_freq = 1.0f / powf(max_period, (float)i / (float)half);
        float angle = pos * inv_freq; /* rope.rs:54 */
        cos_out[i] = round_act(cosf(angle), act_dtype);
        sin_out[i] = round_act(sinf(angle), act_dtype);
    }
}

void orc_rotate(int head_dim, float *x, const float *c, const float *s, int act_dtype) {
    for (int i = 0; i < head_dim / 2; i++) {
        float x0 = x[2 * i], x1 = x[2 * i + 1];
        float a = x0 * c[i], b = x1 * s[i];
        float e = x0 * s[i], f = x1 * c[i];
        x[2 * i] = round_act(a - b, act_dtype);
        x[2 * i + 1] = round_act(e + f, act_dtype);
    }
}

/* ---------------------------------------------------------------------------------------- */
/* stream state                                                                             */

struct orc_stream {
    int L, H, KVH, D, cap, cdt, adt;
    float theta;
    void *kc[2];  /* [L][cap][H][D] keys (0) and values (1), element type by cdt */
    float *sc[2]; /* int8: [L][nblk][H] scales */
    int nblk;
    int current_end;
    int ring, write, filled, prefix, shift;
    uint8_t *valid; /* [cap] */
};

static size_t esize(int dt) { return dt == ORC_F32 ? 4 : dt == ORC_BF16 ? 2 : 1; }

orc_stream *orc_open(int layers, int heads, int kv_heads, int head_dim, int capacity,
                     int cache_dtype, int act_dtype, float max_period) {
    if (layers <= 0 || heads <= 0 || head_dim <= 0 || head_dim > 256 || (head_dim & 1) || capacity < 0) {
        fail("bad shape");
        return NULL;
    }
    if (kv_heads <= 0 || heads % kv_heads) {
        fail("the config's %d key/value heads do not divide its %d attention heads", kv_heads,
             heads);
        return NULL;
    }
    if (cache_dtype < 0 || cache_dtype > 2 || act_dtype < 0 || act_dtype > 1) {
        fail("bad dtype");
        return NULL;
    }
    orc_stream *st = calloc(1, sizeof *st);
    st->L = layers;
    st->H = heads;
    st->KVH = kv_heads;
    st->D = head_dim;
    st->cap = capacity;
    st->cdt = cache_dtype;
    st->adt = act_dtype;
    st->theta = max_period;
    st->nblk = (capacity + ORC_BLOCK - 1) / ORC_BLOCK;
    size_t n = (size_t)layers * capacity * heads * head_dim;
    for (int kv = 0; kv < 2; kv++) {
        st->kc[kv] = calloc(n ? n : 1, esize(cache_dtype));
        if (cache_dtype == ORC_I8)
            st->sc[kv] = calloc((size_t)layers * (st->nblk ? st->nblk : 1) * heads, 4);
    }
    st->valid = calloc(capacity ? capacity : 1, 1);
    return st;
}

void orc_close(orc_stream *st) {
    if (!st) return;
    for (int kv = 0; kv < 2; kv++) {
        free(st->kc[kv]);
        free(st->sc[kv]);
    }
    free(st->valid);
    free(st);
}

int orc_current_end(const orc_stream *st) { return st->current_end; }
int orc_capacity(const orc_stream *st) { return st->cap; }

void orc_ring_info(const orc_stream *st, int *mode, int *write, int *filled, int *prefix,
                   int *shift, uint8_t *valid) {
    if (mode) *mode = st->ring;
    if (write) *write = st->write;
    if (filled) *filled = st->filled;
    if (prefix) *prefix = st->prefix;
    if (shift) *shift = st->shift;
    if (valid) memcpy(valid, st->valid, st->cap);
}

static inline size_t idx(const orc_stream *st, int layer, int slot, int h) {
    return (((size_t)layer * st->cap + slot) * st->H + h) * st->D;
}

static inline float *scale_at(const orc_stream *st, int kv, int layer, int blk, int h) {
    return &st->sc[kv][((size_t)layer * st->nblk + blk) * st->H + h];
}

/* The stored element as f32 (dequantized for int8: q * scale, one f32 product). */
static inline float get(const orc_stream *st, int kv, int layer, int slot, int h, int d) {
    size_t i = idx(st, layer, slot, h) + d;
    switch (st->cdt) {
    case ORC_F32: return ((float *)st->kc[kv])[i];
    case ORC_BF16: return bf16_value(((uint16_t *)st->kc[kv])[i]);
    default: return (float)((int8_t *)st->kc[kv])[i] * *scale_at(st, kv, layer, slot / ORC_BLOCK, h);
    }
}

/* Whether a row other than `slot` in slot's block can still be attended to: the int8 rule for
 * starting a block's scale afresh.  Without a ring the rows before `slot` are the filled ones. */
static int block_has_other_row(const orc_stream *st, int slot) {
    int b0 = slot / ORC_BLOCK * ORC_BLOCK;
    if (st->ring == ORC_RING_NONE) return slot > b0;
    int b1 = b0 + ORC_BLOCK < st->cap ? b0 + ORC_BLOCK : st->cap;
    for (int s = b0; s < b1; s++)
        if (s != slot && st->valid[s]) return 1;
    return 0;
}

/* Store one head row x[D] (activation values) at `slot`.  For int8: per-(block, head) scale
 * amax/127; a block holding another live row keeps its scale unless the row needs a larger
 * one, and then every other row of the block is requantized to the larger scale. */
static void store_row(orc_stream *st, int kv, int layer, int slot, int h, const float *x) {
    size_t base = idx(st, layer, slot, h);
    int D = st->D;
    if (st->cdt == ORC_F32) {
        memcpy((float *)st->kc[kv] + base, x, D * 4);
        return;
    }
    if (st->cdt == ORC_BF16) {
        uint16_t *p = (uint16_t *)st->kc[kv] + base;
        for (int d = 0; d < D; d++) p[d] = bf16_bits(x[d]);
        return;
    }
    int8_t *q = (int8_t *)st->kc[kv];
    float *sp = scale_at(st, kv, layer, slot / ORC_BLOCK, h);
    float amax = 0.0f;
    for (int d = 0; d < D; d++) amax = fmaxf(amax, fabsf(x[d]));
    float s_row = amax / 127.0f;
    int fresh = !block_has_other_row(st, slot);
    float s_old = *sp;
    float s_new = fresh ? s_row : fmaxf(s_old, s_row);
    if (!fresh && s_new > s_old) {
        int b0 = slot / ORC_BLOCK * ORC_BLOCK;
        int b1 = b0 + ORC_BLOCK < st->cap ? b0 + ORC_BLOCK : st->cap;
        for (int s = b0; s < b1; s++) {
            if (s == slot) continue;
            int8_t *r = q + idx(st, layer, s, h);
            for (int d = 0; d < D; d++) r[d] = orc_quant((float)r[d] * s_old, s_new);
        }
    }
    for (int d = 0; d < D; d++) q[base + d] = orc_quant(x[d], s_new);
    *sp = s_new;
}

/* The slot the step's row i goes to, or -1 with the error set. */
static int check_append(const orc_stream *st, int t) {
    if (t <= 0) return fail("a step appends at least one row, not %d", t);
    if (st->ring != ORC_RING_NONE) {
        if (t != 1) return fail("a ring cache takes one row at a time, not %d", t);
        if (st->valid[st->write])
            return fail("ring slot %d still holds a row, evict it first", st->write);
        return 0;
    }
    if (st->current_end + t > st->cap)
        return fail("no room left: the cache holds %d positions", st->cap);
    return 0;
}

/* The RoPE position of a key written now at `slot`, step row i. */
static float key_pos(const orc_stream *st, int slot, int i) {
    int p = st->current_end + i;
    if (st->ring == ORC_RING_ABSOLUTE && slot >= st->prefix) p += st->shift;
    return (float)p;
}

int orc_append(orc_stream *st, int layer, int t, const float *k, const float *v) {
    if (layer < 0 || layer >= st->L) return fail("layer %d of %d", layer, st->L);
    if (check_append(st, t)) return -1;
    int H = st->H, D = st->D, group = st->H / st->KVH;
    float *cs = malloc(sizeof(float) * D), *sn = cs + D / 2;
    float *x = malloc(sizeof(float) * D);
    for (int i = 0; i < t; i++) {
        int slot = st->ring != ORC_RING_NONE ? st->write : st->current_end + i;
        orc_rope_row(D, st->theta, key_pos(st, slot, i), st->adt, cs, sn);
        for (int h = 0; h < H; h++) {
            /* transformer.rs:199-211: kv head j serves query heads j*group .. j*group+group-1 */
            const float *src = k + ((size_t)i * st->KVH + h / group) * D;
            memcpy(x, src, D * 4);
            orc_rotate(D, x, cs, sn, st->adt);
            store_row(st, 0, layer, slot, h, x);
            store_row(st, 1, layer, slot, h, v + ((size_t)i * st->KVH + h / group) * D);
        }
    }
    free(cs);
    free(x);
    return 0;
}

/* Row `slot` of head h as f32 (dequantized for int8: q * scale, one f32 product). */
static void load_row(const orc_stream *st, int kv, int layer, int slot, int h, float *out) {
    size_t i = idx(st, layer, slot, h);
    int D = st->D;
    if (st->cdt == ORC_F32) {
        memcpy(out, (float *)st->kc[kv] + i, D * 4);
    } else if (st->cdt == ORC_BF16) {
        const uint16_t *p = (const uint16_t *)st->kc[kv] + i;
        for (int d = 0; d < D; d++) out[d] = bf16_value(p[d]);
    } else {
        const int8_t *p = (const int8_t *)st->kc[kv] + i;
        float s = *scale_at(st, kv, layer, slot / ORC_BLOCK, h);
        for (int d = 0; d < D; d++) out[d] = (float)p[d] * s;
    }
}

/* Attention of step row i, head h, with rotated query rows qw (keys past the prefix) and qp
 * (keys before it; the same as qw except on an absolute ring).  f32 in key order; the f64
 * companion (when out64 is given) from the same operands. */
static void attend_one(const orc_stream *st, int layer, int i, int h, const float *qw,
                       const float *qp, float scale, float *out, double *out64,
                       float *sbuf, double *dbuf) {
    int D = st->D;
    int ring = st->ring != ORC_RING_NONE;
    int span = ring ? (st->filled > st->write + 1 ? st->filled : st->write + 1)
                    : st->current_end + i + 1;
    float kbuf[256];
    float m = -INFINITY;
    double md = -INFINITY;
    for (int j = 0; j < span; j++) {
        int seen = !ring || j == st->write || st->valid[j];
        if (!seen) {
            sbuf[j] = -INFINITY;
            if (out64) dbuf[j] = -INFINITY;
            continue;
        }
        const float *qq = (st->ring == ORC_RING_ABSOLUTE && j < st->prefix) ? qp : qw;
        load_row(st, 0, layer, j, h, kbuf);
        float s = 0.0f;
        for (int d = 0; d < D; d++) s = s + qq[d] * kbuf[d];
        s = s * scale;
        sbuf[j] = s;
        if (s > m) m = s;
        if (out64) {
            double sd = 0.0;
            for (int d = 0; d < D; d++) sd += (double)qq[d] * (double)kbuf[d];
            sd *= (double)scale;
            dbuf[j] = sd;
            if (sd > md) md = sd;
        }
    }
    float l = 0.0f;
    double ld = 0.0;
    for (int j = 0; j < span; j++) {
        float e = sbuf[j] == -INFINITY ? 0.0f : expf(sbuf[j] - m);
        sbuf[j] = e;
        l = l + e;
        if (out64) {
            double ed = dbuf[j] == -INFINITY ? 0.0 : exp(dbuf[j] - md);
            dbuf[j] = ed;
            ld += ed;
        }
    }
    float o[256];
    double od[256];
    for (int d = 0; d < D; d++) {
        o[d] = 0.0f;
        od[d] = 0.0;
    }
    for (int j = 0; j < span; j++) {
        int seen = !ring || j == st->write || st->valid[j];
        if (!seen) continue;
        load_row(st, 1, layer, j, h, kbuf);
        for (int d = 0; d < D; d++) o[d] = o[d] + sbuf[j] * kbuf[d];
        if (out64)
            for (int d = 0; d < D; d++) od[d] += dbuf[j] * (double)kbuf[d];
    }
    for (int d = 0; d < D; d++) {
        out[d] = round_act(o[d] / l, st->adt);
        if (out64) out64[d] = od[d] / ld;
    }
}

int orc_attention(orc_stream *st, int layer, int t, const float *q, float scale, float *out,
                  double *out64) {
    if (layer < 0 || layer >= st->L) return fail("layer %d of %d", layer, st->L);
    if (check_append(st, t)) return -1;
    int H = st->H, D = st->D;
    float *cs = malloc(sizeof(float) * D), *sn = cs + D / 2;
    float *qw = malloc(sizeof(float) * D * 2), *qp = qw + D;
    int span_max = (st->ring != ORC_RING_NONE ? st->cap : st->current_end + t) + 1;
    float *sbuf = malloc(sizeof(float) * span_max);
    double *dbuf = malloc(sizeof(double) * span_max);
    for (int i = 0; i < t; i++) {
        for (int h = 0; h < H; h++) {
            const float *src = q + ((size_t)i * H + h) * D;
            int p = st->current_end + i;
            int pw = p + (st->ring == ORC_RING_ABSOLUTE ? st->shift : 0);
            memcpy(qw, src, D * 4);
            orc_rope_row(D, st->theta, (float)pw, st->adt, cs, sn);
            orc_rotate(D, qw, cs, sn, st->adt);
            memcpy(qp, src, D * 4);
            orc_rope_row(D, st->theta, (float)p, st->adt, cs, sn);
            orc_rotate(D, qp, cs, sn, st->adt);
            attend_one(st, layer, i, h, qw, qp, scale, out + ((size_t)i * H + h) * D,
                       out64 ? out64 + ((size_t)i * H + h) * D : NULL, sbuf, dbuf);
        }
    }
    free(cs);
    free(qw);
    free(sbuf);
    free(dbuf);
    return 0;
}

/* Appending row i of a ring before attending to it: attention must see the new row, which in
 * the reference is valid from complete_kv on (transformer.rs:74-79).  The oracle keeps the ring
 * fields untouched until orc_commit, so attention treats the write slot as seen explicitly. */
int orc_attend(orc_stream *st, int layer, int t, const float *q, const float *k,
               const float *v, float scale, float *out, double *out64) {
    if (orc_append(st, layer, t, k, v)) return -1;
    return orc_attention(st, layer, t, q, scale, out, out64);
}

int orc_commit(orc_stream *st, int t) {
    if (check_append(st, t)) return -1;
    if (st->ring != ORC_RING_NONE) {
        st->valid[st->write] = 1;
        if (st->write + 1 > st->filled) st->filled = st->write + 1;
    }
    st->current_end += t;
    return 0;
}

int orc_advance(orc_stream *st, int n) {
    if (st->ring != ORC_RING_NONE) return fail("a ring cache steps one row at a time");
    if (n < 0 || st->current_end + n > st->cap)
        return fail("no room left: the cache holds %d positions", st->cap);
    st->current_end += n;
    return 0;
}

/* ---------------------------------------------------------------------------------------- */
/* ring: transformer.rs:842-929                                                             */

int orc_start_ring(orc_stream *st, int mode, int prefix) {
    if (mode != ORC_RING_SHIFT && mode != ORC_RING_ABSOLUTE) return fail("bad ring mode %d", mode);
    if (st->ring != ORC_RING_NONE) return fail("the cache is a ring already");
    if (prefix < 0 || prefix > st->cap) return fail("prefix %d of a %d-slot cache", prefix, st->cap);
    int used = st->current_end;
    for (int s = 0; s < st->cap; s++) st->valid[s] = s < used;
    st->ring = mode;
    st->write = used;
    st->filled = used;
    st->prefix = mode == ORC_RING_ABSOLUTE ? prefix : 0;
    st->shift = 0;
    return 0;
}

int orc_ring_restore(orc_stream *st, int mode, int write, int filled, int prefix, int shift,
                     int current_end, const uint8_t *valid) {
    if (mode != ORC_RING_SHIFT && mode != ORC_RING_ABSOLUTE) return fail("bad ring mode %d", mode);
    if (write < 0 || write >= st->cap || filled < 0 || filled > st->cap) return fail("bad ring fields");
    st->ring = mode;
    st->write = write;
    st->filled = filled;
    st->prefix = prefix;
    st->shift = shift;
    st->current_end = current_end;
    memcpy(st->valid, valid, st->cap);
    return 0;
}

int orc_set_ring_slot(orc_stream *st, int slot) {
    if (st->ring == ORC_RING_NONE) return fail("not a ring cache, see start_ring");
    if (slot < 0 || slot >= st->cap) return fail("slot %d of a %d-slot ring", slot, st->cap);
    st->write = slot;
    return 0;
}

int orc_evict(orc_stream *st, int prefix, const int *slots, int count) {
    if (st->ring == ORC_RING_NONE) return fail("not a ring cache, see start_ring");
    if (count > st->current_end)
        return fail("cannot evict %d of %d positions", count, st->current_end);
    if (st->ring == ORC_RING_ABSOLUTE && prefix != st->prefix)
        return fail("an absolute ring evicts past its prefix %d, not %d", st->prefix, prefix);
    if (st->ring == ORC_RING_SHIFT && st->cdt == ORC_I8)
        return fail("an int8 cache evicts on an absolute ring");
    /* Every slot is checked before any changes (transformer.rs:896-901). */
    for (int j = 0; j < count; j++) {
        int s = slots[j];
        if (s < prefix || s < 0 || s >= st->cap || !st->valid[s])
            return fail("slot %d holds no row past the prefix", s);
    }
    for (int j = 0; j < count; j++) st->valid[slots[j]] = 0;
    if (st->ring == ORC_RING_SHIFT && count > 0) {
        /* transformer.rs:905-925: every kept row past the prefix is rotated by -count where
         * it lies, with the shift_back table of rope.rs:26-35 (rows of position -count). */
        int D = st->D;
        float *cs = malloc(sizeof(float) * D), *sn = cs + D / 2, *x = malloc(sizeof(float) * D);
        orc_rope_row(D, st->theta, -(float)count, st->adt, cs, sn);
        for (int s = prefix; s < st->filled; s++) {
            if (!st->valid[s]) continue;
            for (int layer = 0; layer < st->L; layer++)
                for (int h = 0; h < st->H; h++) {
                    for (int d = 0; d < D; d++) x[d] = get(st, 0, layer, s, h, d);
                    orc_rotate(D, x, cs, sn, st->adt);
                    store_row(st, 0, layer, s, h, x);
                }
        }
        free(cs);
        free(x);
    }
    if (st->ring == ORC_RING_ABSOLUTE) st->shift += count;
    st->current_end -= count;
    return 0;
}

/* ---------------------------------------------------------------------------------------- */
/* with_seq_budget: transformer.rs:350-392                                                  */

orc_stream *orc_with_seq_budget(const orc_stream *st, int budget) {
    if (st->ring != ORC_RING_NONE) {
        fail("a ring cache cannot be resized");
        return NULL;
    }
    int used = st->current_end;
    if (used > budget) {
        fail("cannot fit %d filled KV positions into a budget of %d", used, budget);
        return NULL;
    }
    orc_stream *dst = orc_open(st->L, st->H, st->KVH, st->D, budget, st->cdt, st->adt, st->theta);
    size_t row = (size_t)st->H * st->D * esize(st->cdt);
    for (int kv = 0; kv < 2; kv++)
        for (int layer = 0; layer < st->L; layer++) {
            memcpy((char *)dst->kc[kv] + idx(dst, layer, 0, 0) * esize(st->cdt),
                   (char *)st->kc[kv] + idx(st, layer, 0, 0) * esize(st->cdt), row * used);
            if (st->cdt == ORC_I8) {
                int nb = (used + ORC_BLOCK - 1) / ORC_BLOCK;
                memcpy(scale_at(dst, kv, layer, 0, 0), scale_at(st, kv, layer, 0, 0),
                       sizeof(float) * nb * st->H);
            }
        }
    dst->current_end = used;
    return dst;
}

/* ---------------------------------------------------------------------------------------- */
/* raw rows                                                                                 */

static int check_rows(const orc_stream *st, int layer, int kv, int slot0, int n) {
    if (layer < 0 || layer >= st->L || kv < 0 || kv > 1) return fail("bad layer or kv");
    if (slot0 < 0 || n < 0 || slot0 + n > st->cap)
        return fail("rows %d..%d of a %d-slot cache", slot0, slot0 + n, st->cap);
    return 0;
}

int orc_read_rows(const orc_stream *st, int layer, int kv, int slot0, int n, float *vals,
                  int8_t *q8, float *scales) {
    if (check_rows(st, layer, kv, slot0, n)) return -1;
    int H = st->H, D = st->D;
    for (int s = 0; s < n; s++)
        for (int h = 0; h < H; h++)
            for (int d = 0; d < D; d++) {
                size_t o = ((size_t)s * H + h) * D + d;
                if (vals) vals[o] = get(st, kv, layer, slot0 + s, h, d);
                if (q8 && st->cdt == ORC_I8)
                    q8[o] = ((int8_t *)st->kc[kv])[idx(st, layer, slot0 + s, h) + d];
            }
    if (scales && st->cdt == ORC_I8 && n > 0) {
        int b0 = slot0 / ORC_BLOCK, b1 = (slot0 + n - 1) / ORC_BLOCK;
        for (int b = b0; b <= b1; b++)
            memcpy(scales + (size_t)(b - b0) * H, scale_at(st, kv, layer, b, 0), sizeof(float) * H);
    }
    return 0;
}

int orc_write_rows(orc_stream *st, int layer, int kv, int slot0, int n, const float *vals,
                   const int8_t *q8, const float *scales) {
    if (check_rows(st, layer, kv, slot0, n)) return -1;
    int H = st->H, D = st->D;
    for (int s = 0; s < n; s++)
        for (int h = 0; h < H; h++) {
            size_t o = ((size_t)s * H + h) * D;
            size_t i = idx(st, layer, slot0 + s, h);
            if (st->cdt == ORC_F32)
                memcpy((float *)st->kc[kv] + i, vals + o, D * 4);
            else if (st->cdt == ORC_BF16)
                for (int d = 0; d < D; d++) ((uint16_t *)st->kc[kv])[i + d] = bf16_bits(vals[o + d]);
            else
                memcpy((int8_t *)st->kc[kv] + i, q8 + o, D);
        }
    if (st->cdt == ORC_I8 && n > 0) {
        int b0 = slot0 / ORC_BLOCK, b1 = (slot0 + n - 1) / ORC_BLOCK;
        for (int b = b0; b <= b1; b++)
            memcpy(scale_at(st, kv, layer, b, 0), scales + (size_t)(b - b0) * H, sizeof(float) * H);
    }
    return 0;
}

/* voice_from_kv_cache (ptts-wasm/src/lib.rs:291-325): the voice's f32 rows kv [2][n][H][D]
 * (keys, already rotated, then values) become rows [0, n) of one layer, stored in the cache dtype.
 * int8 has no counterpart in the reference; the policy here is one scale per (block, head),
 * amax / 127 over the block's rows, and codes rint(x / s), as a block whose rows all arrive at
 * once would take them. */
int orc_load_kv(orc_stream *st, int layer, const float *kv, int n) {
    if (check_rows(st, layer, 0, 0, n)) return -1;
    if (st->ring != ORC_RING_NONE) return fail("a voice loads into a plain cache, not a ring");
    if (n != st->current_end)
        return fail("a %d-row voice loads into a stream holding exactly as many rows, not %d", n,
                    st->current_end);
    const int H = st->H, D = st->D;
    for (int which = 0; which < 2; which++) {
        const float *src = kv + (size_t)which * n * H * D;
        if (st->cdt != ORC_I8) {
            if (orc_write_rows(st, layer, which, 0, n, src, NULL, NULL)) return -1;
            continue;
        }
        for (int b0 = 0; b0 < n; b0 += ORC_BLOCK) {
            const int rows = n - b0 < ORC_BLOCK ? n - b0 : ORC_BLOCK;
            for (int h = 0; h < H; h++) {
                float amax = 0.f;
                for (int r = 0; r < rows; r++)
                    for (int d = 0; d < D; d++)
                        amax = fmaxf(amax, fabsf(src[((size_t)(b0 + r) * H + h) * D + d]));
                const float sc = amax / 127.0f;
                for (int r = 0; r < rows; r++) {
                    int8_t *dst = (int8_t *)st->kc[which] + idx(st, layer, b0 + r, h);
                    for (int d = 0; d < D; d++) dst[d] = orc_quant(src[((size_t)(b0 + r) * H + h) * D + d], sc);
                }
                *scale_at(st, which, layer, b0 / ORC_BLOCK, h) = sc;
            }
        }
    }
    return 0;
}

/* ---------------------------------------------------------------------------------------- */
/* Mimi's attention cache: KvCache (transformer.rs:257-318), MimiStreamingMultiheadAttention::  */
/* forward (:428-468) and the window mask of StreamingTransformer::forward (:764-781)          */

struct orc_window {
    int L, H, D, context, rows_max, adt;
    float theta;
    float *k, *v; /* [L][context - 1 + rows_max][H][D]: the kept rows then this step's, in order */
    int len;      /* KvCache::current_seq_len: rows kept between steps (at most context - 1) */
    int offset;   /* KvCache::absolute_offset: rows appended so far */
};

orc_window *orc_window_open(int layers, int heads, int head_dim, int context, int rows_max, int act_dtype,
                            float max_period) {
    if (layers <= 0 || heads <= 0 || head_dim <= 0 || head_dim > 256 || (head_dim & 1) || context <= 0 ||
        rows_max <= 0 || act_dtype < 0 || act_dtype > 1) {
        fail("bad window shape");
        return NULL;
    }
    orc_window *w = calloc(1, sizeof *w);
    w->L = layers, w->H = heads, w->D = head_dim, w->context = context, w->rows_max = rows_max;
    w->adt = act_dtype, w->theta = max_period;
    const size_t n = (size_t)layers * (context - 1 + rows_max) * heads * head_dim;
    w->k = calloc(n, sizeof(float));
    w->v = calloc(n, sizeof(float));
    return w;
}

void orc_window_close(orc_window *w) {
    if (!w) return;
    free(w->k);
    free(w->v);
    free(w);
}

int orc_window_len(const orc_window *w) { return w->len; }
int orc_window_offset(const orc_window *w) { return w->offset; }

static float *win_row(const orc_window *w, float *base, int layer, int r, int h) {
    return base + (((size_t)layer * (w->context - 1 + w->rows_max) + r) * w->H + h) * w->D;
}

/* One layer of a step of t rows: append (KvCache::append, keys rotated at absolute_offset + i as
 * RotaryEmbedding::new(head_dim, offset, t) gives them, stored in the activation dtype), then row
 * i attends key j of the len + t rows when j <= len + i < j + context (:771-775; with t = 1 the
 * reference passes no mask, and every row is inside the window).  Softmax in f32 in key order, as
 * orc_attention; out64 (nullable) the f64 companion. */
int orc_window_attend(orc_window *w, int layer, int t, const float *q, const float *k, const float *v, float scale,
                      float *out, double *out64) {
    if (layer < 0 || layer >= w->L) return fail("layer %d of %d", layer, w->L);
    if (t <= 0 || t > w->rows_max) return fail("a step of %d rows, at most %d", t, w->rows_max);
    const int H = w->H, D = w->D, n = w->len + t;
    float cs[256], qr[256], x[256], kb[256];
    float *sn = cs + D / 2;
    float *sbuf = malloc(sizeof(float) * n);
    double *dbuf = malloc(sizeof(double) * n);
    for (int i = 0; i < t; i++) {
        orc_rope_row(D, w->theta, (float)(w->offset + i), w->adt, cs, sn);
        for (int h = 0; h < H; h++) {
            memcpy(x, k + ((size_t)i * H + h) * D, D * 4);
            orc_rotate(D, x, cs, sn, w->adt);
            memcpy(win_row(w, w->k, layer, w->len + i, h), x, D * 4);
            const float *vs = v + ((size_t)i * H + h) * D;
            float *vd = win_row(w, w->v, layer, w->len + i, h);
            for (int d = 0; d < D; d++) vd[d] = round_act(vs[d], w->adt);
        }
    }
    for (int i = 0; i < t; i++) {
        const int seq = w->len + i;
        orc_rope_row(D, w->theta, (float)(w->offset + i), w->adt, cs, sn);
        for (int h = 0; h < H; h++) {
            memcpy(qr, q + ((size_t)i * H + h) * D, D * 4);
            orc_rotate(D, qr, cs, sn, w->adt);
            float m = -INFINITY;
            double md = -INFINITY;
            for (int j = 0; j < n; j++) {
                if (!(j <= seq && seq < j + w->context)) {
                    sbuf[j] = -INFINITY;
                    dbuf[j] = -INFINITY;
                    continue;
                }
                const float *kr = win_row(w, w->k, layer, j, h);
                float sc = 0.0f;
                double sd = 0.0;
                for (int d = 0; d < D; d++) {
                    sc = sc + qr[d] * kr[d];
                    sd += (double)qr[d] * (double)kr[d];
                }
                sbuf[j] = sc * scale;
                dbuf[j] = sd * (double)scale;
                if (sbuf[j] > m) m = sbuf[j];
                if (dbuf[j] > md) md = dbuf[j];
            }
            float l = 0.0f;
            double ld = 0.0;
            for (int j = 0; j < n; j++) {
                sbuf[j] = sbuf[j] == -INFINITY ? 0.0f : expf(sbuf[j] - m);
                dbuf[j] = dbuf[j] == -INFINITY ? 0.0 : exp(dbuf[j] - md);
                l = l + sbuf[j];
                ld += dbuf[j];
            }
            float o[256];
            double od[256];
            for (int d = 0; d < D; d++) o[d] = 0.0f, od[d] = 0.0;
            for (int j = 0; j < n; j++) {
                if (!(j <= seq && seq < j + w->context)) continue;
                memcpy(kb, win_row(w, w->v, layer, j, h), D * 4);
                for (int d = 0; d < D; d++) {
                    o[d] = o[d] + sbuf[j] * kb[d];
                    od[d] += dbuf[j] * (double)kb[d];
                }
            }
            for (int d = 0; d < D; d++) {
                out[((size_t)i * H + h) * D + d] = round_act(o[d] / l, w->adt);
                if (out64) out64[((size_t)i * H + h) * D + d] = od[d] / ld;
            }
        }
    }
    free(sbuf);
    free(dbuf);
    return 0;
}

/* After every layer took the step: absolute_offset += t, then KvCache::trim (:300-316) keeps the
 * last context - 1 rows. */
int orc_window_commit(orc_window *w, int t) {
    if (t <= 0 || t > w->rows_max) return fail("a step of %d rows, at most %d", t, w->rows_max);
    w->offset += t;
    const int n = w->len + t, keep = w->context - 1;
    if (n <= keep) {
        w->len = n;
        return 0;
    }
    const int drop = n - keep;
    for (int l = 0; l < w->L; l++) {
        memmove(win_row(w, w->k, l, 0, 0), win_row(w, w->k, l, drop, 0), sizeof(float) * keep * w->H * w->D);
        memmove(win_row(w, w->v, l, 0, 0), win_row(w, w->v, l, drop, 0), sizeof(float) * keep * w->H * w->D);
    }
    w->len = keep;
    return 0;
}

/* The kept rows [len][H][D] of one layer, keys (kv 0) or values (1), oldest first. */
int orc_window_rows(const orc_window *w, int layer, int kv, float *rows) {
    if (layer < 0 || layer >= w->L || kv < 0 || kv > 1) return fail("bad layer or kv");
    memcpy(rows, win_row(w, kv ? w->v : w->k, layer, 0, 0), sizeof(float) * w->len * w->H * w->D);
    return 0;
}

/* ---------------------------------------------------------------------------------------- */
/* the rest of the layer: transformer.rs:591-634                                            */

void orc_layer_norm(const float *x, int rows, int dim, const float *w, const float *b, float eps,
                    int act_dtype, float *out) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * dim;
        float sum = 0.f;
        for (int i = 0; i < dim; i++) sum += xr[i];
        const float mean = sum / (float)dim;
        float sq = 0.f;
        for (int i = 0; i < dim; i++) {
            float d = xr[i] - mean;
            sq += d * d;
        }
        const float rstd = 1.0f / sqrtf(sq / (float)dim + eps);
        float *o = out + (size_t)r * dim;
        for (int i = 0; i < dim; i++) {
            float y = (xr[i] - mean) * rstd;
            o[i] = round_act(y * w[i] + b[i], act_dtype);
        }
    }
}

void orc_quantize_rows(const float *w, int rows, int cols, int8_t *q, float *scales) {
    for (int r = 0; r < rows; r++) {
        const float *wr = w + (size_t)r * cols;
        float amax = 0.f;
        for (int i = 0; i < cols; i++) amax = fmaxf(amax, fabsf(wr[i]));
        const float s = amax / 127.0f;
        scales[r] = s;
        for (int i = 0; i < cols; i++) q[(size_t)r * cols + i] = orc_quant(wr[i], s);
    }
}

void orc_linear_q8(const float *x, int rows, int k, const int8_t *q, const float *s, int n,
                   int act_dtype, float *y) {
    for (int m = 0; m < rows; m++)
        for (int j = 0; j < n; j++) {
            const float *xr = x + (size_t)m * k;
            const int8_t *qr = q + (size_t)j * k;
            float acc = 0.f;
            for (int i = 0; i < k; i++) acc += xr[i] * (float)qr[i];
            y[(size_t)m * n + j] = round_act(s[j] * acc, act_dtype);
        }
}

float orc_gelu(float x, int kind) {
    if (kind == 1) {
        const float c = 0.7978845608028654f; /* sqrt(2 / pi) */
        return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
    }
    return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f));
}

static int layer_step_one(orc_stream *st, int t, int layer, const orc_layer_weights *w, float scale,
                          float *x) {
    const int dm = w->d_model, H = st->H, KVH = st->KVH, D = st->D, adt = st->adt;
    const int qd = H * D, kd = KVH * D, nqkv = qd + 2 * kd;
    float *h = malloc(sizeof(float) * (size_t)t * dm);
    float *qkv = malloc(sizeof(float) * (size_t)t * nqkv);
    float *q = malloc(sizeof(float) * (size_t)t * qd);
    float *k = malloc(sizeof(float) * (size_t)t * kd);
    float *v = malloc(sizeof(float) * (size_t)t * kd);
    float *att = malloc(sizeof(float) * (size_t)t * qd);
    float *y = malloc(sizeof(float) * (size_t)t * dm);
    float *f = malloc(sizeof(float) * (size_t)t * w->ff);
    /* self-attention block: x + layer_scale_1(attn(norm1(x))) */
    orc_layer_norm(x, t, dm, w->ln1_w, w->ln1_b, 1e-5f, adt, h);
    orc_linear_q8(h, t, dm, w->wqkv, w->sqkv, nqkv, adt, qkv);
    for (int i = 0; i < t; i++) { /* narrow into q, k, v (transformer.rs:195-211) */
        memcpy(q + (size_t)i * qd, qkv + (size_t)i * nqkv, sizeof(float) * qd);
        memcpy(k + (size_t)i * kd, qkv + (size_t)i * nqkv + qd, sizeof(float) * kd);
        memcpy(v + (size_t)i * kd, qkv + (size_t)i * nqkv + qd + kd, sizeof(float) * kd);
    }
    int rc = orc_attend(st, layer, t, q, k, v, scale, att, NULL);
    if (rc == 0) {
        orc_linear_q8(att, t, qd, w->wout, w->sout, dm, adt, y);
        for (size_t i = 0; i < (size_t)t * dm; i++) {
            float a = w->ls1 ? round_act(y[i] * w->ls1[i % dm], adt) : y[i];
            x[i] = round_act(x[i] + a, adt);
        }
        /* feed-forward block: x + layer_scale_2(linear2(gelu(linear1(norm2(x))))) */
        orc_layer_norm(x, t, dm, w->ln2_w, w->ln2_b, 1e-5f, adt, h);
        orc_linear_q8(h, t, dm, w->w1, w->s1, w->ff, adt, f);
        for (size_t i = 0; i < (size_t)t * w->ff; i++) f[i] = round_act(orc_gelu(f[i], w->gelu), adt);
        orc_linear_q8(f, t, w->ff, w->w2, w->s2, dm, adt, y);
        for (size_t i = 0; i < (size_t)t * dm; i++) {
            float a = w->ls2 ? round_act(y[i] * w->ls2[i % dm], adt) : y[i];
            x[i] = round_act(x[i] + a, adt);
        }
    }
    free(h); free(qkv); free(q); free(k); free(v); free(att); free(y); free(f);
    return rc;
}

int orc_layer_step(orc_stream **streams, int n, int t, int layer, const orc_layer_weights *w,
                   float scale, float *x) {
    if (n <= 0) return 0;
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(| : bad)
    for (int i = 0; i < n; i++)
        bad |= layer_step_one(streams[i], t, layer, w, scale, x + (size_t)i * t * w->d_model) != 0;
    return bad ? fail("a stream refused the step") : 0;
}

/* ---------------------------------------------------------------------------------------- */
/* the flow LM around the transformer (flow_lm.rs, mlp.rs, conditioners.rs), f32            */

#define ORC_MAXL 64

typedef struct {
    size_t embed, in_lin, bos;
    size_t ln1_w[ORC_MAXL], ln1_b[ORC_MAXL], wqkv[ORC_MAXL], wout[ORC_MAXL];
    size_t ln2_w[ORC_MAXL], ln2_b[ORC_MAXL], w1[ORC_MAXL], w2[ORC_MAXL];
    size_t on_w, on_b, z_proj, eos_w, eos_b;
    size_t te_freqs[2], te_w1[2], te_b1[2], te_w2[2], te_b2[2], te_alpha[2];
    size_t cond_w, cond_b, inp_w, inp_b;
    size_t rb_lnw[ORC_MAXL], rb_lnb[ORC_MAXL], rb_w1[ORC_MAXL], rb_b1[ORC_MAXL];
    size_t rb_w2[ORC_MAXL], rb_b2[ORC_MAXL], rb_aw[ORC_MAXL], rb_ab[ORC_MAXL];
    size_t fin_aw, fin_ab, fin_w, fin_b;
    size_t total;
    int zd; /* the width out_eos and cond_embed read: z_dim, else d_model */
    int ad; /* the attention's query and output width: attn_dim, else d_model */
    int kd; /* its key and value width: ad / num_heads x num_kv_heads (transformer.rs:162) */
} flow_layout;

static int flow_layout_of(const orc_flow_lm_desc *d, flow_layout *L) {
    const int ad = d->attn_dim ? d->attn_dim : d->d_model, kvh = d->num_kv_heads ? d->num_kv_heads : d->num_heads;
    if (d->num_layers <= 0 || d->num_layers > ORC_MAXL || d->flow_depth < 0 || d->flow_depth > ORC_MAXL ||
        d->d_model <= 0 || d->num_heads <= 0 || d->ldim <= 0 || d->flow_dim <= 0 || d->ff <= 0 ||
        d->n_bins <= 0 || d->z_dim < 0 || d->attn_dim < 0 || d->num_kv_heads < 0 || ad % d->num_heads ||
        kvh > d->num_heads || d->num_heads % kvh || d->flow_type < 0 || d->flow_type > 2 ||
        (d->flow_type == 0 && d->lsd_steps <= 0) || d->precision < 0 || d->precision > 1)
        return fail("bad flow LM shape");
    const size_t dm = d->d_model, F = d->flow_dim, ld = d->ldim, ff = d->ff, fq = ORC_FREQ_DIM;
    const size_t zd = d->z_dim ? (size_t)d->z_dim : dm;
    L->zd = (int)zd;
    L->ad = ad;
    L->kd = ad / d->num_heads * kvh;
    size_t o = 0;
#define TAKE(field, n) (L->field = o, o += (size_t)(n))
    TAKE(embed, (d->n_bins + 1) * dm);
    TAKE(in_lin, dm * ld);
    TAKE(bos, ld);
    for (int l = 0; l < d->num_layers; l++) {
        TAKE(ln1_w[l], dm); TAKE(ln1_b[l], dm);
        TAKE(wqkv[l], ((size_t)L->ad + 2 * (size_t)L->kd) * dm); TAKE(wout[l], dm * (size_t)L->ad);
        TAKE(ln2_w[l], dm); TAKE(ln2_b[l], dm);
        TAKE(w1[l], ff * dm); TAKE(w2[l], dm * ff);
    }
    TAKE(on_w, dm); TAKE(on_b, dm);
    TAKE(z_proj, d->z_dim ? zd * dm : 0);
    TAKE(eos_w, zd); TAKE(eos_b, 1);
    for (int i = 0; i < (d->flow_type == 0 ? 2 : 0); i++) { /* num_time_conds: 2 for Lsd, else 0 */
        TAKE(te_freqs[i], fq / 2); TAKE(te_w1[i], F * fq); TAKE(te_b1[i], F);
        TAKE(te_w2[i], F * F); TAKE(te_b2[i], F); TAKE(te_alpha[i], F);
    }
    TAKE(cond_w, F * zd); TAKE(cond_b, F);
    TAKE(inp_w, F * ld); TAKE(inp_b, F);
    for (int j = 0; j < d->flow_depth; j++) {
        TAKE(rb_lnw[j], F); TAKE(rb_lnb[j], F);
        TAKE(rb_w1[j], F * F); TAKE(rb_b1[j], F);
        TAKE(rb_w2[j], F * F); TAKE(rb_b2[j], F);
        TAKE(rb_aw[j], 3 * F * F); TAKE(rb_ab[j], 3 * F);
    }
    TAKE(fin_aw, 2 * F * F); TAKE(fin_ab, 2 * F);
    TAKE(fin_w, ld * F); TAKE(fin_b, ld);
#undef TAKE
    L->total = o;
    return 0;
}

long long orc_flow_lm_size(const orc_flow_lm_desc *d) {
    flow_layout L;
    if (flow_layout_of(d, &L)) return -1;
    return (long long)L.total;
}

/* y[m][j] = sum_k x[m][k] w[j][k] (+ b[j]), f32, k ascending: xn's Linear (load: no bias; load_b). */
void orc_linear_f32(const float *x, int rows, int k, const float *w, const float *b, int n, float *y) {
    /* output channels in parallel: each is summed by one thread in the same order, so the result
     * does not depend on the thread count */
#pragma omp parallel for collapse(2) schedule(static) if ((long long)rows * n * k >= (1 << 18))
    for (int m = 0; m < rows; m++)
        for (int j = 0; j < n; j++) {
            const float *xr = x + (size_t)m * k, *wr = w + (size_t)j * k;
            float acc = 0.f;
            for (int i = 0; i < k; i++) acc += xr[i] * wr[i];
            y[(size_t)m * n + j] = b ? acc + b[j] : acc;
        }
}

static inline float silu(float x) { return x / (1.0f + expf(-x)); }

/* TimestepEmbedder::forward (mlp.rs:55-67) for one time t, then its norm (mlp.rs:69-86). */
static void time_embed_one(const orc_flow_lm_desc *d, const float *blob, const flow_layout *L, int i, float t,
                           float *out) {
    const int F = d->flow_dim, half = ORC_FREQ_DIM / 2;
    float emb[ORC_FREQ_DIM];
    const float *fr = blob + L->te_freqs[i];
    for (int j = 0; j < half; j++) {
        float a = t * fr[j];
        emb[j] = cosf(a);
        emb[half + j] = sinf(a);
    }
    float *h = malloc(sizeof(float) * F);
    orc_linear_f32(emb, 1, ORC_FREQ_DIM, blob + L->te_w1[i], blob + L->te_b1[i], F, h);
    for (int j = 0; j < F; j++) h[j] = silu(h[j]);
    orc_linear_f32(h, 1, F, blob + L->te_w2[i], blob + L->te_b2[i], F, out);
    const float *alpha = blob + L->te_alpha[i];
    const float eps = 1e-5f, n = (float)F;
    if (d->time_norm == 1) { /* RmsVar: centred, unbiased variance */
        float s = 0.f;
        for (int j = 0; j < F; j++) s += out[j];
        const float mean = s * (1.0f / n);
        float v = 0.f;
        for (int j = 0; j < F; j++) {
            float e = out[j] - mean;
            v += e * e;
        }
        const float inv = 1.0f / sqrtf(v * (1.0f / (n - 1.0f)) + eps);
        for (int j = 0; j < F; j++) out[j] = out[j] * inv * alpha[j];
    } else { /* Rms: x * alpha / sqrt(mean(x^2) + eps) */
        float s = 0.f;
        for (int j = 0; j < F; j++) s += out[j] * out[j];
        const float inv = 1.0f / sqrtf(s * (1.0f / n) + eps);
        for (int j = 0; j < F; j++) out[j] = out[j] * inv * alpha[j];
    }
    free(h);
}

int orc_flow_time_embedding(const orc_flow_lm_desc *d, const float *blob, float s, float t, float *out) {
    flow_layout L;
    if (flow_layout_of(d, &L)) return -1;
    if (d->flow_type != 0) return fail("a head without time conditions has no time embedding");
    const int F = d->flow_dim;
    float *b = malloc(sizeof(float) * F);
    time_embed_one(d, blob, &L, 0, s, out);
    time_embed_one(d, blob, &L, 1, t, b);
    for (int j = 0; j < F; j++) out[j] = (out[j] + b[j]) * 0.5f; /* mlp.rs:205-212 */
    free(b);
    return 0;
}

/* LayerNorm without rounding, f32, optional affine, then modulate (mlp.rs:4-11) when shift/scale
 * are given: y * (1 + scale) + shift. */
static void ln_mod(const float *x, int n, const float *w, const float *b, float eps, const float *shift,
                   const float *scale, float *out) {
    float s = 0.f;
    for (int i = 0; i < n; i++) s += x[i];
    const float mean = s / (float)n;
    float q = 0.f;
    for (int i = 0; i < n; i++) {
        float e = x[i] - mean;
        q += e * e;
    }
    const float rstd = 1.0f / sqrtf(q / (float)n + eps);
    for (int i = 0; i < n; i++) {
        float y = (x[i] - mean) * rstd;
        if (w) y = y * w[i] + b[i];
        if (shift) y = y * (scale[i] + 1.0f) + shift[i];
        out[i] = y;
    }
}

int orc_flow_net(const orc_flow_lm_desc *d, const float *blob, const float *c, const float *t_emb,
                 const float *x0, float *out) {
    flow_layout L;
    if (flow_layout_of(d, &L)) return -1;
    const int F = d->flow_dim, ld = d->ldim;
    float *x = malloc(sizeof(float) * F), *y = malloc(sizeof(float) * F), *ya = malloc(sizeof(float) * F);
    float *ada = malloc(sizeof(float) * 3 * F), *h = malloc(sizeof(float) * F), *h2 = malloc(sizeof(float) * F);
    orc_linear_f32(x0, 1, ld, blob + L.inp_w, blob + L.inp_b, F, x);     /* input_proj */
    orc_linear_f32(c, 1, L.zd, blob + L.cond_w, blob + L.cond_b, F, y); /* cond_embed */
    for (int j = 0; j < F; j++) ya[j] = silu(t_emb ? t_emb[j] + y[j] : y[j]); /* y = t + c (or c); silu */
    for (int r = 0; r < d->flow_depth; r++) {                            /* ResBlock (mlp.rs:113-131) */
        orc_linear_f32(ya, 1, F, blob + L.rb_aw[r], blob + L.rb_ab[r], 3 * F, ada);
        ln_mod(x, F, blob + L.rb_lnw[r], blob + L.rb_lnb[r], 1e-6f, ada, ada + F, h);
        orc_linear_f32(h, 1, F, blob + L.rb_w1[r], blob + L.rb_b1[r], F, h2);
        for (int j = 0; j < F; j++) h2[j] = silu(h2[j]);
        orc_linear_f32(h2, 1, F, blob + L.rb_w2[r], blob + L.rb_b2[r], F, h);
        for (int j = 0; j < F; j++) x[j] = x[j] + ada[2 * F + j] * h[j];
    }
    orc_linear_f32(ya, 1, F, blob + L.fin_aw, blob + L.fin_ab, 2 * F, ada); /* FinalLayer (mlp.rs:155-163) */
    ln_mod(x, F, NULL, NULL, 1e-6f, ada, ada + F, h);
    orc_linear_f32(h, 1, F, blob + L.fin_w, blob + L.fin_b, ld, out);
    free(x); free(y); free(ya); free(ada); free(h); free(h2);
    return 0;
}

/* The transformer over t rows of one stream (transformer.rs:591-634, f32 weights), x [t][d]. */
static int flow_transformer(const orc_flow_lm_desc *d, const float *blob, const flow_layout *L, orc_stream *st,
                            int t, float *x) {
    const int dm = d->d_model, ff = d->ff, H = d->num_heads, ad = L->ad, kd = L->kd, D = ad / H, nq = ad + 2 * kd;
    float *h = malloc(sizeof(float) * (size_t)t * dm), *qkv = malloc(sizeof(float) * (size_t)t * nq);
    float *q = malloc(sizeof(float) * (size_t)t * ad), *k = malloc(sizeof(float) * (size_t)t * kd);
    float *v = malloc(sizeof(float) * (size_t)t * kd), *att = malloc(sizeof(float) * (size_t)t * ad);
    float *f = malloc(sizeof(float) * (size_t)t * ff);
    int rc = 0;
    for (int l = 0; l < d->num_layers && rc == 0; l++) {
        orc_layer_norm(x, t, dm, blob + L->ln1_w[l], blob + L->ln1_b[l], 1e-5f, ORC_F32, h);
        orc_linear_f32(h, t, dm, blob + L->wqkv[l], NULL, nq, qkv);
        for (int i = 0; i < t; i++) { /* q, then k, then v (transformer.rs:195-211) */
            memcpy(q + (size_t)i * ad, qkv + (size_t)i * nq, sizeof(float) * ad);
            memcpy(k + (size_t)i * kd, qkv + (size_t)i * nq + ad, sizeof(float) * kd);
            memcpy(v + (size_t)i * kd, qkv + (size_t)i * nq + ad + kd, sizeof(float) * kd);
        }
        rc = orc_attend(st, l, t, q, k, v, 1.0f / sqrtf((float)D), att, NULL);
        if (rc) break;
        orc_linear_f32(att, t, ad, blob + L->wout[l], NULL, dm, h);
        for (size_t i = 0; i < (size_t)t * dm; i++) x[i] += h[i];
        orc_layer_norm(x, t, dm, blob + L->ln2_w[l], blob + L->ln2_b[l], 1e-5f, ORC_F32, h);
        orc_linear_f32(h, t, dm, blob + L->w1[l], NULL, ff, f);
        for (size_t i = 0; i < (size_t)t * ff; i++) f[i] = orc_gelu(f[i], d->gelu);
        orc_linear_f32(f, t, ff, blob + L->w2[l], NULL, dm, h);
        for (size_t i = 0; i < (size_t)t * dm; i++) x[i] += h[i];
    }
    if (rc == 0) rc = orc_commit(st, t);
    free(h); free(qkv); free(q); free(k); free(v); free(att); free(f);
    return rc;
}

int orc_flow_lm_prompt_text(const orc_flow_lm_desc *d, const float *blob, orc_stream *st, const int *ids, int n) {
    flow_layout L;
    if (flow_layout_of(d, &L)) return -1;
    if (n <= 0) return 0;
    const int dm = d->d_model;
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] > d->n_bins) return fail("token id %d is past the %d-entry embedding table", ids[i], d->n_bins + 1);
    float *x = malloc(sizeof(float) * (size_t)n * dm);
    for (int i = 0; i < n; i++) memcpy(x + (size_t)i * dm, blob + L.embed + (size_t)ids[i] * dm, sizeof(float) * dm);
    int rc = flow_transformer(d, blob, &L, st, n, x); /* tts_model.rs:297-307, 455-466 */
    free(x);
    return rc;
}

int orc_flow_lm_step(const orc_flow_lm_desc *d, const float *blob, orc_stream *st, const float *latent_in,
                     const float *cond, const float *noise, float *latent_out, float *eos_logit) {
    flow_layout L;
    if (flow_layout_of(d, &L)) return -1;
    if (d->precision != 0) return fail("a q8 flow LM steps through orc_flow_q8_step");
    const int dm = d->d_model, F = d->flow_dim, ld = d->ldim;
    float *x = malloc(sizeof(float) * dm), *t_out = malloc(sizeof(float) * dm), *temb = malloc(sizeof(float) * F);
    float *cur = malloc(sizeof(float) * ld), *dir = malloc(sizeof(float) * ld);
    float *z = malloc(sizeof(float) * L.zd);
    /* input_linear of the previous latent, or of bos_emb on the first step (flow_lm.rs:314-324) */
    orc_linear_f32(latent_in ? latent_in : blob + L.bos, 1, ld, blob + L.in_lin, NULL, dm, x);
    if (cond) /* the conditions, broadcast-added to the step input (flow_lm.rs:304-307) */
        for (int j = 0; j < dm; j++) x[j] = x[j] + cond[j];
    int rc = flow_transformer(d, blob, &L, st, 1, x);
    if (rc == 0) {
        ln_mod(x, dm, blob + L.on_w, blob + L.on_b, 1e-5f, NULL, NULL, t_out); /* out_norm (flow_lm.rs:315) */
        if (d->z_dim) orc_linear_f32(t_out, 1, dm, blob + L.z_proj, NULL, d->z_dim, z); /* :320-323 */
        else memcpy(z, t_out, sizeof(float) * dm);
        orc_linear_f32(z, 1, L.zd, blob + L.eos_w, blob + L.eos_b, 1, eos_logit);
        memcpy(cur, noise, sizeof(float) * ld);
        if (d->flow_type == 0) {
            const float step_scale = 1.0f / (float)d->lsd_steps;
            for (int i = 0; i < d->lsd_steps; i++) { /* lsd_decode (flow_lm.rs:97-110) */
                orc_flow_time_embedding(d, blob, (float)i / (float)d->lsd_steps, (float)(i + 1) / (float)d->lsd_steps,
                                        temb);
                orc_flow_net(d, blob, z, temb, cur, dir);
                for (int j = 0; j < ld; j++) cur[j] = cur[j] + dir[j] * step_scale;
            }
        } else { /* Drifting: flow_net(c, None, noise); Pointwise: noise + the same (:380-381) */
            orc_flow_net(d, blob, z, NULL, noise, dir);
            for (int j = 0; j < ld; j++) cur[j] = d->flow_type == 2 ? noise[j] + dir[j] : dir[j];
        }
        memcpy(latent_out, cur, sizeof(float) * ld);
    }
    free(x); free(t_out); free(temb); free(cur); free(dir); free(z);
    return rc;
}

/* ---------------------------------------------------------------------------------------- */
/* the flow LM in q8 precision: int8 per-channel weights, bf16 activations                   */

/* The flow net's q8 linear (the batched frame's GEMM and its epilogues): y = bf16(s[j] * sum_k
 * bf16(x[m][k]) q[j][k] (+ b[j])), then epi 0 store; 4 silu; 5 silu(bf16(y + aux[j])); 6
 * out = bf16(out + bf16(aux[m][j] * y)); 7 out = bf16(bf16(aux[m][j]) + bf16(y * alpha)); 8 store (the
 * f32 output is the bf16 value).  out [rows][ldo] (read by 6), aux rows of stride ld_aux. */
void orc_flow_linear_q8(const float *x, int rows, int k, const int8_t *q, const float *s, const float *b, int n,
                        int epi, float *out, int ldo, const float *aux, int ld_aux, float alpha) {
    for (int m = 0; m < rows; m++)
        for (int j = 0; j < n; j++) {
            const float *xr = x + (size_t)m * k;
            const int8_t *qr = q + (size_t)j * k;
            float acc = 0.f;
            for (int i = 0; i < k; i++) acc += orc_bf16_round(xr[i]) * (float)qr[i];
            const float y = orc_bf16_round(b ? s[j] * acc + b[j] : s[j] * acc);
            float *o = out + (size_t)m * ldo + j;
            switch (epi) {
            case 4: *o = orc_bf16_round(silu(y)); break;
            case 5: *o = orc_bf16_round(silu(orc_bf16_round(y + aux[j]))); break;
            case 6: *o = orc_bf16_round(*o + orc_bf16_round(aux[(size_t)m * ld_aux + j] * y)); break;
            case 7:
                *o = orc_bf16_round(orc_bf16_round(aux[(size_t)m * ld_aux + j]) + orc_bf16_round(y * alpha));
                break;
            case 9: *o = orc_bf16_round(orc_bf16_round(aux[(size_t)m * ld_aux + j]) + y); break;
            default: *o = y;
            }
        }
}

/* LayerNorm of bf16 rows (w, b: the affine, or NULL) rounded once, then, when shift is given, the
 * AdaLN modulation in bf16 steps: bf16(bf16(y * bf16(scale + 1)) + shift) (shift and scale rows of
 * stride ld_mod). */
void orc_layer_norm_mod(const float *x, int rows, int dim, const float *w, const float *b, float eps,
                        const float *shift, const float *scale, int ld_mod, float *out) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * dim;
        float sum = 0.f;
        for (int i = 0; i < dim; i++) sum += xr[i];
        const float mean = sum / (float)dim;
        float q = 0.f;
        for (int i = 0; i < dim; i++) {
            float e = xr[i] - mean;
            q += e * e;
        }
        const float rstd = 1.0f / sqrtf(q / (float)dim + eps);
        for (int i = 0; i < dim; i++) {
            float y = (xr[i] - mean) * rstd;
            if (w) y = y * w[i] + b[i];
            y = orc_bf16_round(y);
            if (shift) {
                const float sc1 = orc_bf16_round(scale[(size_t)r * ld_mod + i] + 1.0f);
                y = orc_bf16_round(orc_bf16_round(y * sc1) + shift[(size_t)r * ld_mod + i]);
            }
            out[(size_t)r * dim + i] = y;
        }
    }
}

typedef struct {
    int8_t *q;
    float *s;
    int n, k;
} qlin;

struct orc_flow_q8 {
    orc_flow_lm_desc d;
    flow_layout L;
    const float *blob; /* the caller's: biases, norms, the LUT */
    qlin in_lin, wqkv[ORC_MAXL], wout[ORC_MAXL], w1[ORC_MAXL], w2[ORC_MAXL], z, eos, cond, inp;
    qlin rb1[ORC_MAXL], rb2[ORC_MAXL], rba[ORC_MAXL], fina, finw;
    orc_layer_weights lw[ORC_MAXL];
    float *temb; /* [steps][F], rounded to bf16 */
};

static void qlin_make(qlin *w, const float *src, int n, int k) {
    w->n = n, w->k = k;
    w->q = malloc((size_t)n * k);
    w->s = malloc(sizeof(float) * n);
    orc_quantize_rows(src, n, k, w->q, w->s);
}

static void qlin_free(qlin *w) {
    free(w->q);
    free(w->s);
}

/* the flow net's q8 linear on one prepared weight */
static void q8lin_epi(const float *x, int rows, const qlin *w, const float *b, int epi, float *out, const float *aux,
                      int ld_aux, float alpha) {
    orc_flow_linear_q8(x, rows, w->k, w->q, w->s, b, w->n, epi, out, w->n, aux, ld_aux, alpha);
}

static void q8lin(const float *x, int rows, const qlin *w, const float *b, float *y) {
    q8lin_epi(x, rows, w, b, 0, y, NULL, 0, 1.f);
}

orc_flow_q8 *orc_flow_q8_prepare(const orc_flow_lm_desc *d, const float *blob) {
    flow_layout L;
    if (flow_layout_of(d, &L)) return NULL;
    if (d->precision != 1) {
        fail("orc_flow_q8_prepare takes a q8 desc");
        return NULL;
    }
    orc_flow_q8 *m = calloc(1, sizeof *m);
    m->d = *d, m->L = L, m->blob = blob;
    const int dm = d->d_model, F = d->flow_dim, ld = d->ldim, ff = d->ff, zd = L.zd;
    qlin_make(&m->in_lin, blob + L.in_lin, dm, ld);
    for (int l = 0; l < d->num_layers; l++) {
        qlin_make(&m->wqkv[l], blob + L.wqkv[l], L.ad + 2 * L.kd, dm);
        qlin_make(&m->wout[l], blob + L.wout[l], dm, L.ad);
        qlin_make(&m->w1[l], blob + L.w1[l], ff, dm);
        qlin_make(&m->w2[l], blob + L.w2[l], dm, ff);
        orc_layer_weights *w = &m->lw[l];
        w->d_model = dm, w->ff = ff, w->gelu = d->gelu;
        w->wqkv = m->wqkv[l].q, w->sqkv = m->wqkv[l].s, w->wout = m->wout[l].q, w->sout = m->wout[l].s;
        w->w1 = m->w1[l].q, w->s1 = m->w1[l].s, w->w2 = m->w2[l].q, w->s2 = m->w2[l].s;
        w->ln1_w = blob + L.ln1_w[l], w->ln1_b = blob + L.ln1_b[l];
        w->ln2_w = blob + L.ln2_w[l], w->ln2_b = blob + L.ln2_b[l];
    }
    if (d->z_dim) qlin_make(&m->z, blob + L.z_proj, d->z_dim, dm);
    qlin_make(&m->eos, blob + L.eos_w, 1, zd);
    qlin_make(&m->cond, blob + L.cond_w, F, zd);
    qlin_make(&m->inp, blob + L.inp_w, F, ld);
    for (int r = 0; r < d->flow_depth; r++) {
        qlin_make(&m->rb1[r], blob + L.rb_w1[r], F, F);
        qlin_make(&m->rb2[r], blob + L.rb_w2[r], F, F);
        qlin_make(&m->rba[r], blob + L.rb_aw[r], 3 * F, F);
    }
    qlin_make(&m->fina, blob + L.fin_aw, 2 * F, F);
    qlin_make(&m->finw, blob + L.fin_w, ld, F);
    const int steps = d->flow_type == 0 ? d->lsd_steps : 0;
    m->temb = calloc((size_t)(steps ? steps : 1) * F, sizeof(float));
    for (int i = 0; i < steps; i++) {
        float *t = m->temb + (size_t)i * F;
        orc_flow_time_embedding(d, blob, (float)i / (float)steps, (float)(i + 1) / (float)steps, t);
        for (int j = 0; j < F; j++) t[j] = orc_bf16_round(t[j]);
    }
    return m;
}

void orc_flow_q8_free(orc_flow_q8 *m) {
    if (!m) return;
    qlin_free(&m->in_lin);
    for (int l = 0; l < m->d.num_layers; l++) {
        qlin_free(&m->wqkv[l]);
        qlin_free(&m->wout[l]);
        qlin_free(&m->w1[l]);
        qlin_free(&m->w2[l]);
    }
    if (m->d.z_dim) qlin_free(&m->z);
    qlin_free(&m->eos);
    qlin_free(&m->cond);
    qlin_free(&m->inp);
    for (int r = 0; r < m->d.flow_depth; r++) {
        qlin_free(&m->rb1[r]);
        qlin_free(&m->rb2[r]);
        qlin_free(&m->rba[r]);
    }
    qlin_free(&m->fina);
    qlin_free(&m->finw);
    free(m->temb);
    free(m);
}

static int q8_transformer(orc_flow_q8 *m, orc_stream *st, int t, float *x) {
    const float scale = 1.0f / sqrtf((float)(m->L.ad / m->d.num_heads));
    for (int l = 0; l < m->d.num_layers; l++)
        if (layer_step_one(st, t, l, &m->lw[l], scale, x)) return -1;
    return orc_commit(st, t);
}

int orc_flow_q8_prompt_text(orc_flow_q8 *m, orc_stream *st, const int *ids, int n) {
    if (n <= 0) return 0;
    const int dm = m->d.d_model;
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] > m->d.n_bins)
            return fail("token id %d is past the %d-entry embedding table", ids[i], m->d.n_bins + 1);
    float *x = malloc(sizeof(float) * (size_t)n * dm);
    for (int i = 0; i < n; i++)
        for (int j = 0; j < dm; j++)
            x[(size_t)i * dm + j] = orc_bf16_round(m->blob[m->L.embed + (size_t)ids[i] * dm + j]);
    int rc = q8_transformer(m, st, n, x);
    free(x);
    return rc;
}

int orc_flow_q8_step(orc_flow_q8 *m, orc_stream *st, const float *latent_in, const float *cond, const float *noise,
                     float *latent_out, float *eos_logit) {
    const orc_flow_lm_desc *d = &m->d;
    const flow_layout *L = &m->L;
    const float *blob = m->blob;
    const int dm = d->d_model, F = d->flow_dim, ld = d->ldim, zd = L->zd;
    float *x = malloc(sizeof(float) * dm), *t_out = malloc(sizeof(float) * dm), *z = malloc(sizeof(float) * zd);
    float *ya = malloc(sizeof(float) * F), *xf = malloc(sizeof(float) * F), *ada = malloc(sizeof(float) * 3 * F);
    float *h = malloc(sizeof(float) * F), *h2 = malloc(sizeof(float) * F), *cur = malloc(sizeof(float) * ld);
    q8lin(latent_in ? latent_in : blob + L->bos, 1, &m->in_lin, NULL, x); /* input_linear (flow_lm.rs:314-324) */
    if (cond) /* the conditions, a bf16 tensor add (flow_lm.rs:304-307) */
        for (int j = 0; j < dm; j++) x[j] = orc_bf16_round(x[j] + orc_bf16_round(cond[j]));
    int rc = q8_transformer(m, st, 1, x);
    if (rc == 0) {
        orc_layer_norm_mod(x, 1, dm, blob + L->on_w, blob + L->on_b, 1e-5f, NULL, NULL, 0, t_out); /* out_norm */
        if (d->z_dim) q8lin(t_out, 1, &m->z, NULL, z);
        else memcpy(z, t_out, sizeof(float) * dm);
        q8lin(z, 1, &m->eos, blob + L->eos_b, eos_logit);
        memcpy(cur, noise, sizeof(float) * ld);
        const int steps = d->flow_type == 0 ? d->lsd_steps : 1;
        const float alpha = d->flow_type == 0 ? 1.0f / (float)steps : 1.0f;
        for (int i = 0; i < steps; i++) {
            /* cond_embed, then y = t + c (or c), silu (mlp.rs:214-238) */
            q8lin_epi(z, 1, &m->cond, blob + L->cond_b, d->flow_type == 0 ? 5 : 4, ya, m->temb + (size_t)i * F, 0, 1.f);
            q8lin(cur, 1, &m->inp, blob + L->inp_b, xf); /* input_proj (x rounded to bf16 as it is read) */
            for (int r = 0; r < d->flow_depth; r++) {  /* ResBlock (mlp.rs:113-131) */
                q8lin(ya, 1, &m->rba[r], blob + L->rb_ab[r], ada);
                orc_layer_norm_mod(xf, 1, F, blob + L->rb_lnw[r], blob + L->rb_lnb[r], 1e-6f, ada, ada + F, 3 * F, h);
                q8lin_epi(h, 1, &m->rb1[r], blob + L->rb_b1[r], 4, h2, NULL, 0, 1.f);
                q8lin_epi(h2, 1, &m->rb2[r], blob + L->rb_b2[r], 6, xf, ada + 2 * F, 3 * F, 1.f);
            }
            q8lin(ya, 1, &m->fina, blob + L->fin_ab, ada); /* FinalLayer (mlp.rs:155-163) */
            orc_layer_norm_mod(xf, 1, F, NULL, NULL, 1e-6f, ada, ada + F, 2 * F, h);
            /* Lsd: x + v / steps; Pointwise: noise + v; Drifting: v */
            q8lin_epi(h, 1, &m->finw, blob + L->fin_b, d->flow_type == 1 ? 8 : 7, cur, cur, ld, alpha);
        }
        memcpy(latent_out, cur, sizeof(float) * ld);
    }
    free(x); free(t_out); free(z); free(ya); free(xf); free(ada); free(h); free(h2); free(cur);
    return rc;
}

/* ---------------------------------------------------------------------------------------- */
/* batched CPU step (the CPU baseline): one thread per stream, OpenMP across streams        */

int orc_batch_attend(orc_stream **streams, int n, int layer, const float *q, const float *k,
                     const float *v, float scale, float *out) {
    if (n <= 0) return 0;
    int H = streams[0]->H, KVH = streams[0]->KVH, D = streams[0]->D;
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(| : bad)
    for (int i = 0; i < n; i++) {
        bad |= orc_attend(streams[i], layer, 1, q + (size_t)i * H * D, k + (size_t)i * KVH * D,
                          v + (size_t)i * KVH * D, scale, out + (size_t)i * H * D, NULL) != 0;
    }
    return bad ? fail("a stream refused the step") : 0;
}

int orc_batch_commit(orc_stream **streams, int n) {
    for (int i = 0; i < n; i++)
        if (orc_commit(streams[i], 1)) return -1;
    return 0;
}

/* One single-row ring step on each of n streams, OpenMP across streams: evict slot drop[i] after
 * prefix 0 when drop[i] >= 0, take slot set[i] for the next row, then append row i of k and v to
 * `layer` (q null) or attend with row i of q as well (orc_attend, out row i), and commit the row.
 * The per-stream calls of the s2s session loop (s2s.rs:324-333: evict, set_ring_slot, then the
 * step) composed, for tests that mirror many streams. */
int orc_batch_ring_step(orc_stream **streams, int n, int layer, const int *drop, const int *set, const float *q,
                        const float *k, const float *v, float scale, float *out) {
    if (n <= 0) return 0;
    int H = streams[0]->H, KVH = streams[0]->KVH, D = streams[0]->D;
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 16) reduction(| : bad)
    for (int i = 0; i < n; i++) {
        orc_stream *st = streams[i];
        const float *ki = k + (size_t)i * KVH * D, *vi = v + (size_t)i * KVH * D;
        if (drop[i] >= 0 && orc_evict(st, 0, &drop[i], 1)) { bad = 1; continue; }
        if (orc_set_ring_slot(st, set[i])) { bad = 1; continue; }
        const int rc = q ? orc_attend(st, layer, 1, q + (size_t)i * H * D, ki, vi, scale, out + (size_t)i * H * D, NULL)
                         : orc_append(st, layer, 1, ki, vi);
        if (rc) { bad = 1; continue; }
        bad |= orc_commit(st, 1) != 0;
    }
    return bad ? fail("a stream refused the ring step") : 0;
}

void orc_set_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
