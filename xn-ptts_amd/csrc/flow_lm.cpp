// Host side of the flow LM around the paged transformer (ptts/src/flow_lm.rs, mlp.rs,
// conditioners.rs, tts_model.rs:297-378): weights uploaded once, then text prompts and frames for
// batches of a pool's streams.  Two precisions: f32 (k_layer.hip's f32 linears with the norms
// fused, the pool's xnp_attend), and q8 (int8 weights on the MFMA GEMM with its epilogues, bf16
// activations, the transformer as xnp_layer_step).
#include "../../include/xnp_kv.h"
#include "xnp_internal.h"

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

using namespace xnp;

namespace {

constexpr int kFreqDim = 256; // the time embedders' frequency embedding (mlp.rs:186-193)
constexpr int kMaxLayers = 64;

// Offsets (in floats) of the weight blob's tensors, in the order include/xnp_kv.h documents.
struct Layout {
    size_t embed, in_lin, bos;
    size_t ln1_w[kMaxLayers], ln1_b[kMaxLayers], wqkv[kMaxLayers], wout[kMaxLayers];
    size_t ln2_w[kMaxLayers], ln2_b[kMaxLayers], w1[kMaxLayers], w2[kMaxLayers];
    size_t on_w, on_b, z_proj, eos_w, eos_b;
    size_t te_freqs[2], te_w1[2], te_b1[2], te_w2[2], te_b2[2], te_alpha[2];
    size_t cond_w, cond_b, inp_w, inp_b;
    size_t rb_lnw[kMaxLayers], rb_lnb[kMaxLayers], rb_w1[kMaxLayers], rb_b1[kMaxLayers];
    size_t rb_w2[kMaxLayers], rb_b2[kMaxLayers], rb_aw[kMaxLayers], rb_ab[kMaxLayers];
    size_t fin_aw, fin_ab, fin_w, fin_b;
    size_t total;
    int zd; // the width out_eos and cond_embed read: z_dim, else d_model
    int ad; // the attention's query and output width: attn_dim, else d_model
    int kd; // its key and value width: ad / num_heads x num_kv_heads
};

bool layout_of(const xnp_flow_lm_desc &d, Layout &L) {
    const int ad = d.attn_dim ? d.attn_dim : d.d_model, kvh = d.num_kv_heads ? d.num_kv_heads : d.num_heads;
    if (d.num_layers <= 0 || d.num_layers > kMaxLayers || d.flow_depth < 0 || d.flow_depth > kMaxLayers ||
        d.d_model <= 0 || d.num_heads <= 0 || d.ldim <= 0 || d.flow_dim <= 0 || d.ff <= 0 || d.n_bins <= 0 ||
        d.z_dim < 0 || d.attn_dim < 0 || d.num_kv_heads < 0 || ad % d.num_heads || kvh > d.num_heads ||
        d.num_heads % kvh || d.flow_type < XNP_FLOW_LSD || d.flow_type > XNP_FLOW_POINTWISE ||
        (d.flow_type == XNP_FLOW_LSD && d.lsd_steps <= 0) || (d.precision != XNP_FLOW_F32 && d.precision != XNP_FLOW_Q8))
        return false;
    const size_t dm = d.d_model, F = d.flow_dim, ld = d.ldim, ff = d.ff, fq = kFreqDim;
    const size_t zd = d.z_dim ? (size_t)d.z_dim : dm;
    L.zd = (int)zd;
    L.ad = ad;
    L.kd = ad / d.num_heads * kvh; // StreamingMultiheadAttention::load's kv_dim (transformer.rs:162)
    const size_t qkv = (size_t)L.ad + 2 * (size_t)L.kd;
    size_t o = 0;
    auto take = [&](size_t &field, size_t n) { field = o, o += n; };
    take(L.embed, ((size_t)d.n_bins + 1) * dm);
    take(L.in_lin, dm * ld);
    take(L.bos, ld);
    for (int l = 0; l < d.num_layers; l++) {
        take(L.ln1_w[l], dm), take(L.ln1_b[l], dm), take(L.wqkv[l], qkv * dm), take(L.wout[l], dm * L.ad);
        take(L.ln2_w[l], dm), take(L.ln2_b[l], dm), take(L.w1[l], ff * dm), take(L.w2[l], dm * ff);
    }
    take(L.on_w, dm), take(L.on_b, dm), take(L.z_proj, d.z_dim ? zd * dm : 0);
    take(L.eos_w, zd), take(L.eos_b, 1);
    for (int i = 0; i < (d.flow_type == XNP_FLOW_LSD ? 2 : 0); i++) { // num_time_conds (flow_lm.rs:225-228)
        take(L.te_freqs[i], fq / 2), take(L.te_w1[i], F * fq), take(L.te_b1[i], F);
        take(L.te_w2[i], F * F), take(L.te_b2[i], F), take(L.te_alpha[i], F);
    }
    take(L.cond_w, F * zd), take(L.cond_b, F), take(L.inp_w, F * ld), take(L.inp_b, F);
    for (int j = 0; j < d.flow_depth; j++) {
        take(L.rb_lnw[j], F), take(L.rb_lnb[j], F), take(L.rb_w1[j], F * F), take(L.rb_b1[j], F);
        take(L.rb_w2[j], F * F), take(L.rb_b2[j], F), take(L.rb_aw[j], 3 * F * F), take(L.rb_ab[j], 3 * F);
    }
    take(L.fin_aw, 2 * F * F), take(L.fin_ab, 2 * F), take(L.fin_w, ld * F), take(L.fin_b, ld);
    L.total = o;
    return true;
}

float host_bf16(float x) { return bf16_round_host(x); }

uint16_t host_bf16_bits(float x) {
    const float r = bf16_round_host(x);
    uint32_t u;
    std::memcpy(&u, &r, 4);
    return (uint16_t)(u >> 16);
}

// y = x W^T + b on the host, f32, k ascending (the time embedders, computed once at load).
void host_linear(const float *x, int k, const float *w, const float *b, int n, float *y) {
    for (int j = 0; j < n; j++) {
        float acc = 0.f;
        for (int i = 0; i < k; i++) acc += x[i] * w[(size_t)j * k + i];
        y[j] = acc + b[j];
    }
}

// TimestepEmbedder::forward and its norm (mlp.rs:55-86) for time t.
void host_time_embed(const xnp_flow_lm_desc &d, const float *blob, const Layout &L, int i, float t, float *out) {
    const int F = d.flow_dim, half = kFreqDim / 2;
    float emb[kFreqDim];
    for (int j = 0; j < half; j++) {
        const float a = t * blob[L.te_freqs[i] + j];
        emb[j] = cosf(a);
        emb[half + j] = sinf(a);
    }
    std::vector<float> h(F);
    host_linear(emb, kFreqDim, blob + L.te_w1[i], blob + L.te_b1[i], F, h.data());
    for (int j = 0; j < F; j++) h[j] = h[j] / (1.0f + expf(-h[j]));
    host_linear(h.data(), F, blob + L.te_w2[i], blob + L.te_b2[i], F, out);
    const float *alpha = blob + L.te_alpha[i];
    const float eps = 1e-5f, n = (float)F;
    if (d.time_norm == XNP_TIME_RMS_VAR) { // centred, unbiased variance
        float s = 0.f;
        for (int j = 0; j < F; j++) s += out[j];
        const float mean = s * (1.0f / n);
        float v = 0.f;
        for (int j = 0; j < F; j++) {
            const float e = out[j] - mean;
            v += e * e;
        }
        const float inv = 1.0f / sqrtf(v * (1.0f / (n - 1.0f)) + eps);
        for (int j = 0; j < F; j++) out[j] = out[j] * inv * alpha[j];
    } else { // x * alpha / sqrt(mean(x^2) + eps)
        float s = 0.f;
        for (int j = 0; j < F; j++) s += out[j] * out[j];
        const float inv = 1.0f / sqrtf(s * (1.0f / n) + eps);
        for (int j = 0; j < F; j++) out[j] = out[j] * inv * alpha[j];
    }
}

} // namespace

// A linear's int8 weights [n][k] and f32 scales [n] on the device.
struct Q8Lin {
    int8_t *q = nullptr;
    float *s = nullptr;
};

// A recorded frame: the launches of xnp_flow_lm_step for one batch size and one set of buffers.
struct FlowGraph {
    hipGraphExec_t exec = nullptr;
    int32_t n = 0;
    const float *latent_in = nullptr, *noise = nullptr, *cond = nullptr;
    float *latent_out = nullptr, *eos = nullptr;
    hipStream_t stream = nullptr;
    BatchLaunchKey key; // the batch's kernel choice when recorded
};

struct xnp_flow_lm {
    FlowGraph graph;
    xnp_pool *pool = nullptr;
    xnp_flow_lm_desc d{};
    Layout L{};
    float *w = nullptr;    // the weight blob on the device
    float *temb = nullptr; // [lsd_steps][F]: SimpleMLPAdaLN::time_embedding of each solver step (q8: rounded)
    // every residual block's adaLN_modulation then the final layer's, stacked: [na][F] and [na].
    // They all read the same conditioning vector, so one launch computes them together.
    float *adaw = nullptr, *adab = nullptr;
    int32_t na = 0; // flow_depth * 3F + 2F
    // f32 scratch for max_rows rows
    float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *f = nullptr;
    float *ya = nullptr, *ada = nullptr, *xf = nullptr, *h2 = nullptr, *z = nullptr;
    // q8: int8 weights with per-output-channel scales (device), the LUT rounded to bf16, bos_emb
    // repeated per row (input_linear's A operand), the layer step's weights and workspace, and
    // bf16 scratch for max_rows rows
    Q8Lin in_lin, wqkv[kMaxLayers], wout[kMaxLayers], w1[kMaxLayers], w2[kMaxLayers], zp, eos, cond, inp;
    Q8Lin rb1[kMaxLayers], rb2[kMaxLayers], adaq, finw;
    uint16_t *lut = nullptr;
    float *bos_rows = nullptr;
    xnp_layer_weights lw[kMaxLayers]{};
    void *ws = nullptr;
    uint64_t ws_bytes = 0;
    uint16_t *bx = nullptr, *btout = nullptr, *bz = nullptr, *bya = nullptr, *bxf = nullptr, *bada = nullptr;
    uint16_t *bh = nullptr, *bh2 = nullptr;
    int32_t *dids = nullptr;
    int32_t *hids = nullptr; // pinned staging of token ids
    float *cond_vec = nullptr; // [d_model]: the model's summed conditions (condition_providers)
    bool has_cond = false;     // cond_vec is set
    std::vector<void *> allocs;
    const float *W(size_t off) const { return w + off; }
};

static void fl_free(xnp_flow_lm *lm) {
    if (lm->graph.exec) (void)hipGraphExecDestroy(lm->graph.exec);
    for (void *p : lm->allocs) (void)hipFree(p);
    if (lm->hids) (void)hipHostFree(lm->hids);
    delete lm;
}

extern "C" xnp_status xnp_flow_lm_weights_size(const xnp_flow_lm_desc *desc, int64_t *nfloats) {
    if (!desc || !nfloats) return pool_fail(XNP_E_INVALID, "null argument");
    Layout L;
    if (!layout_of(*desc, L)) return pool_fail(XNP_E_INVALID, "bad flow LM shape");
    *nfloats = (int64_t)L.total;
    return XNP_OK;
}

extern "C" xnp_status xnp_flow_lm_create(xnp_pool *pool, const xnp_flow_lm_desc *desc, const float *weights,
                                         int64_t nfloats, xnp_flow_lm **out) {
    if (!pool || !desc || !weights || !out) return pool_fail(XNP_E_INVALID, "null argument");
    *out = nullptr;
    const xnp_pool_desc &pd = *pool_desc(pool);
    const xnp_flow_lm_desc &d = *desc;
    Layout L;
    if (!layout_of(d, L)) return pool_fail(XNP_E_INVALID, "bad flow LM shape");
    if ((int64_t)L.total != nfloats)
        return pool_fail(XNP_E_INVALID, "the weights hold %lld floats; the layout needs %lld", (long long)nfloats,
                         (long long)L.total);
    if (pool_host_only(pool)) return pool_fail(XNP_E_STATE, "a host-only pool has no device");
    const bool q8 = d.precision == XNP_FLOW_Q8;
    if (!q8 && (pd.cache_dtype != XNP_F32 || pd.act_dtype != XNP_F32))
        return pool_fail(XNP_E_INVALID, "the f32 flow LM runs on an f32 pool (f32 cache and activations)");
    if (q8 && (pd.cache_dtype != XNP_BF16 || pd.act_dtype != XNP_BF16))
        return pool_fail(XNP_E_INVALID, "the q8 flow LM runs on a bf16 pool (bf16 cache and activations)");
    if (pd.num_layers != d.num_layers || pd.num_heads != d.num_heads ||
        pd.num_kv_heads != (d.num_kv_heads ? d.num_kv_heads : d.num_heads) || pd.head_dim * d.num_heads != L.ad)
        return pool_fail(XNP_E_INVALID, "the pool's layers and heads do not match the flow LM's (%d x %d heads of %d "
                                        "for an attention %d wide)", pd.num_layers, pd.num_heads, pd.head_dim, L.ad);
    if (d.max_rows <= 0) return pool_fail(XNP_E_INVALID, "max_rows %d", d.max_rows);
    if (d.d_model > 2048 || d.flow_dim > 2048 || d.ff > 2048 || d.ldim > 2048 || L.zd > 2048 || L.ad > 2048)
        return pool_fail(XNP_E_INVALID, "widths above 2048 are not supported");
    if (q8 && (d.d_model % 512 || d.flow_dim % 512 || d.ff % 64 || d.ldim % 16 || L.zd % 16))
        return pool_fail(XNP_E_INVALID, "the q8 flow LM takes d_model and flow_dim multiples of 512, ff of 64, "
                                        "ldim and z_dim of 16");
    if (d.gelu != XNP_GELU_ERF && d.gelu != XNP_GELU_TANH) return pool_fail(XNP_E_INVALID, "gelu %d", d.gelu);
    if (d.time_norm != XNP_TIME_RMS && d.time_norm != XNP_TIME_RMS_VAR)
        return pool_fail(XNP_E_INVALID, "time norm %d", d.time_norm);

    xnp_flow_lm *lm = new (std::nothrow) xnp_flow_lm();
    if (!lm) return pool_fail(XNP_E_INVALID, "out of host memory");
    lm->pool = pool;
    lm->d = d;
    lm->L = L;
    hipError_t e = hipSetDevice(pd.device);
    auto fail_hip = [&](hipError_t err, const char *what) {
        fl_free(lm);
        return pool_fail(XNP_E_HIP, "%s: %s", what, hipGetErrorString(err));
    };
    if (e != hipSuccess) return fail_hip(e, "hipSetDevice");
    auto dalloc = [&](void **p, size_t bytes) {
        hipError_t r = hipMalloc(p, bytes);
        if (r == hipSuccess) lm->allocs.push_back(*p);
        return r;
    };
    const size_t M = d.max_rows, dm = d.d_model, F = d.flow_dim, ld = d.ldim, zd = L.zd;
    const size_t na = (size_t)d.flow_depth * 3 * F + 2 * F;
    const int steps = d.flow_type == XNP_FLOW_LSD ? d.lsd_steps : 0;
    lm->na = (int32_t)na;
    struct {
        float **p;
        size_t n;
    } common[] = {{&lm->w, L.total}, {&lm->temb, (size_t)(steps ? steps : 1) * F}, {&lm->adab, na}, {&lm->cond_vec, dm}};
    for (auto &b : common)
        if ((e = dalloc((void **)b.p, sizeof(float) * b.n)) != hipSuccess) return fail_hip(e, "flow LM buffers");
    if ((e = dalloc((void **)&lm->dids, sizeof(int32_t) * M)) != hipSuccess) return fail_hip(e, "flow LM ids");
    if ((e = hipHostMalloc((void **)&lm->hids, sizeof(int32_t) * M, hipHostMallocDefault)) != hipSuccess)
        return fail_hip(e, "pinned ids");
    if ((e = hipMemcpy(lm->w, weights, sizeof(float) * L.total, hipMemcpyHostToDevice)) != hipSuccess)
        return fail_hip(e, "weight upload");
    // every block's adaLN_modulation rows, then the final layer's, stacked
    std::vector<float> adaw_h(na * F), adab_h(na);
    for (int r = 0; r <= d.flow_depth; r++) {
        const bool fin = r == d.flow_depth;
        const size_t rows = (fin ? 2 : 3) * F, row0 = (size_t)r * 3 * F;
        std::memcpy(adaw_h.data() + row0 * F, weights + (fin ? L.fin_aw : L.rb_aw[r]), sizeof(float) * rows * F);
        std::memcpy(adab_h.data() + row0, weights + (fin ? L.fin_ab : L.rb_ab[r]), sizeof(float) * rows);
    }
    if ((e = hipMemcpy(lm->adab, adab_h.data(), sizeof(float) * na, hipMemcpyHostToDevice)) != hipSuccess)
        return fail_hip(e, "adaLN bias upload");
    // lsd_time_embeddings (flow_lm.rs:82-95): times (i / steps, (i + 1) / steps), averaged over the
    // two embedders (mlp.rs:201-212).  They depend on nothing but the weights: once, at load.
    std::vector<float> temb((size_t)(steps ? steps : 1) * F, 0.f), b(F);
    for (int i = 0; i < steps; i++) {
        float *o = temb.data() + (size_t)i * F;
        host_time_embed(d, weights, L, 0, (float)i / (float)steps, o);
        host_time_embed(d, weights, L, 1, (float)(i + 1) / (float)steps, b.data());
        for (size_t j = 0; j < F; j++) o[j] = (o[j] + b[j]) * 0.5f;
        if (q8)
            for (size_t j = 0; j < F; j++) o[j] = host_bf16(o[j]);
    }
    if ((e = hipMemcpy(lm->temb, temb.data(), sizeof(float) * temb.size(), hipMemcpyHostToDevice)) != hipSuccess)
        return fail_hip(e, "time embedding upload");

    if (!q8) {
        struct {
            float **p;
            size_t n;
        } bufs[] = {{&lm->x, M * dm}, {&lm->q, M * L.ad}, {&lm->k, M * L.kd}, {&lm->v, M * L.kd}, {&lm->att, M * L.ad},
                    {&lm->f, M * (size_t)d.ff}, {&lm->ya, M * F}, {&lm->ada, M * na}, {&lm->xf, M * F},
                    {&lm->h2, M * F}, {&lm->z, M * zd}, {&lm->adaw, na * F}};
        for (auto &bf : bufs)
            if ((e = dalloc((void **)bf.p, sizeof(float) * bf.n)) != hipSuccess) return fail_hip(e, "flow LM buffers");
        if ((e = hipMemcpy(lm->adaw, adaw_h.data(), sizeof(float) * na * F, hipMemcpyHostToDevice)) != hipSuccess)
            return fail_hip(e, "adaLN weight upload");
        *out = lm;
        return XNP_OK;
    }

    // q8: quantize every linear's rows on the host (xnp_quantize_rows), upload codes and scales
    std::vector<int8_t> qh;
    std::vector<float> sh;
    auto upload_q8 = [&](const float *src, size_t n, size_t k, Q8Lin &w) -> hipError_t {
        qh.resize(n * k);
        sh.resize(n);
        (void)xnp_quantize_rows(src, (int32_t)n, (int32_t)k, qh.data(), sh.data());
        hipError_t r = dalloc((void **)&w.q, n * k);
        if (r == hipSuccess) r = dalloc((void **)&w.s, sizeof(float) * n);
        if (r == hipSuccess) r = hipMemcpy(w.q, qh.data(), n * k, hipMemcpyHostToDevice);
        if (r == hipSuccess) r = hipMemcpy(w.s, sh.data(), sizeof(float) * n, hipMemcpyHostToDevice);
        return r;
    };
    const size_t ff = d.ff;
    if ((e = upload_q8(weights + L.in_lin, dm, ld, lm->in_lin)) != hipSuccess) return fail_hip(e, "q8 weights");
    for (int l = 0; l < d.num_layers; l++) {
        if ((e = upload_q8(weights + L.wqkv[l], (size_t)L.ad + 2 * (size_t)L.kd, dm, lm->wqkv[l])) != hipSuccess ||
            (e = upload_q8(weights + L.wout[l], dm, L.ad, lm->wout[l])) != hipSuccess ||
            (e = upload_q8(weights + L.w1[l], ff, dm, lm->w1[l])) != hipSuccess ||
            (e = upload_q8(weights + L.w2[l], dm, ff, lm->w2[l])) != hipSuccess)
            return fail_hip(e, "q8 weights");
        xnp_layer_weights &w = lm->lw[l];
        w.d_model = d.d_model, w.ff = d.ff, w.gelu = d.gelu;
        w.wqkv = lm->wqkv[l].q, w.sqkv = lm->wqkv[l].s, w.wout = lm->wout[l].q, w.sout = lm->wout[l].s;
        w.w1 = lm->w1[l].q, w.s1 = lm->w1[l].s, w.w2 = lm->w2[l].q, w.s2 = lm->w2[l].s;
        w.ln1_w = lm->W(L.ln1_w[l]), w.ln1_b = lm->W(L.ln1_b[l]), w.ln2_w = lm->W(L.ln2_w[l]), w.ln2_b = lm->W(L.ln2_b[l]);
        w.ls1 = w.ls2 = nullptr;
    }
    if ((d.z_dim && (e = upload_q8(weights + L.z_proj, zd, dm, lm->zp)) != hipSuccess) ||
        (e = upload_q8(weights + L.eos_w, 1, zd, lm->eos)) != hipSuccess ||
        (e = upload_q8(weights + L.cond_w, F, zd, lm->cond)) != hipSuccess ||
        (e = upload_q8(weights + L.inp_w, F, ld, lm->inp)) != hipSuccess ||
        (e = upload_q8(adaw_h.data(), na, F, lm->adaq)) != hipSuccess ||
        (e = upload_q8(weights + L.fin_w, ld, F, lm->finw)) != hipSuccess)
        return fail_hip(e, "q8 weights");
    for (int r = 0; r < d.flow_depth; r++)
        if ((e = upload_q8(weights + L.rb_w1[r], F, F, lm->rb1[r])) != hipSuccess ||
            (e = upload_q8(weights + L.rb_w2[r], F, F, lm->rb2[r])) != hipSuccess)
            return fail_hip(e, "q8 weights");
    // the LUT rows rounded to bf16; bos_emb once per row
    {
        const size_t nl = ((size_t)d.n_bins + 1) * dm;
        std::vector<uint16_t> lut(nl);
        for (size_t i = 0; i < nl; i++) lut[i] = host_bf16_bits(weights[L.embed + i]);
        std::vector<float> bos(M * ld);
        for (size_t r = 0; r < M; r++) std::memcpy(bos.data() + r * ld, weights + L.bos, sizeof(float) * ld);
        if ((e = dalloc((void **)&lm->lut, sizeof(uint16_t) * nl)) != hipSuccess ||
            (e = hipMemcpy(lm->lut, lut.data(), sizeof(uint16_t) * nl, hipMemcpyHostToDevice)) != hipSuccess ||
            (e = dalloc((void **)&lm->bos_rows, sizeof(float) * M * ld)) != hipSuccess ||
            (e = hipMemcpy(lm->bos_rows, bos.data(), sizeof(float) * M * ld, hipMemcpyHostToDevice)) != hipSuccess)
            return fail_hip(e, "q8 tables");
    }
    struct {
        uint16_t **p;
        size_t n;
    } bb[] = {{&lm->bx, M * dm}, {&lm->btout, M * dm}, {&lm->bz, M * zd}, {&lm->bya, M * F},
              {&lm->bxf, M * F}, {&lm->bada, M * na}, {&lm->bh, M * F}, {&lm->bh2, M * F}};
    for (auto &bf : bb)
        if ((e = dalloc((void **)bf.p, sizeof(uint16_t) * bf.n)) != hipSuccess) return fail_hip(e, "flow LM buffers");
    if (xnp_status st = xnp_layer_workspace(pool, (int32_t)M, d.d_model, d.ff, &lm->ws_bytes)) {
        fl_free(lm);
        return st;
    }
    if ((e = dalloc(&lm->ws, lm->ws_bytes)) != hipSuccess) return fail_hip(e, "layer workspace");
    *out = lm;
    return XNP_OK;
}

extern "C" xnp_status xnp_flow_lm_destroy(xnp_flow_lm *lm) {
    if (!lm) return XNP_OK;
    (void)hipSetDevice(pool_desc(lm->pool)->device);
    fl_free(lm);
    return XNP_OK;
}

#define FL_TRY(expr, what)                                                                         \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess) return pool_fail(XNP_E_HIP, "%s: %s", what, hipGetErrorString(e_)); \
    } while (0)

// The transformer (StreamingTransformer::forward, transformer.rs:742-808, with the layers of
// transformer.rs:591-634) over the M rows in lm->x, for the open batch.
static xnp_status fl_transformer(xnp_flow_lm *lm, int M, void *hip_stream) {
    const xnp_flow_lm_desc &d = lm->d;
    const Layout &L = lm->L;
    hipStream_t hs = (hipStream_t)hip_stream;
    const int dm = d.d_model, ff = d.ff, ad = L.ad, kd = L.kd;
    const float scale = 1.0f / std::sqrt((float)(ad / d.num_heads)); // 1 / sqrt(head_dim) (transformer.rs:215)
    for (int l = 0; l < d.num_layers; l++) {
        LinNorm n1; // norm1, applied as in_proj reads x
        n1.w = lm->W(L.ln1_w[l]), n1.b = lm->W(L.ln1_b[l]), n1.eps = 1e-5f;
        LinOut qkv; // q [M][ad], then k and v [M][kd] (transformer.rs:195-211)
        qkv.nseg = 3;
        qkv.out[0] = lm->q, qkv.ld[0] = ad, qkv.col0[0] = 0;
        qkv.out[1] = lm->k, qkv.ld[1] = kd, qkv.col0[1] = ad;
        qkv.out[2] = lm->v, qkv.ld[2] = kd, qkv.col0[2] = ad + kd;
        FL_TRY(launch_linear_f32(lm->x, dm, M, dm, lm->W(L.wqkv[l]), nullptr, ad + 2 * kd, kLinStore, qkv, hs, &n1),
               "in_proj");
        if (xnp_status st = xnp_attend(lm->pool, l, lm->q, lm->k, lm->v, lm->att, scale, hip_stream)) return st;
        LinOut res;
        res.out[0] = lm->x, res.ld[0] = dm;
        FL_TRY(launch_linear_f32(lm->att, ad, M, ad, lm->W(L.wout[l]), nullptr, dm, kLinResidual, res, hs), "out_proj");
        LinNorm n2; // norm2, applied as linear1 reads x
        n2.w = lm->W(L.ln2_w[l]), n2.b = lm->W(L.ln2_b[l]), n2.eps = 1e-5f;
        LinOut hid;
        hid.out[0] = lm->f, hid.ld[0] = ff;
        FL_TRY(launch_linear_f32(lm->x, dm, M, dm, lm->W(L.w1[l]), nullptr, ff,
                                 d.gelu == XNP_GELU_ERF ? kLinGeluErf : kLinGeluTanh, hid, hs, &n2),
               "linear1");
        FL_TRY(launch_linear_f32(lm->f, ff, M, ff, lm->W(L.w2[l]), nullptr, dm, kLinResidual, res, hs), "linear2");
    }
    return XNP_OK;
}

// The q8 transformer: xnp_layer_step per layer over the bf16 rows in lm->bx.
static xnp_status fl_transformer_q8(xnp_flow_lm *lm, void *hip_stream) {
    for (int l = 0; l < lm->d.num_layers; l++)
        if (xnp_status st = xnp_layer_step(lm->pool, l, &lm->lw[l], lm->bx, lm->ws, lm->ws_bytes, hip_stream)) return st;
    return XNP_OK;
}

extern "C" xnp_status xnp_flow_lm_prompt_text(xnp_flow_lm *lm, const int32_t *ids, int32_t n, const int32_t *tokens,
                                              int32_t t, void *hip_stream) {
    if (!lm || (n > 0 && (!ids || !tokens))) return pool_fail(XNP_E_INVALID, "null argument");
    if (n < 0 || t < 0) return pool_fail(XNP_E_INVALID, "%d streams of %d tokens", n, t);
    if (n == 0 || t == 0) return XNP_OK;
    const int64_t M = (int64_t)n * t;
    if (M > lm->d.max_rows) return pool_fail(XNP_E_INVALID, "%lld rows; the flow LM holds %d", (long long)M, lm->d.max_rows);
    for (int64_t i = 0; i < M; i++) // LUTConditioner::embed_tokens refuses ids past its table
        if (tokens[i] < 0 || tokens[i] > lm->d.n_bins)
            return pool_fail(XNP_E_INVALID, "token id %d is past this checkpoint's %d-entry embedding table", tokens[i],
                             lm->d.n_bins + 1);
    hipStream_t hs = (hipStream_t)hip_stream;
    FL_TRY(hipSetDevice(pool_desc(lm->pool)->device), "hipSetDevice");
    // the previous call's upload from the staging buffer has finished once the stream reaches here
    FL_TRY(hipStreamSynchronize(hs), "staging");
    std::memcpy(lm->hids, tokens, sizeof(int32_t) * M);
    FL_TRY(hipMemcpyAsync(lm->dids, lm->hids, sizeof(int32_t) * M, hipMemcpyHostToDevice, hs), "token upload");
    if (xnp_status st = xnp_batch_begin(lm->pool, ids, n, t, hip_stream)) return st;
    xnp_status st;
    if (lm->d.precision == XNP_FLOW_Q8) {
        FL_TRY(launch_gather_rows(lm->lut, lm->dids, (int)M, lm->d.d_model * 2, lm->bx, hs), "embed");
        st = fl_transformer_q8(lm, hip_stream);
    } else {
        FL_TRY(launch_embed_f32(lm->W(lm->L.embed), lm->dids, (int)M, lm->d.d_model, lm->x, hs), "embed");
        st = fl_transformer(lm, (int)M, hip_stream);
    }
    if (st) {
        (void)xnp_batch_abort(lm->pool);
        return st;
    }
    return xnp_batch_end(lm->pool);
}

static xnp_status fl_frame_q8(xnp_flow_lm *lm, int M, const float *latent_in, const float *cond, const float *noise,
                              float *latent_out, float *eos_logit, void *hip_stream);

// The frame's device work after the step's plan is uploaded: input_linear, the transformer, the
// heads and the flow net, all launches on hip_stream (what a graph of the frame records).
// cond: each row's condition (stride d_model), else the model's (one row for all), else none.
static xnp_status fl_frame_launches(xnp_flow_lm *lm, int M, const float *latent_in, const float *cond,
                                    const float *noise, float *latent_out, float *eos_logit, void *hip_stream) {
    if (lm->d.precision == XNP_FLOW_Q8)
        return fl_frame_q8(lm, M, latent_in, cond, noise, latent_out, eos_logit, hip_stream);
    const xnp_flow_lm_desc &d = lm->d;
    const Layout &L = lm->L;
    hipStream_t hs = (hipStream_t)hip_stream;
    const int dm = d.d_model, F = d.flow_dim, ld = d.ldim;
    // input_linear of the previous latents, or of bos_emb for every row (flow_lm.rs:314-324, 423-427),
    // plus the condition row (flow_lm.rs:304-307): y + c, as out = aux + 1 * y
    LinOut xo;
    xo.out[0] = lm->x, xo.ld[0] = dm;
    const float *c_rows = cond ? cond : lm->has_cond ? lm->cond_vec : nullptr;
    if (c_rows) xo.aux = c_rows, xo.ld_aux = cond ? dm : 0, xo.alpha = 1.0f;
    FL_TRY(launch_linear_f32(latent_in ? latent_in : lm->W(L.bos), latent_in ? ld : 0, M, ld, lm->W(L.in_lin), nullptr,
                             dm, c_rows ? kLinAxpy : kLinStore, xo, hs),
           "input_linear");
    if (xnp_status st = fl_transformer(lm, M, hip_stream)) return st;
    // out_norm (flow_lm.rs:315), applied as its readers load x: z_proj (flow_lm.rs:320-323) when the
    // model has one, else the EOS logit (flow_lm.rs:366) and the flow net's cond_embed
    LinNorm on;
    on.w = lm->W(L.on_w), on.b = lm->W(L.on_b), on.eps = 1e-5f;
    const float *c = lm->x;
    const LinNorm *cn = &on;
    if (d.z_dim) {
        LinOut zo;
        zo.out[0] = lm->z, zo.ld[0] = L.zd;
        FL_TRY(launch_linear_f32(lm->x, dm, M, dm, lm->W(L.z_proj), nullptr, L.zd, kLinStore, zo, hs, &on), "z_proj");
        c = lm->z, cn = nullptr;
    }
    LinOut eo;
    eo.out[0] = eos_logit, eo.ld[0] = 1;
    FL_TRY(launch_linear_f32(c, L.zd, M, L.zd, lm->W(L.eos_w), lm->W(L.eos_b), 1, kLinStore, eo, hs, cn), "out_eos");
    // sample_from_noise (flow_lm.rs:363-384): lsd_decode (:97-110), each step x += flow_net(c,
    // t_emb_i, x) / steps; Drifting flow_net(c, None, noise); Pointwise noise + the same
    const bool lsd = d.flow_type == XNP_FLOW_LSD;
    const int steps = lsd ? d.lsd_steps : 1;
    for (int i = 0; i < steps; i++) {
        const float *cur = i == 0 ? noise : latent_out;
        LinOut y;
        y.out[0] = lm->ya, y.ld[0] = F, y.aux = lsd ? lm->temb + (size_t)i * F : nullptr;
        FL_TRY(launch_linear_f32(c, L.zd, M, L.zd, lm->W(L.cond_w), lm->W(L.cond_b), F, lsd ? kLinSiluAddVec : kLinSilu,
                                 y, hs, cn),
               "cond_embed");
        LinOut xf;
        xf.out[0] = lm->xf, xf.ld[0] = F;
        FL_TRY(launch_linear_f32(cur, ld, M, ld, lm->W(L.inp_w), lm->W(L.inp_b), F, kLinStore, xf, hs), "input_proj");
        // every block's adaLN_modulation and the final layer's, in one launch: row m of lm->ada
        // holds block r's (shift, scale, gate) at r * 3F and the final (shift, scale) at depth * 3F
        const int na = lm->na;
        LinOut a;
        a.out[0] = lm->ada, a.ld[0] = na;
        FL_TRY(launch_linear_f32(lm->ya, F, M, F, lm->adaw, lm->adab, na, kLinStore, a, hs), "adaLN_modulation");
        for (int r = 0; r < d.flow_depth; r++) { // ResBlock (mlp.rs:113-131)
            const float *mod = lm->ada + (size_t)r * 3 * F;
            LinNorm in; // in_ln and modulate(shift, scale), applied as mlp.0 reads x
            in.w = lm->W(L.rb_lnw[r]), in.b = lm->W(L.rb_lnb[r]), in.eps = 1e-6f;
            in.shift = mod, in.scale = mod + F, in.ld_mod = na;
            LinOut s1;
            s1.out[0] = lm->h2, s1.ld[0] = F;
            FL_TRY(launch_linear_f32(lm->xf, F, M, F, lm->W(L.rb_w1[r]), lm->W(L.rb_b1[r]), F, kLinSilu, s1, hs, &in),
                   "mlp.0");
            LinOut g;
            g.out[0] = lm->xf, g.ld[0] = F, g.aux = mod + 2 * F, g.ld_aux = na;
            FL_TRY(launch_linear_f32(lm->h2, F, M, F, lm->W(L.rb_w2[r]), lm->W(L.rb_b2[r]), F, kLinGated, g, hs), "mlp.2");
        }
        // FinalLayer (mlp.rs:155-163): norm_final (no affine) and modulate, applied as the final
        // linear reads x
        const float *fmod = lm->ada + (size_t)d.flow_depth * 3 * F;
        LinNorm nf;
        nf.eps = 1e-6f, nf.shift = fmod, nf.scale = fmod + F, nf.ld_mod = na;
        LinOut o;
        o.out[0] = latent_out, o.ld[0] = ld, o.aux = cur, o.ld_aux = ld, o.alpha = lsd ? 1.0f / (float)steps : 1.0f;
        FL_TRY(launch_linear_f32(lm->xf, F, M, F, lm->W(L.fin_w), lm->W(L.fin_b), ld,
                                 d.flow_type == XNP_FLOW_DRIFTING ? kLinStore : kLinAxpy, o, hs, &nf),
               "final linear");
    }
    return XNP_OK;
}

// The q8 frame: the same steps on bf16 rows, the linears on the MFMA GEMM with their epilogues,
// the transformer as xnp_layer_step, the LayerNorms (and modulations) as kernels of their own.
static xnp_status fl_frame_q8(xnp_flow_lm *lm, int M, const float *latent_in, const float *cond, const float *noise,
                              float *latent_out, float *eos_logit, void *hip_stream) {
    const xnp_flow_lm_desc &d = lm->d;
    const Layout &L = lm->L;
    hipStream_t hs = (hipStream_t)hip_stream;
    const int dm = d.d_model, F = d.flow_dim, ld = d.ldim, zd = L.zd, na = lm->na;
    auto gemm = [&](const void *a, bool a_f32, int K, const Q8Lin &w, const float *bias, int N, int epi, void *out,
                    int ldo, const void *aux, int ld_aux, float alpha, const char *what) -> xnp_status {
        GemmOut go;
        go.out[0] = out, go.ld[0] = ldo, go.bias = bias, go.aux = aux, go.ld_aux = ld_aux, go.alpha = alpha;
        go.a_f32 = a_f32;
        FL_TRY(launch_gemm_q8(a, M, K, w.q, w.s, N, epi, go, hs), what);
        return XNP_OK;
    };
#define FL_Q(call)                                                                                 \
    do {                                                                                           \
        if (xnp_status st_ = (call)) return st_;                                                   \
    } while (0)
    // input_linear of the previous latents, or of bos_emb for every row (flow_lm.rs:314-324, 423-427),
    // plus the condition row (flow_lm.rs:304-307) as a bf16 tensor add: bf16(bf16(c) + y)
    const float *c_rows = cond ? cond : lm->has_cond ? lm->cond_vec : nullptr;
    FL_Q(gemm(latent_in ? latent_in : lm->bos_rows, true, ld, lm->in_lin, nullptr, dm, c_rows ? kAddF32 : kStore, lm->bx,
              dm, c_rows, cond ? dm : 0, 1.f, "input_linear"));
    FL_Q(fl_transformer_q8(lm, hip_stream));
    FL_TRY(launch_layer_norm(lm->bx, M, dm, lm->W(L.on_w), lm->W(L.on_b), 1e-5f, lm->btout, hs), "out_norm");
    const uint16_t *c = lm->btout;
    if (d.z_dim) {
        FL_Q(gemm(lm->btout, false, dm, lm->zp, nullptr, zd, kStore, lm->bz, zd, nullptr, 0, 1.f, "z_proj"));
        c = lm->bz;
    }
    FL_Q(gemm(c, false, zd, lm->eos, lm->W(L.eos_b), 1, kStoreF32, eos_logit, 1, nullptr, 0, 1.f, "out_eos"));
    const bool lsd = d.flow_type == XNP_FLOW_LSD;
    const int steps = lsd ? d.lsd_steps : 1;
    for (int i = 0; i < steps; i++) {
        const float *cur = i == 0 ? noise : latent_out;
        FL_Q(gemm(c, false, zd, lm->cond, lm->W(L.cond_b), F, lsd ? kSiluAddVec : kSilu, lm->bya, F,
                  lsd ? lm->temb + (size_t)i * F : nullptr, 0, 1.f, "cond_embed"));
        FL_Q(gemm(cur, true, ld, lm->inp, lm->W(L.inp_b), F, kStore, lm->bxf, F, nullptr, 0, 1.f, "input_proj"));
        // every block's (shift, scale, gate) and the final (shift, scale), one launch
        FL_Q(gemm(lm->bya, false, F, lm->adaq, lm->adab, na, kStore, lm->bada, na, nullptr, 0, 1.f, "adaLN_modulation"));
        for (int r = 0; r < d.flow_depth; r++) { // ResBlock (mlp.rs:113-131)
            const uint16_t *mod = lm->bada + (size_t)r * 3 * F;
            FL_TRY(launch_layer_norm_mod(lm->bxf, M, F, lm->W(L.rb_lnw[r]), lm->W(L.rb_lnb[r]), 1e-6f, mod, mod + F, na,
                                         lm->bh, hs),
                   "in_ln");
            FL_Q(gemm(lm->bh, false, F, lm->rb1[r], lm->W(L.rb_b1[r]), F, kSilu, lm->bh2, F, nullptr, 0, 1.f, "mlp.0"));
            FL_Q(gemm(lm->bh2, false, F, lm->rb2[r], lm->W(L.rb_b2[r]), F, kGated, lm->bxf, F, mod + 2 * F, na, 1.f,
                      "mlp.2"));
        }
        const uint16_t *fmod = lm->bada + (size_t)d.flow_depth * 3 * F; // FinalLayer (mlp.rs:155-163)
        FL_TRY(launch_layer_norm_mod(lm->bxf, M, F, nullptr, nullptr, 1e-6f, fmod, fmod + F, na, lm->bh, hs),
               "norm_final");
        if (d.flow_type == XNP_FLOW_DRIFTING)
            FL_Q(gemm(lm->bh, false, F, lm->finw, lm->W(L.fin_b), ld, kStoreF32, latent_out, ld, nullptr, 0, 1.f,
                      "final linear"));
        else
            FL_Q(gemm(lm->bh, false, F, lm->finw, lm->W(L.fin_b), ld, kAxpyF32, latent_out, ld, cur, ld,
                      lsd ? 1.0f / (float)steps : 1.0f, "final linear"));
    }
#undef FL_Q
    return XNP_OK;
}

static xnp_status fl_step_check(xnp_flow_lm *lm, const int32_t *ids, int32_t n, const float *noise, float *latent_out,
                                float *eos_logit) {
    if (!lm || (n > 0 && (!ids || !noise || !latent_out || !eos_logit))) return pool_fail(XNP_E_INVALID, "null argument");
    if (n < 0 || n > lm->d.max_rows) return pool_fail(XNP_E_INVALID, "%d streams; the flow LM holds %d rows", n, lm->d.max_rows);
    return XNP_OK;
}

extern "C" xnp_status xnp_flow_lm_set_condition(xnp_flow_lm *lm, const float *cond, int32_t dim) {
    if (!lm) return pool_fail(XNP_E_INVALID, "null argument");
    if (!cond) {
        lm->has_cond = false;
        return XNP_OK;
    }
    if (dim != lm->d.d_model) return pool_fail(XNP_E_INVALID, "a condition of %d values for d_model %d", dim, lm->d.d_model);
    FL_TRY(hipSetDevice(pool_desc(lm->pool)->device), "hipSetDevice");
    FL_TRY(hipMemcpy(lm->cond_vec, cond, sizeof(float) * dim, hipMemcpyHostToDevice), "condition upload");
    lm->has_cond = true;
    return XNP_OK;
}

extern "C" xnp_status xnp_flow_lm_step(xnp_flow_lm *lm, const int32_t *ids, int32_t n, const float *latent_in,
                                       const float *conditions, const float *noise, float *latent_out, float *eos_logit,
                                       void *hip_stream) {
    if (xnp_status st = fl_step_check(lm, ids, n, noise, latent_out, eos_logit)) return st;
    if (n == 0) return XNP_OK;
    FL_TRY(hipSetDevice(pool_desc(lm->pool)->device), "hipSetDevice");
    if (xnp_status st = xnp_batch_begin(lm->pool, ids, n, 1, hip_stream)) return st;
    if (xnp_status st = fl_frame_launches(lm, n, latent_in, conditions, noise, latent_out, eos_logit, hip_stream)) {
        (void)xnp_batch_abort(lm->pool);
        return st;
    }
    return xnp_batch_end(lm->pool);
}

extern "C" xnp_status xnp_flow_lm_step_graph(xnp_flow_lm *lm, const int32_t *ids, int32_t n, const float *latent_in,
                                             const float *conditions, const float *noise, float *latent_out,
                                             float *eos_logit, void *hip_stream) {
    if (xnp_status st = fl_step_check(lm, ids, n, noise, latent_out, eos_logit)) return st;
    if (n == 0) return XNP_OK;
    if (!hip_stream) return pool_fail(XNP_E_INVALID, "a graph is recorded on a stream of the caller's, not the null stream");
    hipStream_t hs = (hipStream_t)hip_stream;
    FL_TRY(hipSetDevice(pool_desc(lm->pool)->device), "hipSetDevice");
    // the plan (positions, pages) is uploaded eagerly; the frame's launches read it from the
    // pool's device buffers, so one recording serves every step with the same rows and buffers
    if (xnp_status st = xnp_batch_begin(lm->pool, ids, n, 1, hip_stream)) return st;
    FlowGraph &G = lm->graph;
    // the recorded kernels were chosen by the batch that recorded them: a ring prefix taken up since
    // (s2s.rs:174) changes the decode's template, and the plan sets the waves per group
    const BatchLaunchKey key = batch_launch_key(lm->pool);
    // the condition source is part of the recording: a step's own rows, the model's, or none
    const float *cond_src = conditions ? conditions : lm->has_cond ? lm->cond_vec : nullptr;
    const bool same = G.exec && G.n == n && G.latent_in == latent_in && G.noise == noise && G.latent_out == latent_out &&
                      G.eos == eos_logit && G.stream == hs && G.key == key && G.cond == cond_src;
    if (!same) {
        if (G.exec) (void)hipGraphExecDestroy(G.exec);
        G = FlowGraph();
        hipGraph_t graph = nullptr;
        hipError_t e = hipStreamBeginCapture(hs, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) {
            (void)xnp_batch_abort(lm->pool);
            return pool_fail(XNP_E_HIP, "graph capture: %s", hipGetErrorString(e));
        }
        xnp_status st = fl_frame_launches(lm, n, latent_in, conditions, noise, latent_out, eos_logit, hip_stream);
        e = hipStreamEndCapture(hs, &graph);
        if (st == XNP_OK && e == hipSuccess) e = hipGraphInstantiate(&G.exec, graph, nullptr, nullptr, 0);
        if (graph) (void)hipGraphDestroy(graph);
        if (st != XNP_OK || e != hipSuccess) {
            G = FlowGraph();
            (void)xnp_batch_abort(lm->pool);
            return st != XNP_OK ? st : pool_fail(XNP_E_HIP, "graph capture: %s", hipGetErrorString(e));
        }
        G.n = n, G.latent_in = latent_in, G.noise = noise, G.latent_out = latent_out, G.eos = eos_logit, G.stream = hs;
        G.cond = cond_src;
        G.key = key;
    }
    hipError_t e = hipGraphLaunch(G.exec, hs);
    if (e != hipSuccess) {
        (void)xnp_batch_abort(lm->pool);
        return pool_fail(XNP_E_HIP, "graph launch: %s", hipGetErrorString(e));
    }
    return xnp_batch_end(lm->pool);
}
