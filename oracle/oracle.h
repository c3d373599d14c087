/*
 * oracle.h -- CPU restatement of the reference's flow-LM KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker that the HIP library is compared against:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  Nothing in
 * the product (xn-ptts_amd/) links, imports or calls it.
 *
 * It restates, per stream and batch 1, what the reference computes below the projections of
 * StreamingMultiheadAttention::forward (ptts/src/transformer.rs:183-251):
 *   - the contiguous cache [S_cap][H][D] per layer for K and V (StreamingMHAState,
 *     transformer.rs:14-25; init_state 169-180), zero-filled;
 *   - RoPE tables (rope.rs:37-63) and the interleaved-pair rotation (rope.rs:74-95);
 *   - complete_kv (transformer.rs:61-92): append at current_end or at the ring's write slot;
 *   - single-query decode attention (sdpa_decode, transformer.rs:223,230) and causal prefill
 *     (transformer.rs:231-248), both over the cache after the append;
 *   - the ring: start_ring / set_ring_slot / evict (transformer.rs:842-929) and its decode mask
 *     (transformer.rs:42-52);
 *   - with_seq_budget (transformer.rs:350-392) and advance (transformer.rs:337-344).
 * Two things the reference does not have are restated the way the HIP library defines them:
 * the int8 cache with per-(block, head) scales, and the "absolute" ring whose eviction keeps
 * keys at their write-time rotation (see orc_start_ring).
 *
 * Arithmetic: f32, no contraction (built with -ffp-contract=off), left-to-right sums.  Every
 * output also has an f64 companion computed from the same rounded operands.
 */
#ifndef XNP_ORACLE_H
#define XNP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_I8 = 2 };
enum { ORC_RING_NONE = 0, ORC_RING_SHIFT = 1, ORC_RING_ABSOLUTE = 2 };
#define ORC_BLOCK 16

typedef struct orc_stream orc_stream;

/* --- element helpers ---------------------------------------------------------------------- */
float orc_bf16_round(float x);
/* Quantize y against scale s: 0 when s == 0, else rint(y / s) clamped to [-127, 127]. */
int8_t orc_quant(float y, float s);

/* --- RoPE (rope.rs:37-63, 74-95) ------------------------------------------------------------ */
/* cos/sin of one position: inv_freq[i] = 1 / theta^(i / (D/2)), angle = pos * inv_freq[i],
 * each value rounded to the activation dtype (T::from_f32 in rope.rs:55-56). */
void orc_rope_row(int head_dim, float max_period, float pos, int act_dtype, float *cos_out,
                  float *sin_out);
/* Rotate pairs (2i, 2i+1) of x[head_dim] in place, then round to act_dtype. */
void orc_rotate(int head_dim, float *x, const float *cos_row, const float *sin_row,
                int act_dtype);

/* --- one stream's state ---------------------------------------------------------------------- */
orc_stream *orc_open(int layers, int heads, int kv_heads, int head_dim, int capacity,
                     int cache_dtype, int act_dtype, float max_period);
void orc_close(orc_stream *st);
int orc_current_end(const orc_stream *st);
int orc_capacity(const orc_stream *st);
/* ring fields: mode, write, filled, prefix, shift; valid[capacity] copied when non-null */
void orc_ring_info(const orc_stream *st, int *mode, int *write, int *filled, int *prefix,
                   int *shift, uint8_t *valid);

/* One layer of one step: rotate q and k at the step's position, append k and v (complete_kv),
 * attend.  q [t][H][D], k and v [t][KVH][D] hold activation values (bf16-representable when
 * act_dtype is bf16), out [t][H][D] receives the attention output rounded to act_dtype and
 * out64 (nullable) the same in f64 without the final rounding.  Every layer of a step appends
 * at the same position; orc_commit(t) then advances the stream, as complete_kv does per layer.
 * Returns 0, or -1 with orc_last_error() set and nothing changed. */
int orc_attend(orc_stream *st, int layer, int t, const float *q, const float *k,
               const float *v, float scale, float *out, double *out64);
/* The two halves of orc_attend, as the HIP library also exposes them. */
int orc_append(orc_stream *st, int layer, int t, const float *k, const float *v);
int orc_attention(orc_stream *st, int layer, int t, const float *q, float scale, float *out,
                  double *out64);
int orc_commit(orc_stream *st, int t);
/* Count n more filled positions written by orc_write_rows (transformer.rs:337-344). */
int orc_advance(orc_stream *st, int n);

int orc_start_ring(orc_stream *st, int mode, int prefix);
/* Set a ring's fields directly (a snapshot restored): the CPU baseline starts windowed streams
 * this way instead of replaying every row.  valid[capacity]. */
int orc_ring_restore(orc_stream *st, int mode, int write, int filled, int prefix, int shift,
                     int current_end, const uint8_t *valid);
int orc_set_ring_slot(orc_stream *st, int slot);
int orc_evict(orc_stream *st, int prefix, const int *slots, int count);
/* with_seq_budget: a fresh stream of `budget` positions holding a copy of the filled prefix. */
orc_stream *orc_with_seq_budget(const orc_stream *st, int budget);

/* Raw cache rows [slot0, slot0+n) of one layer, kv = 0 (keys) or 1 (values).
 * vals [n][H][D]: the stored values as f32 (dequantized for int8).
 * q8 [n][H][D] and scales [nblk][H] (blocks slot0/16 .. (slot0+n-1)/16): int8 caches only. */
int orc_read_rows(const orc_stream *st, int layer, int kv, int slot0, int n, float *vals,
                  int8_t *q8, float *scales);
int orc_write_rows(orc_stream *st, int layer, int kv, int slot0, int n, const float *vals,
                   const int8_t *q8, const float *scales);
/* voice_from_kv_cache (ptts-wasm/src/lib.rs:291-325): kv [2][n][H][D] f32 (keys, already
 * rotated, then values) stored as rows [0, n) of one layer; the stream must hold exactly n rows
 * and no ring.  int8: per (block, head) s = amax / 127 over the block's rows, q = rint(x / s). */
int orc_load_kv(orc_stream *st, int layer, const float *kv, int n);

/* --- Mimi's attention cache (transformer.rs:257-318, 428-468, 764-781) ------------------------ */
/* KvCache with context `context`: between steps it keeps the last context - 1 rows; a step of t
 * rows (at most rows_max) rotates them at absolute_offset + i and each attends the rows within
 * `context` positions before it, itself included.  Values stored in the activation dtype. */
typedef struct orc_window orc_window;
orc_window *orc_window_open(int layers, int heads, int head_dim, int context, int rows_max, int act_dtype,
                            float max_period);
void orc_window_close(orc_window *w);
int orc_window_attend(orc_window *w, int layer, int t, const float *q, const float *k, const float *v, float scale,
                      float *out, double *out64);
int orc_window_commit(orc_window *w, int t);
int orc_window_len(const orc_window *w);
int orc_window_offset(const orc_window *w);
int orc_window_rows(const orc_window *w, int layer, int kv, float *rows);

/* --- the rest of a flow-LM transformer layer (transformer.rs:591-634) ------------------------ */
/* LayerNorm over the last dimension, as norm1/norm2 (transformer.rs:547-548, eps 1e-5): per row,
 * mean and biased variance in f32 (ascending sums), then (x - mean) * (1 / sqrt(var + eps)) * w + b,
 * rounded to act_dtype.  x and out [rows][dim] may alias. */
void orc_layer_norm(const float *x, int rows, int dim, const float *w, const float *b, float eps,
                    int act_dtype, float *out);
/* Per-row int8 weights, the quantization this build defines for the projections: s = amax / 127
 * (0 for an all-zero row), q = rint(w / s) clamped to [-127, 127]. */
void orc_quantize_rows(const float *w, int rows, int cols, int8_t *q, float *scales);
/* y[m][j] = round_act(s[j] * sum_k x[m][k] * q[j][k]), the sum in f32 with k ascending:
 * a q8 linear without bias (the flow LM's in_proj, out_proj, linear1, linear2). */
void orc_linear_q8(const float *x, int rows, int k, const int8_t *q, const float *s, int n,
                   int act_dtype, float *y);
/* GELU: kind 0 erf (0.5 x (1 + erf(x / sqrt 2))), kind 1 tanh approximation. */
float orc_gelu(float x, int kind);

typedef struct orc_layer_weights {
    int d_model, ff, gelu;                  /* gelu: 0 erf, 1 tanh */
    const int8_t *wqkv; const float *sqkv; /* [(H + 2 KVH) D][d_model] */
    const int8_t *wout; const float *sout; /* [d_model][H D] */
    const int8_t *w1; const float *s1;     /* [ff][d_model] */
    const int8_t *w2; const float *s2;     /* [d_model][ff] */
    const float *ln1_w, *ln1_b, *ln2_w, *ln2_b; /* [d_model] */
    const float *ls1, *ls2;                 /* [d_model] layer scales (layer_scale.rs), or NULL */
} orc_layer_weights;

/* One layer of StreamingTransformerLayer::forward (transformer.rs:591-634) for t rows of each of
 * n streams (OpenMP across streams): x [n][t][d_model] holds activation values and is updated in
 * place.  norm1 -> in_proj -> split q/k/v (transformer.rs:195-211) -> orc_attend -> out_proj ->
 * layer scale -> residual; norm2 -> linear1 -> gelu -> linear2 -> layer scale -> residual.  Every
 * tensor is rounded to the activation dtype as it is produced.  The streams are not committed. */
int orc_layer_step(orc_stream **streams, int n, int t, int layer, const orc_layer_weights *w,
                   float scale, float *x);

/* --- the flow LM around the transformer (flow_lm.rs, mlp.rs, conditioners.rs), f32 ------------ */
#define ORC_FREQ_DIM 256 /* the time embedders' frequency embedding (mlp.rs:186-193) */
typedef struct orc_flow_lm_desc {
    int d_model, num_heads, num_layers, ff;  /* the transformer (no layer scale: flow_lm.rs:239-249) */
    int ldim, n_bins, flow_dim, flow_depth;  /* latent width, LUT rows - 1, flow net width, res blocks */
    int lsd_steps;                           /* LSD solver steps (lsd_decode_steps) */
    int gelu;                                /* 0 erf, 1 tanh */
    int time_norm;                           /* 0 Rms, 1 RmsVar (mlp.rs:17-28) */
    int z_dim;                               /* 0: no z_proj; else its width (flow_lm.rs:135, 239-240) */
    int flow_type;                           /* 0 Lsd, 1 Drifting, 2 Pointwise (flow_lm.rs:372-381) */
    int precision;                           /* 0 f32; 1 q8: int8 weights, bf16 activations */
    int num_kv_heads;                        /* 0: num_heads; else grouped-query kv heads (flow_lm.rs:143-145) */
    int attn_dim;                            /* 0: d_model; else the attention width (flow_lm.rs:139-141) */
} orc_flow_lm_desc;
/* Floats of the weight blob: every tensor f32, row-major [out][in], in this order (zd = z_dim when
 * set, else d; a = attn_dim when set, else d; kv = a / num_heads x num_kv_heads) --
 * conditioner.embed [n_bins+1][d]; input_linear [d][ldim]; bos_emb [ldim];
 * per layer: norm1 w, b [d]; in_proj [a + 2 kv][d]; out_proj [d][a]; norm2 w, b [d];
 *   linear1 [ff][d]; linear2 [d][ff];
 * out_norm w, b [d]; z_proj [z][d] when z_dim; out_eos w [1][zd], b [1];
 * per time embedder (2, Lsd only): freqs [128]; mlp.0 w [F][256], b [F]; mlp.2 w [F][F], b [F];
 *   alpha [F];
 * cond_embed w [F][zd], b [F]; input_proj w [F][ldim], b [F];
 * per res block: in_ln w, b [F]; mlp.0 w [F][F], b [F]; mlp.2 w [F][F], b [F];
 *   adaLN_modulation.1 w [3F][F], b [3F];
 * final_layer: adaLN_modulation.1 w [2F][F], b [2F]; linear w [ldim][F], b [ldim].
 * Returns -1 for a bad shape. */
long long orc_flow_lm_size(const orc_flow_lm_desc *d);
/* y[m][j] = sum_k x[m][k] w[j][k] (+ b[j] when b is not NULL), f32, k ascending. */
void orc_linear_f32(const float *x, int rows, int k, const float *w, const float *b, int n, float *y);
/* SimpleMLPAdaLN::time_embedding([s, t]) (mlp.rs:201-212): out [flow_dim]. */
int orc_flow_time_embedding(const orc_flow_lm_desc *d, const float *blob, float s, float t, float *out);
/* SimpleMLPAdaLN::forward (mlp.rs:214-238) on one row, f32: c [zd], t_emb [flow_dim] (NULL: a head
 * without time conditions), x0 [ldim]. */
int orc_flow_net(const orc_flow_lm_desc *d, const float *blob, const float *c, const float *t_emb,
                 const float *x0, float *out);
/* TTSModel::prompt_text (tts_model.rs:297-307): the LUT rows of the tokens through the transformer
 * (f32 stream), committed.  No text sink. */
int orc_flow_lm_prompt_text(const orc_flow_lm_desc *d, const float *blob, orc_stream *st,
                            const int *ids, int n);
/* One frame (generate_step_parts, tts_model.rs:365-378): input_linear of latent_in (NULL: bos_emb)
 * plus cond [d_model] when not NULL (the conditions, flow_lm.rs:304-307), the transformer
 * (committed), out_norm, z_proj, the EOS logit (out_eos) and the flow head on noise [ldim]
 * conditioned on the output (sample_from_noise, flow_lm.rs:363-384): latent_out [ldim], eos_logit
 * [1].  f32 desc only.  A stream of a grouped-head desc holds num_kv_heads heads of a / num_heads. */
int orc_flow_lm_step(const orc_flow_lm_desc *d, const float *blob, orc_stream *st, const float *latent_in,
                     const float *cond, const float *noise, float *latent_out, float *eos_logit);

/* The q8 precision (desc->precision 1), the batched frame's definition: every linear's weight rows
 * quantized as orc_quantize_rows does (biases, norms and the LUT stay f32, the LUT rows and bos
 * rounded to bf16 when read), activations bf16, each op rounding its output once as a bf16 tensor
 * op does -- linear: bf16(s * acc (+ b)); LayerNorm (affine inside): once; modulate:
 * bf16(bf16(y * bf16(scale + 1)) + shift); y + t, silu, gate * h, x + gate * h, x + v / steps: once
 * each.  The time embeddings are computed in f32 (as the f32 path) and rounded once.  The
 * transformer is orc_layer_step's.  Streams are bf16 caches with bf16 activations. */
/* Its pieces.  The q8 linear: y = bf16(s[j] * sum_k bf16(x[m][k]) q[j][k] (+ b[j])), then epi 0:
 * store; 4: silu; 5: silu(bf16(y + aux[j])); 6: out = bf16(out + bf16(aux[m][j] * y)) (the AdaLN
 * gate); 7: out = bf16(bf16(aux[m][j]) + bf16(y * alpha)) (the solver step); 8: store; 9: out =
 * bf16(bf16(aux[m][j]) + y) (a condition added to the step input).  Every result is rounded to
 * bf16 once.  out [rows][ldo], aux rows of stride ld_aux (0: one row for every row). */
void orc_flow_linear_q8(const float *x, int rows, int k, const int8_t *q, const float *s, const float *b, int n,
                        int epi, float *out, int ldo, const float *aux, int ld_aux, float alpha);
/* LayerNorm of rows (affine w, b or NULL) rounded to bf16, then when shift is given the AdaLN
 * modulation (mlp.rs:4-11) in bf16 steps: bf16(bf16(y * bf16(scale + 1)) + shift). */
void orc_layer_norm_mod(const float *x, int rows, int dim, const float *w, const float *b, float eps,
                        const float *shift, const float *scale, int ld_mod, float *out);
typedef struct orc_flow_q8 orc_flow_q8;
orc_flow_q8 *orc_flow_q8_prepare(const orc_flow_lm_desc *d, const float *blob);
void orc_flow_q8_free(orc_flow_q8 *m);
int orc_flow_q8_prompt_text(orc_flow_q8 *m, orc_stream *st, const int *ids, int n);
int orc_flow_q8_step(orc_flow_q8 *m, orc_stream *st, const float *latent_in, const float *cond, const float *noise,
                     float *latent_out, float *eos_logit);

/* Many streams, one layer: the CPU baseline's batched step (OpenMP over streams). */
int orc_batch_attend(orc_stream **streams, int n, int layer, const float *q, const float *k,
                     const float *v, float scale, float *out);
int orc_batch_commit(orc_stream **streams, int n);
/* Each stream i: evict slot drop[i] (if >= 0, prefix 0), set_ring_slot(set[i]), then append row i
 * of k and v to `layer` (q null) or attend with row i of q (out row i), commit 1 (OpenMP over
 * streams). */
int orc_batch_ring_step(orc_stream **streams, int n, int layer, const int *drop, const int *set, const float *q,
                        const float *k, const float *v, float scale, float *out);
int orc_threads(void);
void orc_set_threads(int n);

const char *orc_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
