/*
 * oracle.h -- CPU restatement of hobby-rs's single-sequence decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product (hobbylm_amd/, include/hobby_gpu.h) never links it.
 *
 * Each function follows one reference function; the file:line it restates is
 * given beside it (paths relative to the HobbyLM repository root).
 */
#ifndef HOBBY_ORACLE_H
#define HOBBY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors hobby-rs/src/config.rs:8-32 (diffusion fields omitted: out of path). */
typedef struct orc_config {
    uint32_t d_model, n_layers, n_dense, n_heads, n_kv_heads, head_dim;
    uint32_t dense_ffn, expert_ffn, n_experts, top_k, n_shared;
    uint32_t vocab_size, context_length;
    float rms_eps, rope_theta, expert_weights_scale;
    int32_t expert_weights_norm, gating_sigmoid;
    uint32_t mask_token_id;
} orc_config;

typedef struct orc_model orc_model;
typedef struct orc_kv orc_kv;

/* error text of the last failing call on this thread */
const char *orc_last_error(void);
void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- gguf.rs ---- */
float orc_half_to_f32(uint16_t h);                                  /* gguf.rs:329-341 */
void orc_dequant_q8_0(const uint8_t *b, size_t n, float *y);        /* gguf.rs:365-375 */
void orc_dequant_f16(const uint8_t *b, size_t n, float *y);         /* gguf.rs:361-363 */
void orc_dequant_q5_0(const uint8_t *b, size_t n, float *y);        /* gguf.rs:377-397 */
void orc_dequant_q4_k(const uint8_t *b, size_t n, float *y);        /* gguf.rs:410-439 */
void orc_dequant_q6_k(const uint8_t *b, size_t n, float *y);        /* gguf.rs:441-468 */
int orc_gguf_load_tensor(const char *path, const char *name, float *out, uint64_t cap, uint64_t *n);

/* ---- quant.rs ---- */
/* Q8Tensor::quantize (quant.rs:78-102): w[out*in] -> scales[out*in/32], qs[out*in] */
void orc_q8_quantize(const float *w, size_t out, size_t in, float *scales, int8_t *qs);
/* activation quantization inside Q8Tensor::matvec (quant.rs:111-123) */
void orc_quantize_act(const float *x, size_t n, int8_t *qx, float *dx);
/* qrow_dot_avx2 (quant.rs:44-67), the AVX2 intrinsic sequence */
float orc_qrow_dot(const int8_t *qw, const int8_t *qa, const float *sw, const float *dx, size_t nb);
/* Q8Tensor::matvec (quant.rs:106-136) */
void orc_q8_matvec(const float *scales, const int8_t *qs, size_t out, size_t in,
                   const float *x, float *y);
/* Q8Tensor::matmul (quant.rs:144-194): x[tn*in] -> y[tn*out] */
void orc_q8_matmul(const float *scales, const int8_t *qs, size_t out, size_t in,
                   const float *x, float *y, size_t tn);

/* ---- ops.rs ---- */
float orc_dot(const float *a, const float *b, size_t n);            /* ops.rs:7-36 */
void orc_matvec_f32(const float *w, const float *x, float *y, size_t out, size_t in); /* ops.rs:40-53 */
float orc_sigmoid(float x);                                         /* ops.rs:75-77 */
float orc_silu(float x);                                            /* ops.rs:80-82 */
float orc_expf(float x);                                            /* f32::exp -> libm expf */
void orc_rmsnorm(const float *x, const float *w, float eps, float *out, size_t n); /* ops.rs:85-96 */
void orc_softmax(float *x, size_t n);                               /* ops.rs:112-128 */
void orc_norm_head(float *v, const float *w, float eps, size_t n);  /* model.rs:753-763 */
/* Rope::new (ops.rs:139-152): cos/sin[max_pos*hd/2] */
void orc_rope_table(size_t head_dim, size_t max_pos, float theta, float *cos_t, float *sin_t);
/* Rope::apply (ops.rs:155-166) */
void orc_rope_apply(const float *cos_t, const float *sin_t, size_t head_dim, float *v, size_t pos);
uint32_t orc_argmax(const float *logits, size_t n);                 /* sample.rs:53-63 */
uint64_t orc_rng_next_u64(uint64_t *state);                         /* sample.rs:10-17 */
float orc_rng_next_f32(uint64_t *state);                            /* sample.rs:18-20 */
uint32_t orc_sample(const float *logits, size_t n, float temp, float top_p, uint64_t *state); /* sample.rs:66-112 */
/* Router decision of one row (model.rs:270-293): sigmoid (or softmax) gate, sel = score +
 * bias, descending sort, top_k ids in rank order, their un-biased scores (renormalised when
 * weights_norm), and gap = sel[k-th] - sel[(k+1)-th]. */
int orc_route(const float *logits, const float *bias, uint32_t n_experts, uint32_t top_k,
              int gating_sigmoid, int weights_norm, uint32_t *idx, float *w, float *gap);

/* One decode-attention layer as in Model::attention (model.rs:199-233), without the
 * projections: q[n_heads*hd], k[n_kv*hd], v[n_kv*hd] are the raw QKV outputs.  Applies
 * QK-norm + RoPE at pos, appends k/v at row `pos` of kcache/vcache ([cap][n_kv*hd]),
 * and writes the attention output out[n_heads*hd].  q and k are updated in place. */
void orc_attention_decode(float *q, float *k, const float *v, const float *q_norm,
                          const float *k_norm, const float *cos_t, const float *sin_t,
                          float eps, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                          uint32_t pos, float *kcache, float *vcache, float *out);

/* ---- model.rs / lib.rs ---- */
int orc_model_load(const char *path, int quant, orc_model **out);   /* Engine::load, lib.rs:85-92 */
void orc_model_free(orc_model *m);
int orc_model_config(const orc_model *m, orc_config *cfg);
uint64_t orc_weight_bytes(const orc_model *m);                      /* model.rs:134-149 */
int orc_kv_new(const orc_model *m, orc_kv **out);                   /* KvCache::new, model.rs:67-74 */
void orc_kv_free(orc_kv *kv);
uint32_t orc_kv_len(const orc_kv *kv);
/* copy cache rows [0,len) of one layer into k/v ([len][kv_dim]) */
int orc_kv_read(const orc_kv *kv, uint32_t layer, float *k, float *v);
/* overwrite the whole cache contents with len rows per layer (k/v: [L][len][kv_dim]) */
int orc_kv_load(orc_kv *kv, uint32_t len, const float *k, const float *v);
int orc_token_embedding(const orc_model *m, uint32_t id, float *out); /* model.rs:332-335 */
int orc_forward(const orc_model *m, orc_kv *kv, uint32_t token, uint32_t pos, float *logits); /* model.rs:152 */
int orc_forward_x(const orc_model *m, orc_kv *kv, const float *x, uint32_t pos, float *logits); /* model.rs:160 */
int orc_prefill(const orc_model *m, orc_kv *kv, const float *inputs, uint32_t tn, float *logits); /* model.rs:340 */
/* Routing of the last forward/prefill row: idx[L*top_k], weight[L*top_k] (rank order;
 * dense layers hold UINT32_MAX / 0) and gap[L] = sel(k-th) - sel(k+1-th). */
int orc_last_routing(const orc_kv *kv, uint32_t *idx, float *weight, float *gap);
/* Engine::generate at temp 0 (lib.rs:107-162) over token ids: prefill, then greedy
 * steps with the id>=min(50257,vocab) mask, optional repetition penalty, EOS and
 * context stops.  Returns the number of generated ids written to out_ids. */
/* DiffOpts (lib.rs:45-65) */
typedef struct orc_diff_opts {
    uint32_t gen_len, block, steps;
    float temp, rep_penalty;
    uint32_t remask_steps;
    float remask_frac;
    uint64_t seed;
    uint32_t cached;
    float threshold;
} orc_diff_opts;
uint32_t orc_gumbel_argmax(const float *logits, size_t n, float temp, uint64_t *state); /* sample.rs:32-50 */
int orc_run_block(const orc_model *m, orc_kv *kv, const float *block, uint32_t b, uint32_t base, float *logits,
                  float *bk, float *bv);                            /* model.rs:471-585 */
int orc_forward_bidir(const orc_model *m, const float *inputs, uint32_t tn, float *logits); /* model.rs:443-468 */
int orc_generate_diffusion(const orc_model *m, const uint32_t *prompt, uint32_t n_prompt, const orc_diff_opts *o,
                           uint32_t eos, uint32_t *out_ids, uint32_t *n_out); /* lib.rs:214-495 */
int orc_generate(const orc_model *m, orc_kv *kv, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_new,
                 float temp, float top_p, uint64_t seed, float rep_penalty, uint32_t eos, uint32_t *out_ids,
                 uint32_t *n_out);                                  /* lib.rs:107-162 */
int orc_generate_greedy(const orc_model *m, orc_kv *kv, const uint32_t *prompt, uint32_t n_prompt,
                        uint32_t max_new, float rep_penalty, uint32_t eos, uint32_t *out_ids,
                        uint32_t *n_out);

#ifdef __cplusplus
}
#endif
#endif
