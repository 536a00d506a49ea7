/*
 * hobby_gpu.h -- C ABI of the MI355X (gfx950) decode backend for hobbylm GGUF models.
 *
 * Drop-in boundary for hobby-rs's model-load / forward-token API.  Every entry point
 * names the reference item it replaces (paths relative to the HobbyLM repository root).
 *
 * Conventions
 *   - Functions returning int return HG_OK (0) or a negative HG_ERR_* code; the message
 *     of the last failure on the calling thread is hg_last_error().  Nothing aborts or
 *     throws across this boundary (the reference panics with panic=abort instead,
 *     hobby-rs/Cargo.toml:23).
 *   - Caller buffers are host memory; the library owns all device memory.
 *   - An hg_model is immutable after load and may be shared by threads (the reference
 *     shares Arc<Engine>, hobby-chat/src-tauri/src/server.rs:15,28-30).  An hg_kv owns a
 *     HIP stream, its KV cache and its scratch, and must be used by one thread at a time
 *     (the reference's &mut KvCache).
 *   - Numerics: every operation of the step follows the reference's operation order: the
 *     Q8_0 matvec reproduces qrow_dot_avx2's lane order and FMAs (quant.rs:44-67), ops::dot
 *     its f32x8 accumulators, and RMSNorm's sum of squares and attention's softmax and P.V
 *     sums run sequentially as in ops.rs / model.rs, with an expf equal to glibc's.  Logits,
 *     expert routing and KV-cache contents are therefore bit-identical to hobby-rs's AVX2
 *     path.  A cache created with HG_KV_FAST reassociates those three sums as trees; its
 *     logits differ in the last bits, and because the sigmoid router selects experts by
 *     gaps as small as 1e-4, such last-bit differences can flip a routing decision and
 *     move the logits by percents: HG_KV_FAST is not a parity mode.
 */
#ifndef HOBBY_GPU_H
#define HOBBY_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HG_OK 0
#define HG_ERR_IO (-1)          /* file cannot be opened / mapped */
#define HG_ERR_FORMAT (-2)      /* malformed or truncated GGUF, missing tensor or metadata */
#define HG_ERR_UNSUPPORTED (-3) /* a ggml type or shape this backend does not handle */
#define HG_ERR_ARG (-4)         /* bad argument: token >= vocab, pos out of order or >= context */
#define HG_ERR_DEVICE (-5)      /* HIP runtime failure or no gfx950 device */
#define HG_ERR_NOMEM (-6)       /* device or host allocation failed */

/* hg_kv_new flags */
#define HG_KV_FAST 1u /* tree reductions in RMSNorm and attention instead of the reference's
                         sequential order: not bit-identical, and near-tied expert routing can
                         then differ from hobby-rs (see the numerics note above) */

typedef struct hg_model hg_model;
typedef struct hg_kv hg_kv;
typedef struct hg_q8_tensor hg_q8_tensor;

/* Model hyperparameters; mirrors Config (hobby-rs/src/config.rs:8-32, diffusion fields
 * omitted). */
typedef struct hg_config {
    uint32_t d_model, n_layers, n_dense, n_heads, n_kv_heads, head_dim;
    uint32_t dense_ffn, expert_ffn, n_experts, top_k, n_shared;
    uint32_t vocab_size, context_length;
    float rms_eps, rope_theta, expert_weights_scale;
    int32_t expert_weights_norm, gating_sigmoid;
    uint32_t mask_token_id;   /* the diffusion canvas's [MASK] id (config.rs:93, default 50257) */
} hg_config;

/* Message of the last failing call on this thread ("" if none). */
const char *hg_last_error(void);

/* ---- model (hobby-rs/src/lib.rs, model.rs) ------------------------------------------ */

/* Engine::load(path, quant) (lib.rs:85-92) -> Gguf::open (gguf.rs:166-212),
 * Config::from_gguf (config.rs:35-97), Model::load (model.rs:79-131).  quant != 0 keeps
 * every matrix as Q8_0 after the load-time requantization of Q8Tensor::quantize
 * (quant.rs:78-102), from any matrix type Gguf::load reads (F32, F16, Q5_0, Q8_0, Q4_K,
 * Q6_K); quant == 0 keeps every matrix as f32 (Mat::Owned, quant.rs:198-222) and applies it
 * with ops::matvec / ops::matmul (ops.rs:40-71: ops::dot per output, ops.rs:7-36) -- in that
 * mode hg_forward, hg_forward_x, hg_prefill (one step per prompt row), the generate entry
 * points and hg_last_routing work, with reference-order caches only (HG_KV_FAST is refused),
 * while the batched prompt path (hg_run_block, hg_forward_bidir, hg_generate_diffusion) and
 * batched decode (hg_batch_*) return HG_ERR_UNSUPPORTED.  The file is parsed and
 * checked on the host before any device call, so format errors are reported (HG_ERR_IO,
 * HG_ERR_FORMAT, HG_ERR_UNSUPPORTED) on a machine without a GPU too.  The tokenizer is not
 * built: token ids cross this boundary. */
int hg_model_load(const char *path, int quant, hg_model **out);
void hg_model_free(hg_model *m);
/* Gguf::open (gguf.rs:166-212) + Gguf::load (gguf.rs:250-269): tensor `name` of the file at
 * `path` as f32, dequantized from F32, F16, Q5_0, Q8_0, Q4_K or Q6_K (gguf.rs:361-468).  *n
 * receives the element count; out (NULL: query the count only) holds cap floats.  Host work
 * only: no device is needed. */
int hg_gguf_load_tensor(const char *path, const char *name, float *out, uint64_t cap, uint64_t *n);
/* Engine.cfg (lib.rs:79) */
int hg_model_config(const hg_model *m, hg_config *out);
/* Engine::weight_bytes (lib.rs:100-102) -> Model::weight_bytes (model.rs:134-149): bytes
 * the reference holds for the matrices (one f32 scale + 32 int8 per block).  The device
 * copy stores each scale as the f16 it came from when that is exact (34 B per block). */
uint64_t hg_weight_bytes(const hg_model *m);
/* Device bytes actually resident for the matrices. */
uint64_t hg_device_weight_bytes(const hg_model *m);
/* Model::token_embedding (model.rs:332-335) */
int hg_token_embedding(const hg_model *m, uint32_t id, float *out);

/* ---- KV cache + decode step ---------------------------------------------------------- */

/* KvCache::new (model.rs:67-74): a device-resident cache for max_ctx positions
 * (0 = context_length), layer-major, head-major within a layer.  flags: 0 or HG_KV_FAST. */
int hg_kv_new(const hg_model *m, uint32_t max_ctx, uint32_t flags, hg_kv **out);
void hg_kv_free(hg_kv *kv);
/* KvCache.len (model.rs:63) */
uint32_t hg_kv_len(const hg_kv *kv);
/* `cache.len = len` on the reference's pub field (model.rs:63): keep rows [0, len) and
 * decode on from len (len <= hg_kv_len; later rows are overwritten). */
int hg_kv_truncate(hg_kv *kv, uint32_t len);
/* Cache rows [0, len) of one layer in the reference layout KvCache.k[layer] /
 * KvCache.v[layer] ([len][n_kv_heads*head_dim], model.rs:60-64, 210-211). */
int hg_kv_read(const hg_kv *kv, uint32_t layer, float *k, float *v);
/* Assigning the reference's pub fields KvCache.k / .v / .len (model.rs:60-64): rows [0, len)
 * of every layer from k, v ([n_layers][len][n_kv_heads*head_dim]), then len; later decode
 * steps continue from len. */
int hg_kv_load(hg_kv *kv, uint32_t len, const float *k, const float *v);

/* Model::forward(token, pos, cache) (model.rs:152-156).  pos must equal hg_kv_len(kv)
 * and be < max_ctx.  logits (may be NULL) receives vocab_size floats; next (may be NULL)
 * receives the greedy token of Engine::generate at temp 0 (lib.rs:132-142 with
 * rep_penalty 1: ids >= min(50257, vocab) masked, then sample::argmax, sample.rs:53-63). */
int hg_forward(const hg_model *m, hg_kv *kv, uint32_t token, uint32_t pos, float *logits,
               uint32_t *next);
/* Model::forward_x(x, pos, cache) (model.rs:160-184): x is d_model floats. */
int hg_forward_x(const hg_model *m, hg_kv *kv, const float *x, uint32_t pos, float *logits,
                 uint32_t *next);
/* Model::prefill(inputs, cache) (model.rs:340-370): tn rows of d_model floats appended at
 * positions len..len+tn-1 with the prompt path's arithmetic (Q8Tensor::matmul order,
 * quant.rs:171-184; experts accumulated in expert-id order, model.rs:707-731); logits and
 * next are those of the last row. */
int hg_prefill(const hg_model *m, hg_kv *kv, const float *inputs, uint32_t tn, float *logits,
               uint32_t *next);
/* n_steps greedy decode steps without a host round trip per token: step i forwards the
 * previous step's greedy token (first_token for i = 0) at pos = len and writes the greedy
 * token it produces to out_ids[i].  Equivalent to n_steps calls of hg_forward with
 * token = previous *next, which is the loop of Engine::generate (lib.rs:131-160) at temp 0
 * with no EOS stop. */
int hg_decode_greedy(const hg_model *m, hg_kv *kv, uint32_t first_token, uint32_t n_steps,
                     uint32_t *out_ids);
/* Engine::generate (lib.rs:107-162) at temp 0 over token ids: prefill of the prompt, then
 * greedy steps with the 50257 mask, the repetition penalty of lib.rs:136-141 (1.0 = off),
 * the EOS stop (lib.rs:143-145) and the context stop (lib.rs:155-157).  Writes at most
 * max_new ids; *n_out receives the count. */
int hg_generate_greedy(const hg_model *m, hg_kv *kv, const uint32_t *prompt, uint32_t n_prompt,
                       uint32_t max_new, float rep_penalty, uint32_t eos, uint32_t *out_ids,
                       uint32_t *n_out);
/* GenOpts (lib.rs:29-41): temp <= 0 is greedy; top_p outside (0, 1) disables the nucleus;
 * rep_penalty 1.0 is off. */
typedef struct hg_gen_opts {
    uint32_t max_new;
    float temp;
    float top_p;
    uint64_t seed;
    float rep_penalty;
} hg_gen_opts;
/* Engine::generate (lib.rs:107-162) over token ids with sampling on the device: prefill of the
 * prompt, then per step the 50257 mask, the repetition penalty once per earlier occurrence,
 * sample::sample (sample.rs:66-112) with the xorshift64* Rng seeded by opts->seed, the EOS stop
 * and the context stop.  The logits never leave the GPU; the host reads the picks every 16
 * steps.  Writes at most max_new ids; *n_out receives the count; the cache then holds the
 * prompt and the forwarded ids.  Equal probabilities in the nucleus order by ascending id
 * (sample.rs:86's sort_unstable_by leaves that order unspecified). */
int hg_generate(const hg_model *m, hg_kv *kv, const uint32_t *prompt, uint32_t n_prompt, const hg_gen_opts *opts,
                uint32_t eos, uint32_t *out_ids, uint32_t *n_out);
/* sample::sample (sample.rs:66-112) of host logits[0 .. n) on the device, with the RNG state
 * *rng_state (Rng's u64: the seed clamped to >= 1), which it advances; the pick in *out. */
int hg_sample(const float *logits, uint32_t n, float temp, float top_p, uint64_t *rng_state, uint32_t *out);
/* ---- the diffusion block path (model.rs:440-651, lib.rs:164-495) ---------------------- */

/* Model::run_block (model.rs:471-585): the b block rows (residual inputs, b x d_model floats)
 * at positions base .. base + b - 1 attend to the cache's rows 0 .. base - 1 and to every block
 * row (bidirectional within the block).  logits [b][vocab] and the block's K/V rows bk / bv
 * [n_layers][b][kv_dim] when not NULL.  append == 0 leaves the cache as it was (run_block is
 * non-destructive); append != 0 (base must equal the cache length) also appends the block's
 * rows, as lib.rs:374-381 does when a block is finalized. */
int hg_run_block(const hg_model *m, hg_kv *kv, const float *block, uint32_t b, uint32_t base, int append,
                 float *logits, float *bk, float *bv);
/* Model::forward_bidir (model.rs:443-468): all tn rows with full bidirectional attention and no
 * cache; logits [tn][vocab]. */
int hg_forward_bidir(const hg_model *m, const float *inputs, uint32_t tn, float *logits);
/* DiffOpts (lib.rs:45-65). */
typedef struct hg_diff_opts {
    uint32_t gen_len, block, steps;
    float temp, rep_penalty;
    uint32_t remask_steps;
    float remask_frac;
    uint64_t seed;
    uint32_t cached;
    float threshold;
} hg_diff_opts;
/* Engine::generate_diffusion (lib.rs:214-495) over token ids: the prefix-cached (cached != 0,
 * lib.rs:269-407) or the uncached (lib.rs:410-495) semi-autoregressive denoising of gen_len ids
 * after the prompt, with the block's logits scored on the device (the mask, the presence
 * penalty, the pick and its softmax confidences; only those cross PCIe).  Writes the generated
 * ids up to the first eos (at most gen_len); *n_out receives the count.  temp > 0 draws the
 * picks as sample::gumbel_argmax (sample.rs:32-50) with the seeded Rng: -ln(-ln(u)) comes from a
 * table of the Rng's 2^24 possible u computed with the host libm's logf (64 MB on the device,
 * built once per process), each lane's draws from a GF(2) jump of the xorshift state. */
int hg_generate_diffusion(const hg_model *m, const uint32_t *prompt, uint32_t n_prompt, const hg_diff_opts *opts,
                          uint32_t eos, uint32_t *out_ids, uint32_t *n_out);

/* Routing of the last processed row, per layer in rank order (model.rs:282-293):
 * idx[L*top_k] (UINT32_MAX for dense layers) and the scaled weights w[L*top_k]. */
int hg_last_routing(const hg_kv *kv, uint32_t *idx, float *w);

/* ---- batched decode over a paged KV cache ------------------------------------------------
 * hobby-rs serves concurrent generations by giving each its own KvCache (model.rs:60-75) and
 * calling Model::forward for each (hobby-chat/src-tauri/src/server.rs:21-31 shares one
 * Arc<Engine> between them); it has no batched step.  An hg_batch runs one decode step of
 * many sequences at once: every sequence's step is Model::forward (model.rs:152-184) on its
 * own cache, with logits, expert routing and cache rows bit-identical to its own hg_forward.
 * The Q8 matrix products of all sequences run as int8 MFMA GEMMs that keep qrow_dot_avx2's
 * order per sequence; the routed experts' rows run once per expert over the sequences that
 * picked it (the grouping of ffn_prefill, model.rs:676-731, with each sequence keeping the
 * decode path's rank-order combine, model.rs:306-323).  Cache rows live in a pool of pages of
 * HG_PAGE positions; each sequence has a block table of page ids.  An hg_batch owns a HIP
 * stream and must be used by one thread at a time. */
#define HG_PAGE 16u
typedef struct hg_batch hg_batch;
/* A batch of up to max_seqs sequences of at most max_ctx positions (0 = context_length) over a
 * pool of n_pages pages (a page holds HG_PAGE positions of one sequence, every layer). */
int hg_batch_new(const hg_model *m, uint32_t max_seqs, uint32_t max_ctx, uint32_t n_pages, hg_batch **out);
void hg_batch_free(hg_batch *b);
/* Sequence seq's block table: pages[i] holds its positions HG_PAGE i .. HG_PAGE i + HG_PAGE - 1.
 * The sequence's length becomes 0 (an empty KvCache::new, model.rs:67-74). */
int hg_batch_set_pages(hg_batch *b, uint32_t seq, const uint32_t *pages, uint32_t n);
/* KvCache.len of sequence seq. */
uint32_t hg_batch_len(const hg_batch *b, uint32_t seq);
/* Sequence seq's KvCache.k / .v / .len = rows [0, len) of every layer from k, v
 * ([n_layers][len][n_kv_heads*head_dim]), as hg_kv_load. */
int hg_batch_load(hg_batch *b, uint32_t seq, uint32_t len, const float *k, const float *v);
/* Rows [0, len) of one layer of sequence seq ([len][n_kv_heads*head_dim]), as hg_kv_read. */
int hg_batch_read(hg_batch *b, uint32_t seq, uint32_t layer, float *k, float *v);
/* Model::forward(tokens[s], len_s, cache_s) for sequences s = 0 .. n-1 in one step.
 * logits (may be NULL) receives [n][vocab_size]; next (may be NULL) the greedy token of each
 * (as hg_forward's next). */
int hg_batch_forward(const hg_model *m, hg_batch *b, const uint32_t *tokens, uint32_t n, float *logits,
                     uint32_t *next);
/* n_steps batched greedy steps of sequences 0 .. n-1 without host round trips: step i forwards
 * each sequence's previous greedy token (first[s] for i = 0); out_ids receives [n_steps][n]. */
int hg_batch_decode_greedy(const hg_model *m, hg_batch *b, const uint32_t *first, uint32_t n, uint32_t n_steps,
                           uint32_t *out_ids);
/* Routing of sequence seq's last step, as hg_last_routing. */
int hg_batch_routing(hg_batch *b, uint32_t seq, uint32_t *idx, float *w);

/* ---- instrumentation (no counterpart in the reference) -------------------------------- */

#define HG_PROF_CLASSES 12
/* Rows [0, len) of every layer of batch sequence seq set to seeded pseudo-random values of unit
 * variance (a hash of seed, layer, position and element), written on the device; the length
 * becomes len.  For timing workloads whose caches would take long to upload. */
int hg_batch_fill(hg_batch *b, uint32_t seq, uint32_t len, uint64_t seed);
/* Time one decode step per kernel class, for measurement tools: the step at pos = len is
 * replayed `reps` times on the cache's own stream, every kernel launched with a start/stop
 * HIP event pair recorded by its own dispatch (hipExtLaunchKernelGGL), i.e. kernel execution
 * time; the cache length does not advance, and the row written at len is overwritten by the
 * next real step.  us[c] = mean microseconds per step spent in class c, launches[c] = kernel
 * launches per step; arrays of HG_PROF_CLASSES. */
int hg_profile_step(const hg_model *m, hg_kv *kv, uint32_t token, uint32_t reps, float *us,
                    uint32_t *launches);
/* Name of profile class c ("" when out of range). */
const char *hg_profile_class(uint32_t c);

/* ---- operator level (hobby-rs/src/quant.rs, model.rs:199-233) ------------------------ */

/* Q8Tensor::quantize(w, out, in) (quant.rs:78-102) from f32 weights [out][in]. */
int hg_q8_tensor_quantize(const float *w, uint32_t out, uint32_t in, hg_q8_tensor **t);
/* The GGUF load path of one Q8_0 matrix: dequant_q8_0 (gguf.rs:365-375) then
 * Q8Tensor::quantize.  blocks: out*in/32 GGML blocks {f16 d; int8 q[32]}. */
int hg_q8_tensor_from_q8_0(const void *blocks, uint32_t out, uint32_t in, hg_q8_tensor **t);
void hg_q8_tensor_free(hg_q8_tensor *t);
/* Q8Tensor::bytes (quant.rs:138-140) */
uint64_t hg_q8_tensor_bytes(const hg_q8_tensor *t);
/* Q8Tensor::matvec (quant.rs:106-136): y[out] = W x[in]. */
int hg_q8_tensor_matvec(const hg_q8_tensor *t, const float *x, float *y);
/* No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops and harnesses that forbid hipMalloc).  hg_q8_tensor_matvec
 * (Q8Tensor::matvec, quant.rs:106-136) on device-resident x_dev[in] and y_dev[out], enqueued on
 * `stream` (a hipStream_t; NULL = the null stream) with nothing allocated: the quantized
 * activation is kept in a fixed library-held device buffer of HG_NOALLOC_SCRATCH_BYTES per GPU
 * (held until the process ends), which bounds in to HG_NOALLOC_MAX_IN (larger tensors:
 * HG_ERR_ARG).  Results are bit-identical to hg_q8_tensor_matvec.  Every call on one GPU uses
 * that GPU's one buffer: calls that overlap on a GPU (other streams, other threads) race.
 * Returns once the work is enqueued; the caller synchronizes the stream. */
#define HG_NOALLOC_MAX_IN 32768u
#define HG_NOALLOC_SCRATCH_BYTES ((HG_NOALLOC_MAX_IN / 128u) * 144u)
int hg_q8_tensor_matvec_noalloc(const hg_q8_tensor *t, const float *x_dev, float *y_dev, void *stream);
/* Q8Tensor::matmul (quant.rs:144-194): y[tn][out] = x[tn][in] W^T. */
int hg_q8_tensor_matmul(const hg_q8_tensor *t, const float *x, float *y, uint32_t tn);
/* The routed-expert matvec: t holds n_mat stacked matrices of rows_per_mat rows each
 * (split_experts, model.rs:17-21); y[i][rows_per_mat] = W[ids[i]] x for i < n_ids. */
int hg_q8_tensor_matvec_gather(const hg_q8_tensor *t, uint32_t rows_per_mat, const uint32_t *ids,
                               uint32_t n_ids, const float *x, float *y);

/* One decode-attention layer of Model::attention (model.rs:199-233) after the QKV
 * projection: QK-norm (model.rs:753-763) and RoPE (ops.rs:139-166, theta, table of
 * rope_len positions) on q[n_heads*hd] and k[n_kv*hd], append of k and v at row pos of
 * the caches kc/vc ([pos+1][n_kv*hd] host arrays; rows < pos are inputs, row pos is
 * written), GQA attention over rows 0..pos, output out[n_heads*hd].  flags: HG_KV_FAST. */
int hg_attention_decode(const float *q, const float *k, const float *v, const float *q_norm,
                        const float *k_norm, float eps, float theta, uint32_t rope_len,
                        uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t pos, float *kc,
                        float *vc, float *out, uint32_t flags);

/* The sequential binary32 sum out = ((0 + x[0]) + x[1]) + ... + x[n-1] that ops::rmsnorm
 * (`ss += v * v`, ops.rs:101-104) and ops::softmax (`sum += *v`, ops.rs:119-122) form, computed
 * on the device by the method the decode kernels use for it: methods 1..7 = the workgroup
 * layouts of those kernels (waves x terms per lane: 8x4, 4x4, 4x4 on waves 0,5,6,7, 2x8, 4x8,
 * 4x12, 8x32; identical bits for non-negative terms; other inputs or n beyond the layout fall
 * back to one lane), method 0 = one lane adding in index order (n <= 4096 in LDS; method 7:
 * n <= 16384). */
int hg_seq_sum(const float *x, uint32_t n, uint32_t method, float *out);

/* ---- measurement (no counterpart in the reference) ------------------------------------ */

/* Kernel time of t's matvec on device-resident data: x[in] is quantized once on the device,
 * then `reps` matvecs (ids != NULL: the gather of hg_q8_tensor_matvec_gather, one launch)
 * run back to back, each timed by events its own dispatch records.  copies > 1 replicates
 * the weights that many times and rotates through the replicas (cold caches when
 * copies * bytes exceeds the last-level cache).  us = mean microseconds per call. */
int hg_q8_tensor_time_matvec(const hg_q8_tensor *t, const float *x, uint32_t reps, uint32_t copies,
                             uint32_t rows_per_mat, const uint32_t *ids, uint32_t n_ids, float *us);
/* Kernel time of one decode-attention layer (the two kernels of hg_attention_decode) at
 * context ctx on seeded device-resident q, k, v and cache (unit QK-norm gains, theta
 * 10000), run `reps` times: us[0] = scores (or split partials with HG_KV_FAST), us[1] =
 * softmax + P.V (or merge), mean microseconds per layer. */
int hg_attention_time(uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t ctx, uint32_t reps,
                      uint32_t flags, float *us);

#ifdef __cplusplus
}
#endif
#endif
