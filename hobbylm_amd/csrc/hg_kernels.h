// hg_kernels.h -- host-side launchers of the gfx950 decode kernels (hg_kernels.hip).
#pragma once
#include "hg_common.h"

#include <string>
#include <vector>

namespace hg {

// Kernel-execution timing of every launch issued while installed (profiling only).
struct LaunchTimer {
    int cls = 0;                                           // class tag of the next launches
    std::vector<int> tags;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
    void add(hipEvent_t a, hipEvent_t b) { ev.emplace_back(a, b); tags.push_back(cls); }
};
void set_launch_timer(LaunchTimer *t);
LaunchTimer *launch_timer();   // this thread's, or null
// First launch error recorded on this thread since the last take (hipSuccess if none), with
// the kernel it concerns; taking clears it.
hipError_t take_launch_error(std::string &msg);
hipError_t take_launch_error_reset();
void note_launch_error(hipError_t e, const std::string &what);

hipError_t init_kernel_attributes();
// LDS ring slots of the reference-order P.V kernel for a cache of cap positions (>= 2 needed).
__host__ __device__ uint32_t pv_ring_slots(uint32_t cap);
// Whether the V slice and products of a cache of cap positions fit the LDS-resident P.V kernel.
__host__ __device__ bool pv_res_fits(uint32_t cap);
void launch_embed(hipStream_t st, const float *emb, uint32_t d, const StepParams *p, float *x);
void launch_load_row(hipStream_t st, const float *inputs, uint32_t d, const StepParams *p, float *x);
void launch_advance(hipStream_t st, StepParams *p);
void launch_rmsnorm_quant(hipStream_t st, bool exact, const float *x, const float *w, float eps, uint32_t d,
                          float *h, uint8_t *q, float *dq);
// The same for `rows` rows of d floats (x, h row-major; q, dq one quantized row each).
void launch_rmsnorm_quant_rows(hipStream_t st, bool exact, uint32_t rows, const float *x, const float *w, float eps,
                               uint32_t d, float *h, uint8_t *q, float *dq);
void launch_quant_vec(hipStream_t st, const float *x, uint32_t n, uint8_t *q, float *dq);
uint32_t matvec_blocks(uint32_t N, uint32_t threads);
// dq == nullptr: q points to an f32 activation that each workgroup quantizes in its prologue.
void launch_matvec(hipStream_t st, int order, int epi, const Q8Mat &W, const uint8_t *q, const float *dq, float *y,
                   uint32_t threads, uint32_t valid, float *pv, uint32_t *pi);
// out = the q | k | v rows of W times quant(rmsnorm(x, w)), with q and k normed (qn, kn) and
// rotated at p->pos, and k, v appended to the caches at row p->pos; one workgroup per head.
bool launch_qkv_head(hipStream_t st, bool exact, int order, uint32_t hd, const Q8Mat &W, const float *x,
                     const float *w, float eps, const float *qn, const float *kn, const float *cs, const float *sn,
                     const StepParams *p, uint32_t n_heads, uint32_t n_kv, float *kc, float *vc, uint32_t cap,
                     float *out);
// Reference order, head_dim 64, a window the LDS-resident softmax + P.V kernel takes: the QKV
// step and the attention scores in one launch (workgroups that each form one q head and score
// one split of at most QKV_SCORE_POS positions, t < pos; qkv_score_splits splits), then
// launch_attn_pv_self for the softmax + P.V, which forms the score at pos itself.
// launch_qkv_scores returns false, launching nothing, where qkv_scores_ok does not hold;
// scores and pmax as launch_attn's scratch and part.
constexpr uint32_t QKV_SCORE_POS = 256;
uint32_t qkv_score_splits(uint32_t win, uint32_t n_heads, uint32_t n_kv);
bool qkv_scores_ok(bool exact, uint32_t hd, uint32_t win, uint32_t n_heads, uint32_t n_kv, uint32_t d);
bool launch_qkv_scores(hipStream_t st, int order, const Q8Mat &W, const float *x, const float *w, float eps,
                       const float *qn, const float *kn, const float *cs, const float *sn, const StepParams *p,
                       uint32_t n_heads, uint32_t n_kv, float *kc, float *vc, uint32_t cap, uint32_t win, float *out,
                       float *scores, float *pmax);
void launch_attn_pv_self(hipStream_t st, const float *qkv, const StepParams *p, float *vc, uint32_t cap, uint32_t win,
                         uint32_t n_heads, uint32_t n_kv, float *part, float *scratch, float *o_out);
// The same head steps for a q | k | v vector computed elsewhere (rewritten in place).
bool launch_qk_rope_append(hipStream_t st, uint32_t hd, float *qkv, const float *qn, const float *kn, float eps,
                           const float *cs, const float *sn, const StepParams *p, uint32_t n_heads, uint32_t n_kv,
                           float *kc, float *vc, uint32_t cap);
// The matvecs of matrices ids[0..n_ids) of a stack of rows_per_mat-row matrices, one launch.
void launch_matvec_gather(hipStream_t st, const Q8Mat &W, uint32_t rows_per_mat, const uint32_t *ids, uint32_t n_ids,
                          const uint8_t *q, const float *dq, float *y);
void launch_argmax_final(hipStream_t st, const float *pv, const uint32_t *pi, uint32_t n, StepParams *p,
                         uint32_t *out_ids);
size_t attn_fast_shm(uint32_t hd, uint32_t rep, uint32_t cap, uint32_t S);
// which = 0: scores (reference order) or split partials (fast); which = 1: softmax + P.V or merge.
// qkv holds q and k normed and rotated, and the caches row pos already (launch_qkv_head or
// launch_qk_rope_append); qn, kn, eps, cs, sn are not read.
// cap is the cache's row stride; win (pos + 1 <= win <= cap) the context extent the launches
// are sized for (splits, LDS, kernel choice), so their cost follows the live context.
// Reference order with q_out == nullptr leaves the quantization of o to its consumer.
bool launch_attn(hipStream_t st, bool exact, int which, uint32_t hd, const float *qkv, const float *qn,
                 const float *kn, float eps, const float *cs, const float *sn, const StepParams *p, float *kc,
                 float *vc, uint32_t cap, uint32_t win, uint32_t n_heads, uint32_t n_kv, uint32_t S, float *part,
                 float *scratch, float *o_out, uint8_t *q_out, float *d_out);
// Attention splits of a window of win positions (at most 256 positions per split).
inline uint32_t attn_splits(uint32_t win) {
    const uint32_t s = div_up(win, 256);
    return s > 64 ? s : 64;
}
// Router row permutation the kernel expects in Wp (d a multiple of 32): element k of a row is
// stored at 32 (k / 32) + 4 (k % 8) + (k % 32) / 8, so the chains k % 32 = l, 8 + l, 16 + l,
// 24 + l of a 32-wide step are the four consecutive floats 4 l .. 4 l + 3.
__host__ __device__ inline uint32_t router_perm(uint32_t k) {
    return (k / 32) * 32 + 4 * (k % 8) + (k % 32) / 8;
}
void launch_ffn_router(hipStream_t st, bool exact, const float *x, const float *w, float eps, uint32_t d,
                       const float *Wr, const float *Wp, const float *bias, uint32_t E, uint32_t top_k,
                       int gating_sigmoid, int weights_norm, float weights_scale, uint8_t *q, float *dq,
                       uint32_t *topk_idx, float *topk_w, uint32_t *order, uint32_t *rec_idx, float *rec_w);
// The router of `rows` rows: row r reads and writes its pointers advanced by r times rs.
void launch_ffn_router_rows(hipStream_t st, bool exact, uint32_t rows, RowStrides rs, const float *x, const float *w,
                            float eps, uint32_t d, const float *Wr, const float *Wp, const float *bias, uint32_t E,
                            uint32_t top_k, int gating_sigmoid, int weights_norm, float weights_scale, uint8_t *q,
                            float *dq, uint32_t *topk_idx, float *topk_w, uint32_t *order, uint32_t *rec_idx,
                            float *rec_w);
// ffn_norm + router + gate/up of every slot in one launch (E == 0: the dense FFN, slot 0);
// false when the shapes are outside what it handles (the caller then uses the router and
// gate/up launches).
bool launch_ffn_front(hipStream_t st, bool exact, int order, const float *x, const float *w, float eps, uint32_t d,
                      const float *Wp, const float *bias, uint32_t E, uint32_t top_k, int gating_sigmoid,
                      int weights_norm, float weights_scale, const Q8Mat &Wg, const Q8Mat &Wu, const Q8Mat &Sg,
                      const Q8Mat &Su, uint32_t n_slots, uint32_t f, uint32_t *topk_idx, float *topk_w,
                      uint32_t *ord, uint32_t *rec_idx, float *rec_w, float *a);
// One workgroup forms 0 + x[0] + ... + x[n-1] in binary32 (method 1: the parallel exact
// method, method 0: one lane).
void launch_seq_sum(hipStream_t st, const float *x, uint32_t n, int method, float *out);
void launch_ffn_gateup(hipStream_t st, int order, const Q8Mat &Wg, const Q8Mat &Wu, const Q8Mat &Sg,
                       const Q8Mat &Su, const uint32_t *topk_idx, uint32_t top_k, uint32_t n_slots, uint32_t f,
                       const uint8_t *q, const float *dq, float *a);
void launch_ffn_down(hipStream_t st, int order, const Q8Mat &Wd, const Q8Mat &Sd, const uint32_t *topk_idx,
                     const float *topk_w, const uint32_t *ord, uint32_t top_k, uint32_t n_slots, int dense,
                     uint32_t d, uint32_t f, const float *a, float *x);

}  // namespace hg
