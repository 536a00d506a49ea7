// hg_batch.h -- device layouts and launchers of the batched decode step (hg_batch_kernels.hip).
#pragma once
#include <string>

#include "hg_common.h"

namespace hg {

constexpr uint32_t PAGE = 16;                   // positions per KV page
constexpr uint32_t ACH = 256;                   // positions per attention score chunk
constexpr uint32_t MAX_GROUPS = 256;            // experts + the shared expert
constexpr size_t BPV_LDS_BUDGET = 150 * 1024;   // softmax + P.V: e_t and the product ring

// The KV pages of one layer: [page][kv head][PAGE][hd] floats for K and for V, and the block
// tables [sequence][bt_stride] (position t of sequence s is in page bt[s][t / PAGE]).
struct PagedKV {
    float *k, *v;
    const uint32_t *bt;
    uint32_t bt_stride, n_heads, n_kv;
};

__host__ __device__ inline size_t kv_row_off(uint32_t page, uint32_t g, uint32_t slot, uint32_t n_kv, uint32_t hd) {
    return (((size_t)page * n_kv + g) * PAGE + slot) * hd;
}

// One column tile of a batched GEMM: entries entry0 .. entry0 + count - 1 of the entry tables
// (act_row: which activation row, out_row: which output row) against matrix group grp of
// matrix set `mat` (rows grp * rows .. + rows - 1; set 0: the plain or routed matrices, set 1:
// the shared expert's).
struct GemmTile {
    uint32_t grp, entry0, count, mat;
};

enum { GM_STORE = 0, GM_RESID = 1, GM_GATEUP = 2 };

// A batched GEMM launch: the matrices (W; U the up matrices of GM_GATEUP), the column tiles
// and entry tables, the quantized activation rows and the output rows.
struct GemmArgs {
    Q8Mat W[2], U[2];               // matrix set 0 (plain or routed) and 1 (the shared expert)
    uint32_t rows;                  // rows of one matrix group (tile.row0 .. + rows)
    const uint32_t *n_tiles;        // device count of valid column tiles
    const GemmTile *tiles;
    const uint32_t *act_row, *out_row;
    const uint8_t *aq;              // activation chunks, aqs bytes per activation row
    const float *ad;                // activation scales, ads floats per activation row
    uint32_t aqs, ads;
    float *y;                       // output rows of ys floats
    uint32_t ys;
};

hipError_t init_batch_kernel_attributes();
void launch_b_embed(hipStream_t st, const float *emb, uint32_t d, const uint32_t *tokens, uint32_t n, float *x);
void launch_b_quant_rows(hipStream_t st, const float *x, uint32_t xs, uint32_t n_elems, uint32_t rows, uint8_t *q,
                         uint32_t qs, float *dq, uint32_t ds);
bool launch_b_gemm(hipStream_t st, int mode, uint32_t tt, const GemmArgs &a, uint32_t max_tiles);
bool launch_b_qk_rope_append(hipStream_t st, uint32_t hd, float *qkv, uint32_t qkv_stride, const float *qn,
                             const float *kn, float eps, const float *cs, const float *sn, const uint32_t *pos,
                             const PagedKV &kv, uint32_t n);
// Scores and softmax + P.V of n sequences over their pages; o [n][n_heads * hd].  false if
// the head size or the context bound is not supported.
bool launch_b_attention(hipStream_t st, uint32_t hd, const float *qkv, uint32_t qkv_stride, const uint32_t *pos,
                        const PagedKV &kv, uint32_t n, uint32_t max_ctx, float *scores, float *pmax, float *o,
                        uint32_t *err);
// LDS product-ring slots of the softmax + P.V kernel for contexts up to max_ctx (>= 2 needed).
uint32_t bpv_slots(uint32_t max_ctx, uint32_t hd);
// Group the (sequence, rank) picks of n sequences by expert into entry tables and column
// tiles of at most tt entries (the shared expert last, slot top_k of every sequence).
void launch_b_group(hipStream_t st, const uint32_t *topk_idx, uint32_t n, uint32_t top_k, uint32_t E,
                    uint32_t n_slots, uint32_t tt, uint32_t *act_row, uint32_t *out_row, GemmTile *tiles,
                    uint32_t *n_tiles);
void launch_b_page_copy(hipStream_t st, float *flat, float *pool, const uint32_t *bt, uint32_t npg,
                        uint32_t page_floats, int dir);
void launch_b_combine(hipStream_t st, const float *y, const float *topk_w, uint32_t top_k, uint32_t n_slots,
                      uint32_t d, uint32_t n, float *x);
void launch_b_argmax(hipStream_t st, const float *logits, uint32_t V, uint32_t valid, uint32_t *pos, uint32_t *tokens,
                     uint32_t *out_ids, const uint32_t *step, uint32_t n, uint32_t feedback);
void launch_b_step_advance(hipStream_t st, uint32_t *step);
void note_launch_error(hipError_t e, const std::string &what);

}  // namespace hg
