// hg_batch.h -- device layouts and launchers of the batched decode step (hg_batch_kernels.hip).
#pragma once
#include <string>

#include "hg_common.h"

namespace hg {

constexpr uint32_t PAGE = 16;                   // positions per KV page
constexpr uint32_t ACH = 256;                   // positions per attention score chunk
constexpr uint32_t MAX_GROUPS = 256;            // experts + the shared expert
constexpr size_t BSM_LDS_MAX = 150 * 1024;      // softmax: e_t of the longest context

// The KV pages of one layer: per page and kv head a tile of PAGE * hd floats for K and one for
// V, and the block tables [sequence][bt_stride] (position t of sequence s is in page
// bt[s][t / PAGE]).  Tiles are laid out for 16-byte loads whose lanes cover contiguous memory:
// K [element quad][slot][4 elements] (lane = position: a row in hd/4 loads, a page's 16 lanes
// reading 256 contiguous bytes), V [slot quad][element][4 slots] (lane = element: 16
// positions in 4 loads, 64 lanes reading 1 KiB contiguous).
struct PagedKV {
    float *k, *v;
    const uint32_t *bt;
    uint32_t bt_stride, n_heads, n_kv;
};

__host__ __device__ inline size_t kv_tile(uint32_t page, uint32_t g, uint32_t n_kv, uint32_t hd) {
    return ((size_t)page * n_kv + g) * PAGE * hd;
}
__host__ __device__ inline uint32_t k_el(uint32_t e, uint32_t slot) { return ((e / 4) * PAGE + slot) * 4 + e % 4; }
__host__ __device__ inline uint32_t v_el(uint32_t e, uint32_t slot, uint32_t hd) {
    return ((slot / 4) * hd + e) * 4 + slot % 4;
}

// One column tile of a batched GEMM: entries entry0 .. entry0 + count - 1 (count <= 8) of the entry tables
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
// A GEMM over column tiles of at most 8 entries (max_tiles: the grid's bound on *n_tiles).
bool launch_b_gemm(hipStream_t st, int mode, const GemmArgs &a, uint32_t max_tiles);
bool launch_b_qk_rope_append(hipStream_t st, uint32_t hd, float *qkv, uint32_t qkv_stride, const float *qn,
                             const float *kn, float eps, const float *cs, const float *sn, const uint32_t *pos,
                             const PagedKV &kv, uint32_t n);
// Scores, softmax and P.V of n sequences over their pages; o [n][n_heads * hd]; *err |= 1 if
// a bounded wait of the P.V hand-off ran out.  false if the head size or the context bound is
// not supported.
bool launch_b_attention(hipStream_t st, uint32_t hd, const float *qkv, uint32_t qkv_stride, const uint32_t *pos,
                        const uint32_t *order, const PagedKV &kv, uint32_t n, uint32_t max_ctx, float *scores,
                        float *pmax, float *o, uint32_t *err);
// order[r] = the sequence of rank r by length, longest first.
void launch_b_order(hipStream_t st, const uint32_t *pos, uint32_t n, uint32_t *order);
// Floats per row of attention scores (one row per (sequence, query head)): max_ctx rounded up
// to 64, so that rows are 16-byte aligned and 16-byte loads near the end stay in the row.
inline uint32_t b_sc_stride(uint32_t max_ctx) { return (max_ctx + 63) / 64 * 64; }
// Whether the attention kernels hold contexts of max_ctx positions (LDS).
bool batch_ctx_ok(uint32_t max_ctx);
// Group the (sequence, rank) picks of n sequences by expert into entry tables and column
// tiles of at most tt entries (the shared expert last, slot top_k of every sequence).
void launch_b_group(hipStream_t st, const uint32_t *topk_idx, uint32_t n, uint32_t top_k, uint32_t E,
                    uint32_t n_slots, uint32_t tt, uint32_t *act_row, uint32_t *out_row, GemmTile *tiles,
                    uint32_t *n_tiles);
void launch_b_page_copy(hipStream_t st, float *flat, float *pool, const uint32_t *bt, uint32_t npg,
                        uint32_t page_floats, int dir);
void launch_b_page_fill(hipStream_t st, float *kpool, float *vpool, const uint32_t *bt, uint32_t len, uint32_t n_layers,
                        uint32_t n_kv, uint32_t hd, size_t layer_floats, uint64_t seed);
// order == nullptr: rank order (decode); else the ranks in ascending expert id per sequence (prompt).
void launch_b_combine(hipStream_t st, const float *y, const float *topk_w, const uint32_t *order, uint32_t top_k,
                      uint32_t n_slots, uint32_t d, uint32_t n, float *x);
void launch_b_argmax(hipStream_t st, const float *logits, uint32_t V, uint32_t valid, uint32_t *pos, uint32_t *tokens,
                     uint32_t *out_ids, const uint32_t *step, uint32_t n, uint32_t feedback);
void launch_b_step_advance(hipStream_t st, uint32_t *step);
void note_launch_error(hipError_t e, const std::string &what);

// ---- prompt path (Model::prefill, model.rs:340-439, 653-750) on the same kernels
constexpr size_t PGEMM_LDS_MAX = 96 * 1024;   // prompt GEMM: staged activations of one column tile
// Entries per column tile of a prompt-order GEMM over K = 128 nc (64, 32 or 16; 0: too long).
uint32_t pgemm_tile(uint32_t nc);
// A GEMM in Q8Tensor::matmul's order over column tiles of at most tt entries (16, 32 or 64).
bool launch_p_gemm(hipStream_t st, int mode, const GemmArgs &a, uint32_t max_tiles, uint32_t tt);
void launch_p_kv_store(hipStream_t st, const float *qkv, uint32_t qw, uint32_t qd, uint32_t kvd, uint32_t hd,
                       uint32_t n_kv, uint32_t base, uint32_t rows, uint32_t cap, float *kc, float *vc);
void launch_p_kv_pages(hipStream_t st, const float *kc, const float *vc, uint32_t cap, uint32_t n_kv, uint32_t hd,
                       uint32_t npos, float *kpg, float *vpg);
void launch_p_rev(hipStream_t st, uint32_t n, uint32_t *order);
// Causal attention of n prompt rows (row r: positions 0 .. pos[r]) over pages shared by the
// rows: the decode step's scores and softmax, then a P.V kernel that shares each V load
// among the rows and heads of a wave.  Arguments as launch_b_attention.
bool launch_p_attention(hipStream_t st, uint32_t hd, const float *qkv, uint32_t qkv_stride, const uint32_t *pos,
                        const uint32_t *order, const PagedKV &kv, uint32_t n, uint32_t max_ctx, float *scores,
                        float *pmax, float *o, uint32_t *err);

}  // namespace hg
