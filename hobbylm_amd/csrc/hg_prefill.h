// hg_prefill.h -- the prompt path of a single-sequence cache (Model::prefill, model.rs:340-439)
// as batched MFMA GEMMs and paged attention over all prompt rows at once (hg_prefill.hip).
#pragma once
#include "hg_model.h"

namespace hg {

// Device work buffers of the batched prompt path, owned by a cache and grown on demand.
struct PrefillWork {
    uint32_t rows = 0, win = 0, tn = 0;   // chunk rows, attention window and prompt rows they are sized for
    DevBuf xall, pos, apos, order, err, kpg, vpg, ident, ptiles, pn, scores, pmax;
    DevBuf xq, xd, qkv, o, oq, od, topk_idx, topk_w, ord, rec_idx, rec_w;
    DevBuf ent_act, ent_out, etiles, n_etiles, a, aq, ad, y;
};

// Whether the batched prompt path runs prompts of a cache of `cap` positions with this model
// (Q8 matrices, head size, expert count, attention window and GEMM tile limits).
bool prefill_batched_ok(const hg_model *m, uint32_t cap);

// Prompt rows inputs[0 .. tn) (host, d floats each) at positions base .. base + tn - 1 of a
// single-sequence cache (kc, vc: [L] layers as the decode step lays them out, cap positions):
// every layer's K/V rows appended, the last row's final residual into x_last and its routing
// records into rec_idx / rec_w ([L][top_k]).  Each row's arithmetic is Model::prefill's.
int prefill_batched(const hg_model *m, PrefillWork &w, hipStream_t st, const float *inputs, uint32_t base,
                    uint32_t tn, float *kc, float *vc, uint32_t cap, float *x_last, uint32_t *rec_idx, float *rec_w);

// Model::run_block (model.rs:471-585) on the same kernels: the b block rows (host rows of d
// floats, or with block == nullptr the embeddings of the device ids `ids`) at positions
// base .. base + b - 1 attend to the cache's rows 0 .. base - 1 and to every block row.  logits
// (device, [b][V]) and the block's K/V rows per layer (device, [L][b][kvd]) when not null;
// append: the block's K/V rows also go into the cache at base (finalizing a block).
// HG_ERR_UNSUPPORTED if the block does not fit one chunk.
int run_block_batched(const hg_model *m, PrefillWork &w, hipStream_t st, const float *block, const uint32_t *ids,
                      uint32_t base, uint32_t b, float *kc, float *vc, uint32_t cap, bool append, float *logits,
                      float *bk, float *bv);

}  // namespace hg
