// hg_batch.hip -- the batch context behind hg_batch_* (include/hobby_gpu.h): many sequences,
// each with its own paged KV cache, decoded one token per sequence per step.
//
// Per step and layer: attn_norm of every sequence's residual (one workgroup per sequence), the
// QKV rows as one MFMA GEMM over all sequences, QK-norm + RoPE + append into each sequence's
// page, paged attention (scores, then softmax + P.V per (sequence, head)), the O rows with the
// residual, then for MoE layers ffn_norm + router per sequence, the grouping of the picks by
// expert, the gate/up and down rows of every expert as grouped GEMMs over the sequences that
// picked it, and the rank-order combine with the residual; dense layers run gate/up and down
// over all sequences.  The step ends with output_norm, the lm_head GEMM and a greedy argmax per
// sequence that advances its position (and, for device-side greedy loops, its token).  Every
// sequence's arithmetic is that of its own single-sequence step (model.rs:152-327), so logits,
// routing and cache rows equal separate hg_forward calls bit for bit.  The step reads tokens
// and positions from device memory and is captured once per batch size as a HIP graph.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hobby_gpu.h"
#include "hg_batch.h"
#include "hg_common.h"
#include "hg_kernels.h"
#include "hg_model.h"

using namespace hg;

static_assert(HG_PAGE == PAGE, "page size of the header and the kernels");

struct hg_batch {
    const hg_model *m = nullptr;
    hipStream_t st = nullptr;
    uint32_t max_seqs = 0, max_ctx = 0, n_pages = 0, bt_stride = 0, out_cap = 0, max_tiles_e = 0;
    std::vector<uint32_t> lens, bt_host;   // per sequence: length, block table [max_seqs][bt_stride]
    std::vector<uint32_t> n_bt;            // pages assigned per sequence
    DevBuf kpool, vpool;                   // [L][n_pages][n_kv][PAGE][hd]
    DevBuf bt, pos, tokens, step, err, seq_order;
    DevBuf x, xq, xd, qkv, scores, pmax, o, oq, od;
    DevBuf topk_idx, topk_w, order, rec_idx, rec_w;
    DevBuf ent_act, ent_out, etiles, n_etiles;
    DevBuf ident, ptiles, pn;              // identity entries; plain tiles of 8 entries per batch size
    DevBuf a, aq, ad, y, logits, out_ids, flat;
    std::map<uint32_t, hipGraphExec_t> graphs;   // captured step per batch size
    uint32_t cur_n = 0;                          // batch size of the step being enqueued
};

namespace {

constexpr uint32_t PT_MAX = 64;   // plain tiles per batch size (>= max_seqs / 8)

// Plain tile tables: for batch size n, the div_up(n, 8) tiles of 8 entries at
// ptiles[n * PT_MAX], their count at pn[n].
const GemmTile *plain_tiles(const hg_batch *b, uint32_t n) { return b->ptiles.as<GemmTile>() + (size_t)n * PT_MAX; }
const uint32_t *plain_count(const hg_batch *b, uint32_t n) { return b->pn.as<uint32_t>() + n; }

PagedKV layer_kv(const hg_batch *b, uint32_t l) {
    const hg_config &c = b->m->c;
    const size_t per = (size_t)b->n_pages * c.n_kv_heads * PAGE * c.head_dim;
    PagedKV kv;
    kv.k = b->kpool.as<float>() + per * l;
    kv.v = b->vpool.as<float>() + per * l;
    kv.bt = b->bt.as<uint32_t>();
    kv.bt_stride = b->bt_stride;
    kv.n_heads = c.n_heads;
    kv.n_kv = c.n_kv_heads;
    return kv;
}

// A GEMM over all n sequences of the step (identity entries) in column tiles of 8.
GemmArgs plain_gemm(const hg_batch *b, const Q8Mat &W, const uint8_t *aq, const float *ad, float *y, uint32_t ys) {
    GemmArgs g{};
    g.W[0] = W;
    g.rows = W.N;
    g.n_tiles = plain_count(b, b->cur_n);
    g.tiles = plain_tiles(b, b->cur_n);
    g.act_row = g.out_row = b->ident.as<uint32_t>();
    g.aq = aq;
    g.ad = ad;
    g.aqs = W.nc * CHUNK_BYTES;
    g.ads = W.nc * 4;
    g.y = y;
    g.ys = ys;
    return g;
}

void enqueue_step(hg_batch *b) {
    const hg_model *m = b->m;
    const hg_config &c = m->c;
    hipStream_t st = b->st;
    const uint32_t n = b->cur_n, d = c.d_model, hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    const uint32_t qw = qd + 2 * kvd, f = c.expert_ffn, ns = m->n_slots;
    const uint32_t ncd = div_up(d / QK, 4), ncq = div_up(qd / QK, 4), pt = div_up(n, 8);   // plain tiles
    float *x = b->x.as<float>();
    uint8_t *xq = b->xq.as<uint8_t>();
    float *xd = b->xd.as<float>();
    uint32_t *pos = b->pos.as<uint32_t>();
    launch_b_embed(st, m->token_embd.as<float>(), d, b->tokens.as<uint32_t>(), n, x);
    launch_b_order(st, pos, n, b->seq_order.as<uint32_t>());
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const Layer &L = *m->layers[l];
        const PagedKV kv = layer_kv(b, l);
        // attention (model.rs:164-171, 186-234)
        launch_rmsnorm_quant_rows(st, true, n, x, L.attn_norm.as<float>(), c.rms_eps, d, nullptr, xq, xd);
        if (!launch_b_gemm(st, GM_STORE, plain_gemm(b, L.qkv.m, xq, xd, b->qkv.as<float>(), qw), pt))
            note_launch_error(hipErrorInvalidConfiguration, "QKV GEMM");
        if (!launch_b_qk_rope_append(st, hd, b->qkv.as<float>(), qw, L.q_norm.as<float>(), L.k_norm.as<float>(),
                                     c.rms_eps, m->rope_cos.as<float>(), m->rope_sin.as<float>(), pos, kv, n))
            note_launch_error(hipErrorInvalidConfiguration, "QK-norm / RoPE");
        if (!launch_b_attention(st, hd, b->qkv.as<float>(), qw, pos, b->seq_order.as<uint32_t>(), kv, n, b->max_ctx,
                                b->scores.as<float>(), b->pmax.as<float>(), b->o.as<float>(), b->err.as<uint32_t>()))
            note_launch_error(hipErrorInvalidConfiguration, "paged attention");
        launch_b_quant_rows(st, b->o.as<float>(), qd, qd, n, b->oq.as<uint8_t>(), ncq * CHUNK_BYTES, b->od.as<float>(),
                            ncq * 4);
        if (!launch_b_gemm(st, GM_RESID, plain_gemm(b, L.o.m, b->oq.as<uint8_t>(), b->od.as<float>(), x, d), pt))
            note_launch_error(hipErrorInvalidConfiguration, "O GEMM");
        if (L.moe) {
            // ffn_norm + router + top-k per sequence (model.rs:259-293), h quantized into xq
            const RowStrides rs{d, ncd * CHUNK_BYTES, ncd * 4, c.top_k, c.n_layers * c.top_k};
            launch_ffn_router_rows(st, true, n, rs, x, L.ffn_norm.as<float>(), c.rms_eps, d, L.router.as<float>(),
                                   L.router_p.as<float>(), L.bias.as<float>(), c.n_experts, c.top_k, c.gating_sigmoid,
                                   c.expert_weights_norm, c.expert_weights_scale, xq, xd, b->topk_idx.as<uint32_t>(),
                                   b->topk_w.as<float>(), b->order.as<uint32_t>(),
                                   b->rec_idx.as<uint32_t>() + (size_t)l * c.top_k,
                                   b->rec_w.as<float>() + (size_t)l * c.top_k);
            launch_b_group(st, b->topk_idx.as<uint32_t>(), n, c.top_k, c.n_experts, ns, 8, b->ent_act.as<uint32_t>(),
                           b->ent_out.as<uint32_t>(), b->etiles.as<GemmTile>(), b->n_etiles.as<uint32_t>());
            GemmArgs gu{};
            gu.W[0] = L.gate_e.m;
            gu.U[0] = L.up_e.m;
            if (c.n_shared) {
                gu.W[1] = L.gate_sh.m;
                gu.U[1] = L.up_sh.m;
            }
            gu.rows = f;
            gu.n_tiles = b->n_etiles.as<uint32_t>();
            gu.tiles = b->etiles.as<GemmTile>();
            gu.act_row = b->ent_act.as<uint32_t>();
            gu.out_row = b->ent_out.as<uint32_t>();
            gu.aq = xq;
            gu.ad = xd;
            gu.aqs = ncd * CHUNK_BYTES;
            gu.ads = ncd * 4;
            gu.y = b->a.as<float>();
            gu.ys = f;
            if (!launch_b_gemm(st, GM_GATEUP, gu, b->max_tiles_e))
                note_launch_error(hipErrorInvalidConfiguration, "expert gate/up GEMM");
            const uint32_t ncf = div_up(f / QK, 4);
            launch_b_quant_rows(st, b->a.as<float>(), f, f, n * ns, b->aq.as<uint8_t>(), ncf * CHUNK_BYTES,
                                b->ad.as<float>(), ncf * 4);
            GemmArgs dn{};
            dn.W[0] = L.down_e.m;
            if (c.n_shared) dn.W[1] = L.down_sh.m;
            dn.rows = d;
            dn.n_tiles = gu.n_tiles;
            dn.tiles = gu.tiles;
            dn.act_row = dn.out_row = b->ent_out.as<uint32_t>();
            dn.aq = b->aq.as<uint8_t>();
            dn.ad = b->ad.as<float>();
            dn.aqs = ncf * CHUNK_BYTES;
            dn.ads = ncf * 4;
            dn.y = b->y.as<float>();
            dn.ys = d;
            if (!launch_b_gemm(st, GM_STORE, dn, b->max_tiles_e))
                note_launch_error(hipErrorInvalidConfiguration, "expert down GEMM");
            launch_b_combine(st, b->y.as<float>(), b->topk_w.as<float>(), nullptr, c.top_k, ns, d, n, x);
        } else {
            // dense FFN (model.rs:243-255)
            const uint32_t df = c.dense_ffn, ncf = div_up(df / QK, 4);
            launch_rmsnorm_quant_rows(st, true, n, x, L.ffn_norm.as<float>(), c.rms_eps, d, nullptr, xq, xd);
            GemmArgs gu = plain_gemm(b, L.gate.m, xq, xd, b->a.as<float>(), df);
            gu.U[0] = L.up.m;
            if (!launch_b_gemm(st, GM_GATEUP, gu, pt))
                note_launch_error(hipErrorInvalidConfiguration, "dense gate/up GEMM");
            launch_b_quant_rows(st, b->a.as<float>(), df, df, n, b->aq.as<uint8_t>(), ncf * CHUNK_BYTES,
                                b->ad.as<float>(), ncf * 4);
            if (!launch_b_gemm(st, GM_RESID, plain_gemm(b, L.down.m, b->aq.as<uint8_t>(), b->ad.as<float>(), x, d), pt))
                note_launch_error(hipErrorInvalidConfiguration, "dense down GEMM");
        }
    }
    // output_norm + lm_head + greedy pick (model.rs:180-183, lib.rs:132-142)
    launch_rmsnorm_quant_rows(st, true, n, x, m->output_norm.as<float>(), c.rms_eps, d, nullptr, xq, xd);
    if (!launch_b_gemm(st, GM_STORE, plain_gemm(b, m->output.m, xq, xd, b->logits.as<float>(), c.vocab_size), pt))
        note_launch_error(hipErrorInvalidConfiguration, "lm_head GEMM");
    launch_b_argmax(st, b->logits.as<float>(), c.vocab_size, std::min(c.vocab_size, 50257u), pos,
                    b->tokens.as<uint32_t>(), b->out_ids.as<uint32_t>(), b->step.as<uint32_t>(), n, 1);
    launch_b_step_advance(st, b->step.as<uint32_t>());
}

// Replay the step for batch size n (capturing it on first use), or with HG_GRAPH=0 launch it
// eagerly (for tracers that do not follow graph launches).
int run_step(hg_batch *b, uint32_t n) {
    b->cur_n = n;
    std::string msg;
    (void)take_launch_error(msg);
    static const bool eager = [] {
        const char *ge = getenv("HG_GRAPH");
        return ge && ge[0] == '0';
    }();
    if (eager) {
        enqueue_step(b);
        if (take_launch_error(msg) != hipSuccess) return fail(HG_ERR_DEVICE, "batched step: " + msg);
        return HG_OK;
    }
    hipGraphExec_t &exec = b->graphs[n];
    if (!exec) {
        hipGraph_t graph = nullptr;
        HIP_TRY(hipStreamBeginCapture(b->st, hipStreamCaptureModeThreadLocal));
        enqueue_step(b);
        const hipError_t le = take_launch_error(msg);
        hipError_t e = hipStreamEndCapture(b->st, &graph);
        if (le != hipSuccess) {
            if (graph) (void)hipGraphDestroy(graph);
            return fail(HG_ERR_DEVICE, "batched step: " + msg);
        }
        if (e != hipSuccess) return fail(HG_ERR_DEVICE, std::string("graph capture: ") + hipGetErrorString(e));
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (e != hipSuccess) {
            exec = nullptr;
            return fail(HG_ERR_DEVICE, std::string("graph instantiate: ") + hipGetErrorString(e));
        }
    }
    HIP_TRY(hipGraphLaunch(exec, b->st));
    return HG_OK;
}

int check_batch(const hg_model *m, const hg_batch *b, uint32_t n, uint32_t steps) {
    if (!m || !b || b->m != m) return fail(HG_ERR_ARG, "batch does not belong to this model");
    if (n == 0 || n > b->max_seqs)
        return fail(HG_ERR_ARG, "batch of " + std::to_string(n) + " sequences (at most " + std::to_string(b->max_seqs) + ")");
    for (uint32_t s = 0; s < n; ++s) {
        const uint64_t end = (uint64_t)b->lens[s] + steps;
        if (end > b->max_ctx)
            return fail(HG_ERR_ARG, "sequence " + std::to_string(s) + ": position " + std::to_string(end - 1) +
                                        " beyond the batch context (" + std::to_string(b->max_ctx) + ")");
        if (end > (uint64_t)b->n_bt[s] * PAGE)
            return fail(HG_ERR_ARG, "sequence " + std::to_string(s) + " has pages for " +
                                        std::to_string(b->n_bt[s] * PAGE) + " positions, needs " + std::to_string(end));
        if (end > b->m->c.context_length)
            return fail(HG_ERR_ARG, "sequence " + std::to_string(s) + ": position beyond context_length");
    }
    return HG_OK;
}

int upload_state(hg_batch *b, const uint32_t *tokens, uint32_t n) {
    HIP_TRY(hipMemcpyAsync(b->tokens.p, tokens, (size_t)n * 4, hipMemcpyHostToDevice, b->st));
    HIP_TRY(hipMemcpyAsync(b->pos.p, b->lens.data(), (size_t)n * 4, hipMemcpyHostToDevice, b->st));
    HIP_TRY(hipMemsetAsync(b->step.p, 0, 4, b->st));
    return HG_OK;
}

// The device error word of the step's bounded waits (then cleared).
int check_err(hg_batch *b) {
    uint32_t e = 0;
    HIP_TRY(hipMemcpyAsync(&e, b->err.p, 4, hipMemcpyDeviceToHost, b->st));
    HIP_TRY(hipStreamSynchronize(b->st));
    if (e) {
        HIP_TRY(hipMemsetAsync(b->err.p, 0, 4, b->st));
        HIP_TRY(hipStreamSynchronize(b->st));
        return fail(HG_ERR_DEVICE, "a batched attention hand-off wait exceeded its bound");
    }
    return HG_OK;
}

}  // namespace

extern "C" {

int hg_batch_new(const hg_model *m, uint32_t max_seqs, uint32_t max_ctx, uint32_t n_pages, hg_batch **out) {
    return guard([&]() -> int {
        if (!m || !out) return fail(HG_ERR_ARG, "NULL argument");
        *out = nullptr;
        const hg_config &c = m->c;
        if (max_seqs == 0 || max_seqs > 8 * PT_MAX) return fail(HG_ERR_ARG, "max_seqs out of range (1..512)");
        if (max_ctx == 0 || max_ctx > c.context_length) max_ctx = c.context_length;
        if (m->f32) return fail(HG_ERR_UNSUPPORTED, "batched decode needs Q8 matrices (load with quant = true)");
        if (c.head_dim != 64 && c.head_dim != 128) return fail(HG_ERR_UNSUPPORTED, "batched decode: head_dim 64 or 128");
        if (c.n_experts + 1 > MAX_GROUPS) return fail(HG_ERR_UNSUPPORTED, "batched decode: too many experts");
        if (!batch_ctx_ok(max_ctx))
            return fail(HG_ERR_UNSUPPORTED, "batched decode: max_ctx " + std::to_string(max_ctx) + " too long");
        if (n_pages == 0) return fail(HG_ERR_ARG, "the page pool is empty");
        int rc = check_device();
        if (rc) return rc;
        if (init_batch_kernel_attributes() != hipSuccess) return fail(HG_ERR_DEVICE, "hipFuncSetAttribute failed");
        auto b = std::make_unique<hg_batch>();
        b->m = m;
        b->max_seqs = max_seqs;
        b->max_ctx = max_ctx;
        b->n_pages = n_pages;
        b->bt_stride = div_up(max_ctx, PAGE);
        b->out_cap = 4096;
        b->lens.assign(max_seqs, 0);
        b->n_bt.assign(max_seqs, 0);
        b->bt_host.assign((size_t)max_seqs * b->bt_stride, 0);
        HIP_TRY(hipStreamCreateWithFlags(&b->st, hipStreamNonBlocking));
        const uint32_t S = max_seqs, d = c.d_model, hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
        const uint32_t ns = std::max(m->n_slots, 1u), f = c.expert_ffn, df = c.dense_ffn;
        const uint32_t ncd = div_up(d / QK, 4), ncq = div_up(qd / QK, 4);
        const uint32_t ncf = std::max(div_up(f / QK, 4), div_up(df / QK, 4));
        const uint32_t ng = c.n_experts + 1;
        b->max_tiles_e = ng + div_up(S * ns, 8);
        const size_t pool = (size_t)c.n_layers * n_pages * c.n_kv_heads * PAGE * hd * 4;
        const uint32_t nch = div_up(max_ctx, ACH);
        if ((rc = b->kpool.alloc(pool)) || (rc = b->vpool.alloc(pool)) ||
            (rc = b->bt.alloc((size_t)S * b->bt_stride * 4)) || (rc = b->pos.alloc((size_t)S * 4)) ||
            (rc = b->tokens.alloc((size_t)S * 4)) || (rc = b->step.alloc(4)) || (rc = b->err.alloc(4)) ||
            (rc = b->seq_order.alloc((size_t)S * 4)) ||
            (rc = b->x.alloc((size_t)S * d * 4)) || (rc = b->xq.alloc((size_t)S * ncd * CHUNK_BYTES)) ||
            (rc = b->xd.alloc((size_t)S * ncd * 16)) || (rc = b->qkv.alloc((size_t)S * (qd + 2 * kvd) * 4)) ||
            (rc = b->scores.alloc((size_t)S * c.n_heads * b_sc_stride(max_ctx) * 4)) ||
            (rc = b->pmax.alloc((size_t)S * c.n_heads * nch * 4)) || (rc = b->o.alloc((size_t)S * qd * 4)) ||
            (rc = b->oq.alloc((size_t)S * ncq * CHUNK_BYTES)) || (rc = b->od.alloc((size_t)S * ncq * 16)) ||
            (rc = b->topk_idx.alloc((size_t)S * std::max(c.top_k, 1u) * 4)) ||
            (rc = b->topk_w.alloc((size_t)S * std::max(c.top_k, 1u) * 4)) ||
            (rc = b->order.alloc((size_t)S * std::max(c.top_k, 1u) * 4)) ||
            (rc = b->rec_idx.alloc((size_t)S * c.n_layers * std::max(c.top_k, 1u) * 4)) ||
            (rc = b->rec_w.alloc((size_t)S * c.n_layers * std::max(c.top_k, 1u) * 4)) ||
            (rc = b->ent_act.alloc((size_t)S * ns * 4)) || (rc = b->ent_out.alloc((size_t)S * ns * 4)) ||
            (rc = b->etiles.alloc((size_t)b->max_tiles_e * sizeof(GemmTile))) || (rc = b->n_etiles.alloc(4)) ||
            (rc = b->a.alloc((size_t)S * std::max(ns * f, df) * 4)) ||
            (rc = b->aq.alloc((size_t)S * ns * ncf * CHUNK_BYTES)) || (rc = b->ad.alloc((size_t)S * ns * ncf * 16)) ||
            (rc = b->y.alloc((size_t)S * ns * d * 4)) || (rc = b->logits.alloc((size_t)S * c.vocab_size * 4)) ||
            (rc = b->out_ids.alloc((size_t)b->out_cap * S * 4)))
            return rc;
        HIP_TRY(hipMemset(b->kpool.p, 0, b->kpool.n));
        HIP_TRY(hipMemset(b->vpool.p, 0, b->vpool.n));
        HIP_TRY(hipMemset(b->bt.p, 0, b->bt.n));
        HIP_TRY(hipMemset(b->err.p, 0, 4));
        HIP_TRY(hipMemset(b->rec_idx.p, 0xff, b->rec_idx.n));
        HIP_TRY(hipMemset(b->rec_w.p, 0, b->rec_w.n));
        // identity entries and the plain column tiles of every batch size
        std::vector<uint32_t> ident(S);
        for (uint32_t i = 0; i < S; ++i) ident[i] = i;
        std::vector<GemmTile> pt((size_t)(S + 1) * PT_MAX);
        std::vector<uint32_t> pn(S + 1);
        for (uint32_t n = 1; n <= S; ++n) {
            pn[n] = div_up(n, 8);
            for (uint32_t q = 0; q < pn[n]; ++q) pt[(size_t)n * PT_MAX + q] = GemmTile{0, q * 8, std::min(8u, n - q * 8), 0};
        }
        if ((rc = b->ident.upload(ident.data(), ident.size() * 4)) ||
            (rc = b->ptiles.upload(pt.data(), pt.size() * sizeof(GemmTile))) ||
            (rc = b->pn.upload(pn.data(), pn.size() * 4)))
            return rc;
        HIP_TRY(hipDeviceSynchronize());
        *out = b.release();
        return HG_OK;
    });
}

void hg_batch_free(hg_batch *b) {
    if (!b) return;
    if (b->st) (void)hipStreamSynchronize(b->st);
    for (auto &g : b->graphs)
        if (g.second) (void)hipGraphExecDestroy(g.second);
    if (b->st) (void)hipStreamDestroy(b->st);
    delete b;
}

int hg_batch_set_pages(hg_batch *b, uint32_t seq, const uint32_t *pages, uint32_t n) {
    return guard([&]() -> int {
        if (!b || (n && !pages)) return fail(HG_ERR_ARG, "NULL argument");
        if (seq >= b->max_seqs) return fail(HG_ERR_ARG, "sequence index out of range");
        if (n > b->bt_stride) return fail(HG_ERR_ARG, "more pages than max_ctx needs");
        for (uint32_t i = 0; i < n; ++i)
            if (pages[i] >= b->n_pages) return fail(HG_ERR_ARG, "page id " + std::to_string(pages[i]) + " out of range");
        uint32_t *row = b->bt_host.data() + (size_t)seq * b->bt_stride;
        std::fill(row, row + b->bt_stride, 0u);
        std::copy(pages, pages + n, row);
        b->n_bt[seq] = n;
        b->lens[seq] = 0;
        HIP_TRY(hipStreamSynchronize(b->st));
        HIP_TRY(hipMemcpy(b->bt.as<uint32_t>() + (size_t)seq * b->bt_stride, row, (size_t)b->bt_stride * 4,
                          hipMemcpyHostToDevice));
        return HG_OK;
    });
}

uint32_t hg_batch_len(const hg_batch *b, uint32_t seq) { return b && seq < b->max_seqs ? b->lens[seq] : 0; }

// Rows [0, len) of every layer of sequence seq to / from the reference layout
// ([n_layers][len][kv_dim]) through the sequence's pages.
static int batch_rows(hg_batch *b, uint32_t seq, uint32_t len, float *k, float *v, bool write, int layer) {
    const hg_config &c = b->m->c;
    const uint32_t hd = c.head_dim, nkv = c.n_kv_heads, kvd = nkv * hd, npg = div_up(len, PAGE);
    const uint32_t pf = nkv * PAGE * hd;   // floats per page of one layer
    const size_t per = (size_t)b->n_pages * pf;
    if (!npg) return HG_OK;
    int rc;
    if (b->flat.n < (size_t)npg * pf * 4 && (rc = b->flat.alloc((size_t)npg * pf * 4))) return rc;
    std::vector<float> host((size_t)npg * pf, 0.0f);
    const uint32_t *bt = b->bt.as<uint32_t>() + (size_t)seq * b->bt_stride;
    const uint32_t l0 = layer < 0 ? 0 : (uint32_t)layer, l1 = layer < 0 ? c.n_layers : (uint32_t)layer + 1;
    for (uint32_t l = l0; l < l1; ++l)
        for (int which = 0; which < 2; ++which) {
            float *src = (which ? v : k) + (layer < 0 ? (size_t)l * len * kvd : 0);
            float *pool = (which ? b->vpool : b->kpool).as<float>() + per * l;
            if (write) {
                for (uint32_t t = 0; t < len; ++t)
                    for (uint32_t g = 0; g < nkv; ++g) {
                        const float *row = src + (size_t)t * kvd + g * hd;
                        float *tile = &host[(size_t)(t / PAGE) * pf + kv_tile(0, g, nkv, hd)];
                        for (uint32_t e = 0; e < hd; ++e) tile[which ? v_el(e, t % PAGE, hd) : k_el(e, t % PAGE)] = row[e];
                    }
                HIP_TRY(hipMemcpyAsync(b->flat.p, host.data(), host.size() * 4, hipMemcpyHostToDevice, b->st));
                launch_b_page_copy(b->st, b->flat.as<float>(), pool, bt, npg, pf, 0);
                HIP_TRY(hipStreamSynchronize(b->st));
            } else {
                launch_b_page_copy(b->st, b->flat.as<float>(), pool, bt, npg, pf, 1);
                HIP_TRY(hipMemcpyAsync(host.data(), b->flat.p, host.size() * 4, hipMemcpyDeviceToHost, b->st));
                HIP_TRY(hipStreamSynchronize(b->st));
                for (uint32_t t = 0; t < len; ++t)
                    for (uint32_t g = 0; g < nkv; ++g) {
                        float *row = src + (size_t)t * kvd + g * hd;
                        const float *tile = &host[(size_t)(t / PAGE) * pf + kv_tile(0, g, nkv, hd)];
                        for (uint32_t e = 0; e < hd; ++e) row[e] = tile[which ? v_el(e, t % PAGE, hd) : k_el(e, t % PAGE)];
                    }
            }
        }
    std::string msg;
    if (take_launch_error(msg) != hipSuccess) return fail(HG_ERR_DEVICE, msg);
    return HG_OK;
}

int hg_batch_load(hg_batch *b, uint32_t seq, uint32_t len, const float *k, const float *v) {
    return guard([&]() -> int {
        if (!b || (len && (!k || !v))) return fail(HG_ERR_ARG, "NULL argument");
        if (seq >= b->max_seqs) return fail(HG_ERR_ARG, "sequence index out of range");
        if (len > b->max_ctx || len > b->n_bt[seq] * PAGE)
            return fail(HG_ERR_ARG, "len " + std::to_string(len) + " beyond the sequence's pages");
        HIP_TRY(hipStreamSynchronize(b->st));
        int rc = batch_rows(b, seq, len, const_cast<float *>(k), const_cast<float *>(v), true, -1);
        if (rc) return rc;
        b->lens[seq] = len;
        return HG_OK;
    });
}

int hg_batch_fill(hg_batch *b, uint32_t seq, uint32_t len, uint64_t seed) {
    return guard([&]() -> int {
        if (!b) return fail(HG_ERR_ARG, "NULL argument");
        if (seq >= b->max_seqs) return fail(HG_ERR_ARG, "sequence index out of range");
        if (len > b->max_ctx || len > b->n_bt[seq] * PAGE)
            return fail(HG_ERR_ARG, "len " + std::to_string(len) + " beyond the sequence's pages");
        const hg_config &c = b->m->c;
        const size_t layer_floats = (size_t)b->n_pages * c.n_kv_heads * PAGE * c.head_dim;
        std::string msg;
        (void)take_launch_error(msg);
        launch_b_page_fill(b->st, b->kpool.as<float>(), b->vpool.as<float>(), b->bt.as<uint32_t>() + (size_t)seq * b->bt_stride,
                           len, c.n_layers, c.n_kv_heads, c.head_dim, layer_floats, seed);
        if (take_launch_error(msg) != hipSuccess) return fail(HG_ERR_DEVICE, msg);
        HIP_TRY(hipStreamSynchronize(b->st));
        b->lens[seq] = len;
        return HG_OK;
    });
}

int hg_batch_read(hg_batch *b, uint32_t seq, uint32_t layer, float *k, float *v) {
    return guard([&]() -> int {
        if (!b || !k || !v) return fail(HG_ERR_ARG, "NULL argument");
        if (seq >= b->max_seqs || layer >= b->m->c.n_layers) return fail(HG_ERR_ARG, "index out of range");
        HIP_TRY(hipStreamSynchronize(b->st));
        return batch_rows(b, seq, b->lens[seq], k, v, false, (int)layer);
    });
}

int hg_batch_forward(const hg_model *m, hg_batch *b, const uint32_t *tokens, uint32_t n, float *logits,
                     uint32_t *next) {
    return guard([&]() -> int {
        if (!tokens) return fail(HG_ERR_ARG, "tokens is NULL");
        int rc = check_batch(m, b, n, 1);
        if (rc) return rc;
        for (uint32_t s = 0; s < n; ++s)
            if (tokens[s] >= m->c.vocab_size) return fail(HG_ERR_ARG, "token " + std::to_string(tokens[s]) + " out of range");
        if ((rc = upload_state(b, tokens, n)) || (rc = run_step(b, n))) return rc;
        if (logits)
            HIP_TRY(hipMemcpyAsync(logits, b->logits.p, (size_t)n * m->c.vocab_size * 4, hipMemcpyDeviceToHost, b->st));
        std::vector<uint32_t> ids(n);
        HIP_TRY(hipMemcpyAsync(ids.data(), b->out_ids.p, (size_t)n * 4, hipMemcpyDeviceToHost, b->st));
        if ((rc = check_err(b))) return rc;
        if (next) memcpy(next, ids.data(), (size_t)n * 4);
        for (uint32_t s = 0; s < n; ++s) b->lens[s] += 1;
        return HG_OK;
    });
}

int hg_batch_decode_greedy(const hg_model *m, hg_batch *b, const uint32_t *first, uint32_t n, uint32_t n_steps,
                           uint32_t *out_ids) {
    return guard([&]() -> int {
        if (!first || (n_steps && !out_ids)) return fail(HG_ERR_ARG, "NULL argument");
        int rc = check_batch(m, b, n, n_steps);
        if (rc) return rc;
        for (uint32_t s = 0; s < n; ++s)
            if (first[s] >= m->c.vocab_size) return fail(HG_ERR_ARG, "token out of range");
        if (n_steps > b->out_cap) return fail(HG_ERR_ARG, "at most " + std::to_string(b->out_cap) + " steps per call");
        if (n_steps == 0) return HG_OK;
        if ((rc = upload_state(b, first, n))) return rc;
        for (uint32_t i = 0; i < n_steps; ++i)
            if ((rc = run_step(b, n))) return rc;
        HIP_TRY(hipMemcpyAsync(out_ids, b->out_ids.p, (size_t)n_steps * n * 4, hipMemcpyDeviceToHost, b->st));
        if ((rc = check_err(b))) return rc;
        for (uint32_t s = 0; s < n; ++s) b->lens[s] += n_steps;
        return HG_OK;
    });
}

int hg_batch_routing(hg_batch *b, uint32_t seq, uint32_t *idx, float *w) {
    return guard([&]() -> int {
        if (!b) return fail(HG_ERR_ARG, "NULL argument");
        if (seq >= b->max_seqs) return fail(HG_ERR_ARG, "sequence index out of range");
        const size_t per = (size_t)b->m->c.n_layers * b->m->c.top_k;
        HIP_TRY(hipStreamSynchronize(b->st));
        if (idx) HIP_TRY(hipMemcpy(idx, b->rec_idx.as<uint32_t>() + seq * per, per * 4, hipMemcpyDeviceToHost));
        if (w) HIP_TRY(hipMemcpy(w, b->rec_w.as<float>() + seq * per, per * 4, hipMemcpyDeviceToHost));
        return HG_OK;
    });
}

}  // extern "C"
