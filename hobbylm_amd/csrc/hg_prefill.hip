// hg_prefill.hip -- Model::prefill (model.rs:340-439) for a single-sequence cache, all prompt
// rows at once: the Q8 products as int8-MFMA GEMMs in Q8Tensor::matmul's order (quant.rs:164-184),
// QK-norm + RoPE per row, the rows appended to the cache, causal attention as the paged
// attention of the batched decode step (row r is a sequence of base + r + 1 positions over
// pages that hold the cache layer), and the expert-grouped FFN (model.rs:653-750) with its
// expert-id-order combine.  Long prompts run in chunks of rows (each chunk sees the rows of the
// earlier ones through the cache), which changes no row's arithmetic.
#include <stdlib.h>

#include <algorithm>
#include <string>

#include "../../include/hobby_gpu.h"
#include "hg_batch.h"
#include "hg_common.h"
#include "hg_kernels.h"
#include "hg_prefill.h"

namespace hg {
namespace {

constexpr size_t SCORE_BUDGET = 512ull << 20;   // bytes of attention scores per chunk
constexpr uint32_t CHUNK_MAX = 2048;            // prompt rows per chunk

uint32_t window_for(uint32_t n) { return div_up(n, 256) * 256; }

// Prompt rows per chunk: as many as the score budget allows for this window (a multiple of
// 64, at most CHUNK_MAX, or HG_PREFILL_CHUNK if that is smaller), or the whole prompt if it is
// shorter.
uint32_t chunk_rows(const hg_config &c, uint32_t win, uint32_t tn) {
    const size_t per = (size_t)c.n_heads * b_sc_stride(win) * 4;
    uint32_t r = (uint32_t)std::min<size_t>(CHUNK_MAX, SCORE_BUDGET / per);
    r = std::max(r / 64 * 64, 64u);
    if (const char *e = getenv("HG_PREFILL_CHUNK")) {
        const long v = strtol(e, nullptr, 10);
        if (v > 0 && (uint32_t)v < r) r = (uint32_t)v;
    }
    return std::min(r, tn);
}

// Per chunk of n rows at positions base0 ..: pos[i] = base0 + i, order[i] = n - 1 - i (longest
// context first) and the plain column tiles of 16, 32 and 64 entries (tables at k tmax, counts
// at counts[k]).
__global__ void k_p_setup(uint32_t n, uint32_t base0, uint32_t tmax, uint32_t *pos, uint32_t *apos, uint32_t bidir,
                          uint32_t *order, GemmTile *tiles, uint32_t *counts) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        pos[i] = base0 + i;
        apos[i] = bidir ? base0 + n - 1 : base0 + i;   // the last position each row attends to
        order[i] = n - 1 - i;
#pragma unroll
        for (uint32_t k = 0; k < 3; ++k) {
            const uint32_t tt = 16u << k;
            if (i * tt < n) {
                GemmTile t;
                t.grp = 0;
                t.entry0 = i * tt;
                t.count = min(tt, n - i * tt);
                t.mat = 0;
                tiles[k * tmax + i] = t;
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < 3) counts[threadIdx.x] = div_up(n, 16u << threadIdx.x);
}

// Rows r = blockIdx.y of the chunk's k and v (normed and rotated) into bk / bv [R][kvd].
__global__ void k_p_rows_out(const float *__restrict__ qkv, uint32_t qw, uint32_t qd, uint32_t kvd, float *bk,
                             float *bv) {
    const uint32_t r = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= kvd) return;
    const float *row = qkv + (size_t)r * qw + qd;
    if (bk) bk[(size_t)r * kvd + i] = row[i];
    if (bv) bv[(size_t)r * kvd + i] = row[kvd + i];
}

__global__ void k_p_iota(uint32_t n, uint32_t *out) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = i;
}

uint32_t tile_slot(uint32_t tt) { return tt == 16 ? 0u : tt == 32 ? 1u : 2u; }

struct Shapes {
    uint32_t d, hd, qd, kvd, qw, f, df, ns, ncd, ncq, ncf, ncdf;
    uint32_t tt_d, tt_q, tt_e, tt_df;   // column tiles: K = d, K = qd, the experts, K = dense_ffn
};

Shapes shapes_of(const hg_model *m) {
    const hg_config &c = m->c;
    Shapes s{};
    s.d = c.d_model;
    s.hd = c.head_dim;
    s.qd = c.n_heads * s.hd;
    s.kvd = c.n_kv_heads * s.hd;
    s.qw = s.qd + 2 * s.kvd;
    s.f = c.expert_ffn;
    s.df = c.dense_ffn;
    s.ns = std::max(m->n_slots, 1u);
    s.ncd = div_up(s.d / QK, 4);
    s.ncq = div_up(s.qd / QK, 4);
    s.ncf = div_up(s.f / QK, 4);
    s.ncdf = div_up(s.df / QK, 4);
    s.tt_d = pgemm_tile(s.ncd);
    s.tt_q = pgemm_tile(s.ncq);
    s.tt_e = std::min(s.tt_d, pgemm_tile(s.ncf));
    s.tt_df = pgemm_tile(s.ncdf);
    return s;
}

bool has_moe(const hg_model *m) {
    for (const auto &L : m->layers)
        if (L->moe) return true;
    return false;
}
bool has_dense(const hg_model *m) {
    for (const auto &L : m->layers)
        if (!L->moe) return true;
    return false;
}

int grow(PrefillWork &w, const hg_model *m, const Shapes &s, uint32_t R, uint32_t win, uint32_t tn) {
    const hg_config &c = m->c;
    int rc;
    if (tn > w.tn) {
        if ((rc = w.xall.alloc((size_t)tn * s.d * 4))) return rc;
        w.tn = tn;
    }
    if (win > w.win || R > w.rows) {   // the window-sized buffers
        const uint32_t wn = std::max(win, w.win), rn = std::max(R, w.rows);
        const size_t pagef = (size_t)div_up(wn, PAGE) * c.n_kv_heads * PAGE * s.hd;
        if ((rc = w.kpg.alloc(pagef * 4)) || (rc = w.vpg.alloc(pagef * 4)) ||
            (rc = w.scores.alloc((size_t)rn * c.n_heads * b_sc_stride(wn) * 4)) ||
            (rc = w.pmax.alloc((size_t)rn * c.n_heads * div_up(wn, ACH) * 4)) ||
            (rc = w.ident.alloc((size_t)std::max(rn, div_up(wn, PAGE)) * 4)))
            return rc;
        HIP_TRY(hipMemset(w.kpg.p, 0, w.kpg.n));
        HIP_TRY(hipMemset(w.vpg.p, 0, w.vpg.n));
        const uint32_t ni = (uint32_t)(w.ident.n / 4);
        hipLaunchKernelGGL(k_p_iota, dim3(div_up(ni, 256)), dim3(256), 0, nullptr, ni, w.ident.as<uint32_t>());
        HIP_TRY(hipGetLastError());
        HIP_TRY(hipDeviceSynchronize());
        w.win = wn;
    }
    if (R > w.rows) {
        const uint32_t tk = std::max(c.top_k, 1u), ns = s.ns, tmax = div_up(R, 16);
        const uint32_t max_te = c.n_experts + 1 + div_up(R * ns, std::max(s.tt_e, 16u));
        const size_t arows = std::max((size_t)ns * s.f, (size_t)s.df), qrows = std::max((size_t)ns * s.ncf, (size_t)s.ncdf);
        if ((rc = w.pos.alloc((size_t)R * 4)) || (rc = w.apos.alloc((size_t)R * 4)) || (rc = w.order.alloc((size_t)R * 4)) ||
            (rc = w.ptiles.alloc((size_t)3 * tmax * sizeof(GemmTile))) || (rc = w.pn.alloc(3 * 4)) ||
            (rc = w.xq.alloc((size_t)R * s.ncd * CHUNK_BYTES)) || (rc = w.xd.alloc((size_t)R * s.ncd * 16)) ||
            (rc = w.qkv.alloc((size_t)R * s.qw * 4)) || (rc = w.o.alloc((size_t)R * s.qd * 4)) ||
            (rc = w.oq.alloc((size_t)R * s.ncq * CHUNK_BYTES)) || (rc = w.od.alloc((size_t)R * s.ncq * 16)) ||
            (rc = w.topk_idx.alloc((size_t)R * tk * 4)) || (rc = w.topk_w.alloc((size_t)R * tk * 4)) ||
            (rc = w.ord.alloc((size_t)R * tk * 4)) || (rc = w.rec_idx.alloc((size_t)R * c.n_layers * tk * 4)) ||
            (rc = w.rec_w.alloc((size_t)R * c.n_layers * tk * 4)) || (rc = w.ent_act.alloc((size_t)R * ns * 4)) ||
            (rc = w.ent_out.alloc((size_t)R * ns * 4)) || (rc = w.etiles.alloc((size_t)max_te * sizeof(GemmTile))) ||
            (rc = w.n_etiles.alloc(4)) || (rc = w.a.alloc((size_t)R * arows * 4)) ||
            (rc = w.aq.alloc((size_t)R * qrows * CHUNK_BYTES)) || (rc = w.ad.alloc((size_t)R * qrows * 16)) ||
            (rc = w.y.alloc((size_t)R * ns * s.d * 4)))
            return rc;
        if (!w.err.p) {
            if ((rc = w.err.alloc(4))) return rc;
            HIP_TRY(hipMemset(w.err.p, 0, 4));
        }
        w.rows = R;
    }
    return HG_OK;
}

// A GEMM over the chunk's rows in order (identity entries), column tiles of tt entries.
GemmArgs plain(const PrefillWork &w, const Q8Mat &W, const uint8_t *aq, const float *ad, float *y, uint32_t ys,
               uint32_t tt) {
    GemmArgs g{};
    g.W[0] = W;
    g.rows = W.N;
    g.n_tiles = w.pn.as<uint32_t>() + tile_slot(tt);
    g.tiles = w.ptiles.as<GemmTile>() + (size_t)tile_slot(tt) * div_up(w.rows, 16);
    g.act_row = g.out_row = w.ident.as<uint32_t>();
    g.aq = aq;
    g.ad = ad;
    g.aqs = W.nc * CHUNK_BYTES;
    g.ads = W.nc * 4;
    g.y = y;
    g.ys = ys;
    return g;
}

void gemm(hipStream_t st, int mode, const GemmArgs &g, uint32_t max_tiles, uint32_t tt, const char *what) {
    if (!launch_p_gemm(st, mode, g, max_tiles, tt)) note_launch_error(hipErrorInvalidConfiguration, what);
}

// What a chunk does besides the layers: prompt rows (causal, appended to the cache) or a
// run_block block (every row attends to all block rows; appended only when finalizing; its K/V
// rows per layer to bk / bv [L][R][kvd]; logits of every row).
struct ChunkMode {
    bool bidir = false, store = true;
    float *bk = nullptr, *bv = nullptr, *logits = nullptr;
};

// The layers over one chunk of R rows at positions base0 .. base0 + R - 1 (x: their residuals).
void enqueue_chunk(const hg_model *m, PrefillWork &w, const Shapes &s, hipStream_t st, float *x, uint32_t base0,
                   uint32_t R, float *kc, float *vc, uint32_t cap, const ChunkMode &cm = ChunkMode()) {
    const hg_config &c = m->c;
    const uint32_t win = window_for(base0 + R), d = s.d, hd = s.hd, nkv = c.n_kv_heads;
    const uint32_t tmax = div_up(w.rows, 16);
    hipLaunchKernelGGL(k_p_setup, dim3(div_up(R, 256)), dim3(256), 0, st, R, base0, tmax, w.pos.as<uint32_t>(),
                       w.apos.as<uint32_t>(), cm.bidir ? 1u : 0u, w.order.as<uint32_t>(), w.ptiles.as<GemmTile>(),
                       w.pn.as<uint32_t>());
    const hipError_t le = hipGetLastError();
    if (le != hipSuccess) note_launch_error(le, "k_p_setup");
    PagedKV kvp;
    kvp.k = w.kpg.as<float>();
    kvp.v = w.vpg.as<float>();
    kvp.bt = w.ident.as<uint32_t>();
    kvp.bt_stride = 0;   // every row reads the one identity block table
    kvp.n_heads = c.n_heads;
    kvp.n_kv = nkv;
    uint8_t *xq = w.xq.as<uint8_t>();
    float *xd = w.xd.as<float>();
    const uint32_t *pos = w.pos.as<uint32_t>();
    const uint32_t nt_d = div_up(R, s.tt_d), nt_q = div_up(R, s.tt_q);
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const Layer &L = *m->layers[l];
        float *Lk = kc + (size_t)l * nkv * cap * hd;
        float *Lv = vc + (size_t)l * v_layer_floats(cap, nkv, hd);
        // attention (model.rs:354-398)
        launch_p_kv_pages(st, Lk, Lv, cap, nkv, hd, base0, kvp.k, kvp.v);
        launch_rmsnorm_quant_rows(st, true, R, x, L.attn_norm.as<float>(), c.rms_eps, d, nullptr, xq, xd);
        gemm(st, GM_STORE, plain(w, L.qkv.m, xq, xd, w.qkv.as<float>(), s.qw, s.tt_d), nt_d, s.tt_d, "QKV GEMM");
        if (!launch_b_qk_rope_append(st, hd, w.qkv.as<float>(), s.qw, L.q_norm.as<float>(), L.k_norm.as<float>(),
                                     c.rms_eps, m->rope_cos.as<float>(), m->rope_sin.as<float>(), pos, kvp, R))
            note_launch_error(hipErrorInvalidConfiguration, "QK-norm / RoPE");
        if (cm.store) launch_p_kv_store(st, w.qkv.as<float>(), s.qw, s.qd, s.kvd, hd, nkv, base0, R, cap, Lk, Lv);
        if (cm.bk || cm.bv) {
            hipLaunchKernelGGL(k_p_rows_out, dim3(div_up(s.kvd, 256), R), dim3(256), 0, st, w.qkv.as<float>(), s.qw,
                               s.qd, s.kvd, cm.bk ? cm.bk + (size_t)l * R * s.kvd : nullptr,
                               cm.bv ? cm.bv + (size_t)l * R * s.kvd : nullptr);
            const hipError_t e2 = hipGetLastError();
            if (e2 != hipSuccess) note_launch_error(e2, "k_p_rows_out");
        }
        if (!launch_p_attention(st, hd, w.qkv.as<float>(), s.qw, w.apos.as<uint32_t>(), w.order.as<uint32_t>(), kvp, R, win,
                                w.scores.as<float>(), w.pmax.as<float>(), w.o.as<float>(), w.err.as<uint32_t>()))
            note_launch_error(hipErrorInvalidConfiguration, "causal attention");
        launch_b_quant_rows(st, w.o.as<float>(), s.qd, s.qd, R, w.oq.as<uint8_t>(), s.ncq * CHUNK_BYTES,
                            w.od.as<float>(), s.ncq * 4);
        gemm(st, GM_RESID, plain(w, L.o.m, w.oq.as<uint8_t>(), w.od.as<float>(), x, d, s.tt_q), nt_q, s.tt_q,
             "O GEMM");
        if (L.moe) {
            // ffn_norm + router + top-k per row (model.rs:674-700), h quantized into xq
            const RowStrides rs{d, s.ncd * CHUNK_BYTES, s.ncd * 4, c.top_k, c.n_layers * c.top_k};
            launch_ffn_router_rows(st, true, R, rs, x, L.ffn_norm.as<float>(), c.rms_eps, d, L.router.as<float>(),
                                   L.router_p.as<float>(), L.bias.as<float>(), c.n_experts, c.top_k,
                                   c.gating_sigmoid, c.expert_weights_norm, c.expert_weights_scale, xq, xd,
                                   w.topk_idx.as<uint32_t>(), w.topk_w.as<float>(), w.ord.as<uint32_t>(),
                                   w.rec_idx.as<uint32_t>() + (size_t)l * c.top_k,
                                   w.rec_w.as<float>() + (size_t)l * c.top_k);
            // rows grouped by expert (model.rs:701-705), each expert's rows one GEMM (:707-724)
            launch_b_group(st, w.topk_idx.as<uint32_t>(), R, c.top_k, c.n_experts, s.ns, s.tt_e,
                           w.ent_act.as<uint32_t>(), w.ent_out.as<uint32_t>(), w.etiles.as<GemmTile>(),
                           w.n_etiles.as<uint32_t>());
            const uint32_t max_te = c.n_experts + 1 + div_up(R * s.ns, s.tt_e);
            GemmArgs gu{};
            gu.W[0] = L.gate_e.m;
            gu.U[0] = L.up_e.m;
            if (c.n_shared) {
                gu.W[1] = L.gate_sh.m;
                gu.U[1] = L.up_sh.m;
            }
            gu.rows = s.f;
            gu.n_tiles = w.n_etiles.as<uint32_t>();
            gu.tiles = w.etiles.as<GemmTile>();
            gu.act_row = w.ent_act.as<uint32_t>();
            gu.out_row = w.ent_out.as<uint32_t>();
            gu.aq = xq;
            gu.ad = xd;
            gu.aqs = s.ncd * CHUNK_BYTES;
            gu.ads = s.ncd * 4;
            gu.y = w.a.as<float>();
            gu.ys = s.f;
            gemm(st, GM_GATEUP, gu, max_te, s.tt_e, "expert gate/up GEMM");
            launch_b_quant_rows(st, w.a.as<float>(), s.f, s.f, R * s.ns, w.aq.as<uint8_t>(), s.ncf * CHUNK_BYTES,
                                w.ad.as<float>(), s.ncf * 4);
            GemmArgs dn{};
            dn.W[0] = L.down_e.m;
            if (c.n_shared) dn.W[1] = L.down_sh.m;
            dn.rows = d;
            dn.n_tiles = gu.n_tiles;
            dn.tiles = gu.tiles;
            dn.act_row = dn.out_row = w.ent_out.as<uint32_t>();
            dn.aq = w.aq.as<uint8_t>();
            dn.ad = w.ad.as<float>();
            dn.aqs = s.ncf * CHUNK_BYTES;
            dn.ads = s.ncf * 4;
            dn.y = w.y.as<float>();
            dn.ys = d;
            gemm(st, GM_STORE, dn, max_te, s.tt_e, "expert down GEMM");
            // out = 0 + (experts in id order) + shared, then x += out (model.rs:718-735, 366-368)
            launch_b_combine(st, w.y.as<float>(), w.topk_w.as<float>(), w.ord.as<uint32_t>(), c.top_k, s.ns, d, R, x);
        } else {
            // dense FFN (model.rs:656-668)
            launch_rmsnorm_quant_rows(st, true, R, x, L.ffn_norm.as<float>(), c.rms_eps, d, nullptr, xq, xd);
            GemmArgs gu = plain(w, L.gate.m, xq, xd, w.a.as<float>(), s.df, s.tt_d);
            gu.U[0] = L.up.m;
            gemm(st, GM_GATEUP, gu, nt_d, s.tt_d, "dense gate/up GEMM");
            launch_b_quant_rows(st, w.a.as<float>(), s.df, s.df, R, w.aq.as<uint8_t>(), s.ncdf * CHUNK_BYTES,
                                w.ad.as<float>(), s.ncdf * 4);
            gemm(st, GM_RESID, plain(w, L.down.m, w.aq.as<uint8_t>(), w.ad.as<float>(), x, d, s.tt_df),
                 div_up(R, s.tt_df), s.tt_df, "dense down GEMM");
        }
    }
    if (cm.logits) {   // every row's logits: output_norm rows, output.matmul (model.rs:504-507)
        launch_rmsnorm_quant_rows(st, true, R, x, m->output_norm.as<float>(), c.rms_eps, d, nullptr, xq, xd);
        gemm(st, GM_STORE, plain(w, m->output.m, xq, xd, cm.logits, c.vocab_size, s.tt_d), nt_d, s.tt_d,
             "lm_head GEMM");
    }
}

}  // namespace

bool prefill_batched_ok(const hg_model *m, uint32_t cap) {
    const hg_config &c = m->c;
    if (m->f32) return false;   // the prompt GEMMs are Q8 (the F32 mode runs one step per row)
    if (c.head_dim != 32 && c.head_dim != 64 && c.head_dim != 128) return false;
    const uint32_t rep = c.n_heads / c.n_kv_heads;
    if (c.head_dim == 32 && rep != 1 && rep != 2 && rep != 4 && rep != 8) return false;
    if (c.n_experts + 1 > MAX_GROUPS) return false;
    if (!batch_ctx_ok(window_for(cap))) return false;
    const Shapes s = shapes_of(m);
    if (!s.tt_d || !s.tt_q) return false;
    if (has_moe(m) && !s.tt_e) return false;
    if (has_dense(m) && !s.tt_df) return false;
    return true;
}

int run_block_batched(const hg_model *m, PrefillWork &w, hipStream_t st, const float *block, const uint32_t *ids,
                      uint32_t base, uint32_t b, float *kc, float *vc, uint32_t cap, bool append, float *logits,
                      float *bk, float *bv) {
    const hg_config &c = m->c;
    const Shapes s = shapes_of(m);
    const uint32_t win = window_for(base + b);
    const uint32_t R = chunk_rows(c, win, b);
    if (R < b) return fail(HG_ERR_UNSUPPORTED, "run_block: a block of " + std::to_string(b) + " rows at this context");
    HIP_TRY(hipStreamSynchronize(st));
    int rc = grow(w, m, s, b, win, b);
    if (rc) return rc;
    std::string msg;
    (void)take_launch_error(msg);
    if (block) HIP_TRY(hipMemcpyAsync(w.xall.p, block, (size_t)b * s.d * 4, hipMemcpyHostToDevice, st));
    else launch_b_embed(st, m->token_embd.as<float>(), s.d, ids, b, w.xall.as<float>());
    ChunkMode cm;
    cm.bidir = true;
    cm.store = append;
    cm.bk = bk;
    cm.bv = bv;
    cm.logits = logits;
    enqueue_chunk(m, w, s, st, w.xall.as<float>(), base, b, kc, vc, cap, cm);
    if (take_launch_error(msg) != hipSuccess) {
        (void)hipStreamSynchronize(st);
        return fail(HG_ERR_DEVICE, "run_block: " + msg);
    }
    uint32_t e = 0;
    HIP_TRY(hipMemcpyAsync(&e, w.err.p, 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    if (e) {
        HIP_TRY(hipMemset(w.err.p, 0, 4));
        return fail(HG_ERR_DEVICE, "run_block: an attention hand-off wait exceeded its bound");
    }
    return HG_OK;
}

int prefill_batched(const hg_model *m, PrefillWork &w, hipStream_t st, const float *inputs, uint32_t base,
                    uint32_t tn, float *kc, float *vc, uint32_t cap, float *x_last, uint32_t *rec_idx, float *rec_w) {
    const hg_config &c = m->c;
    const Shapes s = shapes_of(m);
    const uint32_t winmax = window_for(base + tn);
    const uint32_t R = chunk_rows(c, winmax, tn);
    HIP_TRY(hipStreamSynchronize(st));   // (the work buffers may be reallocated)
    int rc = grow(w, m, s, R, winmax, tn);
    if (rc) return rc;
    std::string msg;
    (void)take_launch_error(msg);
    float *xall = w.xall.as<float>();
    HIP_TRY(hipMemcpyAsync(xall, inputs, (size_t)tn * s.d * 4, hipMemcpyHostToDevice, st));
    uint32_t last = 0;
    for (uint32_t off = 0; off < tn; off += R) {
        const uint32_t n = std::min(R, tn - off);
        enqueue_chunk(m, w, s, st, xall + (size_t)off * s.d, base + off, n, kc, vc, cap);
        last = off + n - 1;
    }
    HIP_TRY(hipMemcpyAsync(x_last, xall + (size_t)last * s.d, (size_t)s.d * 4, hipMemcpyDeviceToDevice, st));
    if (c.top_k && has_moe(m)) {   // the last row's routing records
        const size_t per = (size_t)c.n_layers * c.top_k, at = (size_t)(last % R) * per;
        HIP_TRY(hipMemcpyAsync(rec_idx, w.rec_idx.as<uint32_t>() + at, per * 4, hipMemcpyDeviceToDevice, st));
        HIP_TRY(hipMemcpyAsync(rec_w, w.rec_w.as<float>() + at, per * 4, hipMemcpyDeviceToDevice, st));
    }
    if (take_launch_error(msg) != hipSuccess) {
        (void)hipStreamSynchronize(st);
        return fail(HG_ERR_DEVICE, "prefill: " + msg);
    }
    uint32_t e = 0;
    HIP_TRY(hipMemcpyAsync(&e, w.err.p, 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    if (e) {
        HIP_TRY(hipMemset(w.err.p, 0, 4));
        return fail(HG_ERR_DEVICE, "prefill: an attention hand-off wait exceeded its bound");
    }
    return HG_OK;
}

}  // namespace hg
