// hg_engine.hip -- model load, device residency, KV cache and the decode step behind the
// C ABI of include/hobby_gpu.h.
//
// One decode step is a fixed sequence of kernels per layer (norm+quant, QKV, attention,
// attn_output+residual, norm+router or norm, gate/up, down+residual) plus the lm_head tail.
// The sequence reads its token and position from a device StepParams block, so it is
// captured once per cache as a HIP graph and replayed per token; in the greedy loop the
// argmax kernel advances StepParams itself and steps chain on the device.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <memory>
#include <stdexcept>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hobby_gpu.h"
#include "hg_batch.h"
#include "hg_common.h"
#include "hg_gguf.h"
#include "hg_kernels.h"
#include "hg_model.h"
#include "hg_prefill.h"
#include "hg_sample.h"

using namespace hg;

namespace hg {
thread_local std::string g_err;
}  // namespace hg

namespace {

// ---- the allocation-free matvec's scratch --------------------------------------------------
// The quantized activation of hg_q8_tensor_matvec_noalloc (chunks + scales, as k_quant_vec
// writes them) lives in this fixed device array, one per GPU for the life of the process.  In
// host code `scratch` only names the symbol: its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and kept in g_scratch_ptr.
constexpr uint32_t NOALLOC_MAX_IN = HG_NOALLOC_MAX_IN;
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)(NOALLOC_MAX_IN / 128) * (CHUNK_BYTES + 16);
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
static_assert(NOALLOC_SCRATCH_BYTES == HG_NOALLOC_SCRATCH_BYTES, "header and library disagree");

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES] = {};

// The device address of `scratch` on the current device (looked up on first use there).
int scratch_ptr(void **out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) return fail(HG_ERR_DEVICE, "device ordinal out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(HG_ERR_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return HG_OK;
}


}  // namespace

int hg::check_device() {
    static std::once_flag once;
    static int status = HG_OK;
    static std::string msg;
    std::call_once(once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
            status = HG_ERR_DEVICE;
            msg = "no HIP device available";
            return;
        }
        int dev = 0;
        (void)hipGetDevice(&dev);
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
            status = HG_ERR_DEVICE;
            msg = "hipGetDeviceProperties failed";
            return;
        }
        if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
            status = HG_ERR_DEVICE;
            msg = std::string("this build targets gfx950; device is ") + prop.gcnArchName;
            return;
        }
        if (init_kernel_attributes() != hipSuccess) {
            status = HG_ERR_DEVICE;
            msg = "hipFuncSetAttribute failed";
            return;
        }
        void *sp = nullptr;   // set-up of the allocation-free entry point's scratch on this device
        if (scratch_ptr(&sp) != HG_OK) {
            status = HG_ERR_DEVICE;
            msg = g_err;
        }
    });
    if (status) g_err = msg;
    return status;
}

namespace {

// The model as parsed and packed on the host, before any device call: every format error of
// the file surfaces here, in the reference's load order (model.rs:79-131).
// A matrix as the load keeps it: packed Q8 (quant = true) or f32 rows in F32Mat's layout.
struct HostMat {
    PackedQ8 q8;
    std::vector<float> f32;
    uint32_t N = 0, K = 0;
};
struct HostLayer {
    bool moe = false;
    std::vector<float> attn_norm, q_norm, k_norm, ffn_norm, router, router_p, bias;
    HostMat qkv, o, gate, up, down, gate_e, up_e, down_e, gate_sh, up_sh, down_sh;
};
struct HostModel {
    hg_config c{};
    bool quant = true;
    std::vector<HostLayer> layers;
    std::vector<float> token_embd, output_norm, rope_cos, rope_sin;
    HostMat output;
    uint64_t ref_bytes = 0;
};

}  // namespace

struct hg_kv {
    const hg_model *m = nullptr;
    hipStream_t st = nullptr;
    uint32_t cap = 0, len = 0, flags = 0;
    bool exact = false;
    uint32_t win = 0;       // attention window of the step being enqueued (see window_of)
    uint32_t lm_threads = 256, n_part = 0;
    DevBuf kc, vc;          // [L][n_kv][cap][hd]; V: each layer also [n_kv][hd][vt_stride(cap)]
    DevBuf x, qkv, o, part, scores, a, logits, pv, pi, qa, da, topk_idx, topk_w, order, rec_idx, rec_w, params,
        out_ids, inputs;
    DevBuf h, y;            // F32 mode: the normed activation, the expert slots' down outputs
    uint32_t inputs_rows = 0;
    StepParams *h_params = nullptr;
    uint32_t *h_ids = nullptr;
    float *h_logits = nullptr;
    // captured steps, one per attention window (decode, prompt-row body), and the prompt tail
    std::map<uint32_t, hipGraphExec_t> g_decode, g_body;
    hipGraphExec_t g_tail = nullptr;
    bool use_graph = true;
    bool no_fuse = false;          // HG_QKV_SCORES=0: scores in their own launch (the unfused kernels)
    LaunchTimer *timer = nullptr;  // hg_profile_step: per-dispatch timing
    std::unique_ptr<PrefillWork> pw;   // the batched prompt path's buffers (on first use)
    std::unique_ptr<SampleWork> sw;    // the device sampler's buffers (on first use)
    DevBuf picks;                      // sampled ids of hg_generate
    ~hg_kv();
};

namespace {

// Attention window of a step over n = pos + 1 positions of a cache of cap positions: n rounded
// up to 256 positions (1024 past 3072), at most cap.  The attention launches are sized for the
// window, not the capacity, so a step costs what its live context needs; each window has its
// own captured graph.
uint32_t window_of(uint32_t n, uint32_t cap) {
    const uint32_t w = n <= 3072 ? div_up(n, 256) * 256 : div_up(n, 1024) * 1024;
    return std::min(w, cap);
}

int load_norm(const Gguf &g, const std::string &name, size_t want, std::vector<float> &dst) {
    int rc = g.f32(name, dst, g_err);
    if (rc) return rc;
    if (dst.size() != want)
        return fail(HG_ERR_FORMAT, "tensor `" + name + "` has " + std::to_string(dst.size()) + " elements, expected " +
                                       std::to_string(want));
    return HG_OK;
}

// Gguf::load + Mat::build(.., quant) (model.rs:87-89, 121, quant.rs:213-222): requantize and
// pack (quant = true), or keep the (dequantized) f32 rows (quant = false).
int load_q8(const Gguf &g, const std::string &name, uint32_t N, uint32_t K, HostMat &dst, HostModel &hm) {
    const TensorInfo *t;
    const uint8_t *raw;
    size_t nbytes;
    int rc = g.raw(name, t, raw, nbytes, g_err);
    if (rc) return rc;
    if (t->n_elems() != (uint64_t)N * K)
        return fail(HG_ERR_FORMAT, "tensor `" + name + "` has " + std::to_string(t->n_elems()) + " elements, expected " +
                                       std::to_string((uint64_t)N * K));
    dst.N = N;
    dst.K = K;
    if (!hm.quant) {
        std::vector<float> w;
        if ((rc = g.load(name, w, g_err))) return rc;
        permute_f32_rows(w.data(), N, K, dst.f32);
        hm.ref_bytes += (uint64_t)N * K * 4;
        return HG_OK;
    }
    if (K % QK) return fail(HG_ERR_UNSUPPORTED, "Q8_0 needs in_ divisible by 32 (got " + std::to_string(K) + ")");
    if (t->type == GGML_Q8_0) pack_q8_from_q8_0(raw, N, K, dst.q8);
    else {
        std::vector<float> w;
        rc = g.load(name, w, g_err);
        if (rc) return rc;
        pack_q8_from_f32(w.data(), N, K, dst.q8);
    }
    hm.ref_bytes += dst.q8.ref_bytes();
    return HG_OK;
}

int validate(const hg_config &c) {
    auto bad = [](const std::string &s) { return fail(HG_ERR_UNSUPPORTED, s); };
    if (!c.d_model || !c.n_layers || !c.n_heads || !c.n_kv_heads || c.n_heads % c.n_kv_heads)
        return bad("unsupported head configuration");
    if (c.head_dim != 32 && c.head_dim != 64 && c.head_dim != 128)
        return bad("head_dim " + std::to_string(c.head_dim) + " not in {32, 64, 128}");
    if (c.n_heads / c.n_kv_heads > 8) return bad("more than 8 query heads per kv head");
    if (c.d_model % QK || c.expert_ffn % QK || c.dense_ffn % QK)
        return bad("Q8_0 and the F32 kernels need in_ divisible by 32");
    if (c.n_experts > 256 || c.top_k > 64 || c.top_k > c.n_experts) return bad("expert count out of range");
    if (c.n_dense < c.n_layers && (slots_of(c) == 0 || slots_of(c) > 16)) return bad("more than 16 expert slots");
    if (!c.context_length) return bad("context_length is 0");
    if (c.context_length > (1u << 20)) return bad("context_length above 2^20");
    return HG_OK;
}

// Gguf::open + Config::from_gguf + Model::load on the host (no device call).
int parse_model(const char *path, bool quant, HostModel &hm) {
    hm.quant = quant;
    Gguf g;
    int rc = g.open(path, g_err);
    if (rc) return rc;
    rc = config_from_gguf(g, hm.c, g_err);
    if (rc) return rc;
    rc = validate(hm.c);
    if (rc) return rc;
    const hg_config &c = hm.c;
    const uint32_t d = c.d_model, f = c.expert_ffn, hd = c.head_dim;
    const uint32_t qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    hm.layers.resize(c.n_layers);
    for (uint32_t i = 0; i < c.n_layers; ++i) {
        HostLayer &L = hm.layers[i];
        const std::string p = "blk." + std::to_string(i) + ".";
        L.moe = i >= c.n_dense;
        if (L.moe) {
            if ((rc = g.load(p + "ffn_gate_inp.weight", L.router, g_err))) return rc;
            if (L.router.size() != (size_t)c.n_experts * d)
                return fail(HG_ERR_FORMAT, "tensor `" + p + "ffn_gate_inp.weight` has wrong size");
            L.router_p.resize(L.router.size());   // the router kernel's 16-byte-per-step row layout
            for (size_t e = 0; e < c.n_experts; ++e)
                for (uint32_t k = 0; k < d; ++k) L.router_p[e * d + router_perm(k)] = L.router[e * d + k];
            if ((rc = load_norm(g, p + "exp_probs_b.bias", c.n_experts, L.bias))) return rc;
            if ((rc = load_q8(g, p + "ffn_gate_exps.weight", c.n_experts * f, d, L.gate_e, hm))) return rc;
            if ((rc = load_q8(g, p + "ffn_up_exps.weight", c.n_experts * f, d, L.up_e, hm))) return rc;
            if ((rc = load_q8(g, p + "ffn_down_exps.weight", c.n_experts * d, f, L.down_e, hm))) return rc;
            if ((rc = load_q8(g, p + "ffn_gate_shexp.weight", f, d, L.gate_sh, hm))) return rc;
            if ((rc = load_q8(g, p + "ffn_up_shexp.weight", f, d, L.up_sh, hm))) return rc;
            if ((rc = load_q8(g, p + "ffn_down_shexp.weight", d, f, L.down_sh, hm))) return rc;
        } else {
            if ((rc = load_q8(g, p + "ffn_gate.weight", c.dense_ffn, d, L.gate, hm))) return rc;
            if ((rc = load_q8(g, p + "ffn_up.weight", c.dense_ffn, d, L.up, hm))) return rc;
            if ((rc = load_q8(g, p + "ffn_down.weight", d, c.dense_ffn, L.down, hm))) return rc;
        }
        if ((rc = load_norm(g, p + "attn_norm.weight", d, L.attn_norm))) return rc;
        if ((rc = load_q8(g, p + "attn_qkv.weight", qd + 2 * kvd, d, L.qkv, hm))) return rc;
        if ((rc = load_norm(g, p + "attn_q_norm.weight", hd, L.q_norm))) return rc;
        if ((rc = load_norm(g, p + "attn_k_norm.weight", hd, L.k_norm))) return rc;
        if ((rc = load_q8(g, p + "attn_output.weight", d, qd, L.o, hm))) return rc;
        if ((rc = load_norm(g, p + "ffn_norm.weight", d, L.ffn_norm))) return rc;
    }
    if ((rc = load_q8(g, "output.weight", c.vocab_size, d, hm.output, hm))) return rc;
    if ((rc = g.load("token_embd.weight", hm.token_embd, g_err))) return rc;
    if (hm.token_embd.size() != (size_t)c.vocab_size * d)
        return fail(HG_ERR_FORMAT, "tensor `token_embd.weight` has wrong size");
    if ((rc = load_norm(g, "output_norm.weight", d, hm.output_norm))) return rc;
    rope_table(hd, c.context_length, c.rope_theta, hm.rope_cos, hm.rope_sin);
    return HG_OK;
}

int upload_vec(const std::vector<float> &v, DevBuf &dst) { return dst.upload(v.data(), v.size() * 4); }

// Device residency of a parsed model.  Q8 matrices keep f16 scales if every scale of every
// matrix is an exact f16 value (GGUF Q8_0 files: the on-disk 34 bytes per block), else all f32.
int upload_model(HostModel &hm, hg_model *m) {
    m->c = hm.c;
    m->f32 = !hm.quant;
    m->n_slots = slots_of(hm.c);
    m->ref_bytes = hm.ref_bytes;
    std::vector<std::pair<HostMat *, DevQ8 *>> mats;
    std::vector<std::pair<HostMat *, DevF32 *>> fmats;
    m->layers.resize(hm.layers.size());
    for (size_t i = 0; i < hm.layers.size(); ++i) {
        HostLayer &H = hm.layers[i];
        m->layers[i] = std::make_unique<Layer>();
        Layer &L = *m->layers[i];
        L.moe = H.moe;
        HostMat *hp[] = {&H.qkv, &H.o, &H.gate, &H.up, &H.down, &H.gate_e, &H.up_e, &H.down_e, &H.gate_sh,
                         &H.up_sh, &H.down_sh};
        DevQ8 *dp[] = {&L.qkv, &L.o, &L.gate, &L.up, &L.down, &L.gate_e, &L.up_e, &L.down_e, &L.gate_sh,
                       &L.up_sh, &L.down_sh};
        DevF32 *fp[] = {&L.fqkv, &L.fo, &L.fgate, &L.fup, &L.fdown, &L.fgate_e, &L.fup_e, &L.fdown_e, &L.fgate_sh,
                        &L.fup_sh, &L.fdown_sh};
        for (size_t k = 0; k < sizeof hp / sizeof hp[0]; ++k) {
            if (!hp[k]->N) continue;
            if (hm.quant) mats.emplace_back(hp[k], dp[k]);
            else fmats.emplace_back(hp[k], fp[k]);
        }
        int rc;
        if ((rc = upload_vec(H.attn_norm, L.attn_norm)) || (rc = upload_vec(H.q_norm, L.q_norm)) ||
            (rc = upload_vec(H.k_norm, L.k_norm)) || (rc = upload_vec(H.ffn_norm, L.ffn_norm)) ||
            (rc = upload_vec(H.router, L.router)) || (rc = upload_vec(H.router_p, L.router_p)) ||
            (rc = upload_vec(H.bias, L.bias)))
            return rc;
    }
    if (hm.quant) mats.emplace_back(&hm.output, &m->output);
    else fmats.emplace_back(&hm.output, &m->foutput);
    bool all_f16 = true;
    for (auto &pm : mats) all_f16 = all_f16 && pm.first->q8.f16_exact;
    for (auto &pm : mats) {
        pm.first->q8.set_scale_storage(!all_f16);
        int rc = pm.second->upload(pm.first->q8);
        if (rc) return rc;
        m->dev_bytes += pm.second->dev_bytes();
        pm.first->q8 = PackedQ8();
    }
    for (auto &pm : fmats) {
        int rc = pm.second->upload(pm.first->f32, pm.first->N, pm.first->K);
        if (rc) return rc;
        m->dev_bytes += pm.second->w.n;
        std::vector<float>().swap(pm.first->f32);
    }
    int rc;
    if ((rc = upload_vec(hm.token_embd, m->token_embd)) || (rc = upload_vec(hm.output_norm, m->output_norm)) ||
        (rc = upload_vec(hm.rope_cos, m->rope_cos)) || (rc = upload_vec(hm.rope_sin, m->rope_sin)))
        return rc;
    return HG_OK;
}

}  // namespace

// ======================================================================= C ABI
extern "C" {

const char *hg_last_error(void) { return g_err.c_str(); }

int hg_model_load(const char *path, int quant, hg_model **out) {
    return guard([&]() -> int {
        if (!out) return fail(HG_ERR_ARG, "out is NULL");
        *out = nullptr;
        if (!path) return fail(HG_ERR_ARG, "path is NULL");
        auto hm = std::make_unique<HostModel>();
        int rc = parse_model(path, quant != 0, *hm);
        if (rc) return rc;
        if ((rc = check_device())) return rc;
        auto m = std::make_unique<hg_model>();
        if ((rc = upload_model(*hm, m.get()))) return rc;
        *out = m.release();
        return HG_OK;
    });
}

int hg_gguf_load_tensor(const char *path, const char *name, float *out, uint64_t cap, uint64_t *n) {
    return guard([&]() -> int {
        if (!path || !name || !n) return fail(HG_ERR_ARG, "NULL argument");
        *n = 0;
        Gguf g;
        int rc = g.open(path, g_err);
        if (rc) return rc;
        std::vector<float> v;
        if ((rc = g.load(name, v, g_err))) return rc;
        *n = v.size();
        if (!out) return HG_OK;
        if (cap < v.size())
            return fail(HG_ERR_ARG, "output holds " + std::to_string(cap) + " floats, tensor has " +
                                        std::to_string(v.size()));
        memcpy(out, v.data(), v.size() * 4);
        return HG_OK;
    });
}

void hg_model_free(hg_model *m) { delete m; }

int hg_model_config(const hg_model *m, hg_config *out) {
    return guard([&]() -> int {
        if (!m || !out) return fail(HG_ERR_ARG, "NULL argument");
        *out = m->c;
        return HG_OK;
    });
}

uint64_t hg_weight_bytes(const hg_model *m) { return m ? m->ref_bytes : 0; }
uint64_t hg_device_weight_bytes(const hg_model *m) { return m ? m->dev_bytes : 0; }

int hg_token_embedding(const hg_model *m, uint32_t id, float *out) {
    return guard([&]() -> int {
        if (!m || !out) return fail(HG_ERR_ARG, "NULL argument");
        if (id >= m->c.vocab_size) return fail(HG_ERR_ARG, "token " + std::to_string(id) + " out of range");
        HIP_TRY(hipMemcpy(out, m->token_embd.as<float>() + (size_t)id * m->c.d_model, m->c.d_model * 4,
                          hipMemcpyDeviceToHost));
        return HG_OK;
    });
}

}  // extern "C"

// ======================================================================= step enqueue
namespace {

enum ProfClass { P_EMBED, P_NORM, P_QKV, P_ATTN_A, P_ATTN_B, P_OPROJ, P_ROUTER, P_GATEUP, P_DOWN, P_LMHEAD,
                 P_ARGMAX, P_OTHER, P_COUNT };
const char *const kProfNames[P_COUNT] = {"embed", "rmsnorm_quant", "attn_norm_qkv_matvec", "attn_scores", "attn_softmax_pv",
                                         "o_proj_matvec", "ffn_norm_router", "expert_gate_up", "expert_down",
                                         "lm_head_matvec", "argmax", "other"};

// Tag the following launches with class c (profiling only).
void mark(hg_kv *kv, int c) {
    if (kv->timer) kv->timer->cls = c;
}

float *layer_k(const hg_kv *kv, uint32_t l) {
    const hg_config &c = kv->m->c;
    return kv->kc.as<float>() + (size_t)l * c.n_kv_heads * kv->cap * c.head_dim;
}
float *layer_v(const hg_kv *kv, uint32_t l) {
    const hg_config &c = kv->m->c;
    return kv->vc.as<float>() + (size_t)l * v_layer_floats(kv->cap, c.n_kv_heads, c.head_dim);
}

// The F32 mode's layers (model.rs:164-184 with every Mat::matvec an ops::matvec): the norms,
// QK-norm + RoPE + append, attention, router and combine of the Q8 step, the products in
// ops::dot's order.  order: ORDER_DECODE adds the routed experts in rank order (Model::ffn,
// model.rs:299-311), ORDER_PREFILL in expert-id order (ffn_prefill, model.rs:707-731).
void enqueue_layers_f32(hg_kv *kv, int order) {
    const hg_model *m = kv->m;
    const hg_config &c = m->c;
    hipStream_t st = kv->st;
    const uint32_t d = c.d_model;
    float *x = kv->x.as<float>(), *h = kv->h.as<float>(), *qkv = kv->qkv.as<float>();
    uint8_t *qa = kv->qa.as<uint8_t>();
    float *da = kv->da.as<float>();
    StepParams *p = kv->params.as<StepParams>();
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const Layer &L = *m->layers[l];
        mark(kv, P_QKV);   // attn_norm, qkv, QK-norm + RoPE + append (model.rs:164-165, 194-211)
        launch_rmsnorm_quant(st, true, x, L.attn_norm.as<float>(), c.rms_eps, d, h, qa, da);
        launch_f32_matvec(st, EPI_STORE, L.fqkv.m, h, qkv, 0, nullptr, nullptr);
        launch_qk_rope_append(st, c.head_dim, qkv, L.q_norm.as<float>(), L.k_norm.as<float>(), c.rms_eps,
                              m->rope_cos.as<float>(), m->rope_sin.as<float>(), p, c.n_heads, c.n_kv_heads,
                              layer_k(kv, l), layer_v(kv, l), kv->cap);
        for (int part = 0; part < 2; ++part) {
            mark(kv, part == 0 ? P_ATTN_A : P_ATTN_B);
            launch_attn(st, true, part, c.head_dim, qkv, L.q_norm.as<float>(), L.k_norm.as<float>(), c.rms_eps,
                        m->rope_cos.as<float>(), m->rope_sin.as<float>(), p, layer_k(kv, l), layer_v(kv, l), kv->cap,
                        kv->win, c.n_heads, c.n_kv_heads, attn_splits(kv->win), kv->part.as<float>(),
                        kv->scores.as<float>(), kv->o.as<float>(), nullptr, da);
        }
        mark(kv, P_OPROJ);   // x += attn_output(o) (model.rs:168-171, 233)
        launch_f32_matvec(st, EPI_RESID, L.fo.m, kv->o.as<float>(), x, 0, nullptr, nullptr);
        mark(kv, P_ROUTER);
        launch_rmsnorm_quant(st, true, x, L.ffn_norm.as<float>(), c.rms_eps, d, h, qa, da);
        if (L.moe) {   // router + top-k (model.rs:270-293), the slots' experts, the combine (model.rs:295-324)
            launch_ffn_router(st, true, x, L.ffn_norm.as<float>(), c.rms_eps, d, L.router.as<float>(),
                              L.router_p.as<float>(), L.bias.as<float>(), c.n_experts, c.top_k, c.gating_sigmoid,
                              c.expert_weights_norm, c.expert_weights_scale, qa, da, kv->topk_idx.as<uint32_t>(),
                              kv->topk_w.as<float>(), kv->order.as<uint32_t>(),
                              kv->rec_idx.as<uint32_t>() + (size_t)l * c.top_k,
                              kv->rec_w.as<float>() + (size_t)l * c.top_k);
            mark(kv, P_GATEUP);
            launch_f32_gateup(st, L.fgate_e.m, L.fup_e.m, L.fgate_sh.m, L.fup_sh.m, kv->topk_idx.as<uint32_t>(),
                              c.top_k, m->n_slots, c.expert_ffn, h, kv->a.as<float>());
            mark(kv, P_DOWN);
            launch_f32_down(st, L.fdown_e.m, L.fdown_sh.m, kv->topk_idx.as<uint32_t>(), c.top_k, m->n_slots, d,
                            c.expert_ffn, kv->a.as<float>(), kv->y.as<float>());
            launch_b_combine(st, kv->y.as<float>(), kv->topk_w.as<float>(),
                             order == ORDER_PREFILL ? kv->order.as<uint32_t>() : nullptr, c.top_k, m->n_slots, d, 1, x);
        } else {   // the dense SwiGLU (model.rs:243-255), x += down(silu(g) * u)
            mark(kv, P_GATEUP);
            launch_f32_gateup(st, L.fgate.m, L.fup.m, L.fgate.m, L.fup.m, nullptr, 0, 1, c.dense_ffn, h,
                              kv->a.as<float>());
            mark(kv, P_DOWN);
            launch_f32_matvec(st, EPI_RESID, L.fdown.m, kv->a.as<float>(), x, 0, nullptr, nullptr);
        }
    }
}

void enqueue_layers(hg_kv *kv, int order) {
    if (kv->m->f32) {
        enqueue_layers_f32(kv, order);
        return;
    }
    const hg_model *m = kv->m;
    const hg_config &c = m->c;
    hipStream_t st = kv->st;
    const uint32_t d = c.d_model;
    float *x = kv->x.as<float>();
    uint8_t *qa = kv->qa.as<uint8_t>();
    float *da = kv->da.as<float>();
    StepParams *p = kv->params.as<StepParams>();
    const bool fused =
        !kv->no_fuse && qkv_scores_ok(kv->exact, c.head_dim, kv->win, c.n_heads, c.n_kv_heads, c.d_model);
    for (uint32_t l = 0; l < c.n_layers; ++l) {
        const Layer &L = *m->layers[l];
        mark(kv, P_QKV);   // attn_norm + attn_qkv + QK-norm + RoPE + append (model.rs:164-165, 194-211)
        // + the attention scores where the launch takes them (the softmax + P.V then forms the
        // score at pos)
        const bool fz = fused && launch_qkv_scores(st, order, L.qkv.m, x, L.attn_norm.as<float>(), c.rms_eps,
                                                   L.q_norm.as<float>(), L.k_norm.as<float>(),
                                                   m->rope_cos.as<float>(), m->rope_sin.as<float>(), p, c.n_heads,
                                                   c.n_kv_heads, layer_k(kv, l), layer_v(kv, l), kv->cap, kv->win,
                                                   kv->qkv.as<float>(), kv->scores.as<float>(), kv->part.as<float>());
        if (fz) {
            mark(kv, P_ATTN_B);
            launch_attn_pv_self(st, kv->qkv.as<float>(), p, layer_v(kv, l), kv->cap, kv->win, c.n_heads,
                                c.n_kv_heads, kv->part.as<float>(), kv->scores.as<float>(), kv->o.as<float>());
        } else {
            launch_qkv_head(st, kv->exact, order, c.head_dim, L.qkv.m, x, L.attn_norm.as<float>(), c.rms_eps,
                            L.q_norm.as<float>(), L.k_norm.as<float>(), m->rope_cos.as<float>(),
                            m->rope_sin.as<float>(), p, c.n_heads, c.n_kv_heads, layer_k(kv, l), layer_v(kv, l),
                            kv->cap, kv->qkv.as<float>());
        }
        for (int part = 0; part < 2 && !fz; ++part) {
            mark(kv, part == 0 ? P_ATTN_A : P_ATTN_B);
            launch_attn(st, kv->exact, part, c.head_dim, kv->qkv.as<float>(), L.q_norm.as<float>(),
                        L.k_norm.as<float>(), c.rms_eps, m->rope_cos.as<float>(), m->rope_sin.as<float>(), p,
                        layer_k(kv, l), layer_v(kv, l), kv->cap, kv->win, c.n_heads, c.n_kv_heads,
                        attn_splits(kv->win), kv->part.as<float>(), kv->scores.as<float>(), kv->o.as<float>(),
                        kv->exact ? nullptr : qa, da);
        }
        mark(kv, P_OPROJ);
        if (kv->exact)  // attn_output quantizes o itself
            launch_matvec(st, order, EPI_RESID, L.o.m, reinterpret_cast<const uint8_t *>(kv->o.as<float>()), nullptr,
                          x, 128, 0, nullptr, nullptr);
        else
            launch_matvec(st, order, EPI_RESID, L.o.m, qa, da, x, 64, 0, nullptr, nullptr);
        if (L.moe) mark(kv, P_ROUTER);   // ffn_norm + router (+ gate/up when fused)
        if (L.moe && launch_ffn_front(st, kv->exact, order, x, L.ffn_norm.as<float>(), c.rms_eps, d,
                                      L.router_p.as<float>(), L.bias.as<float>(), c.n_experts, c.top_k,
                                      c.gating_sigmoid, c.expert_weights_norm, c.expert_weights_scale, L.gate_e.m,
                                      L.up_e.m, L.gate_sh.m, L.up_sh.m, m->n_slots, c.expert_ffn,
                                      kv->topk_idx.as<uint32_t>(), kv->topk_w.as<float>(), kv->order.as<uint32_t>(),
                                      kv->rec_idx.as<uint32_t>() + (size_t)l * c.top_k,
                                      kv->rec_w.as<float>() + (size_t)l * c.top_k, kv->a.as<float>())) {
            mark(kv, P_DOWN);
            launch_ffn_down(st, order, L.down_e.m, L.down_sh.m, kv->topk_idx.as<uint32_t>(), kv->topk_w.as<float>(),
                            kv->order.as<uint32_t>(), c.top_k, m->n_slots, 0, d, c.expert_ffn, kv->a.as<float>(), x);
        } else if (L.moe) {
            launch_ffn_router(st, kv->exact, x, L.ffn_norm.as<float>(), c.rms_eps, d, L.router.as<float>(),
                              L.router_p.as<float>(), L.bias.as<float>(), c.n_experts, c.top_k, c.gating_sigmoid, c.expert_weights_norm,
                              c.expert_weights_scale, qa, da, kv->topk_idx.as<uint32_t>(), kv->topk_w.as<float>(),
                              kv->order.as<uint32_t>(), kv->rec_idx.as<uint32_t>() + (size_t)l * c.top_k,
                              kv->rec_w.as<float>() + (size_t)l * c.top_k);
            mark(kv, P_GATEUP);
            launch_ffn_gateup(st, order, L.gate_e.m, L.up_e.m, L.gate_sh.m, L.up_sh.m, kv->topk_idx.as<uint32_t>(),
                              c.top_k, m->n_slots, c.expert_ffn, qa, da, kv->a.as<float>());
            mark(kv, P_DOWN);
            launch_ffn_down(st, order, L.down_e.m, L.down_sh.m, kv->topk_idx.as<uint32_t>(), kv->topk_w.as<float>(),
                            kv->order.as<uint32_t>(), c.top_k, m->n_slots, 0, d, c.expert_ffn, kv->a.as<float>(), x);
        } else {
            mark(kv, P_NORM);
            launch_rmsnorm_quant(st, kv->exact, x, L.ffn_norm.as<float>(), c.rms_eps, d, nullptr, qa, da);
            mark(kv, P_GATEUP);
            launch_ffn_gateup(st, order, L.gate.m, L.up.m, L.gate.m, L.up.m, nullptr, 0, 1, c.dense_ffn, qa, da,
                              kv->a.as<float>());
            mark(kv, P_DOWN);   // x += down(a): the plain matvec, a quantized in its prologue (model.rs:253-254)
            launch_matvec(st, order, EPI_RESID, L.down.m, reinterpret_cast<const uint8_t *>(kv->a.as<float>()), nullptr,
                          x, 128, 0, nullptr, nullptr);
        }
    }
}

// output_norm + lm_head + greedy argmax (model.rs:180-183, lib.rs:132-142).
void enqueue_tail(hg_kv *kv) {
    const hg_model *m = kv->m;
    const hg_config &c = m->c;
    const uint32_t valid = c.vocab_size < 50257 ? c.vocab_size : 50257;
    mark(kv, P_NORM);
    launch_rmsnorm_quant(kv->st, kv->exact, kv->x.as<float>(), m->output_norm.as<float>(), c.rms_eps, c.d_model,
                         m->f32 ? kv->h.as<float>() : nullptr, kv->qa.as<uint8_t>(), kv->da.as<float>());
    mark(kv, P_LMHEAD);
    if (m->f32)
        launch_f32_matvec(kv->st, EPI_LOGITS, m->foutput.m, kv->h.as<float>(), kv->logits.as<float>(), valid,
                          kv->pv.as<float>(), kv->pi.as<uint32_t>());
    else
        launch_matvec(kv->st, ORDER_DECODE, EPI_LOGITS, m->output.m, kv->qa.as<uint8_t>(), kv->da.as<float>(),
                      kv->logits.as<float>(), kv->lm_threads, valid, kv->pv.as<float>(), kv->pi.as<uint32_t>());
    mark(kv, P_ARGMAX);
    launch_argmax_final(kv->st, kv->pv.as<float>(), kv->pi.as<uint32_t>(), kv->n_part, kv->params.as<StepParams>(),
                        kv->out_ids.as<uint32_t>());
}

void enqueue_decode(hg_kv *kv) {
    mark(kv, P_EMBED);
    launch_embed(kv->st, kv->m->token_embd.as<float>(), kv->m->c.d_model, kv->params.as<StepParams>(),
                 kv->x.as<float>());
    enqueue_layers(kv, ORDER_DECODE);
    enqueue_tail(kv);
}

void enqueue_body(hg_kv *kv) {
    launch_load_row(kv->st, kv->inputs.as<float>(), kv->m->c.d_model, kv->params.as<StepParams>(), kv->x.as<float>());
    enqueue_layers(kv, ORDER_PREFILL);
    launch_advance(kv->st, kv->params.as<StepParams>());
}

// A launch the kernels' host code refused or HIP rejected while `fn` enqueued (sticky per
// thread, cleared by the check).
int check_launches(const char *what) {
    std::string msg;
    const hipError_t e = take_launch_error(msg);
    if (e == hipSuccess) return HG_OK;
    return fail(HG_ERR_DEVICE, std::string(what) + ": " + msg);
}

// Run `fn`'s kernels on the cache's stream: replay its captured graph (capturing it on
// first use) or, with HG_GRAPH=0, launch eagerly.  A launch error during capture ends the
// capture and discards the graph, so no step returns HG_OK without having run.
template <class F>
int run(hg_kv *kv, hipGraphExec_t &exec, F fn) {
    (void)take_launch_error_reset();
    if (!kv->use_graph) {
        fn(kv);
        int rc = check_launches("kernel launch");
        if (rc) return rc;
        HIP_TRY(hipGetLastError());
        return HG_OK;
    }
    if (!exec) {
        hipGraph_t graph = nullptr;
        HIP_TRY(hipStreamBeginCapture(kv->st, hipStreamCaptureModeThreadLocal));
        fn(kv);
        const int lrc = check_launches("kernel launch during graph capture");
        hipError_t e = hipStreamEndCapture(kv->st, &graph);
        if (lrc) {
            if (graph) (void)hipGraphDestroy(graph);
            return lrc;
        }
        if (e != hipSuccess) return fail(HG_ERR_DEVICE, std::string("graph capture: ") + hipGetErrorString(e));
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (e != hipSuccess) {
            exec = nullptr;
            return fail(HG_ERR_DEVICE, std::string("graph instantiate: ") + hipGetErrorString(e));
        }
    }
    HIP_TRY(hipGraphLaunch(exec, kv->st));
    return HG_OK;
}

// The captured step for the window of a step at position pos (kv->win is set for enqueue).
hipGraphExec_t &graph_for(hg_kv *kv, std::map<uint32_t, hipGraphExec_t> &set, uint32_t pos) {
    kv->win = window_of(pos + 1, kv->cap);
    return set[kv->win];
}

int set_params(hg_kv *kv, uint32_t token, uint32_t pos, uint32_t feedback, uint32_t embed, uint32_t base) {
    StepParams &hp = *kv->h_params;
    hp = StepParams{};
    hp.token = token;
    hp.pos = pos;
    hp.step = 0;
    hp.feedback = feedback;
    hp.embed = embed;
    hp.base = base;
    const char *sc = getenv("HG_SPIN_CAP");   // (tests: a tiny cap drives the bounded waits' error path)
    hp.spin_cap = sc ? (uint32_t)strtoul(sc, nullptr, 10) : 0u;
    HIP_TRY(hipMemcpyAsync(kv->params.p, kv->h_params, sizeof(StepParams), hipMemcpyHostToDevice, kv->st));
    return HG_OK;
}

// Enqueue the read-back of the step parameters (before the stream sync that ends a call) and,
// after it, the verdict of the attention kernels' bounded waits (StepParams::err).
int fetch_params(hg_kv *kv) {
    HIP_TRY(hipMemcpyAsync(kv->h_params, kv->params.p, sizeof(StepParams), hipMemcpyDeviceToHost, kv->st));
    return HG_OK;
}
int waits_ok(const hg_kv *kv) {
    if (kv->h_params->err)
        return fail(HG_ERR_DEVICE, "a softmax/P.V kernel's wait ran out of polls: the step's results are void");
    return HG_OK;
}

int finish(hg_kv *kv, float *logits, uint32_t *next) {
    const hg_config &c = kv->m->c;
    if (logits)
        HIP_TRY(hipMemcpyAsync(kv->h_logits, kv->logits.p, (size_t)c.vocab_size * 4, hipMemcpyDeviceToHost, kv->st));
    HIP_TRY(hipMemcpyAsync(kv->h_ids, kv->out_ids.p, 4, hipMemcpyDeviceToHost, kv->st));
    int rc = fetch_params(kv);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(kv->st));
    if ((rc = waits_ok(kv))) return rc;
    if (logits) memcpy(logits, kv->h_logits, (size_t)c.vocab_size * 4);
    if (next) *next = kv->h_ids[0];
    return HG_OK;
}

// The prompt path: all rows at once (default; shapes it does not take fall back), with
// HG_PREFILL=rows one replayed decode-shaped step per row (the reference-order kernels of the
// decode step in prompt order), with HG_PREFILL=batched all rows at once or an error.
enum { PF_AUTO, PF_ROWS, PF_BATCHED };
int prefill_mode() {
    const char *e = getenv("HG_PREFILL");
    if (e && strcmp(e, "rows") == 0) return PF_ROWS;
    if (e && strcmp(e, "batched") == 0) return PF_BATCHED;
    return PF_AUTO;
}

int check_step(const hg_model *m, const hg_kv *kv, uint32_t pos, uint32_t n) {
    if (!m || !kv || kv->m != m) return fail(HG_ERR_ARG, "cache does not belong to this model");
    if (pos != kv->len)
        return fail(HG_ERR_ARG, "pos " + std::to_string(pos) + " does not continue the cache (len " +
                                    std::to_string(kv->len) + ")");
    if ((uint64_t)pos + n > kv->cap)
        return fail(HG_ERR_ARG, "pos " + std::to_string(pos) + " + " + std::to_string(n) + " exceeds the cache (" +
                                    std::to_string(kv->cap) + " positions)");
    return HG_OK;
}

}  // namespace

hg_kv::~hg_kv() {
    if (st) (void)hipStreamSynchronize(st);
    for (auto &g : g_decode)
        if (g.second) (void)hipGraphExecDestroy(g.second);
    for (auto &g : g_body)
        if (g.second) (void)hipGraphExecDestroy(g.second);
    if (g_tail) (void)hipGraphExecDestroy(g_tail);
    if (h_params) (void)hipHostFree(h_params);
    if (h_ids) (void)hipHostFree(h_ids);
    if (h_logits) (void)hipHostFree(h_logits);
    if (st) (void)hipStreamDestroy(st);
}

extern "C" {

int hg_kv_new(const hg_model *m, uint32_t max_ctx, uint32_t flags, hg_kv **out) {
    return guard([&]() -> int {
        if (!m || !out) return fail(HG_ERR_ARG, "NULL argument");
        *out = nullptr;
        const hg_config &c = m->c;
        if (max_ctx == 0 || max_ctx > c.context_length) max_ctx = c.context_length;
        auto kv = std::make_unique<hg_kv>();
        kv->m = m;
        kv->cap = max_ctx;
        kv->flags = flags;
        kv->exact = (flags & HG_KV_FAST) == 0;
        const char *ge = getenv("HG_GRAPH");
        kv->use_graph = !(ge && ge[0] == '0');
        const char *qs = getenv("HG_QKV_SCORES");
        kv->no_fuse = qs && qs[0] == '0';
        kv->win = kv->cap;
        if (kv->exact && pv_ring_slots(kv->cap) < 2)
            return fail(HG_ERR_UNSUPPORTED, "a reference-order cache holds at most 32768 positions");
        if (m->f32 && !kv->exact)
            return fail(HG_ERR_UNSUPPORTED, "the F32 mode runs the reference-order attention only (no HG_KV_FAST)");
        HIP_TRY(hipStreamCreateWithFlags(&kv->st, hipStreamNonBlocking));
        const size_t kvsz = (size_t)c.n_layers * c.n_kv_heads * kv->cap * c.head_dim * 4;
        int rc;
        if ((rc = kv->kc.alloc(kvsz)) ||
            (rc = kv->vc.alloc((size_t)c.n_layers * v_layer_floats(kv->cap, c.n_kv_heads, c.head_dim) * 4)))
            return rc;
        const uint32_t qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
        const uint32_t maxk = std::max(std::max(c.d_model, qd), std::max(c.dense_ffn, c.expert_ffn));
        const uint32_t maxnc = div_up(maxk / QK, 4);
        const uint32_t ffw = std::max(c.dense_ffn, c.expert_ffn) * std::max(m->n_slots, 1u);
        kv->n_part = m->f32 ? f32_matvec_blocks(c.vocab_size) : matvec_blocks(c.vocab_size, kv->lm_threads);
        if (m->f32 && ((rc = kv->h.alloc((size_t)c.d_model * 4)) ||
                       (rc = kv->y.alloc((size_t)std::max(m->n_slots, 1u) * c.d_model * 4))))
            return rc;
        if ((rc = kv->x.alloc(c.d_model * 4)) || (rc = kv->qkv.alloc((size_t)(qd + 2 * kvd) * 4)) ||
            (rc = kv->o.alloc((size_t)qd * 4)) ||
            (rc = kv->part.alloc((size_t)c.n_heads * attn_splits(kv->cap) * (c.head_dim + 2) * 4)) ||
            (rc = kv->scores.alloc(kv->exact ? (size_t)c.n_heads * kv->cap * 4 : 4)) ||
            (rc = kv->a.alloc((size_t)ffw * 4)) || (rc = kv->logits.alloc((size_t)c.vocab_size * 4)) ||
            (rc = kv->pv.alloc((size_t)kv->n_part * 4)) || (rc = kv->pi.alloc((size_t)kv->n_part * 4)) ||
            (rc = kv->qa.alloc((size_t)maxnc * CHUNK_BYTES)) || (rc = kv->da.alloc((size_t)maxnc * 4 * 4)) ||
            (rc = kv->topk_idx.alloc(64 * 4)) || (rc = kv->topk_w.alloc(64 * 4)) || (rc = kv->order.alloc(64 * 4)) ||
            (rc = kv->rec_idx.alloc((size_t)c.n_layers * std::max(c.top_k, 1u) * 4)) ||
            (rc = kv->rec_w.alloc((size_t)c.n_layers * std::max(c.top_k, 1u) * 4)) ||
            (rc = kv->params.alloc(sizeof(StepParams))) || (rc = kv->out_ids.alloc((size_t)(kv->cap + 1) * 4)))
            return rc;
        HIP_TRY(hipMemset(kv->rec_idx.p, 0xff, kv->rec_idx.n));
        HIP_TRY(hipMemset(kv->rec_w.p, 0, kv->rec_w.n));
        HIP_TRY(hipMemset(kv->kc.p, 0, kv->kc.n));
        HIP_TRY(hipMemset(kv->vc.p, 0, kv->vc.n));
        HIP_TRY(hipHostMalloc((void **)&kv->h_params, sizeof(StepParams), hipHostMallocDefault));
        HIP_TRY(hipHostMalloc((void **)&kv->h_ids, (size_t)(kv->cap + 1) * 4, hipHostMallocDefault));
        HIP_TRY(hipHostMalloc((void **)&kv->h_logits, (size_t)c.vocab_size * 4, hipHostMallocDefault));
        HIP_TRY(hipDeviceSynchronize());
        *out = kv.release();
        return HG_OK;
    });
}

void hg_kv_free(hg_kv *kv) { delete kv; }

uint32_t hg_kv_len(const hg_kv *kv) { return kv ? kv->len : 0; }

int hg_kv_read(const hg_kv *kv, uint32_t layer, float *k, float *v) {
    return guard([&]() -> int {
        if (!kv || !k || !v) return fail(HG_ERR_ARG, "NULL argument");
        const hg_config &c = kv->m->c;
        if (layer >= c.n_layers) return fail(HG_ERR_ARG, "layer out of range");
        const uint32_t hd = c.head_dim, nkv = c.n_kv_heads, len = kv->len;
        std::vector<float> kb((size_t)nkv * kv->cap * hd), vb(kb.size());
        HIP_TRY(hipStreamSynchronize(kv->st));
        HIP_TRY(hipMemcpy(kb.data(), layer_k(kv, layer), kb.size() * 4, hipMemcpyDeviceToHost));
        HIP_TRY(hipMemcpy(vb.data(), layer_v(kv, layer), vb.size() * 4, hipMemcpyDeviceToHost));
        for (uint32_t t = 0; t < len; ++t)
            for (uint32_t g = 0; g < nkv; ++g) {
                memcpy(k + ((size_t)t * nkv + g) * hd, kb.data() + ((size_t)g * kv->cap + t) * hd, hd * 4);
                memcpy(v + ((size_t)t * nkv + g) * hd, vb.data() + ((size_t)g * kv->cap + t) * hd, hd * 4);
            }
        return HG_OK;
    });
}

int hg_kv_load(hg_kv *kv, uint32_t len, const float *k, const float *v) {
    return guard([&]() -> int {
        if (!kv || (len && (!k || !v))) return fail(HG_ERR_ARG, "NULL argument");
        if (len > kv->cap)
            return fail(HG_ERR_ARG, "len " + std::to_string(len) + " exceeds the cache (" + std::to_string(kv->cap) +
                                        " positions)");
        const hg_config &c = kv->m->c;
        const uint32_t hd = c.head_dim, nkv = c.n_kv_heads, kvd = nkv * hd, vts = vt_stride(kv->cap);
        HIP_TRY(hipStreamSynchronize(kv->st));
        std::vector<float> kh((size_t)len * hd), vh((size_t)len * hd), vt((size_t)hd * len);
        for (uint32_t l = 0; l < c.n_layers; ++l)
            for (uint32_t g = 0; g < nkv; ++g) {
                const float *ks = k + (size_t)l * len * kvd, *vs = v + (size_t)l * len * kvd;
                for (uint32_t t = 0; t < len; ++t) {
                    memcpy(&kh[(size_t)t * hd], ks + (size_t)t * kvd + g * hd, hd * 4);
                    memcpy(&vh[(size_t)t * hd], vs + (size_t)t * kvd + g * hd, hd * 4);
                    for (uint32_t i = 0; i < hd; ++i) vt[(size_t)i * len + t] = vs[(size_t)t * kvd + g * hd + i];
                }
                if (!len) continue;
                float *kd = layer_k(kv, l) + (size_t)g * kv->cap * hd, *vd = layer_v(kv, l) + (size_t)g * kv->cap * hd;
                float *vtd = layer_v(kv, l) + (size_t)nkv * kv->cap * hd + (size_t)g * hd * vts;
                HIP_TRY(hipMemcpy(kd, kh.data(), (size_t)len * hd * 4, hipMemcpyHostToDevice));
                HIP_TRY(hipMemcpy(vd, vh.data(), (size_t)len * hd * 4, hipMemcpyHostToDevice));
                HIP_TRY(hipMemcpy2D(vtd, (size_t)vts * 4, vt.data(), (size_t)len * 4, (size_t)len * 4, hd,
                                    hipMemcpyHostToDevice));
            }
        kv->len = len;
        return HG_OK;
    });
}

int hg_forward(const hg_model *m, hg_kv *kv, uint32_t token, uint32_t pos, float *logits, uint32_t *next) {
    return guard([&]() -> int {
        int rc = check_step(m, kv, pos, 1);
        if (rc) return rc;
        if (token >= m->c.vocab_size)
            return fail(HG_ERR_ARG, "token " + std::to_string(token) + " out of range (vocab " +
                                        std::to_string(m->c.vocab_size) + ")");
        if ((rc = set_params(kv, token, pos, 0, 1, pos))) return rc;
        if ((rc = run(kv, graph_for(kv, kv->g_decode, pos), enqueue_decode))) return rc;
        if ((rc = finish(kv, logits, next))) return rc;
        kv->len = pos + 1;
        return HG_OK;
    });
}

int hg_forward_x(const hg_model *m, hg_kv *kv, const float *x, uint32_t pos, float *logits, uint32_t *next) {
    return guard([&]() -> int {
        int rc = check_step(m, kv, pos, 1);
        if (rc) return rc;
        if (!x) return fail(HG_ERR_ARG, "x is NULL");
        HIP_TRY(hipMemcpyAsync(kv->x.p, x, (size_t)m->c.d_model * 4, hipMemcpyHostToDevice, kv->st));
        if ((rc = set_params(kv, 0, pos, 0, 0, pos))) return rc;
        if ((rc = run(kv, graph_for(kv, kv->g_decode, pos), enqueue_decode))) return rc;
        if ((rc = finish(kv, logits, next))) return rc;
        kv->len = pos + 1;
        return HG_OK;
    });
}

int hg_prefill(const hg_model *m, hg_kv *kv, const float *inputs, uint32_t tn, float *logits, uint32_t *next) {
    return guard([&]() -> int {
        if (!kv) return fail(HG_ERR_ARG, "NULL argument");
        if (tn == 0) return fail(HG_ERR_ARG, "prefill needs at least one input row");
        if (!inputs) return fail(HG_ERR_ARG, "inputs is NULL");
        const uint32_t base = kv->len;
        int rc = check_step(m, kv, base, tn);
        if (rc) return rc;
        const size_t rowb = (size_t)m->c.d_model * 4;
        if (tn > kv->inputs_rows) {
            HIP_TRY(hipStreamSynchronize(kv->st));
            if ((rc = kv->inputs.alloc(rowb * tn))) return rc;
            kv->inputs_rows = tn;
            for (auto &g : kv->g_body)   // the captured bodies read the old buffer
                if (g.second) (void)hipGraphExecDestroy(g.second);
            kv->g_body.clear();
        }
        const int mode = prefill_mode();
        const bool ok = kv->exact && prefill_batched_ok(m, base + tn);
        if (mode == PF_BATCHED && !ok) return fail(HG_ERR_UNSUPPORTED, "HG_PREFILL=batched: shape or cache not supported");
        if (mode != PF_ROWS && ok) {
            if (!kv->pw) kv->pw = std::make_unique<PrefillWork>();
            if ((rc = prefill_batched(m, *kv->pw, kv->st, inputs, base, tn, kv->kc.as<float>(), kv->vc.as<float>(),
                                      kv->cap, kv->x.as<float>(), kv->rec_idx.as<uint32_t>(), kv->rec_w.as<float>())))
                return rc;
            if ((rc = set_params(kv, 0, base + tn, 0, 0, base))) return rc;
            if ((rc = run(kv, kv->g_tail, enqueue_tail))) return rc;
            if ((rc = finish(kv, logits, next))) return rc;
            kv->len = base + tn;
            return HG_OK;
        }
        HIP_TRY(hipMemcpyAsync(kv->inputs.p, inputs, rowb * tn, hipMemcpyHostToDevice, kv->st));
        if ((rc = set_params(kv, 0, base, 0, 0, base))) return rc;
        for (uint32_t t = 0; t < tn; ++t)
            if ((rc = run(kv, graph_for(kv, kv->g_body, base + t), enqueue_body))) return rc;
        if ((rc = run(kv, kv->g_tail, enqueue_tail))) return rc;
        if ((rc = finish(kv, logits, next))) return rc;
        kv->len = base + tn;
        return HG_OK;
    });
}

int hg_decode_greedy(const hg_model *m, hg_kv *kv, uint32_t first_token, uint32_t n_steps, uint32_t *out_ids) {
    return guard([&]() -> int {
        if (!kv) return fail(HG_ERR_ARG, "NULL argument");
        const uint32_t pos = kv->len;
        int rc = check_step(m, kv, pos, n_steps);
        if (rc) return rc;
        if (first_token >= m->c.vocab_size) return fail(HG_ERR_ARG, "token out of range");
        if (n_steps == 0) return HG_OK;
        if (!out_ids) return fail(HG_ERR_ARG, "out_ids is NULL");
        if ((rc = set_params(kv, first_token, pos, 1, 1, pos))) return rc;
        for (uint32_t i = 0; i < n_steps; ++i)
            if ((rc = run(kv, graph_for(kv, kv->g_decode, pos + i), enqueue_decode))) return rc;
        HIP_TRY(hipMemcpyAsync(kv->h_ids, kv->out_ids.p, (size_t)n_steps * 4, hipMemcpyDeviceToHost, kv->st));
        if ((rc = fetch_params(kv))) return rc;
        HIP_TRY(hipStreamSynchronize(kv->st));
        if ((rc = waits_ok(kv))) return rc;
        memcpy(out_ids, kv->h_ids, (size_t)n_steps * 4);
        kv->len = pos + n_steps;
        return HG_OK;
    });
}

int hg_generate(const hg_model *m, hg_kv *kv, const uint32_t *prompt, uint32_t n_prompt, const hg_gen_opts *opts,
                uint32_t eos, uint32_t *out_ids, uint32_t *n_out) {
    return guard([&]() -> int {
        if (!m || !kv || !opts || !n_out) return fail(HG_ERR_ARG, "NULL argument");
        *n_out = 0;
        if (n_prompt > 0 && !prompt) return fail(HG_ERR_ARG, "prompt is NULL");
        if (opts->max_new > 0 && !out_ids) return fail(HG_ERR_ARG, "out_ids is NULL");
        if (kv->m != m) return fail(HG_ERR_ARG, "cache does not belong to this model");
        if (n_prompt == 0) return HG_OK;
        const hg_config &c = m->c;
        const uint32_t d = c.d_model, V = c.vocab_size, valid = V < 50257 ? V : 50257, max_new = opts->max_new;
        std::vector<float> in((size_t)n_prompt * d);
        int rc;
        for (uint32_t i = 0; i < n_prompt; ++i)
            if ((rc = hg_token_embedding(m, prompt[i], in.data() + (size_t)i * d))) return rc;
        uint32_t first = 0;
        if ((rc = hg_prefill(m, kv, in.data(), n_prompt, nullptr, &first))) return rc;   // logits stay on the device
        if (max_new == 0) return HG_OK;
        if (!kv->sw) kv->sw = std::make_unique<SampleWork>();
        if ((rc = sample_init(*kv->sw, V))) return rc;
        const uint64_t seed = opts->seed > 1 ? opts->seed : 1;   // Rng::new (sample.rs:6-8)
        HIP_TRY(hipMemcpy(kv->sw->rng.p, &seed, 8, hipMemcpyHostToDevice));
        if (kv->picks.n < (size_t)max_new * 4 && (rc = kv->picks.alloc((size_t)max_new * 4))) return rc;
        uint32_t *picks = kv->picks.as<uint32_t>();
        const uint32_t p0 = kv->len, stop = std::min(c.context_length, kv->cap);
        uint32_t pos = p0, n = 0, fw = 0;
        bool done = false;
        if ((rc = set_params(kv, 0, pos, 1, 1, pos))) return rc;
        // steps in chunks between host checks of the picks: per step the draw from the logits on
        // the device (it sets the token of the next step), then the decode step at pos
        constexpr uint32_t CH = 16;
        for (uint32_t it = 0; it < max_new && !done;) {
            const uint32_t j0 = it;
            uint32_t fw_chunk = 0;
            bool ctx_stop = false;
            for (; it < max_new && it < j0 + CH; ++it) {
                (void)take_launch_error_reset();
                if (!enqueue_sample(kv->st, *kv->sw, kv->logits.as<float>(), valid, opts->temp, opts->top_p,
                                    opts->rep_penalty, picks + it, kv->params.as<StepParams>()))
                    return fail(HG_ERR_DEVICE, "sampling launch failed");
                if (pos + 1 >= stop) {   // lib.rs:155-157: the token is kept, not forwarded
                    ctx_stop = true;
                    ++it;
                    break;
                }
                if ((rc = run(kv, graph_for(kv, kv->g_decode, pos), enqueue_decode))) return rc;
                ++pos;
                ++fw_chunk;
            }
            HIP_TRY(hipMemcpyAsync(kv->h_ids, picks + j0, (size_t)(it - j0) * 4, hipMemcpyDeviceToHost, kv->st));
            if ((rc = fetch_params(kv))) return rc;
            HIP_TRY(hipStreamSynchronize(kv->st));
            if ((rc = waits_ok(kv))) return rc;
            for (uint32_t j = 0; j < it - j0; ++j) {
                const uint32_t t = kv->h_ids[j];
                if (t == eos) {   // lib.rs:143-145
                    done = true;
                    break;
                }
                out_ids[n++] = t;
                if (j < fw_chunk) ++fw;
            }
            if (ctx_stop) done = true;
        }
        kv->len = p0 + fw;   // the forwarded rows (a step past an eos leaves rows beyond len)
        *n_out = n;
        return HG_OK;
    });
}

int hg_sample(const float *logits, uint32_t n, float temp, float top_p, uint64_t *rng_state, uint32_t *out) {
    return guard([&]() -> int {
        if (!logits || !rng_state || !out) return fail(HG_ERR_ARG, "NULL argument");
        if (n == 0) return fail(HG_ERR_ARG, "no logits");
        int rc = check_device();
        if (rc) return rc;
        SampleWork w;
        DevBuf lg, pick;
        if ((rc = sample_init(w, n)) || (rc = lg.alloc((size_t)n * 4)) || (rc = pick.alloc(4))) return rc;
        HIP_TRY(hipMemcpy(lg.p, logits, (size_t)n * 4, hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(w.rng.p, rng_state, 8, hipMemcpyHostToDevice));
        if (!enqueue_sample(nullptr, w, lg.as<float>(), n, temp, top_p, 1.0f, pick.as<uint32_t>(), nullptr))
            return fail(HG_ERR_DEVICE, "sampling launch failed");
        HIP_TRY(hipMemcpy(out, pick.p, 4, hipMemcpyDeviceToHost));
        HIP_TRY(hipMemcpy(rng_state, w.rng.p, 8, hipMemcpyDeviceToHost));
        return HG_OK;
    });
}

int hg_run_block(const hg_model *m, hg_kv *kv, const float *block, uint32_t b, uint32_t base, int append,
                 float *logits, float *bk, float *bv) {
    return guard([&]() -> int {
        if (!m || !kv || !block) return fail(HG_ERR_ARG, "NULL argument");
        if (kv->m != m) return fail(HG_ERR_ARG, "cache does not belong to this model");
        if (b == 0) return fail(HG_ERR_ARG, "run_block needs at least one row");
        if (base > kv->len) return fail(HG_ERR_ARG, "base beyond the cache length");
        if (append && base != kv->len) return fail(HG_ERR_ARG, "append needs base == the cache length");
        if ((uint64_t)base + b > kv->cap) return fail(HG_ERR_ARG, "block beyond the cache capacity");
        if (!prefill_batched_ok(m, base + b)) return fail(HG_ERR_UNSUPPORTED, "run_block: shape not supported");
        const hg_config &c = m->c;
        const size_t kvd = (size_t)c.n_kv_heads * c.head_dim, lb = (size_t)c.vocab_size * b * 4;
        const size_t kb = (size_t)c.n_layers * b * kvd * 4;
        DevBuf dl, dk, dv;
        int rc;
        if ((logits && (rc = dl.alloc(lb))) || (bk && (rc = dk.alloc(kb))) || (bv && (rc = dv.alloc(kb)))) return rc;
        if (!kv->pw) kv->pw = std::make_unique<PrefillWork>();
        if ((rc = run_block_batched(m, *kv->pw, kv->st, block, nullptr, base, b, kv->kc.as<float>(), kv->vc.as<float>(),
                                    kv->cap, append != 0, dl.as<float>(), dk.as<float>(), dv.as<float>())))
            return rc;
        if (logits) HIP_TRY(hipMemcpy(logits, dl.p, lb, hipMemcpyDeviceToHost));
        if (bk) HIP_TRY(hipMemcpy(bk, dk.p, kb, hipMemcpyDeviceToHost));
        if (bv) HIP_TRY(hipMemcpy(bv, dv.p, kb, hipMemcpyDeviceToHost));
        if (append) kv->len = base + b;
        return HG_OK;
    });
}

int hg_forward_bidir(const hg_model *m, const float *inputs, uint32_t tn, float *logits) {
    return guard([&]() -> int {
        if (!m || !inputs || !logits) return fail(HG_ERR_ARG, "NULL argument");
        hg_kv *kv = nullptr;
        int rc = hg_kv_new(m, tn, 0, &kv);
        if (rc) return rc;
        rc = hg_run_block(m, kv, inputs, tn, 0, 0, logits, nullptr, nullptr);
        hg_kv_free(kv);
        return rc;
    });
}

namespace {

// The scoring state of one Engine::generate_diffusion call (lib.rs:214-495).
struct Diffusion {
    const hg_model *m = nullptr;
    const hg_diff_opts *o = nullptr;
    hg_kv *kv = nullptr;          // cached: the persistent prefix cache; uncached: a scratch cache
    std::vector<uint32_t> canvas; // uncached: the canvas; cached: the committed ids
    size_t committed = 0;
    uint32_t valid = 0, mask = 0;
    DevBuf logits, ids, present, cur, pred, pconf, cconf;
    std::vector<uint8_t> h_present;
    // Gumbel draws (temp > 0): the RNG state (host), the jump matrices, the -ln(-ln(u)) table
    uint64_t rng = 1;
    std::vector<uint64_t> M;
    DevBuf dM, G, count;
    std::vector<uint32_t> h_count;
    ~Diffusion() {
        if (kv) hg_kv_free(kv);
    }

    // Engine::score_block / diffusion_block's scoring (lib.rs:171-205, 226-262) of the block
    // [b0, b0 + len) whose current ids are blk: run_block of the block over the cache (cached) or
    // forward_bidir of canvas[0 .. b0 + len) (uncached), then the rows scored on the device.
    int score(const uint32_t *blk, size_t b0, size_t len, uint32_t *h_pred, float *h_pconf, float *h_cconf) {
        const hg_config &c = m->c;
        const uint32_t V = c.vocab_size;
        hipStream_t st = kv->st;
        const bool cached = o->cached != 0;
        const size_t rows = cached ? len : b0 + len;
        const uint32_t *src = cached ? blk : canvas.data();
        HIP_TRY(hipMemcpyAsync(ids.p, src, rows * 4, hipMemcpyHostToDevice, st));
        int rc = run_block_batched(m, *kv->pw, st, nullptr, ids.as<uint32_t>(), cached ? (uint32_t)b0 : 0u,
                                   (uint32_t)rows, kv->kc.as<float>(), kv->vc.as<float>(), kv->cap, false,
                                   logits.as<float>(), nullptr, nullptr);
        if (rc) return rc;
        const bool pen = o->rep_penalty != 1.0f;
        if (pen) {   // the present ids: committed (or the canvas up to b1) and the block, mask excluded
            std::fill(h_present.begin(), h_present.end(), 0);
            auto mark = [&](uint32_t id) {
                if (id != mask && id < valid) h_present[id] = 1;
            };
            if (cached) {
                for (size_t i = 0; i < committed; ++i) mark(canvas[i]);
                for (size_t i = 0; i < len; ++i) mark(blk[i]);
            } else {
                for (size_t i = 0; i < b0 + len; ++i) mark(canvas[i]);
            }
            HIP_TRY(hipMemcpyAsync(present.p, h_present.data(), valid, hipMemcpyHostToDevice, st));
        }
        HIP_TRY(hipMemcpyAsync(cur.p, blk, len * 4, hipMemcpyHostToDevice, st));
        const float *lg = logits.as<float>() + (cached ? 0 : b0 * (size_t)V);
        const bool gumbel = o->temp > 0.0f;
        GumbelDraws gd{o->temp, rng, dM.as<uint64_t>(), G.as<float>(), count.as<uint32_t>()};
        if (!enqueue_score_rows(st, lg, (uint32_t)len, V, valid, pen ? present.as<uint8_t>() : nullptr, o->rep_penalty,
                                cur.as<uint32_t>(), pred.as<uint32_t>(), pconf.as<float>(), cconf.as<float>(),
                                gumbel ? &gd : nullptr))
            return fail(HG_ERR_DEVICE, "scoring launch failed");
        HIP_TRY(hipMemcpyAsync(h_pred, pred.p, len * 4, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipMemcpyAsync(h_pconf, pconf.p, len * 4, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipMemcpyAsync(h_cconf, cconf.p, len * 4, hipMemcpyDeviceToHost, st));
        if (gumbel) HIP_TRY(hipMemcpyAsync(h_count.data(), count.p, len * 4, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipStreamSynchronize(st));
        if (gumbel) {   // the rows' draws advance the one Rng (lib.rs:275, 312-370)
            uint64_t total = 0;
            for (size_t i = 0; i < len; ++i) total += h_count[i];
            rng = rng_jump_host(rng, total, M.data());
        }
        return HG_OK;
    }
};

}  // namespace

int hg_generate_diffusion(const hg_model *m, const uint32_t *prompt, uint32_t n_prompt, const hg_diff_opts *opts,
                          uint32_t eos, uint32_t *out_ids, uint32_t *n_out) {
    return guard([&]() -> int {
        if (!m || !opts || !n_out) return fail(HG_ERR_ARG, "NULL argument");
        if (m->f32) return fail(HG_ERR_UNSUPPORTED, "diffusion decoding needs Q8 matrices (load with quant = true)");
        *n_out = 0;
        if (n_prompt > 0 && !prompt) return fail(HG_ERR_ARG, "prompt is NULL");
        if (n_prompt == 0) return HG_OK;
        if (opts->block == 0 || opts->steps == 0) return fail(HG_ERR_ARG, "block and steps must be positive");
        if (!out_ids && opts->gen_len > 0) return fail(HG_ERR_ARG, "out_ids is NULL");
        const hg_config &c = m->c;
        const size_t p = n_prompt, V = c.vocab_size, ctx = c.context_length;
        for (size_t i = 0; i < p; ++i)
            if (prompt[i] >= V) return fail(HG_ERR_ARG, "token out of range");
        if (c.mask_token_id >= V) return fail(HG_ERR_UNSUPPORTED, "the mask id is outside the vocabulary");
        Diffusion D;
        D.m = m;
        D.o = opts;
        D.valid = (uint32_t)std::min<size_t>(V, 50257);
        D.mask = c.mask_token_id;
        const bool cached = opts->cached != 0;
        const size_t room = cached ? (ctx > p + opts->block ? ctx - (p + opts->block) : 0) : (ctx > p ? ctx - p : 0);
        const size_t gen_len = std::min<size_t>(opts->gen_len, std::max<size_t>(room, 1));
        const size_t span = cached ? std::max<size_t>(opts->block, p) : p + gen_len;
        int rc = hg_kv_new(m, (uint32_t)std::min<size_t>(ctx, p + gen_len + opts->block), 0, &D.kv);
        if (rc) return rc;
        D.kv->pw = std::make_unique<PrefillWork>();
        if ((rc = D.logits.alloc(span * V * 4)) || (rc = D.ids.alloc(span * 4)) || (rc = D.present.alloc(D.valid)) ||
            (rc = D.cur.alloc(opts->block * 4)) || (rc = D.pred.alloc(opts->block * 4)) ||
            (rc = D.pconf.alloc(opts->block * 4)) || (rc = D.cconf.alloc(opts->block * 4)))
            return rc;
        D.h_present.assign(D.valid, 0);
        D.canvas.assign(prompt, prompt + p);
        if (opts->temp > 0.0f) {   // Rng::new (sample.rs:6-8), the jump matrices and the draw table
            D.rng = opts->seed > 1 ? opts->seed : 1;
            D.M.resize(32 * 64);
            rng_jump_matrices(D.M.data());
            const std::vector<float> &tab = gumbel_table();
            if ((rc = D.dM.upload(D.M.data(), D.M.size() * 8)) || (rc = D.G.upload(tab.data(), tab.size() * 4)) ||
                (rc = D.count.alloc(opts->block * 4 + 4)))
                return rc;
            D.h_count.assign(opts->block + 1, 0);
        }
        if (cached) {   // the bidirectional prompt encode seeds the cache (lib.rs:281-289)
            HIP_TRY(hipMemcpy(D.ids.p, prompt, p * 4, hipMemcpyHostToDevice));
            if ((rc = run_block_batched(m, *D.kv->pw, D.kv->st, nullptr, D.ids.as<uint32_t>(), 0, (uint32_t)p,
                                        D.kv->kc.as<float>(), D.kv->vc.as<float>(), D.kv->cap, true, nullptr, nullptr,
                                        nullptr)))
                return rc;
            D.kv->len = (uint32_t)p;
            D.committed = p;
        } else {
            D.canvas.resize(p + gen_len, D.mask);
        }
        std::vector<uint32_t> blk(opts->block), pred(opts->block);
        std::vector<float> pconf(opts->block), cconf(opts->block);
        size_t result = gen_len;
        for (size_t b0 = p; b0 < p + gen_len;) {
            const size_t b1 = std::min<size_t>(b0 + opts->block, p + gen_len), len = b1 - b0;
            uint32_t *cur = cached ? blk.data() : D.canvas.data() + b0;
            if (cached) std::fill(blk.begin(), blk.begin() + len, D.mask);
            auto any_mask = [&] {
                for (size_t i = 0; i < len; ++i)
                    if (cur[i] == D.mask) return true;
                return false;
            };
            auto score = [&] { return D.score(cur, b0, len, pred.data(), pconf.data(), cconf.data()); };
            if (cached && opts->threshold > 0.0f) {   // confidence-threshold decode (lib.rs:302-327)
                for (size_t it = 0; it < std::max<size_t>(len, 1); ++it) {
                    if (!any_mask()) break;
                    if ((rc = score())) return rc;
                    bool any = false, have = false;
                    size_t best = 0;
                    for (size_t i = 0; i < len; ++i)   // Iterator::max_by: the last of equal maxima
                        if (cur[i] == D.mask && (!have || !(pconf[i] < pconf[best]))) {
                            best = i;
                            have = true;
                        }
                    for (size_t i = 0; i < len; ++i)
                        if (cur[i] == D.mask && pconf[i] >= opts->threshold) {
                            cur[i] = pred[i];
                            any = true;
                        }
                    if (!any) cur[best] = pred[best];
                }
            } else {   // the num_transfer schedule (lib.rs:329-352, 420-451)
                size_t sb = (size_t)roundf((float)(opts->steps * len) / (float)gen_len);
                sb = std::max<size_t>(sb, 1);
                const size_t base_n = len / sb;
                for (size_t s = 0; s < sb; ++s) {
                    const size_t k_step = base_n + (s < len - base_n * sb ? 1 : 0);   // num_transfer (lib.rs:68-76)
                    if ((rc = score())) return rc;
                    std::vector<std::pair<size_t, float>> cand;
                    for (size_t i = 0; i < len; ++i)
                        if (cur[i] == D.mask) cand.emplace_back(i, pconf[i]);
                    if (cand.empty()) break;
                    std::stable_sort(cand.begin(), cand.end(), [](const auto &a, const auto &b) { return a.second > b.second; });
                    for (size_t q = 0; q < std::min(k_step, cand.size()); ++q) cur[cand[q].first] = pred[cand[q].first];
                }
                if (any_mask()) {
                    if ((rc = score())) return rc;
                    for (size_t i = 0; i < len; ++i)
                        if (cur[i] == D.mask) cur[i] = pred[i];
                }
            }
            for (uint32_t rs = 0; rs < opts->remask_steps; ++rs) {   // re-mask the least confident (lib.rs:354-371)
                if ((rc = score())) return rc;
                size_t r = std::max<size_t>((size_t)((float)len * opts->remask_frac), 1);
                std::vector<std::pair<size_t, float>> idx;
                for (size_t i = 0; i < len; ++i) idx.emplace_back(i, cconf[i]);
                std::stable_sort(idx.begin(), idx.end(), [](const auto &a, const auto &b) { return a.second < b.second; });
                for (size_t q = 0; q < std::min(r, len); ++q) cur[idx[q].first] = D.mask;
                if ((rc = score())) return rc;
                for (size_t i = 0; i < len; ++i)
                    if (cur[i] == D.mask) cur[i] = pred[i];
            }
            if (cached) {   // finalize: the block's K/V into the cache (lib.rs:374-381)
                HIP_TRY(hipMemcpy(D.ids.p, blk.data(), len * 4, hipMemcpyHostToDevice));
                if ((rc = run_block_batched(m, *D.kv->pw, D.kv->st, nullptr, D.ids.as<uint32_t>(), (uint32_t)b0,
                                            (uint32_t)len, D.kv->kc.as<float>(), D.kv->vc.as<float>(), D.kv->cap, true,
                                            nullptr, nullptr, nullptr)))
                    return rc;
                D.kv->len = (uint32_t)b1;
                D.canvas.insert(D.canvas.end(), blk.begin(), blk.begin() + len);
                D.committed = b1;
            }
            size_t endpos = b1;
            bool hit = false;
            for (size_t i = p; i < b1; ++i)
                if (D.canvas[i] == eos) {
                    endpos = i;
                    hit = true;
                    break;
                }
            if (hit) {
                result = endpos - p;
                break;
            }
            b0 = b1;
        }
        memcpy(out_ids, D.canvas.data() + p, result * 4);
        *n_out = (uint32_t)result;
        return HG_OK;
    });
}

int hg_generate_greedy(const hg_model *m, hg_kv *kv, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_new,
                       float rep_penalty, uint32_t eos, uint32_t *out_ids, uint32_t *n_out) {
    return guard([&]() -> int {
        if (!m || !kv || !n_out) return fail(HG_ERR_ARG, "NULL argument");
        *n_out = 0;
        if (n_prompt > 0 && !prompt) return fail(HG_ERR_ARG, "prompt is NULL");
        if (max_new > 0 && !out_ids) return fail(HG_ERR_ARG, "out_ids is NULL");
        if (n_prompt == 0) return HG_OK;
        const hg_config &c = m->c;
        const uint32_t d = c.d_model, V = c.vocab_size, valid = V < 50257 ? V : 50257;
        std::vector<float> in((size_t)n_prompt * d);
        int rc;
        for (uint32_t i = 0; i < n_prompt; ++i)
            if ((rc = hg_token_embedding(m, prompt[i], in.data() + (size_t)i * d))) return rc;
        const bool host_sample = rep_penalty != 1.0f;
        std::vector<float> logits(host_sample ? V : 0);
        uint32_t next = 0, pos = kv->len + n_prompt;
        if ((rc = hg_prefill(m, kv, in.data(), n_prompt, host_sample ? logits.data() : nullptr, &next))) return rc;
        const uint32_t stop = std::min(c.context_length, kv->cap);
        uint32_t n = 0;
        for (uint32_t it = 0; it < max_new; ++it) {
            if (host_sample) {
                for (uint32_t i = valid; i < V; ++i) logits[i] = -INFINITY;
                for (uint32_t q = 0; q < n; ++q) {
                    float &l = logits[out_ids[q]];
                    l = l > 0.0f ? l / rep_penalty : l * rep_penalty;
                }
                uint32_t best = 0;
                float bv = -INFINITY;
                for (uint32_t i = 0; i < V; ++i)
                    if (logits[i] > bv) { bv = logits[i]; best = i; }
                next = best;
            }
            if (next == eos) break;
            out_ids[n++] = next;
            if (pos + 1 >= stop) break;
            if ((rc = hg_forward(m, kv, next, pos, host_sample ? logits.data() : nullptr, &next))) {
                *n_out = n;
                return rc;
            }
            ++pos;
        }
        *n_out = n;
        return HG_OK;
    });
}

int hg_profile_step(const hg_model *m, hg_kv *kv, uint32_t token, uint32_t reps, float *us, uint32_t *launches) {
    return guard([&]() -> int {
        if (!m || !kv || kv->m != m || !us || !launches) return fail(HG_ERR_ARG, "NULL argument");
        if (kv->len >= kv->cap) return fail(HG_ERR_ARG, "the cache is full: no free position to replay a step at");
        if (token >= m->c.vocab_size) return fail(HG_ERR_ARG, "token out of range");
        for (int c = 0; c < P_COUNT; ++c) { us[c] = 0.0f; launches[c] = 0; }
        int rc;
        for (uint32_t r = 0; r < reps; ++r) {
            if ((rc = set_params(kv, token, kv->len, 0, 1, kv->len))) return rc;
            LaunchTimer timer;
            kv->timer = &timer;
            kv->win = window_of(kv->len + 1, kv->cap);
            set_launch_timer(&timer);
            enqueue_decode(kv);
            set_launch_timer(nullptr);
            kv->timer = nullptr;
            hipError_t e = hipStreamSynchronize(kv->st);
            for (size_t i = 0; e == hipSuccess && i < timer.ev.size(); ++i) {
                float ms = 0.0f;
                e = hipEventElapsedTime(&ms, timer.ev[i].first, timer.ev[i].second);
                us[timer.tags[i]] += ms * 1000.0f / reps;
                if (r == 0) launches[timer.tags[i]] += 1;
            }
            for (auto &pr : timer.ev) {
                (void)hipEventDestroy(pr.first);
                (void)hipEventDestroy(pr.second);
            }
            if (e != hipSuccess) return fail(HG_ERR_DEVICE, std::string("profile: ") + hipGetErrorString(e));
        }
        return HG_OK;
    });
}

const char *hg_profile_class(uint32_t c) { return c < P_COUNT ? kProfNames[c] : ""; }

int hg_last_routing(const hg_kv *kv, uint32_t *idx, float *w) {
    return guard([&]() -> int {
        if (!kv) return fail(HG_ERR_ARG, "NULL argument");
        const size_t n = (size_t)kv->m->c.n_layers * kv->m->c.top_k;
        HIP_TRY(hipStreamSynchronize(kv->st));
        if (idx) HIP_TRY(hipMemcpy(idx, kv->rec_idx.p, n * 4, hipMemcpyDeviceToHost));
        if (w) HIP_TRY(hipMemcpy(w, kv->rec_w.p, n * 4, hipMemcpyDeviceToHost));
        return HG_OK;
    });
}

}  // extern "C"

// ======================================================================= operator level
struct hg_q8_tensor {
    DevQ8 w;
    hipStream_t st = nullptr;
    ~hg_q8_tensor() {
        if (st) (void)hipStreamDestroy(st);
    }
};

namespace {

int make_tensor(PackedQ8 &p, hg_q8_tensor **t) {
    p.set_scale_storage(!p.f16_exact);
    auto q = std::make_unique<hg_q8_tensor>();
    int rc = q->w.upload(p);
    if (rc) return rc;
    HIP_TRY(hipStreamCreateWithFlags(&q->st, hipStreamNonBlocking));
    *t = q.release();
    return HG_OK;
}

// Quantize x (host) into device (qa, da); then run `body`.
template <class F>
int with_act(const hg_q8_tensor *t, const float *x, uint32_t rows, F body) {
    const Q8Mat &W = t->w.m;
    DevBuf dx, qa, da;
    int rc;
    if ((rc = dx.upload(x, (size_t)rows * W.K * 4))) return rc;
    if ((rc = qa.alloc((size_t)rows * W.nc * CHUNK_BYTES)) || (rc = da.alloc((size_t)rows * W.nc * 16))) return rc;
    for (uint32_t r = 0; r < rows; ++r)
        launch_quant_vec(t->st, dx.as<float>() + (size_t)r * W.K, W.K, qa.as<uint8_t>() + (size_t)r * W.nc * CHUNK_BYTES,
                         da.as<float>() + (size_t)r * W.nc * 4);
    return body(qa, da);
}

}  // namespace

extern "C" {

int hg_q8_tensor_quantize(const float *w, uint32_t out, uint32_t in, hg_q8_tensor **t) {
    return guard([&]() -> int {
        if (!w || !t) return fail(HG_ERR_ARG, "NULL argument");
        if (in % QK || !out || !in) return fail(HG_ERR_ARG, "Q8_0 needs in_ divisible by 32 (got " + std::to_string(in) + ")");
        int rc = check_device();
        if (rc) return rc;
        PackedQ8 p;
        pack_q8_from_f32(w, out, in, p);
        return make_tensor(p, t);
    });
}

int hg_q8_tensor_from_q8_0(const void *blocks, uint32_t out, uint32_t in, hg_q8_tensor **t) {
    return guard([&]() -> int {
        if (!blocks || !t) return fail(HG_ERR_ARG, "NULL argument");
        if (in % QK || !out || !in) return fail(HG_ERR_ARG, "Q8_0 needs in_ divisible by 32 (got " + std::to_string(in) + ")");
        int rc = check_device();
        if (rc) return rc;
        PackedQ8 p;
        pack_q8_from_q8_0(static_cast<const uint8_t *>(blocks), out, in, p);
        return make_tensor(p, t);
    });
}

void hg_q8_tensor_free(hg_q8_tensor *t) { delete t; }

uint64_t hg_q8_tensor_bytes(const hg_q8_tensor *t) { return t ? t->w.ref_bytes : 0; }

int hg_q8_tensor_matvec(const hg_q8_tensor *t, const float *x, float *y) {
    return guard([&]() -> int {
        if (!t || !x || !y) return fail(HG_ERR_ARG, "NULL argument");
        const Q8Mat &W = t->w.m;
        return with_act(t, x, 1, [&](DevBuf &qa, DevBuf &da) -> int {
            DevBuf dy;
            int rc = dy.alloc((size_t)W.N * 4);
            if (rc) return rc;
            launch_matvec(t->st, ORDER_DECODE, EPI_STORE, W, qa.as<uint8_t>(), da.as<float>(), dy.as<float>(), 64, 0,
                          nullptr, nullptr);
            HIP_TRY(hipGetLastError());
            HIP_TRY(hipMemcpyAsync(y, dy.p, (size_t)W.N * 4, hipMemcpyDeviceToHost, t->st));
            HIP_TRY(hipStreamSynchronize(t->st));
            return HG_OK;
        });
    });
}

int hg_q8_tensor_matvec_noalloc(const hg_q8_tensor *t, const float *x_dev, float *y_dev, void *stream) {
    return guard([&]() -> int {
        if (!t || !x_dev || !y_dev) return fail(HG_ERR_ARG, "NULL argument");
        const Q8Mat &W = t->w.m;
        if (W.K > NOALLOC_MAX_IN)
            return fail(HG_ERR_ARG, "in = " + std::to_string(W.K) + " exceeds the allocation-free matvec's maximum of " +
                                        std::to_string(NOALLOC_MAX_IN));
        void *sp = nullptr;
        int rc = scratch_ptr(&sp);
        if (rc) return rc;
        // [nc][128] activation chunks, then [nc][4] f32 scales: every byte the matvec reads is
        // written by the quantization of this call (blocks past in are zeroed), so the previous
        // call's contents never leak into this one
        uint8_t *qa = static_cast<uint8_t *>(sp);
        float *da = reinterpret_cast<float *>(qa + (size_t)W.nc * CHUNK_BYTES);
        hipStream_t st = static_cast<hipStream_t>(stream);
        (void)take_launch_error_reset();
        launch_quant_vec(st, x_dev, W.K, qa, da);
        launch_matvec(st, ORDER_DECODE, EPI_STORE, W, qa, da, y_dev, 64, 0, nullptr, nullptr);
        return check_launches("hg_q8_tensor_matvec_noalloc");
    });
}

int hg_q8_tensor_matmul(const hg_q8_tensor *t, const float *x, float *y, uint32_t tn) {
    return guard([&]() -> int {
        if (!t || !x || !y) return fail(HG_ERR_ARG, "NULL argument");
        if (tn == 0) return HG_OK;
        const Q8Mat &W = t->w.m;
        return with_act(t, x, tn, [&](DevBuf &qa, DevBuf &da) -> int {
            DevBuf dy;
            int rc = dy.alloc((size_t)W.N * tn * 4);
            if (rc) return rc;
            for (uint32_t r = 0; r < tn; ++r)
                launch_matvec(t->st, ORDER_PREFILL, EPI_STORE, W, qa.as<uint8_t>() + (size_t)r * W.nc * CHUNK_BYTES,
                              da.as<float>() + (size_t)r * W.nc * 4, dy.as<float>() + (size_t)r * W.N, 64, 0, nullptr,
                              nullptr);
            HIP_TRY(hipGetLastError());
            HIP_TRY(hipMemcpyAsync(y, dy.p, (size_t)W.N * tn * 4, hipMemcpyDeviceToHost, t->st));
            HIP_TRY(hipStreamSynchronize(t->st));
            return HG_OK;
        });
    });
}

int hg_q8_tensor_matvec_gather(const hg_q8_tensor *t, uint32_t rows_per_mat, const uint32_t *ids, uint32_t n_ids,
                               const float *x, float *y) {
    return guard([&]() -> int {
        if (!t || !ids || !x || !y) return fail(HG_ERR_ARG, "NULL argument");
        const Q8Mat &W = t->w.m;
        if (rows_per_mat == 0 || W.N % rows_per_mat) return fail(HG_ERR_ARG, "rows_per_mat does not divide the rows");
        const uint32_t n_mat = W.N / rows_per_mat;
        for (uint32_t i = 0; i < n_ids; ++i)
            if (ids[i] >= n_mat) return fail(HG_ERR_ARG, "expert id " + std::to_string(ids[i]) + " out of range");
        if (n_ids == 0) return HG_OK;
        return with_act(t, x, 1, [&](DevBuf &qa, DevBuf &da) -> int {
            DevBuf dy, did;
            int rc;
            if ((rc = dy.alloc((size_t)rows_per_mat * n_ids * 4)) || (rc = did.upload(ids, (size_t)n_ids * 4))) return rc;
            launch_matvec_gather(t->st, W, rows_per_mat, did.as<uint32_t>(), n_ids, qa.as<uint8_t>(), da.as<float>(),
                                 dy.as<float>());
            HIP_TRY(hipGetLastError());
            HIP_TRY(hipMemcpyAsync(y, dy.p, (size_t)rows_per_mat * n_ids * 4, hipMemcpyDeviceToHost, t->st));
            HIP_TRY(hipStreamSynchronize(t->st));
            return HG_OK;
        });
    });
}

namespace {
// Mean kernel microseconds of the launches a timer recorded (after the stream is drained).
int timer_mean_us(LaunchTimer &timer, float *us) {
    double tot = 0.0;
    hipError_t e = hipSuccess;
    for (size_t i = 0; e == hipSuccess && i < timer.ev.size(); ++i) {
        float ms = 0.0f;
        e = hipEventElapsedTime(&ms, timer.ev[i].first, timer.ev[i].second);
        tot += ms;
    }
    for (auto &pr : timer.ev) {
        (void)hipEventDestroy(pr.first);
        (void)hipEventDestroy(pr.second);
    }
    if (e != hipSuccess) return fail(HG_ERR_DEVICE, std::string("timing: ") + hipGetErrorString(e));
    *us = timer.ev.empty() ? 0.0f : (float)(tot * 1000.0 / timer.ev.size());
    return HG_OK;
}
}  // namespace

int hg_q8_tensor_time_matvec(const hg_q8_tensor *t, const float *x, uint32_t reps, uint32_t copies,
                             uint32_t rows_per_mat, const uint32_t *ids, uint32_t n_ids, float *us) {
    return guard([&]() -> int {
        if (!t || !x || !us || !reps || !copies) return fail(HG_ERR_ARG, "NULL argument or zero count");
        const Q8Mat &W = t->w.m;
        const bool gather = ids != nullptr;
        if (gather) {
            if (rows_per_mat == 0 || W.N % rows_per_mat || n_ids == 0) return fail(HG_ERR_ARG, "bad gather shape");
            for (uint32_t i = 0; i < n_ids; ++i)
                if (ids[i] >= W.N / rows_per_mat) return fail(HG_ERR_ARG, "expert id out of range");
        }
        const size_t qs_bytes = (size_t)W.N * W.nc * CHUNK_BYTES, sc_bytes = (size_t)W.N * W.nc * 4 * (W.sc_f32 ? 4 : 2);
        return with_act(t, x, 1, [&](DevBuf &qa, DevBuf &da) -> int {
            DevBuf dy, did, rep;
            int rc;
            const uint32_t rows = gather ? rows_per_mat * n_ids : W.N;
            if ((rc = dy.alloc((size_t)rows * 4))) return rc;
            if (gather && (rc = did.upload(ids, (size_t)n_ids * 4))) return rc;
            if (copies > 1) {   // replicas of the weights, each (qs, scales) 256-byte aligned
                const size_t one = (qs_bytes + 255) / 256 * 256 + (sc_bytes + 255) / 256 * 256;
                if ((rc = rep.alloc(one * copies))) return rc;
                for (uint32_t c = 0; c < copies; ++c) {
                    uint8_t *b = rep.as<uint8_t>() + one * c;
                    HIP_TRY(hipMemcpyAsync(b, W.qs, qs_bytes, hipMemcpyDeviceToDevice, t->st));
                    HIP_TRY(hipMemcpyAsync(b + (qs_bytes + 255) / 256 * 256, W.sc, sc_bytes, hipMemcpyDeviceToDevice, t->st));
                }
            }
            const size_t one = (qs_bytes + 255) / 256 * 256 + (sc_bytes + 255) / 256 * 256;
            auto view = [&](uint32_t c) {
                Q8Mat v = W;
                if (copies > 1) {
                    uint8_t *b = rep.as<uint8_t>() + one * c;
                    v.qs = b;
                    v.sc = b + (qs_bytes + 255) / 256 * 256;
                }
                return v;
            };
            auto call = [&](uint32_t r) {
                const Q8Mat v = view(r % copies);
                if (gather)
                    launch_matvec_gather(t->st, v, rows_per_mat, did.as<uint32_t>(), n_ids, qa.as<uint8_t>(), da.as<float>(),
                                         dy.as<float>());
                else
                    launch_matvec(t->st, ORDER_DECODE, EPI_STORE, v, qa.as<uint8_t>(), da.as<float>(), dy.as<float>(), 64, 0,
                                  nullptr, nullptr);
            };
            for (uint32_t r = 0; r < 3; ++r) call(r);   // warm-up
            HIP_TRY(hipStreamSynchronize(t->st));
            LaunchTimer timer;
            set_launch_timer(&timer);
            for (uint32_t r = 0; r < reps; ++r) call(r);
            set_launch_timer(nullptr);
            HIP_TRY(hipGetLastError());
            HIP_TRY(hipStreamSynchronize(t->st));
            return timer_mean_us(timer, us);
        });
    });
}

int hg_attention_decode(const float *q, const float *k, const float *v, const float *q_norm, const float *k_norm,
                        float eps, float theta, uint32_t rope_len, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                        uint32_t pos, float *kc, float *vc, float *out, uint32_t flags) {
    return guard([&]() -> int {
        if (!q || !k || !v || !q_norm || !k_norm || !kc || !vc || !out) return fail(HG_ERR_ARG, "NULL argument");
        if (hd != 32 && hd != 64 && hd != 128) return fail(HG_ERR_UNSUPPORTED, "head_dim not in {32, 64, 128}");
        if (!n_kv || n_heads % n_kv || n_heads / n_kv > 8) return fail(HG_ERR_UNSUPPORTED, "unsupported head grouping");
        if (pos >= rope_len) return fail(HG_ERR_ARG, "pos beyond the RoPE table");
        if (!(flags & HG_KV_FAST) && pv_ring_slots(pos + 1) < 2)
            return fail(HG_ERR_UNSUPPORTED, "reference-order attention supports at most 32768 positions");
        int rc = check_device();
        if (rc) return rc;
        const bool exact = (flags & HG_KV_FAST) == 0;
        const uint32_t qd = n_heads * hd, kvd = n_kv * hd, n = pos + 1, cap = n, S = attn_splits(cap);
        std::vector<float> qkv(qd + 2 * kvd);
        memcpy(qkv.data(), q, qd * 4);
        memcpy(qkv.data() + qd, k, kvd * 4);
        memcpy(qkv.data() + qd + kvd, v, kvd * 4);
        std::vector<float> kh((size_t)n_kv * cap * hd, 0.0f), vh(v_layer_floats(cap, n_kv, hd), 0.0f);
        float *vth = vh.data() + (size_t)n_kv * cap * hd;   // the transposed copy
        for (uint32_t t = 0; t < pos; ++t)
            for (uint32_t g = 0; g < n_kv; ++g) {
                memcpy(&kh[((size_t)g * cap + t) * hd], kc + ((size_t)t * n_kv + g) * hd, hd * 4);
                memcpy(&vh[((size_t)g * cap + t) * hd], vc + ((size_t)t * n_kv + g) * hd, hd * 4);
                for (uint32_t i = 0; i < hd; ++i)
                    vth[((size_t)g * hd + i) * vt_stride(cap) + t] = vc[((size_t)t * n_kv + g) * hd + i];
            }
        std::vector<float> cs, sn;
        rope_table(hd, rope_len, theta, cs, sn);
        StepParams hp{};
        hp.pos = pos;
        DevBuf dqkv, dqn, dkn, dcs, dsn, dk, dv, dp, dpart, dscr, dout, dq, dd;
        if ((rc = dqkv.upload(qkv.data(), qkv.size() * 4)) || (rc = dqn.upload(q_norm, hd * 4)) ||
            (rc = dkn.upload(k_norm, hd * 4)) || (rc = dcs.upload(cs.data(), cs.size() * 4)) ||
            (rc = dsn.upload(sn.data(), sn.size() * 4)) || (rc = dk.upload(kh.data(), kh.size() * 4)) ||
            (rc = dv.upload(vh.data(), vh.size() * 4)) || (rc = dp.upload(&hp, sizeof hp)) ||
            (rc = dpart.alloc((size_t)n_heads * S * (hd + 2) * 4)) || (rc = dscr.alloc((size_t)n_heads * cap * 4)) ||
            (rc = dout.alloc((size_t)qd * 4)) || (rc = dq.alloc((size_t)div_up(qd / QK, 4) * CHUNK_BYTES)) ||
            (rc = dd.alloc((size_t)div_up(qd / QK, 4) * 16)))
            return rc;
        if (!launch_qk_rope_append(nullptr, hd, dqkv.as<float>(), dqn.as<float>(), dkn.as<float>(), eps, dcs.as<float>(),
                                   dsn.as<float>(), dp.as<StepParams>(), n_heads, n_kv, dk.as<float>(), dv.as<float>(), cap))
            return fail(HG_ERR_UNSUPPORTED, "head_dim not supported");
        for (int which = 0; which < 2; ++which)
            if (!launch_attn(nullptr, exact, which, hd, dqkv.as<float>(), dqn.as<float>(), dkn.as<float>(), eps,
                             dcs.as<float>(), dsn.as<float>(), dp.as<StepParams>(), dk.as<float>(), dv.as<float>(), cap,
                             cap, n_heads, n_kv, S, dpart.as<float>(), dscr.as<float>(), dout.as<float>(),
                             dq.as<uint8_t>(), dd.as<float>()))
                return fail(HG_ERR_UNSUPPORTED, "head_dim not supported");
        HIP_TRY(hipGetLastError());
        HIP_TRY(hipDeviceSynchronize());
        StepParams back{};
        HIP_TRY(hipMemcpy(&back, dp.p, sizeof back, hipMemcpyDeviceToHost));
        if (back.err) return fail(HG_ERR_DEVICE, "a softmax/P.V kernel's wait ran out of polls");
        HIP_TRY(hipMemcpy(out, dout.p, (size_t)qd * 4, hipMemcpyDeviceToHost));
        HIP_TRY(hipMemcpy(kh.data(), dk.p, kh.size() * 4, hipMemcpyDeviceToHost));
        HIP_TRY(hipMemcpy(vh.data(), dv.p, vh.size() * 4, hipMemcpyDeviceToHost));
        for (uint32_t g = 0; g < n_kv; ++g) {
            memcpy(kc + ((size_t)pos * n_kv + g) * hd, &kh[((size_t)g * cap + pos) * hd], hd * 4);
            memcpy(vc + ((size_t)pos * n_kv + g) * hd, &vh[((size_t)g * cap + pos) * hd], hd * 4);
        }
        return HG_OK;
    });
}

int hg_seq_sum(const float *x, uint32_t n, uint32_t method, float *out) {
    return guard([&]() -> int {
        if ((!x && n) || !out || method > 7) return fail(HG_ERR_ARG, "NULL argument or unknown method");
        int rc = check_device();
        if (rc) return rc;
        DevBuf dx, dout;
        if ((rc = dx.upload(x, (size_t)n * 4)) || (rc = dout.alloc(4))) return rc;
        launch_seq_sum(nullptr, dx.as<float>(), n, (int)method, dout.as<float>());
        HIP_TRY(hipGetLastError());
        HIP_TRY(hipDeviceSynchronize());
        HIP_TRY(hipMemcpy(out, dout.p, 4, hipMemcpyDeviceToHost));
        return HG_OK;
    });
}

int hg_attention_time(uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t ctx, uint32_t reps, uint32_t flags,
                      float *us) {
    return guard([&]() -> int {
        if (!us || !reps || !ctx) return fail(HG_ERR_ARG, "NULL argument or zero count");
        if (hd != 32 && hd != 64 && hd != 128) return fail(HG_ERR_UNSUPPORTED, "head_dim not in {32, 64, 128}");
        if (!n_kv || n_heads % n_kv || n_heads / n_kv > 8) return fail(HG_ERR_UNSUPPORTED, "unsupported head grouping");
        const bool exact = (flags & HG_KV_FAST) == 0;
        if (exact && !pv_res_fits(ctx) && pv_ring_slots(ctx) < 2)
            return fail(HG_ERR_UNSUPPORTED, "reference-order attention supports at most 32768 positions");
        int rc = check_device();
        if (rc) return rc;
        const uint32_t qd = n_heads * hd, kvd = n_kv * hd, cap = ctx, S = attn_splits(ctx), pos = ctx - 1;
        // seeded N(0,1)-like data: q, k, v and the cache rows 0 .. pos-1; unit QK-norm gains
        uint64_t st = 0x9e3779b97f4a7c15ull;
        auto rnd = [&]() {
            st ^= st << 13; st ^= st >> 7; st ^= st << 17;
            return (float)((double)(st >> 11) * 0x1p-53 * 2.0 - 1.0) * 1.7320508f;
        };
        std::vector<float> qkv(qd + 2 * kvd), kh((size_t)n_kv * cap * hd), vh(v_layer_floats(cap, n_kv, hd)),
            ones(hd, 1.0f), cs, sn;   // (vh: the rows and their transposed copy, random alike: timing only)
        for (float &v : qkv) v = rnd();
        for (float &v : kh) v = rnd();
        for (float &v : vh) v = rnd();
        rope_table(hd, ctx, 10000.0f, cs, sn);
        StepParams hp{};
        hp.pos = pos;
        DevBuf dqkv, dqn, dcs, dsn, dk, dv, dp, dpart, dscr, dout, dq, dd;
        const size_t part_floats = exact ? (size_t)n_heads * S : (size_t)n_heads * S * (hd + 2);
        // the fast path's merge also writes the quantized o (the exact path leaves it to attn_output)
        if ((rc = dq.alloc((size_t)div_up(qd / QK, 4) * CHUNK_BYTES)) || (rc = dd.alloc((size_t)div_up(qd / QK, 4) * 16)))
            return rc;
        uint8_t *q_out = exact ? nullptr : dq.as<uint8_t>();
        float *d_out = exact ? nullptr : dd.as<float>();
        if ((rc = dqkv.upload(qkv.data(), qkv.size() * 4)) || (rc = dqn.upload(ones.data(), hd * 4)) ||
            (rc = dcs.upload(cs.data(), cs.size() * 4)) || (rc = dsn.upload(sn.data(), sn.size() * 4)) ||
            (rc = dk.upload(kh.data(), kh.size() * 4)) || (rc = dv.upload(vh.data(), vh.size() * 4)) ||
            (rc = dp.upload(&hp, sizeof hp)) || (rc = dpart.alloc(std::max(part_floats, (size_t)n_heads * S * (hd + 2)) * 4)) ||
            (rc = dscr.alloc((size_t)n_heads * cap * 4)) || (rc = dout.alloc((size_t)qd * 4)))
            return rc;
        HIP_TRY(hipDeviceSynchronize());
        hipStream_t s0 = nullptr;
        HIP_TRY(hipStreamCreateWithFlags(&s0, hipStreamNonBlocking));
        auto layer = [&]() {
            for (int which = 0; which < 2; ++which)
                launch_attn(s0, exact, which, hd, dqkv.as<float>(), dqn.as<float>(), dqn.as<float>(), 1e-5f,
                            dcs.as<float>(), dsn.as<float>(), dp.as<StepParams>(), dk.as<float>(), dv.as<float>(), cap,
                            cap, n_heads, n_kv, S, dpart.as<float>(), dscr.as<float>(), dout.as<float>(), q_out, d_out);
        };
        // q, k normed and rotated and the row pos appended once (the QKV step's work, not timed)
        launch_qk_rope_append(s0, hd, dqkv.as<float>(), dqn.as<float>(), dqn.as<float>(), 1e-5f, dcs.as<float>(),
                              dsn.as<float>(), dp.as<StepParams>(), n_heads, n_kv, dk.as<float>(), dv.as<float>(), cap);
        for (int r = 0; r < 3; ++r) layer();
        hipError_t e = hipStreamSynchronize(s0);
        LaunchTimer timer;
        if (e == hipSuccess) {
            set_launch_timer(&timer);
            for (uint32_t r = 0; r < reps; ++r) {
                timer.cls = 0;
                launch_attn(s0, exact, 0, hd, dqkv.as<float>(), dqn.as<float>(), dqn.as<float>(), 1e-5f, dcs.as<float>(),
                            dsn.as<float>(), dp.as<StepParams>(), dk.as<float>(), dv.as<float>(), cap, cap, n_heads, n_kv,
                            S, dpart.as<float>(), dscr.as<float>(), dout.as<float>(), q_out, d_out);
                timer.cls = 1;
                launch_attn(s0, exact, 1, hd, dqkv.as<float>(), dqn.as<float>(), dqn.as<float>(), 1e-5f, dcs.as<float>(),
                            dsn.as<float>(), dp.as<StepParams>(), dk.as<float>(), dv.as<float>(), cap, cap, n_heads, n_kv,
                            S, dpart.as<float>(), dscr.as<float>(), dout.as<float>(), q_out, d_out);
            }
            set_launch_timer(nullptr);
            e = hipStreamSynchronize(s0);
        }
        double t[2] = {0.0, 0.0};
        for (size_t i = 0; e == hipSuccess && i < timer.ev.size(); ++i) {
            float ms = 0.0f;
            e = hipEventElapsedTime(&ms, timer.ev[i].first, timer.ev[i].second);
            t[timer.tags[i] ? 1 : 0] += ms;
        }
        for (auto &pr : timer.ev) {
            (void)hipEventDestroy(pr.first);
            (void)hipEventDestroy(pr.second);
        }
        (void)hipStreamDestroy(s0);
        if (e != hipSuccess) return fail(HG_ERR_DEVICE, std::string("attention timing: ") + hipGetErrorString(e));
        us[0] = (float)(t[0] * 1000.0 / reps);
        us[1] = (float)(t[1] * 1000.0 / reps);
        return HG_OK;
    });
}

int hg_kv_truncate(hg_kv *kv, uint32_t len) {
    return guard([&]() -> int {
        if (!kv) return fail(HG_ERR_ARG, "NULL argument");
        if (len > kv->len) return fail(HG_ERR_ARG, "truncate can only shorten the cache");
        kv->len = len;
        return HG_OK;
    });
}

}  // extern "C"
