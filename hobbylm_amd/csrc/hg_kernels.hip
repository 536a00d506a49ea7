// hg_kernels.hip -- gfx950 kernels of the hobbylm single-sequence decode step.
//
// Every kernel restates one piece of hobby-rs's arithmetic (file:line given at each) in the
// same floating-point operation order, except where a comment says "tree": those
// reductions (RMSNorm sum of squares and attention softmax / P.V in the fast path) are
// reassociated.  The build uses -ffp-contract=off; each fmaf() stands where the reference
// issues an FMA.  Wavefronts are 64 wide; a Q8 row is owned by 8 adjacent lanes (see
// hg_common.h for the device row layout).
#include <hip/hip_ext.h>

#include <algorithm>

#include "hg_common.h"
#include "hg_device.h"
#include "hg_expf.h"
#include "hg_kernels.h"

namespace hg {

// Test entry: one workgroup sums x[0..n) (n <= 4096, method 7: n <= 16384, in LDS; larger n:
// one lane over global memory) with the layouts the decode kernels use: method 1: 8 waves x 4
// terms per lane, 2: 4 waves x 4 (waves 0..3), 3: 4 waves x 4 (waves 0, 5, 6, 7), 4: 2 waves x
// 8, 5: 4 waves x 8, 6: 4 waves x 12, 7: 8 waves x 32; method 0: one lane.
constexpr uint32_t SEQSUM_MAX = 16384;
__global__ __launch_bounds__(512) void k_seq_sum(const float *__restrict__ x, uint32_t n, int method, float *out) {
    extern __shared__ __align__(16) float a[];   // SEQSUM_MAX floats (+4)
    __shared__ xsum::Scratch L;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t cap = method == 7 ? SEQSUM_MAX : 4096;
    if (n > cap) {
        if (tid == 0) {
            float s = 0.0f;
            for (uint32_t i = 0; i < n; ++i) s = s + x[i];
            *out = s;
        }
        return;
    }
    for (uint32_t i = tid; i < cap + 4; i += 512) a[i] = i < n ? x[i] : 0.0f;
    if (tid == 0) L.sync = 0;
    __syncthreads();
    float r = 0.0f;
    switch (method) {
    case 1: r = block_seq_sum<8, 4>(a, n, L, wave, lane); break;
    case 2:
        if (wave < 4) r = block_seq_sum<4, 4>(a, n, L, wave, lane);
        break;
    case 3:
        if (wave == 0 || wave >= 5) r = block_seq_sum<4, 4>(a, n, L, wave == 0 ? 0 : wave - 4, lane);
        break;
    case 4:
        if (wave < 2) r = block_seq_sum<2, 8>(a, n, L, wave, lane);
        break;
    case 5:
        if (wave < 4) r = block_seq_sum<4, 8>(a, n, L, wave, lane);
        break;
    case 6:
        if (wave < 4) r = block_seq_sum<4, 12>(a, n, L, wave, lane);
        break;
    case 7: r = block_seq_sum<8, 32>(a, n, L, wave, lane); break;
    default:
        if (tid == 0) r = seq_sum_lds(a, n, 0.0f);
    }
    if (tid == 0) *out = r;
}

// ------------------------------------------------------------------ embedding
// Model::forward (model.rs:154): x = token_embd[token] (F32 table, dequantized at load).
__global__ void k_embed(const float *__restrict__ emb, uint32_t d, const StepParams *p, float *x) {
    if (!p->embed) return;
    const float *row = emb + (size_t)p->token * d;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x) x[i] = row[i];
}

// Prefill: x = inputs[pos - base].
__global__ void k_load_row(const float *__restrict__ inputs, uint32_t d, const StepParams *p, float *x) {
    const float *row = inputs + (size_t)(p->pos - p->base) * d;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x) x[i] = row[i];
}

__global__ void k_advance(StepParams *p) {
    if (threadIdx.x == 0) p->pos += 1;
}

// ------------------------------------------------------------------ RMSNorm + quantize
// rmsnorm (ops.rs:85-96): ss = sum x^2; scale = 1/sqrt(ss/n + eps); h = x*scale*w; then
// the activation quantization of the consuming matvec (quant.rs:111-123).
// EXACT: the squares are formed in parallel and summed in index order (the reference's
// `ss += v * v`) by block_seq_sum; otherwise a tree.
template <bool EXACT>
__global__ __launch_bounds__(256) void k_rmsnorm_quant(const float *__restrict__ x, const float *__restrict__ w,
                                                       float eps, uint32_t d, float *h_out, uint8_t *q_out,
                                                       float *d_out, RowStrides rs) {
    extern __shared__ __align__(16) float ps[];  // d squares
    x += (size_t)blockIdx.x * rs.x;   // row blockIdx.x of a batched launch
    if (h_out) h_out += (size_t)blockIdx.x * rs.x;
    q_out += (size_t)blockIdx.x * rs.q;
    d_out += (size_t)blockIdx.x * rs.d;
    __shared__ float red[4];
    __shared__ float s_ss;
    __shared__ xsum::Scratch xs;
    const int tid = threadIdx.x, j = tid & 7;
    const uint32_t nb = d / QK, nc = div_up(nb, 4), ng = d / 4;
    // thread tid owns the float4 groups g = tid + 256 u: elements 4g..4g+3, i.e. lane j of
    // quantization block g / 8.  x and the gain of the first RQ groups are fetched up front.
    constexpr uint32_t RQ = 4;
    v4f xv[RQ], wv[RQ];
#pragma unroll
    for (uint32_t u = 0; u < RQ; ++u) {
        const uint32_t g = min(tid + 256 * u, ng - 1);
        xv[u] = reinterpret_cast<const v4f *>(x)[g];
        wv[u] = reinterpret_cast<const v4f *>(w)[g];
    }
    float ss = 0.0f;
    auto squares = [&](const v4f a, uint32_t g) {
        if (EXACT) {
            reinterpret_cast<v4f *>(ps)[g] = a * a;
        } else {
            ss += a.x * a.x;
            ss += a.y * a.y;
            ss += a.z * a.z;
            ss += a.w * a.w;
        }
    };
#pragma unroll
    for (uint32_t u = 0; u < RQ; ++u)
        if (tid + 256 * u < ng) squares(xv[u], tid + 256 * u);
    for (uint32_t g = tid + 256 * RQ; g < ng; g += 256) squares(reinterpret_cast<const v4f *>(x)[g], g);
    if (EXACT) {
        if (tid == 0) xs.sync = 0;
        __syncthreads();
        const float r = block_seq_sum<4, 4>(ps, d, xs, tid >> 6, tid & 63);   // ss += v * v in index order
        if (tid == 0) s_ss = r;
    } else {
        for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        if (tid == 0) s_ss = (red[0] + red[1]) + (red[2] + red[3]);
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf(s_ss / (float)d + eps);
    auto emit = [&](const v4f a, const v4f gw, uint32_t g) {
        const float v[4] = {a.x * scale * gw.x, a.y * scale * gw.y, a.z * scale * gw.z, a.w * scale * gw.w};
        if (h_out) reinterpret_cast<v4f *>(h_out)[g] = v4f{v[0], v[1], v[2], v[3]};
        quant_block_lane(v, j, g / 8, q_out, d_out);
    };
#pragma unroll
    for (uint32_t u = 0; u < RQ; ++u)   // a block's 8 groups are all < ng or all >= ng
        if (tid + 256 * u < ng) emit(xv[u], wv[u], tid + 256 * u);
    for (uint32_t g = tid + 256 * RQ; g < ng; g += 256)
        emit(reinterpret_cast<const v4f *>(x)[g], reinterpret_cast<const v4f *>(w)[g], g);
    zero_pad(nb, nc, q_out, d_out, tid, 256);
}

// Quantize a plain f32 vector (the activation of Q8Tensor::matvec, quant.rs:111-123).
__global__ __launch_bounds__(256) void k_quant_vec(const float *__restrict__ x, uint32_t n, uint8_t *q_out,
                                                   float *d_out) {
    const int tid = threadIdx.x, j = tid & 7;
    const uint32_t nb = n / QK, nc = div_up(nb, 4);
    for (uint32_t b0 = blockIdx.x * 32; b0 < nb; b0 += gridDim.x * 32) {
        const uint32_t b = b0 + (tid >> 3);
        if (b < nb) {
            float v[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) v[m] = x[b * QK + j * 4 + m];
            quant_block_lane(v, j, b, q_out, d_out);
        }
    }
    if (blockIdx.x == 0) zero_pad(nb, nc, q_out, d_out, tid, 256);
}

// ------------------------------------------------------------------ Q8 matvec
// Q8Tensor::matvec / matmul row loop (quant.rs:125-135, 168-185) over a pre-quantized
// activation.  8 lanes per row; blockDim.x/8 rows per workgroup.  The weight stream of
// each row is started before the activation is staged into LDS.
//   EPI_STORE:  y[r] = v
//   EPI_RESID:  y[r] = y[r] + v     (x[i] += attn[i], model.rs:169-171)
//   EPI_LOGITS: y[r] = v, plus a per-workgroup (max, first index) over rows < valid for
//               the greedy argmax (sample.rs:53-63 on logits masked per lib.rs:132-134).
template <int ORDER, int EPI, bool SCF32, int NCT, bool AF32 = false>
__global__ __launch_bounds__(256) void k_matvec(Q8Mat W, const uint8_t *__restrict__ gq,
                                                const float *__restrict__ gd, float *y, uint32_t valid,
                                                float *part_v, uint32_t *part_i) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *sq = smem;
    float *sd = reinterpret_cast<float *>(smem + W.nc * CHUNK_BYTES);
    const int tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t row = blockIdx.x * (nthr >> 3) + (tid >> 3);
    const uint32_t lrow = min(row, W.N - 1);
    const int j = tid & 7;
    // the activation's loads are issued before the weight stream (the memory counter retires
    // in order, so the wait for the activation then leaves the weights in flight); the first
    // XQ rounds are held in registers, larger activations finish with a loop
    constexpr uint32_t XQ = 4;
    const uint32_t bstep = (uint32_t)nthr / 8, nb = W.nb, nc = W.nc;
    v4f xv[XQ];
    v4i qv[XQ];
    float dv = 0.0f;
    const float *xf = reinterpret_cast<const float *>(gq);
#pragma unroll
    for (uint32_t u = 0; u < XQ; ++u) {
        if (AF32) {
            const uint32_t b = min(u * bstep + (uint32_t)(tid >> 3), nb - 1);
            xv[u] = *reinterpret_cast<const v4f *>(xf + b * QK + j * 4);
        } else {
            const uint32_t i = min(u * (uint32_t)nthr + (uint32_t)tid, nc * 8 - 1);
            qv[u] = reinterpret_cast<const v4i *>(gq)[i];
        }
    }
    if (!AF32) dv = gd[min((uint32_t)tid, nc * 4 - 1)];
    const float yold = (EPI == EPI_RESID) ? y[min(row, W.N - 1)] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
    Q8Row<ORDER, SCF32, NCT> rd;
    rd.begin(row_qs(W, lrow), row_sc<SCF32>(W, lrow), nb, nc, j);
    __builtin_amdgcn_sched_barrier(0);
    if (AF32) {
#pragma unroll
        for (uint32_t u = 0; u < XQ; ++u) {   // a block's 8 lanes are all in or all out
            const uint32_t b = u * bstep + (uint32_t)(tid >> 3);
            const float v4[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
            quant_block_lane(v4, j, min(b, nb - 1), sq, sd, b < nb);
        }
        for (uint32_t b0 = XQ * bstep; b0 < nb; b0 += bstep) {
            const uint32_t b = b0 + (uint32_t)(tid >> 3);
            if (b < nb) {
                const v4f x4 = *reinterpret_cast<const v4f *>(xf + b * QK + j * 4);
                const float v4[4] = {x4.x, x4.y, x4.z, x4.w};
                quant_block_lane(v4, j, b, sq, sd);
            }
        }
        zero_pad(nb, nc, sq, sd, tid, nthr);
    } else {
#pragma unroll
        for (uint32_t u = 0; u < XQ; ++u)   // (clamped slots rewrite the value they already hold)
            reinterpret_cast<v4i *>(sq)[min(u * (uint32_t)nthr + (uint32_t)tid, nc * 8 - 1)] = qv[u];
        for (uint32_t i = XQ * (uint32_t)nthr + (uint32_t)tid; i < nc * 8; i += nthr)
            reinterpret_cast<v4i *>(sq)[i] = reinterpret_cast<const v4i *>(gq)[i];
        sd[min((uint32_t)tid, nc * 4 - 1)] = dv;
        for (uint32_t i = (uint32_t)tid + nthr; i < nc * 4; i += nthr) sd[i] = gd[i];
    }
    __syncthreads();
    const float v = rd.finish(sq, sd);
    if (row < W.N && j == 0) {
        if (EPI == EPI_RESID) y[row] = yold + v;
        else y[row] = v;
    }
    if (EPI == EPI_LOGITS) {
        __shared__ float bv[32];
        __shared__ uint32_t bi[32];
        float mv = -__builtin_huge_valf();
        uint32_t mi = 0xffffffffu;
        if (j == 0 && row < W.N && row < valid && v > mv) { mv = v; mi = row; }
        // wave reduce: larger value wins, equal values keep the lower row
        for (int m = 8; m < 64; m <<= 1) {
            const float ov = shfl_xor(mv, m);
            const uint32_t oi = (uint32_t)shfl_xor_i((int)mi, m);
            if (ov > mv || (ov == mv && oi < mi)) { mv = ov; mi = oi; }
        }
        if ((tid & 63) == 0) { bv[tid >> 6] = mv; bi[tid >> 6] = mi; }
        __syncthreads();
        if (tid == 0) {
            for (int wv = 1; wv < (nthr >> 6); ++wv)
                if (bv[wv] > mv || (bv[wv] == mv && bi[wv] < mi)) { mv = bv[wv]; mi = bi[wv]; }
            part_v[blockIdx.x] = mv;
            part_i[blockIdx.x] = mi;
        }
    }
}

// Q8Tensor::matvec of the matrices ids[0..n) of a stack of equal matrices (rows_per_mat rows
// each; the expert matvecs of model.rs:301-318 at the operator level), one launch:
// blockIdx.y = position in ids, y[blockIdx.y * rows_per_mat + r].  Same row order as k_matvec.
template <bool SCF32, int NCT>
__global__ __launch_bounds__(256) void k_matvec_gather(Q8Mat W, uint32_t rows_per_mat, const uint32_t *__restrict__ ids,
                                                       const uint8_t *__restrict__ gq, const float *__restrict__ gd,
                                                       float *y) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *sq = smem;
    float *sd = reinterpret_cast<float *>(smem + W.nc * CHUNK_BYTES);
    const int tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t r = blockIdx.x * (nthr >> 3) + (tid >> 3), lr = min(r, rows_per_mat - 1);
    const uint32_t row = ids[blockIdx.y] * rows_per_mat + lr;
    const int j = tid & 7;
    Q8Row<ORDER_DECODE, SCF32, NCT> rd;
    rd.begin(row_qs(W, row), row_sc<SCF32>(W, row), W.nb, W.nc, j);
    stage_act(gq, gd, W.nc, sq, sd, tid, nthr);
    __syncthreads();
    const float v = rd.finish(sq, sd);
    if (r < rows_per_mat && j == 0) y[(size_t)blockIdx.y * rows_per_mat + r] = v;
}

// Final greedy argmax over the per-workgroup partials; writes out_ids[step] and, in
// feedback mode, chains the next step (token = next, pos += 1).
__global__ __launch_bounds__(1024) void k_argmax_final(const float *__restrict__ pv, const uint32_t *__restrict__ pi,
                                                       uint32_t n, StepParams *p, uint32_t *out_ids) {
    __shared__ float bv[16];
    __shared__ uint32_t bi[16];
    const int tid = threadIdx.x;
    float mv = -__builtin_huge_valf();
    uint32_t mi = 0xffffffffu;
    for (uint32_t i = tid; i < n; i += 1024) {
        const float v = pv[i];
        const uint32_t ix = pi[i];
        if (ix != 0xffffffffu && (v > mv || (v == mv && ix < mi))) { mv = v; mi = ix; }
    }
    for (int m = 1; m < 64; m <<= 1) {
        const float ov = shfl_xor(mv, m);
        const uint32_t oi = (uint32_t)shfl_xor_i((int)mi, m);
        if (ov > mv || (ov == mv && oi < mi)) { mv = ov; mi = oi; }
    }
    if ((tid & 63) == 0) { bv[tid >> 6] = mv; bi[tid >> 6] = mi; }
    __syncthreads();
    if (tid == 0) {
        for (int wv = 1; wv < 16; ++wv)
            if (bv[wv] > mv || (bv[wv] == mv && bi[wv] < mi)) { mv = bv[wv]; mi = bi[wv]; }
        // sample::argmax returns 0 when no logit exceeds -inf
        const uint32_t next = (mi == 0xffffffffu) ? 0u : mi;
        out_ids[p->step] = next;
        p->step += 1;
        if (p->feedback) {
            p->token = next;
            p->pos += 1;
        }
    }
}

// The group's q heads, k and v as the QKV matvec produced them ((rep + 2) * HD floats),
// fetched into registers (issue first, store to LDS `raw` later).
template <int HD, int MAXREP>
struct GroupRaw {
    static constexpr uint32_t N = ((MAXREP + 2) * HD + 255) / 256;
    float v[N];
    __device__ inline void load(const float *__restrict__ qkv, uint32_t g, uint32_t rep, uint32_t qd, uint32_t kvd,
                                int tid) {
        const uint32_t nraw = (rep + 2) * HD;
#pragma unroll
        for (uint32_t u = 0; u < N; ++u) {
            const uint32_t i = min(tid + 256 * u, nraw - 1);
            const uint32_t src = i < rep * HD         ? g * rep * HD + i
                                 : i < (rep + 1) * HD ? qd + g * HD + (i - rep * HD)
                                                      : qd + kvd + g * HD + (i - (rep + 1) * HD);
            v[u] = qkv[src];
        }
    }
    __device__ inline void store(float *raw, uint32_t rep, int tid) const {
#pragma unroll
        for (uint32_t u = 0; u < N; ++u)
            if (tid + 256 * u < (rep + 2) * HD) raw[tid + 256 * u] = v[u];
    }
};

// ------------------------------------------------------------------ attention front
// attn_norm + attn_qkv + QK-norm + RoPE + cache append for one head (model.rs:164-165,
// 194-211): rmsnorm (ops.rs:98-109) of x with gain w and its activation quantization
// (quant.rs:111-123), the head's HD rows of the Q8 matvec (quant.rs:125-135), then for a q or
// k head norm_head (model.rs:753-763) and Rope::apply (ops.rs:155-166), and for k and v the
// append of row pos to the caches.  Workgroup hh: q head hh (hh < n_heads), k head
// hh - n_heads, or v head hh - n_heads - n_kv (the rows of W are q | k | v, so rows
// hh*HD .. hh*HD + HD - 1).  Every workgroup forms the norm of the whole x itself, in the
// reference's order; a separate chain wave (HD <= 64) runs it while the row waves fetch their
// weights.  Writes q, k (normed and rotated) and v into out (the q | k | v layout).
// SC (reference order, HD = 64): the attention scores join this launch.  Workgroups
// 0 .. n_heads S2 - 1 each form one q head and the scores s[h][t] = dot(q_h, K_t) / sqrt(HD)
// (model.rs:213-218, ops::dot's order) of split s of the window (positions [s c, s c + c),
// c = ceil(win / S2) <= 256, one position per row thread, the split's K rows fetched into LDS
// behind the weights), for t < pos only, and the split's maximum into pmax[h S2 + s]; the
// score at pos needs this step's k, so the softmax + P.V kernel forms it.  Placement: the rep
// heads of one (kv group, split) share an XCD (one L2 for their K rows) and each kv group's
// splits stay on 8 / n_kv XCDs (its q weights reach that many L2s).  The k and v workgroups
// follow.  Every q head is formed alike by its S2 workgroups; split 0's writes it to out.
template <int HD> struct QkvCfg {
    static constexpr int CW = HD <= 64 ? 64 : 0;   // wave 0: the head's epilogue
    static constexpr int RE = CW + 8 * HD;         // + 8 lanes per row
    static constexpr int SW = HD <= 64 ? 192 : 0;  // + waves that only sum (no weight loads)
    static constexpr int NT = RE + SW;
};
template <bool EXACT, int ORDER, bool SCF32, int NCT, int HD, bool SC = false>
__global__ __launch_bounds__(QkvCfg<HD>::NT) void k_qkv_head(Q8Mat W, const float *__restrict__ x,
                                                            const float *__restrict__ w, float eps,
                                                            const float *__restrict__ qn, const float *__restrict__ kn,
                                                            const float *__restrict__ cs, const float *__restrict__ sn,
                                                            const StepParams *p, uint32_t n_heads, uint32_t n_kv,
                                                            float *kc, float *vc, uint32_t cap, float *out,
                                                            uint32_t win, uint32_t S2, float *scores, float *pmax) {
    constexpr int CW = QkvCfg<HD>::CW, RE = QkvCfg<HD>::RE, NT = QkvCfg<HD>::NT;
    static_assert(!SC || (EXACT && HD == 64), "scores join the exact head-64 launch only");
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *sq = smem;
    float *sd = reinterpret_cast<float *>(smem + W.nc * CHUNK_BYTES);
    float *ps = sd + W.nc * 4;   // the d squares
    __shared__ __align__(16) float hv[HD], ho[HD], tmp[HD];
    __shared__ float red[NT / 64];
    __shared__ float s_ss;
    __shared__ xsum::Scratch xs;
    const int tid = threadIdx.x, lane = tid & 63, j = tid & 7;
    const bool rowt = tid >= CW && tid < RE;
    uint32_t hh = blockIdx.x, spl = 0;   // head, split (SC)
    if constexpr (SC) {
        const uint32_t nsc = n_heads * S2, rep = n_heads / n_kv, L = blockIdx.x;
        if (L < nsc) {
            uint32_t key, r;
            const uint32_t xq = n_kv && n_kv <= 8 && 8 % n_kv == 0 ? 8 / n_kv : 0;   // XCDs per kv group
            if (xq && S2 % xq == 0) {
                // XCD x serves kv group x / xq, splits x % xq, + xq, ...: each q head's weights
                // reach xq L2s, each split's K rows one
                const uint32_t x = L % 8, loc = L / 8, gg = x / xq;
                r = loc % rep;
                key = gg * S2 + (loc / rep) * xq + x % xq;
            } else if ((n_kv * S2) % 8 == 0) {
                const uint32_t slot = L / 8;
                key = L % 8 + 8 * (slot / rep);
                r = slot % rep;
            } else {
                key = L / rep;
                r = L % rep;
            }
            hh = (key / S2) * rep + r;
            spl = key % S2;
        } else {
            hh = n_heads + (L - nsc);
        }
    }
    const uint32_t d = W.K, ng = d / 4;
    // the waves of the index-order sum: wave 0 and the waves past the rows (or, without those,
    // the first four waves)
    const int wave = tid >> 6,
              sp = QkvCfg<HD>::SW ? (wave == 0 ? 0 : (tid >= RE ? 1 + (tid - RE) / 64 : -1)) : (wave < 4 ? wave : -1);
    const uint32_t kind = hh < n_heads ? 0u : (hh < n_heads + n_kv ? 1u : 2u);   // q, k, v
    // x and the gain first, alone in the memory pipeline (the chain waits for them)
    constexpr uint32_t RQ = (1024 / 4 + NT - 1) / NT;
    v4f xv[RQ], wv[RQ];
#pragma unroll
    for (uint32_t u = 0; u < RQ; ++u) {
        const uint32_t g = min(tid + NT * u, ng - 1);
        xv[u] = reinterpret_cast<const v4f *>(x)[g];
        wv[u] = reinterpret_cast<const v4f *>(w)[g];
    }
    const uint32_t pos = p->pos;
    HeadConst<HD> hc;   // gains and RoPE row, used by wave 0 at the end
    if (tid < 64) hc.load(qn, kn, cs, sn, pos, lane);
    const uint32_t row = hh * HD + (rowt ? (uint32_t)(tid - CW) >> 3 : 0u);
    Q8Row<ORDER, SCF32, NCT> rd;
    float ss = 0.0f;
    auto squares = [&](const v4f a, uint32_t g) {
        if (EXACT) {
            reinterpret_cast<v4f *>(ps)[g] = a * a;
        } else {
            ss += a.x * a.x;
            ss += a.y * a.y;
            ss += a.z * a.z;
            ss += a.w * a.w;
        }
    };
#pragma unroll
    for (uint32_t u = 0; u < RQ; ++u)
        if (tid + NT * u < ng) squares(xv[u], tid + NT * u);
    for (uint32_t g = tid + NT * RQ; g < ng; g += NT) squares(reinterpret_cast<const v4f *>(x)[g], g);
    // (SC) the split's K rows, fetched straight into LDS behind the weights: 16-byte piece m of
    // local row i at slot 16 i + (m + i) % 16, so a row read by its thread is bank-conflict free
    float *kbuf = ps + d;
    if (EXACT) {
        if (tid == 0) xs.sync = 0;
        __syncthreads();
        // the row waves issue their weights now (arriving during the sum)
        if (rowt) rd.begin(row_qs(W, row), row_sc<SCF32>(W, row), W.nb, W.nc, j);
        if constexpr (SC) {
            const uint32_t c = div_up(win, S2), t0 = spl * c, t1 = min(win, t0 + c);
            if (kind == 0 && rowt) {   // row wave rw issues 1 KB instructions rw, rw + 8, ... (64 slots each)
                const float *kcg = kc + (size_t)(hh / (n_heads / n_kv)) * cap * HD;
                const uint32_t rw = (uint32_t)(tid - CW) >> 6, ni = div_up(c, 4);
                for (uint32_t I = rw; I < ni; I += (RE - CW) / 64) {
                    const uint32_t sl = I * 64 + (uint32_t)lane, i = sl / 16, m = (sl - i) & 15;
                    const uint32_t tr = min(t0 + i, t1 - 1);   // (rows past the split: its last row)
                    __builtin_amdgcn_global_load_lds(kcg + (size_t)tr * HD + 4 * m, kbuf + (size_t)I * 256, 16, 0, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (sp >= 0) {
            const float r = block_seq_sum<4, 4>(ps, d, xs, sp, lane);   // ss += v * v in index order
            if (tid == 0) s_ss = r;
        }
    } else {
        if (rowt) rd.begin(row_qs(W, row), row_sc<SCF32>(W, row), W.nb, W.nc, j);
        for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
        if (lane == 0) red[tid >> 6] = ss;
        __syncthreads();
        if (tid == 0) {
            float t = 0.0f;
            for (int i = 0; i < NT / 64; ++i) t += red[i];
            s_ss = t;
        }
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf(s_ss / (float)d + eps);
    auto emit = [&](const v4f a, const v4f gw, uint32_t g, bool store) {
        const float v[4] = {a.x * scale * gw.x, a.y * scale * gw.y, a.z * scale * gw.z, a.w * scale * gw.w};
        quant_block_lane(v, j, g / 8, sq, sd, store);
    };
#pragma unroll
    for (uint32_t u = 0; u < RQ; ++u) {   // a block's 8 groups are all < ng or all >= ng
        const uint32_t g = tid + NT * u;
        emit(xv[u], wv[u], min(g, ng - 1), g < ng);
    }
    for (uint32_t g = tid + NT * RQ; g < ng; g += NT)
        emit(reinterpret_cast<const v4f *>(x)[g], reinterpret_cast<const v4f *>(w)[g], g, true);
    zero_pad(W.nb, W.nc, sq, sd, tid, NT);
    __syncthreads();
    if (rowt) {
        const float v = rd.finish(sq, sd);
        if (j == 0) hv[(tid - CW) >> 3] = v;
    }
    const bool scw = SC && kind == 0;   // (uniform) a score workgroup: every thread stays
    if (scw) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's K pieces are in LDS
    __syncthreads();
    if (!scw && tid >= 64) return;
    // (SC) each row thread takes its K row into registers while wave 0 forms the q head
    float kt[SC ? HD : 1];
    if constexpr (SC) {
        const uint32_t i = (uint32_t)(tid - CW);
        if (rowt && i < div_up(win, S2)) {
#pragma unroll
            for (uint32_t m = 0; m < HD / 4; ++m)
                *reinterpret_cast<v4f *>(kt + 4 * m) = *reinterpret_cast<const v4f *>(kbuf + 4 * (16 * i + ((m + i) & 15)));
        }
    }
    if (tid < 64) {
        float *dst = out + (size_t)hh * HD;   // q | k | v regions are contiguous in head order
        if (kind == 2) {
            const uint32_t g = hh - n_heads - n_kv;
            float *vcr = vc + ((size_t)g * cap + pos) * HD;
            float *vtr = vc + (size_t)n_kv * cap * HD + (size_t)g * HD * vt_stride(cap) + pos;
            for (uint32_t i = lane; i < HD; i += 64) {
                dst[i] = hv[i];
                vcr[i] = hv[i];
                vtr[(size_t)i * vt_stride(cap)] = hv[i];
            }
            return;
        }
        norm_rope_head<HD>(hv, ho, hc, kind == 0, eps, tmp, lane);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (!scw || spl == 0)
            for (uint32_t i = lane; i < HD; i += 64) dst[i] = ho[i];
        if (kind == 1) {
            float *kcr = kc + ((size_t)(hh - n_heads) * cap + pos) * HD;
            for (uint32_t i = lane; i < HD; i += 64) kcr[i] = ho[i];
        }
    }
    if constexpr (SC) {
        if (!scw) return;
        __syncthreads();   // q_h (ho)
        const uint32_t c = div_up(win, S2), t0 = spl * c, t1 = min(win, t0 + c);
        const uint32_t t = t0 + (uint32_t)(tid - CW);
        float mx = -__builtin_huge_valf();
        if (rowt && t < t1 && t < pos) {   // (position pos: the softmax + P.V kernel)
            const float v = dot_wide_serial(ho, kt, HD) * (1.0f / sqrtf((float)HD));
            scores[(size_t)hh * cap + t] = v;
            mx = v;
        }
        for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, shfl_xor(mx, m));   // max is order-free
        if (lane == 0) red[tid >> 6] = mx;
        __syncthreads();
        if (tid == 0) {
            for (int i = 1; i < NT / 64; ++i) mx = fmaxf(mx, red[i]);
            pmax[(size_t)hh * S2 + spl] = mx;
        }
    }
}

// QK-norm + RoPE of q and k and the cache append of k and v for a q | k | v vector as the QKV
// matvec produced it (the same steps as k_qkv_head's end, for callers that hold the raw
// vector): workgroup hh as in k_qkv_head, 64 threads; qkv is rewritten in place.
template <int HD>
__global__ __launch_bounds__(64) void k_qk_rope_append(float *qkv, const float *__restrict__ qn,
                                                       const float *__restrict__ kn, float eps,
                                                       const float *__restrict__ cs, const float *__restrict__ sn,
                                                       const StepParams *p, uint32_t n_heads, uint32_t n_kv, float *kc,
                                                       float *vc, uint32_t cap) {
    __shared__ __align__(16) float u[HD], o[HD], tmp[HD];
    const int lane = threadIdx.x;
    const uint32_t hh = blockIdx.x, pos = p->pos;
    float *src = qkv + (size_t)hh * HD;
    HeadConst<HD> hc;
    hc.load(qn, kn, cs, sn, pos, lane);
    for (uint32_t i = lane; i < HD; i += 64) u[i] = src[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (hh >= n_heads + n_kv) {
        const uint32_t g = hh - n_heads - n_kv;
        float *vcr = vc + ((size_t)g * cap + pos) * HD;
        float *vtr = vc + (size_t)n_kv * cap * HD + (size_t)g * HD * vt_stride(cap) + pos;
        for (uint32_t i = lane; i < HD; i += 64) {
            vcr[i] = u[i];
            vtr[(size_t)i * vt_stride(cap)] = u[i];
        }
        return;
    }
    norm_rope_head<HD>(u, o, hc, hh < n_heads, eps, tmp, lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (uint32_t i = lane; i < HD; i += 64) src[i] = o[i];
    if (hh >= n_heads) {
        float *kcr = kc + ((size_t)(hh - n_heads) * cap + pos) * HD;
        for (uint32_t i = lane; i < HD; i += 64) kcr[i] = o[i];
    }
}

// ------------------------------------------------------------------ attention (fast)
// Longest split of a cache of `cap` positions cut in S parts, rounded to whole float4s.
__host__ __device__ inline uint32_t attn_maxchunk(uint32_t cap, uint32_t S) { return div_up(div_up(cap, S), 4) * 4; }

// Decode attention of model.rs:212-233, split over the context (flash-decoding): workgroup
// (g, s) handles kv head g and positions [t0, t1) of split s for the rep = n_heads/n_kv query
// heads of the group, and writes an unnormalised partial (max, sum, o[hd]) per head.  q and k
// arrive normed and rotated, and k, v already appended (model.rs:197-211), from the QKV step.
// Softmax and P.V are reduced as trees across lanes and splits.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_fast(const float *__restrict__ qkv, const float *__restrict__ qn,
                                                   const float *__restrict__ kn, float eps,
                                                   const float *__restrict__ cs, const float *__restrict__ sn,
                                                   const StepParams *p, float *kc, float *vc, uint32_t cap,
                                                   uint32_t win, uint32_t n_heads, uint32_t n_kv, uint32_t S,
                                                   float *part) {
    constexpr int MAXREP = 8;
    constexpr int TPT = HD / 4;       // threads per token (one float4 each)
    constexpr int TOK = 256 / TPT;    // tokens per pass
    extern __shared__ __align__(16) float sm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = blockIdx.x, s = blockIdx.y;
    const uint32_t rep = n_heads / n_kv;
    const uint32_t pos = p->pos, n = pos + 1;
    const uint32_t chunk = div_up(n, S);
    const uint32_t t0 = s * chunk, t1 = min(n, t0 + chunk);
    const uint32_t qd = n_heads * HD, kvd = n_kv * HD;
    float *raw = sm;                         // (rep+2)*HD : q heads, k, v of this step
    float *rot = raw + (rep + 2) * HD;       // (rep+1)*HD : (unused)
    float *tmp = rot + (rep + 1) * HD;       // 4*HD : (unused)
    float *sc = tmp + 4 * HD;                // rep * chunk scores
    const uint32_t maxchunk = attn_maxchunk(win, S);
    float *red = sc + rep * maxchunk;        // TOK * rep * HD partial P.V sums
    float *stat = red + TOK * rep * HD;      // 2*rep (max, sum)
    // q and k are normed and rotated, and k, v appended to the caches, by the QKV step
    GroupRaw<HD, MAXREP> gr;
    gr.load(qkv, g, rep, qd, kvd, tid);
    gr.store(raw, rep, tid);
    __syncthreads();
    const float *qrot = raw;
    const float *krot = raw + rep * HD;
    const float *vnew = raw + (rep + 1) * HD;
    const float *kcg = kc + (size_t)g * cap * HD;
    const float *vcg = vc + (size_t)g * cap * HD;
    float *pout = part + (size_t)(g * rep) * S * (HD + 2);
    if (t0 >= t1) {
        for (uint32_t r = 0; r < rep; ++r) {
            float *pr = pout + ((size_t)r * S + s) * (HD + 2);
            for (uint32_t i = tid; i < HD + 2; i += 256) pr[i] = (i == 0) ? -__builtin_huge_valf() : 0.0f;
        }
        return;
    }
    const uint32_t len = t1 - t0;
    const float scale = 1.0f / sqrtf((float)HD);
    const int tl = tid % TPT, tg = tid / TPT;
    // scores
    for (uint32_t tt = tg; tt < len; tt += TOK) {
        const uint32_t t = t0 + tt;
        const float4 k4 = (t == pos) ? *reinterpret_cast<const float4 *>(krot + tl * 4)
                                     : *reinterpret_cast<const float4 *>(kcg + (size_t)t * HD + tl * 4);
        float acc[MAXREP];
#pragma unroll
        for (int r = 0; r < MAXREP; ++r) {
            if (r < (int)rep) {
                const float4 q4 = *reinterpret_cast<const float4 *>(qrot + r * HD + tl * 4);
                acc[r] = q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
            }
        }
#pragma unroll
        for (int r = 0; r < MAXREP; ++r) {
            if (r < (int)rep) {
                float a = acc[r];
                for (int m = 1; m < TPT; m <<= 1) a += shfl_xor(a, m);
                if (tl == 0) sc[r * maxchunk + tt] = a * scale;
            }
        }
    }
    __syncthreads();
    // softmax statistics per head: one wave per head
    for (uint32_t r = wave; r < rep; r += 4) {
        float m = -__builtin_huge_valf();
        for (uint32_t tt = lane; tt < len; tt += 64) m = fmaxf(m, sc[r * maxchunk + tt]);
        for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, shfl_xor(m, k));
        float l = 0.0f;
        for (uint32_t tt = lane; tt < len; tt += 64) {
            const float e = __expf(sc[r * maxchunk + tt] - m);
            sc[r * maxchunk + tt] = e;
            l += e;
        }
        for (int k = 32; k >= 1; k >>= 1) l += shfl_xor(l, k);
        if (lane == 0) { stat[2 * r] = m; stat[2 * r + 1] = l; }
    }
    __syncthreads();
    // P.V
    float4 o[MAXREP];
#pragma unroll
    for (int r = 0; r < MAXREP; ++r) o[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t tt = tg; tt < len; tt += TOK) {
        const uint32_t t = t0 + tt;
        const float4 v4 = (t == pos) ? *reinterpret_cast<const float4 *>(vnew + tl * 4)
                                     : *reinterpret_cast<const float4 *>(vcg + (size_t)t * HD + tl * 4);
#pragma unroll
        for (int r = 0; r < MAXREP; ++r) {
            if (r < (int)rep) {
                const float pr = sc[r * maxchunk + tt];
                o[r].x += pr * v4.x; o[r].y += pr * v4.y; o[r].z += pr * v4.z; o[r].w += pr * v4.w;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MAXREP; ++r)
        if (r < (int)rep) *reinterpret_cast<float4 *>(red + ((size_t)tg * rep + r) * HD + tl * 4) = o[r];
    __syncthreads();
    for (uint32_t i = tid; i < rep * HD; i += 256) {
        float a = 0.0f;
        for (int q = 0; q < TOK; ++q) a += red[(size_t)q * rep * HD + i];
        const uint32_t r = i / HD, di = i % HD;
        float *pr = pout + ((size_t)r * S + s) * (HD + 2);
        pr[2 + di] = a;
        if (di == 0) { pr[0] = stat[2 * r]; pr[1] = stat[2 * r + 1]; }
    }
}

// Merge of the split partials of one head per workgroup (flash-decoding combine, tree
// order): M = max_s M_s, f_s = exp(M_s - M), o = sum_s f_s P_s / sum_s f_s L_s; then the
// quantization of the head's o blocks for attn_output (quant.rs:111-123).
template <int HD>
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part, uint32_t n_heads, uint32_t S,
                                                      float *o_out, uint8_t *q_out, float *d_out) {
    constexpr uint32_t NG = 256 / HD;   // split groups
    __shared__ float fs[1024];
    __shared__ float red[4];
    __shared__ float acc_s[NG][HD];
    __shared__ float s_m, s_inv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t h = blockIdx.x;
    const float *ph = part + (size_t)h * S * (HD + 2);
    float m = -__builtin_huge_valf();
    for (uint32_t s = tid; s < S; s += 256) m = fmaxf(m, ph[(size_t)s * (HD + 2)]);
    for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, shfl_xor(m, k));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (tid == 0) s_m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    const float M = s_m;
    float l = 0.0f;
    for (uint32_t s = tid; s < S; s += 256) {
        const float *pr = ph + (size_t)s * (HD + 2);
        const float f = (pr[1] == 0.0f) ? 0.0f : __expf(pr[0] - M);
        fs[s] = f;
        l += pr[1] * f;
    }
    for (int k = 32; k >= 1; k >>= 1) l += shfl_xor(l, k);
    __syncthreads();
    if (lane == 0) red[wave] = l;
    __syncthreads();
    if (tid == 0) s_inv = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
    const uint32_t d = tid % HD, sg = tid / HD;
    float a = 0.0f;
    if (sg < NG)
        for (uint32_t s = sg; s < S; s += NG) a += ph[(size_t)s * (HD + 2) + 2 + d] * fs[s];
    if (sg < NG) acc_s[sg][d] = a;
    __syncthreads();
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    const uint32_t nbh = HD / QK;   // blocks of this head
    const uint32_t t = (uint32_t)tid;   // thread t < HD / 4: elements 4t .. 4t+3 of the head
    if (t < HD / 4) {
#pragma unroll
        for (int m4 = 0; m4 < 4; ++m4) {
            float o = 0.0f;
            for (uint32_t g = 0; g < NG; ++g) o += acc_s[g][4 * t + m4];
            v[m4] = o * s_inv;
            if (o_out) o_out[h * HD + 4 * t + m4] = v[m4];
        }
    }
    if (t < nbh * 8) quant_block_lane(v, t & 7, h * nbh + t / 8, q_out, d_out);
    if (h == 0) {
        const uint32_t nb = n_heads * HD / QK;
        zero_pad(nb, div_up(nb, 4), q_out, d_out, tid, 256);
    }
}

// ------------------------------------------------------------------ attention (exact)
// Reference-order decode attention (model.rs:218-233, ops.rs:7-36, 112-128) in three
// launches: scores in parallel over the context, the softmax of each head with a
// sequential sum, then P.V as one sequential chain per output element.


// Scores s[h][t] = dot(q_h, K_t) * (1/sqrt(hd)) (model.rs:213-218, ops::dot's order) for the
// rep query heads of kv head g over split s of the attention window (grid n_kv x S; split s
// covers positions [s c, s c + c) with c = ceil(win / S), a layout independent of the step
// within the window, so the K rows are fetched before the step's position is known), and the
// split maximum of every head.  The window win (<= cap, >= pos + 1) is fixed per captured
// step; cap is the cache's row stride.
// q (normed, rotated) comes from the QKV step's output, K (with this step's row appended) from
// the cache.  Lane l of the workgroup's 256 threads takes head l % R and position
// t0 + l / R (+ 256 / R, ...), R = rep rounded up to a power of two: the R lanes of a position
// read the same K row (one memory request per row).
template <int HD>
__global__ __launch_bounds__(256) void k_attn_scores(const float *__restrict__ qkv, const StepParams *p,
                                                     const float *__restrict__ kc, uint32_t cap, uint32_t win,
                                                     uint32_t n_heads, uint32_t n_kv, uint32_t S, float *scores,
                                                     float *pmax) {
    constexpr int MAXREP = 8;
    __shared__ __align__(16) float qs[MAXREP * HD];
    __shared__ float wm[4][MAXREP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = blockIdx.x, s = blockIdx.y;
    const uint32_t rep = n_heads / n_kv;
    const uint32_t R = rep <= 1 ? 1u : rep <= 2 ? 2u : rep <= 4 ? 4u : 8u;   // lanes per position
    const uint32_t r = (uint32_t)tid % R, pp = 256 / R;                      // head, positions per pass
    const uint32_t chunk = div_up(win, S), t0 = s * chunk, t1 = min(win, t0 + chunk);
    const float *kcg = kc + (size_t)g * cap * HD;
    // loads in issue order: this lane's first K row, the group's q heads, the position
    // Rows past the split are clamped to its last row (already fetched), so a split never pulls
    // in its neighbour's rows.
    float kt[HD];
    {
        const uint32_t tr = min(t0 + (uint32_t)tid / R, t1 - 1);
#pragma unroll
        for (int i = 0; i < HD; i += 4)
            *reinterpret_cast<v4f *>(kt + i) = *reinterpret_cast<const v4f *>(kcg + (size_t)tr * HD + i);
    }
    for (uint32_t i = tid; i < rep * HD; i += 256) qs[i] = qkv[(size_t)g * rep * HD + i];
    const uint32_t n = p->pos + 1;
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    float mx = -__builtin_huge_valf();
    const float *qr = qs + min(r, rep - 1) * HD;
    for (uint32_t tb = t0; tb < t1; tb += pp) {
        const uint32_t t = tb + (uint32_t)tid / R;
        if (tb != t0) {   // splits longer than 256 / R positions: the next K row
            const uint32_t tr = min(t, t1 - 1);
#pragma unroll
            for (int i = 0; i < HD; i += 4)
                *reinterpret_cast<v4f *>(kt + i) = *reinterpret_cast<const v4f *>(kcg + (size_t)tr * HD + i);
        }
        if (r < rep && t < t1 && t < n) {
            const float v = dot_wide_serial(qr, kt, HD) * scale;
            scores[(size_t)(g * rep + r) * cap + t] = v;
            mx = fmaxf(mx, v);
        }
    }
    // split maximum of each head: over the lanes of equal r (xor of the position bits), then waves
    for (uint32_t o = R; o < 64; o <<= 1) mx = fmaxf(mx, shfl_xor(mx, (int)o));
    if ((uint32_t)lane < R) wm[wave][lane] = mx;
    __syncthreads();
    if ((uint32_t)tid < rep)
        pmax[(size_t)(g * rep + tid) * S + s] = fmaxf(fmaxf(wm[0][tid], wm[1][tid]), fmaxf(wm[2][tid], wm[3][tid]));
}

// Softmax and P.V of one query head (ops.rs:112-128, model.rs:227-232):
//   m = max_t s_t (order-free), e_t = exp(s_t - m) with the reference expf (all threads,
//   into LDS); sum = e_0 + e_1 + ... sequentially (one lane), inv = 1/sum, p_t = e_t * inv;
//   o[di] = ((0 + p_0 v_0[di]) + p_1 v_1[di]) + ...  one sequential chain per output element.
// Grid: (n_heads, HD/16); workgroup (h, q) owns the 16 output elements [16q, 16q+16) of head h
// (the softmax is recomputed identically by the HD/16 workgroups of a head).  Wave 0 lanes
// 0..15 run the chains; waves 1-3 and 5-7 are producers (wave 4, on the chain's SIMD, idles):
// producer i forms the rounded products p_t * v_t[di] (the reference's separate multiply) of
// tiles i, i+NP, ... of T positions
// into a ring of R LDS slots, stored [element][position] so the chain reads four positions per
// 16-byte LDS load.  Readiness and release of slots are LDS flags at workgroup scope; every wait
// is bounded: tile k waits only for tile k - R to be consumed, the chain only for tile k to be
// produced.  Producers start their first V fetch before the sum.  Also writes o and its
// quantization for attn_output (quant.rs:111-123).
// The bounded LDS waits of the softmax + P.V kernels: a wait polls at most cap times
// (StepParams::spin_cap, 0 = SPIN_CAP_DEFAULT, ~0.1 s of s_sleep), then records the failure in
// StepParams::err (a vector atomic) and gives up; the kernel runs on to its normal exit with
// whatever the LDS holds, and the host reports HG_ERR_DEVICE for the step.
struct SpinGuard {
    uint32_t cap;
    uint32_t *err;
    __device__ explicit SpinGuard(const StepParams *p)
        : cap(p->spin_cap ? p->spin_cap : SPIN_CAP_DEFAULT), err(const_cast<uint32_t *>(&p->err)) {}
    // One more poll of a wait that has polled `it` times: true after a sleep, false (error
    // recorded) once the cap is reached.
    __device__ bool more(uint32_t &it) const {
        if (++it <= cap) {
            __builtin_amdgcn_s_sleep(1);
            return true;
        }
        atomicOr(err, 1u);
        return false;
    }
};

// Workgroup -> (head h, output quarter q) of the softmax + P.V kernels (1-D grid of
// n_heads * nq).  Workgroups are dealt to the 8 XCDs round-robin by linear id, each XCD with its
// own L2; the rep query heads of a kv group read the same V slice, so the rep workgroups of one
// (kv group, quarter) key are given ids that are equal mod 8, keeping the shared V in one L2.
// A head's score row is then fetched into every L2 (16 heads x 16 quarters: 8 x 131 KB per
// layer at context 2049).  Keeping a head's quarters on 2 or 4 XCDs instead (runs of
// consecutive quarters per XCD) cut the measured fetch from 3.49 MB to 2.68 MB per launch but
// made the launch 0.75 us slower, so this placement stays.
__device__ inline void pv_head_quarter(uint32_t L, uint32_t n_heads, uint32_t n_kv, uint32_t nq, uint32_t *h,
                                       uint32_t *q) {
    const uint32_t rep = n_heads / n_kv, nkeys = n_kv * nq;
    if (nkeys % 8 == 0) {
        const uint32_t slot = L / 8, key = L % 8 + 8 * (slot / rep), r = slot % rep;
        *h = (key / nq) * rep + r;
        *q = key % nq;
    } else {
        *h = L % n_heads;
        *q = L / n_heads;
    }
}

struct PvCfg {
    static constexpr uint32_t D = 16;          // output elements per workgroup
    static constexpr uint32_t T = 128;         // positions per tile
    static constexpr uint32_t TP = T + 4;      // padded row of a slot
    static constexpr uint32_t SLOT = D * TP;   // floats per slot
    static constexpr uint32_t NW = 8;          // waves per workgroup
    static constexpr uint32_t NP = NW - 2;     // producer waves (not wave 0 or wave 4)
    static constexpr uint32_t LPP = D / 4;     // producer lanes per position (one float4 each)
    static constexpr uint32_t PPI = 64 / LPP;  // positions per producer instruction
    static constexpr uint32_t NI = T / PPI;    // float4 per producer lane per tile
    static constexpr uint32_t RMAX = 16;
};
constexpr size_t PV_LDS_BUDGET = 156 * 1024;
constexpr size_t XSUM_FLOATS = (sizeof(xsum::Scratch) + 15) / 16 * 4;   // the exact sum's LDS tables

__host__ __device__ uint32_t pv_ring_slots(uint32_t cap) {
    const size_t e_bytes = (size_t)div_up(cap, 4) * 16 + XSUM_FLOATS * 4;
    const size_t left = PV_LDS_BUDGET > e_bytes ? PV_LDS_BUDGET - e_bytes : 0;
    const uint32_t r = (uint32_t)(left / (PvCfg::SLOT * 4));
    return r > PvCfg::RMAX ? PvCfg::RMAX : r;
}

template <int HD>
__global__ __launch_bounds__(512) void k_attn_softmax_pv(const float *__restrict__ scores,
                                                         const float *__restrict__ pmax,
                                                         const float *__restrict__ qkv, const StepParams *p,
                                                         const float *__restrict__ vc, uint32_t cap, uint32_t win,
                                                         uint32_t S, uint32_t n_heads, uint32_t n_kv, float *o_out,
                                                         uint8_t *q_out, float *d_out) {
    using C = PvCfg;
    constexpr uint32_t T = C::T, TP = C::TP, D = C::D;
    extern __shared__ __align__(16) float lds[];
    __shared__ uint32_t ready[C::RMAX];
    __shared__ uint32_t done;
    __shared__ float s_inv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t h, q;
    pv_head_quarter(blockIdx.x, n_heads, n_kv, HD / D, &h, &q);
    const uint32_t rep = n_heads / n_kv, g = h / rep;
    const uint32_t pos = p->pos, n = pos + 1;
    const SpinGuard sg(p);
    const uint32_t R = pv_ring_slots(win);
    float *e = lds;                                     // [win] e_t, then p_t
    float *ring = lds + (size_t)div_up(win, 4) * 4;     // [R][D][TP]
    xsum::Scratch &xs = *reinterpret_cast<xsum::Scratch *>(ring + (size_t)R * C::SLOT);
    const float *sc = scores + (size_t)h * cap;
    const uint32_t qd = n_heads * HD, kvd = n_kv * HD;
    const float *vcg = vc + (size_t)g * cap * HD + q * D;
    const float *vnew = qkv + qd + kvd + g * HD + q * D;  // row pos, appended this step
    const uint32_t ntiles = div_up(n, T);
    const uint32_t sub = lane / C::LPP, d4 = (lane % C::LPP) * 4;  // producer lane -> (position, elements)
    // waves run on SIMD wave % 4: wave 4 shares SIMD 0 with the chain wave and stays idle so
    // the chain's dependent adds never wait behind a producer's VALU issue
    const int pw = wave == 4 ? -1 : (wave < 4 ? wave - 1 : wave - 2);
    v4f vr[C::NI];
    auto fetch = [&](uint32_t k) {
#pragma unroll
        for (uint32_t i = 0; i < C::NI; ++i) {
            const uint32_t t = min(k * T + i * C::PPI + sub, n - 1);
            const float *src = (t == pos) ? vnew + d4 : vcg + (size_t)t * HD + d4;
            vr[i] = *reinterpret_cast<const v4f *>(src);
        }
    };
    // loads in issue order: the split maxima (one per lane), this thread's first scores, the
    // exp table, then the producers' first V tile, so waiting for the first ones leaves V in
    // flight
    constexpr uint32_t EB = 8;
    float m = pmax[(size_t)h * S + min((uint32_t)lane, S - 1)];
    float sv[EB];
#pragma unroll
    for (uint32_t u = 0; u < EB; ++u) sv[u] = sc[min(u * 512 + tid, n - 1)];
    const WaveExpTab tab = WaveExpTab::load(lane);
    // V does not depend on the softmax.  Every wave fetches (wave 0 and idle producers a
    // clamped tile they do not use): a load under a branch would make the waits for the
    // scores after the join also wait for V.
    fetch(pw < 0 ? 0u : (uint32_t)pw);
    for (uint32_t s = lane + 64; s < S; s += 64) m = fmaxf(m, pmax[(size_t)h * S + s]);
    for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, shfl_xor(m, k));   // max is order-free
    for (uint32_t t0 = 0; t0 < n; t0 += EB * 512) {
        if (t0)
#pragma unroll
            for (uint32_t u = 0; u < EB; ++u) sv[u] = sc[min(t0 + u * 512 + tid, n - 1)];
#pragma unroll
        for (uint32_t u = 0; u < EB; ++u)
            if (t0 + u * 512 < n) {                      // uniform: every lane calls the exp
                const uint32_t t = t0 + u * 512 + tid;
                const float ev = hg_expf_l(sv[u] - m, tab);
                if (t < n) e[t] = ev;
            }
    }
    if (tid < (int)C::RMAX) ready[tid] = 0;
    if (tid == 0) {
        done = 0;
        xs.sync = 0;
    }
    __syncthreads();
    {   // sum += e_t in index order, formed by all 8 waves (16 or 32 terms per lane; past 16384
        // terms block_seq_sum runs the one-lane chain itself)
        const float r = n <= 8192 ? block_seq_sum<8, 16>(e, n, xs, wave, lane) : block_seq_sum<8, 32>(e, n, xs, wave, lane);
        if (tid == 0) s_inv = 1.0f / r;
    }
    __syncthreads();
    const float inv = s_inv;   // p_t = e_t * inv, formed by the producers
    if (pw >= 0) {
        for (uint32_t k = pw; k < ntiles; k += C::NP) {
            if (k != (uint32_t)pw) fetch(k);
            if (k >= R) {
                uint32_t it = 0;
                while (__hip_atomic_load(&done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < k - R + 1)
                    if (!sg.more(it)) break;
            }
            float *slot = ring + (size_t)(k % R) * C::SLOT;
#pragma unroll
            for (uint32_t i = 0; i < C::NI; ++i) {
                const uint32_t tt = i * C::PPI + sub, t = k * T + tt;
                // positions past the context hold -0, the exact identity of the chain's adds
                const bool in = t < n;
                const float pt = in ? e[t] * inv : 0.0f;
                slot[(d4 + 0) * TP + tt] = in ? pt * vr[i].x : -0.0f;
                slot[(d4 + 1) * TP + tt] = in ? pt * vr[i].y : -0.0f;
                slot[(d4 + 2) * TP + tt] = in ? pt * vr[i].z : -0.0f;
                slot[(d4 + 3) * TP + tt] = in ? pt * vr[i].w : -0.0f;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_store(&ready[k % R], k + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    } else if (wave == 0 && lane < (int)D) {
        // Chain lanes 0..15: o += product, position order, 32 positions (eight 16-byte LDS
        // reads) per chunk, the next chunk's reads issued before the current chunk's adds; the
        // instruction order is pinned so the reads stay ahead of the dependent adds.
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's unused V prefetch is done
        float o = 0.0f;
        const uint32_t di = lane;
        auto ready_wait = [&](uint32_t k) {
            uint32_t it = 0;
            while (__hip_atomic_load(&ready[k % R], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != k + 1)
                if (!sg.more(it)) break;
        };
        auto rowp = [&](uint32_t k) {
            return reinterpret_cast<const v4f *>(ring + (size_t)(k % R) * C::SLOT + di * TP);
        };
        v4f ca[8], cb[8];
        auto ld = [&](v4f(&c)[8], const v4f *p) {
#pragma unroll
            for (int u = 0; u < 8; ++u) c[u] = p[u];
        };
        auto add = [&](const v4f(&c)[8]) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                o = o + c[u].x;
                o = o + c[u].y;
                o = o + c[u].z;
                o = o + c[u].w;
            }
        };
        static_assert(T == 128, "four chunks of 32 positions per tile");
        ready_wait(0);
        ld(ca, rowp(0));
        for (uint32_t k = 0; k < ntiles; ++k) {
            const v4f *row = rowp(k);
            __builtin_amdgcn_sched_barrier(0);
            ld(cb, row + 8);
            __builtin_amdgcn_sched_barrier(0);
            add(ca);
            __builtin_amdgcn_sched_barrier(0);
            ld(ca, row + 16);
            __builtin_amdgcn_sched_barrier(0);
            add(cb);
            __builtin_amdgcn_sched_barrier(0);
            ld(cb, row + 24);
            __builtin_amdgcn_sched_barrier(0);
            add(ca);
            __builtin_amdgcn_sched_barrier(0);
            if (k + 1 < ntiles) {
                ready_wait(k + 1);
                ld(ca, rowp(k + 1));
            }
            __builtin_amdgcn_sched_barrier(0);
            add(cb);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_store(&done, k + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        if (o_out) o_out[h * HD + q * D + di] = o;
    }
}

// o = o + p_0 + p_1 + ... + p_63 in order, for the first lane of each row of 16, where lane i
// of the row holds p_4i .. p_4i+3 in a: the row's own four, then lane i's four through a row
// rotation by 16 - i fused into the add.  One asm block, so that no wait states separate the
// adds: an add whose rotated operand was written long before needs none for its other operand
// (the previous add's result), which keeps the chain at the rate of register-fed adds (2.0 ns
// per add, against 2.5-2.9 with the products read from LDS and 5.1 with the compiler's wait
// states between rotated adds; all three bit-identical).  Every lane of the row must be active.
__device__ __forceinline__ void pv_adds64(float &o, const v4f a) {
    const float a0 = a.x, a1 = a.y, a2 = a.z, a3 = a.w;
    asm volatile(
                 "v_add_f32 %0, %0, %1\n"
                 "v_add_f32 %0, %0, %2\n"
                 "v_add_f32 %0, %0, %3\n"
                 "v_add_f32 %0, %0, %4\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:15 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:15 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:15 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:15 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:14 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:14 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:14 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:14 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:13 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:13 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:13 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:13 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:12 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:12 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:12 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:12 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:11 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:11 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:11 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:11 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:10 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:10 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:10 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:10 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:9 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:9 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:9 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:9 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:7 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:7 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:7 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:7 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:6 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:6 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:6 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:6 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:5 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:5 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:5 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:5 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:4 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:4 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:4 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:4 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:3 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:3 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:3 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:3 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:2 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:2 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:2 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:2 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %1, %0 row_ror:1 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %2, %0 row_ror:1 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %3, %0 row_ror:1 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 "v_add_f32_dpp %0, %4, %0 row_ror:1 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
                 : "+v"(o)
                 : "v"(a0), "v"(a1), "v"(a2), "v"(a3));
}

// Softmax and P.V of one query head, as k_attn_softmax_pv, for caches whose V slice and
// products fit in LDS (pv_res_fits): no ring.  Workgroup (h, q), 512 threads, D = 4 output
// elements (one per row of 16 lanes of the chain wave; a workgroup per CU):
//   every wave forms its share of e_t and signals it (no wait); waves 4..7 then stream the
//   D rows of V's transposed copy (contiguous positions) into LDS, P[d][t], flagging each
//   round, while waves 0..3 form the index-order sum of e_t (block_seq_sum).  Once inv is
//   known (a flag, not a barrier), wave 0 replaces the first 4 groups of G positions by the
//   rounded products p_t * V[d][t] (p_t = e_t * inv; -0 past the context, the exact identity
//   of the chain's adds) and waves 1..3 and 5..7 (not wave 4, which shares wave 0's SIMD) the
//   others, flagging them; wave 0 then runs the D sequential chains, a row's lanes holding a
//   group's products and its first lane adding them in order through DPP row rotations
//   (pv_adds64), waiting only for each block of 4 groups' flags.
// LONG = false serves windows up to SHORT positions (one 64-bit ready word, each producer's
// groups in one batch); LONG = true up to MAXR (two ready words, batches of 7 groups, the sum
// as 16 or 28 terms per lane).  SELF (head 64, after the QKV launch that also scores): the
// scores row stops short of pos; wave 0 forms the score at pos from this step's q and k
// (dot64_lanes, ops::dot's order) and the maximum and exps take it in place of the row's.
struct PvResCfg {
    static constexpr uint32_t D = 4;      // output elements per workgroup (4 or 8)
    static constexpr uint32_t G = 64;     // positions per product group (16 lanes x 4)
    static constexpr uint32_t NG = 128;   // product groups: one bit each of the ready mask (2 words)
    static constexpr uint32_t MAXR = 7168;   // positions: the exact sum as 4 waves x 64 lanes x 28 terms
    static constexpr uint32_t SHORT = 3072;  // up to here: 12 terms per lane, one ready word (LONG = false)
    static constexpr uint32_t VB = 8;     // V loads in flight per V thread
};

__host__ __device__ inline uint32_t pv_res_rows(uint32_t cap) { return div_up(cap, 256) * 256; }   // chain blocks
__host__ __device__ inline size_t pv_res_lds(uint32_t cap) {   // e, P, the sum's scratch
    const uint32_t rc = pv_res_rows(cap);
    return ((size_t)rc + (size_t)PvResCfg::D * (rc + 4) + XSUM_FLOATS) * 4;
}
__host__ __device__ bool pv_res_fits(uint32_t cap) {
    return cap >= 1 && pv_res_lds(cap) <= PV_LDS_BUDGET && pv_res_rows(cap) / PvResCfg::G <= PvResCfg::NG &&
           pv_res_rows(cap) <= PvResCfg::MAXR;
}

template <int HD, bool LONG, bool SELF = false>
__global__ __launch_bounds__(512) void k_attn_softmax_pv_res(const float *__restrict__ scores,
                                                             const float *__restrict__ pmax,
                                                             const float *__restrict__ qkv, const StepParams *p,
                                                             const float *__restrict__ vc, uint32_t cap, uint32_t win,
                                                             uint32_t S, uint32_t n_heads, uint32_t n_kv, float *o_out) {
    using C = PvResCfg;
    constexpr uint32_t D = C::D, G = C::G, EB = 8;
    extern __shared__ __align__(16) float lds[];
    __shared__ uint64_t ready[LONG ? 2 : 1];   // bit g % 64 of word g / 64: products of group g written
    __shared__ uint32_t vdone[4];        // V rounds written by V wave 4 + i (its groups i, i + 4, ...)
    __shared__ uint32_t arrived;         // waves whose e_t are written
    __shared__ uint32_t inv_ready;
    __shared__ float s_inv, s_pos;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t h, q;
    pv_head_quarter(blockIdx.x, n_heads, n_kv, HD / D, &h, &q);
    const uint32_t rep = n_heads / n_kv, g = h / rep;
    const uint32_t pos = p->pos, n = pos + 1;
    const SpinGuard sg(p);
    const uint32_t rc = pv_res_rows(win), TPC = rc + 4;   // row stride 4 mod 32 banks
    float *e = lds;                                         // [rc]  e_t
    float *P = lds + rc;                                    // [D][TPC]  V, then the products
    xsum::Scratch &xs = *reinterpret_cast<xsum::Scratch *>(P + (size_t)D * TPC);
    const float *sc = scores + (size_t)h * cap;
    static_assert(D == 4, "a lane moves 16 bytes of one element's row");
    const float *vtg = vc + (size_t)n_kv * cap * HD + ((size_t)g * HD + q * D) * vt_stride(cap);   // rows q D ..
    const uint32_t ng = div_up(n, G), nblk = div_up(n, 4 * G);   // V groups, chain blocks of 4 groups
    // loads in issue order: (SELF, wave 0) this step's q and k elements, the split maxima, this
    // thread's first scores, the exp table
    float qk[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (SELF) {
        if (wave == 0) {
            const float *qh = qkv + (size_t)h * HD, *kp = qkv + (size_t)(n_heads + g) * HD;
            const uint32_t e = (uint32_t)lane & 31;
            qk[0] = qh[e];
            qk[1] = kp[e];
            qk[2] = qh[32 + e];
            qk[3] = kp[32 + e];
        }
    }
    float m = pmax[(size_t)h * S + min((uint32_t)lane, S - 1)];
    float sv[EB];
#pragma unroll
    for (uint32_t u = 0; u < EB; ++u) sv[u] = sc[min(u * 512 + tid, n - 1)];
    const WaveExpTab tab = WaveExpTab::load(lane);
    if (tid == 0) {
        ready[0] = 0;
        if constexpr (LONG) ready[LONG ? 1 : 0] = 0;
        arrived = 0;
        inv_ready = 0;
        xs.sync = 0;
    }
    if constexpr (SELF) {
        // the score at pos, s = dot(q_h, k_pos) / sqrt(HD) (model.rs:213-218, ops::dot's order),
        // from this step's q and k as the QKV launch wrote them (the scores row stops short of pos)
        static_assert(!SELF || HD == 64, "one wave's dot");
        if (wave == 0) {
            const float v = dot64_lanes(qk[0], qk[1], qk[2], qk[3]) * (1.0f / sqrtf((float)HD));
            if (lane == 0) s_pos = v;
        }
    }
    if (tid < 4) vdone[tid] = 0;
    __syncthreads();
    const float spos = SELF ? s_pos : 0.0f;
    if constexpr (SELF) m = fmaxf(m, spos);
    for (uint32_t s = lane + 64; s < S; s += 64) m = fmaxf(m, pmax[(size_t)h * S + s]);
    for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, shfl_xor(m, k));   // max is order-free
    for (uint32_t t0 = 0; t0 < n; t0 += EB * 512) {
        if (t0)
#pragma unroll
            for (uint32_t u = 0; u < EB; ++u) sv[u] = sc[min(t0 + u * 512 + tid, n - 1)];
#pragma unroll
        for (uint32_t u = 0; u < EB; ++u)
            if (t0 + u * 512 < n) {                      // uniform: every lane calls the exp
                const uint32_t t = t0 + u * 512 + tid;
                const float ev = hg_expf_l(((SELF && t == n - 1) ? spos : sv[u]) - m, tab);
                if (t < n) e[t] = ev;
            }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) __hip_atomic_fetch_add(&arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    constexpr uint32_t LP = 1;   // V waves per group
    if (wave >= 4) {
        // V into P[d][t] from the transposed copy: round r, wave 4 + w -> group g = 4 r + w,
        // lane l -> element l / 16, positions 64 g + 4 (l % 16) .. + 3 (16 contiguous bytes; the
        // rows run to vt_stride(cap), positions past the context are replaced by -0 later); VB
        // rounds of loads in flight, then per round its LDS writes and this wave's round count
        const uint32_t w4 = (uint32_t)wave - 4, d4 = (uint32_t)lane >> 4, t4 = 4 * ((uint32_t)lane & 15);
        const float *vrow = vtg + (size_t)d4 * vt_stride(cap) + t4;
        const uint32_t nr = div_up(ng, 4);
        for (uint32_t r0 = 0; r0 < nr; r0 += C::VB) {
            v4f vr[C::VB];
#pragma unroll
            for (uint32_t u = 0; u < C::VB; ++u) {
                const uint32_t gg = min(4 * (r0 + u) + w4, ng - 1);
                vr[u] = *reinterpret_cast<const v4f *>(vrow + G * gg);
            }
#pragma unroll
            for (uint32_t u = 0; u < C::VB; ++u) {
                const uint32_t gg = 4 * (r0 + u) + w4;
                if (r0 + u < nr) {
                    if (gg < ng) *reinterpret_cast<v4f *>(P + d4 * TPC + G * gg + t4) = vr[u];
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");   // (the later rounds' loads stay in flight)
                    if (lane == 0)
                        __hip_atomic_store(&vdone[w4], r0 + u + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
        }
    }
    float inv0 = 0.0f;   // wave 0: 1 / sum
    if (wave < 4) {   // sum += e_t in index order, once every wave's e_t are written
        uint32_t it = 0;
        while (__hip_atomic_load(&arrived, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 8u)
            if (!sg.more(it)) break;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        // terms per lane by context (4 waves x 64 lanes x EPT >= n; a longer sum would fall back
        // to the one-lane chain inside block_seq_sum).  Two layouts per instantiation: more
        // inlined layouts made the kernel measurably slower.
        float r;
        if constexpr (LONG)
            r = n <= 4096 ? block_seq_sum<4, 16>(e, n, xs, wave, lane) : block_seq_sum<4, 28>(e, n, xs, wave, lane);
        else
            r = n <= 2048 ? block_seq_sum<4, 8>(e, n, xs, wave, lane) : block_seq_sum<4, 12>(e, n, xs, wave, lane);
        inv0 = 1.0f / r;
        if (tid == 0) {
            s_inv = inv0;
            __hip_atomic_store(&inv_ready, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    if (wave >= 1 && wave != 4) {
        // products by the six waves off the chain wave's SIMD (wave 4 shares it with wave 0):
        // groups pw, pw + 6, ... (pw = 0..5) past the first block; lane l -> element l / 16,
        // positions 4 (l % 16) .. + 3 of the group.  The first group alone (the chain needs it
        // soon), then the others together: their reads first, one release, one flag update.
        uint32_t it = 0;
        while (__hip_atomic_load(&inv_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0u)
            if (!sg.more(it)) break;
        const float inv = s_inv;
        const uint32_t di = (uint32_t)lane >> 4, tq = (uint32_t)lane & 15;
        const uint32_t pw = (uint32_t)wave - (wave < 4 ? 1 : 2), ngp = 4 * nblk;   // (past the context: -0)
        auto vwait = [&](uint32_t r, uint32_t w0, uint32_t w1) {   // V waves w0..w1 past round r
            uint32_t it = 0;
            for (;;) {
                uint32_t v0 = __hip_atomic_load(&vdone[w0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                for (uint32_t w = w0 + 1; w <= w1; ++w)
                    v0 = min(v0, __hip_atomic_load(&vdone[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
                if (v0 > r || !sg.more(it)) break;
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        };
        auto prod = [&](uint32_t t, const v4f ev, const v4f vv) {
            v4f pr;
            pr.x = t + 0 < n ? (ev.x * inv) * vv.x : -0.0f;
            pr.y = t + 1 < n ? (ev.y * inv) * vv.y : -0.0f;
            pr.z = t + 2 < n ? (ev.z * inv) * vv.z : -0.0f;
            pr.w = t + 3 < n ? (ev.w * inv) * vv.w : -0.0f;
            return pr;
        };
        static_assert(D == 4 && LP == 1, "one 16-byte step per lane and group");
        if (pw >= 4 && pw < ngp) {   // (groups 0..3, the first chain block: wave 0 itself)
            if (pw < ng) vwait(pw / 4, pw % 4, pw % 4);
            const uint32_t t = G * pw + 4 * tq;
            v4f *pv = reinterpret_cast<v4f *>(P + di * TPC + t);
            *pv = prod(t, *reinterpret_cast<const v4f *>(e + t), *pv);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            if (lane == 0) __hip_atomic_fetch_or(&ready[0], 1ull << pw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        if (!LONG && pw + 6 < ngp) {
            constexpr uint32_t KM = 8;   // groups per wave: 4 nblk <= 48
            vwait(div_up(ng, 4) - 1, 0, 3);   // every V round in
            v4f ev[KM], vv[KM];
#pragma unroll
            for (uint32_t k = 1; k < KM; ++k) {
                const uint32_t gi = min(pw + 6 * k, ngp - 1), t = G * gi + 4 * tq;
                ev[k] = *reinterpret_cast<const v4f *>(e + t);
                vv[k] = *reinterpret_cast<const v4f *>(P + di * TPC + t);
            }
            uint64_t mask = 0;
#pragma unroll
            for (uint32_t k = 1; k < KM; ++k) {
                const uint32_t gi = pw + 6 * k, t = G * gi + 4 * tq;
                if (gi < ngp) {
                    *reinterpret_cast<v4f *>(P + di * TPC + t) = prod(t, ev[k], vv[k]);
                    mask |= 1ull << gi;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            if (lane == 0) __hip_atomic_fetch_or(&ready[0], mask, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        if (LONG && pw + 6 < ngp) {
            // the wave's other groups pw + 6 k (k >= 1) in batches of KB: the batch's reads first,
            // then its products, one release and one flag update per ready word
            constexpr uint32_t KB = 7;
            vwait(div_up(ng, 4) - 1, 0, 3);   // every V round in
            for (uint32_t k0 = 1; pw + 6 * k0 < ngp; k0 += KB) {
                v4f ev[KB], vv[KB];
#pragma unroll
                for (uint32_t k = 0; k < KB; ++k) {
                    const uint32_t gi = min(pw + 6 * (k0 + k), ngp - 1), t = G * gi + 4 * tq;
                    ev[k] = *reinterpret_cast<const v4f *>(e + t);
                    vv[k] = *reinterpret_cast<const v4f *>(P + di * TPC + t);
                }
                uint64_t m0 = 0, m1 = 0;
#pragma unroll
                for (uint32_t k = 0; k < KB; ++k) {
                    const uint32_t gi = pw + 6 * (k0 + k), t = G * gi + 4 * tq;
                    if (gi < ngp) {
                        *reinterpret_cast<v4f *>(P + di * TPC + t) = prod(t, ev[k], vv[k]);
                        if (gi < 64) m0 |= 1ull << gi;
                        else m1 |= 1ull << (gi - 64);
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                if (lane == 0) {
                    if (m0) __hip_atomic_fetch_or(&ready[0], m0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    if (m1)
                        __hip_atomic_fetch_or(&ready[LONG ? 1 : 0], m1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
        }
    }
    if (wave == 0) {   // the first block's products (groups 0..3), by the chain wave itself
        const uint32_t di = (uint32_t)lane >> 4, tq = (uint32_t)lane & 15;
        uint32_t it = 0;
        for (;;) {   // round 0 of every V wave in
            uint32_t v0 = __hip_atomic_load(&vdone[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            v0 = min(v0, __hip_atomic_load(&vdone[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            v0 = min(v0, __hip_atomic_load(&vdone[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            v0 = min(v0, __hip_atomic_load(&vdone[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            if (v0 > 0 || !sg.more(it)) break;
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        v4f ev[4], vv[4];
#pragma unroll
        for (uint32_t g4 = 0; g4 < 4; ++g4) {
            const uint32_t t = G * g4 + 4 * tq;
            ev[g4] = *reinterpret_cast<const v4f *>(e + t);
            vv[g4] = *reinterpret_cast<const v4f *>(P + di * TPC + t);
        }
#pragma unroll
        for (uint32_t g4 = 0; g4 < 4; ++g4) {
            const uint32_t t = G * g4 + 4 * tq;
            v4f pr;
            pr.x = t + 0 < n ? (ev[g4].x * inv0) * vv[g4].x : -0.0f;
            pr.y = t + 1 < n ? (ev[g4].y * inv0) * vv[g4].y : -0.0f;
            pr.z = t + 2 < n ? (ev[g4].z * inv0) * vv[g4].z : -0.0f;
            pr.w = t + 3 < n ? (ev[g4].w * inv0) * vv[g4].w : -0.0f;
            *reinterpret_cast<v4f *>(P + di * TPC + t) = pr;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (wave == 0) {
        // chains: row r of the wave (lanes 16 r .. 16 r + 15) owns element r; lane i of the row
        // holds the products of positions 4 i .. 4 i + 3 of the current group, and the row's
        // first lane adds the group's 64 products in order, reading lane i's through a row
        // rotation fused into the add (pv_adds64).  The next group's products are read before
        // the current group's adds; the product flags are checked once per block of 4 groups.
        const uint32_t r4 = (uint32_t)lane >> 4, li = (uint32_t)lane & 15;
        const float *prow = P + r4 * TPC + 4 * li;
        uint64_t known = 0xf;   // ready word kw as last read (block 0: this wave's own products)
        uint32_t kw = 0;
        // (not polled against the cap: ready bits are only ever set, and every producer wave
        // runs to its end through bounded waits setting all of its groups' bits, so this wait
        // always ends; a cap here cost 0.8 us per launch)
        auto block_wait = [&](uint32_t b) {   // groups 4 b .. 4 b + 3: bits 4 b % 64 .. of word b / 16
            const uint32_t wd = LONG ? b >> 4 : 0, sh = (4 * b) & 63;
            if (LONG && wd != kw) {
                kw = wd;
                known = 0;
            }
            while (((known >> sh) & 0xf) != 0xf) {
                known = __hip_atomic_load(&ready[wd], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
                if (((known >> sh) & 0xf) != 0xf) __builtin_amdgcn_s_sleep(1);
            }
        };
        const uint32_t ngp = 4 * nblk;
        float o = 0.0f;
        v4f pa = *reinterpret_cast<const v4f *>(prow);
        for (uint32_t g = 0; g < ngp; ++g) {
            const uint32_t gn = g + 1;
            if (gn < ngp && (gn & 3) == 0) block_wait(gn >> 2);
            const v4f pb = *reinterpret_cast<const v4f *>(prow + G * min(gn, ngp - 1));
            pv_adds64(o, pa);
            pa = pb;
        }
        if (li == 0) o_out[h * HD + q * D + r4] = o;
    }
}

// Quantize the attention output o (f32, [n_heads*HD]) for attn_output (quant.rs:111-123).
__global__ __launch_bounds__(256) void k_quant_o(const float *__restrict__ o, uint32_t n, uint8_t *q_out,
                                                 float *d_out) {
    const int tid = threadIdx.x, j = tid & 7;
    const uint32_t nb = n / QK, nc = div_up(nb, 4);
    for (uint32_t b0 = 0; b0 < nb; b0 += 32) {
        const uint32_t b = b0 + (tid >> 3);
        if (b < nb) {
            float v[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) v[m] = o[b * QK + j * 4 + m];
            quant_block_lane(v, j, b, q_out, d_out);
        }
    }
    zero_pad(nb, nc, q_out, d_out, tid, 256);
}

// ------------------------------------------------------------------ MoE router
// ffn_norm RMSNorm + quantization of h, then the F32 router of Model::ffn (model.rs:270-293):
// logits = W_r h in ops::dot's order, sigmoid (or softmax) gate, sel = score + bias,
// descending rank (equal keys: lower expert first), top-k in rank order, optional
// renormalisation, x weights_scale.  One workgroup of router_threads(E) threads.
// ops::dot (ops.rs:7-36) keeps 32 accumulator chains c = 8a + l (a: the four f32x8
// accumulators, l: the lane) over 32-wide steps; here 8 lanes own an expert row and lane l
// runs the four chains l, 8 + l, 16 + l, 24 + l, so (acc0 + acc1) + (acc2 + acc3) is formed in
// the lane and the 8-lane hsum is the xor 4/2/1 butterfly.  With d % 32 == 0 and d <= 1024 the
// router rows come pre-permuted (Wp[e][32 i + 4 l + a] = W_r[e][32 i + 8 a + l]), so a lane's
// four weights of a step are one 16-byte load, and all of them are fetched before the RMSNorm
// chain; h is kept in LDS both in order (for the quantization) and permuted the same way.
// d must be a multiple of 32 (the Q8_0 rows of the same layer already require it); Wr is the
// row-major router, Wp its permuted copy.
constexpr uint32_t ROUTER_IMAX = 32;   // 32-wide steps held in registers (d <= 1024)
constexpr uint32_t ROUTER_MAXE = 64;   // experts ranked by the register path (wave 0's lanes)

// Wave 0 runs the RMSNorm chain and the final selection; waves 1.. own the expert rows (8
// lanes each), so their row fetch (all of it through this one CU's memory pipeline) is issued
// during the chain instead of before it.
__host__ __device__ inline uint32_t router_threads(uint32_t E) {
    const uint32_t t = 64 + (E * 8 + 63) / 64 * 64;
    return t < 256 ? 256 : (t > 1024 ? 1024 : t);
}

// NST: d / 32 when the rows are prefetched (compile-time, so the steps unroll without guards
// and their LDS reads issue back to back), 0 for the generic path.
template <bool EXACT, int MAXT, int NST>
__global__ __launch_bounds__(MAXT) void k_ffn_router(const float *__restrict__ x, const float *__restrict__ w,
                                                     float eps, uint32_t d, const float *__restrict__ Wr,
                                                     const float *__restrict__ Wp,
                                                     const float *__restrict__ bias, uint32_t E, uint32_t top_k,
                                                     int gating_sigmoid, int weights_norm, float weights_scale,
                                                     uint8_t *q_out, float *d_out, uint32_t *topk_idx,
                                                     float *topk_w, uint32_t *order, uint32_t *rec_idx,
                                                     float *rec_w, RowStrides rs) {
    extern __shared__ __align__(16) float hs[];  // 3*d floats: h, h permuted, the squares
    {   // row blockIdx.x of a batched launch
        const size_t bx = blockIdx.x;
        x += bx * rs.x;
        q_out += bx * rs.q;
        d_out += bx * rs.d;
        topk_idx += bx * rs.k;
        topk_w += bx * rs.k;
        order += bx * rs.k;
        rec_idx += bx * rs.rec;
        rec_w += bx * rs.rec;
    }
    float *hp = hs + d, *ps = hs + 2 * d;
    __shared__ float red[16];
    __shared__ float s_ss;
    __shared__ xsum::Scratch xs;
    __shared__ __align__(16) float lg[256], scr[256], sel[256];
    __shared__ __align__(16) uint32_t tk[64];
    __shared__ __align__(16) float tw[64];
    const int tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63;
    const bool rows = tid >= 64;   // waves 1..: the expert rows
    const uint32_t e8 = rows ? (uint32_t)(tid - 64) >> 3 : 0u, l8 = (uint32_t)tid & 7;
    const uint32_t nrt = (uint32_t)nthr - 64;   // row threads
    const uint32_t main = d - d % 32;
    constexpr bool pre = NST > 0;
    static_assert(NST <= (int)ROUTER_IMAX, "prefetched steps");
    // loads in issue order: x and the norm gain (needed first), the exp table, the bias, then
    // the permuted router rows (unconditional, addresses clamped: a load under a branch makes
    // the compiler's wait for x at the join count as if the weights were not in flight)
    constexpr uint32_t XB = 4;
    float xv[XB], wv[XB];
#pragma unroll
    for (uint32_t u = 0; u < XB; ++u) {
        const uint32_t i = min(tid + u * nthr, d - 1);
        xv[u] = x[i];
        wv[u] = w[i];
    }
    const WaveExpTab tab = WaveExpTab::load(lane);
    const float bv = (uint32_t)tid < E ? bias[tid] : 0.0f;
    const float bv8 = bias[min(e8, E - 1)];   // the bias of this thread's expert row
    v4f wr[NST > 0 ? NST : 1];   // issued once the squares are formed
    auto fetch_rows = [&] {
        const uint32_t e = min(e8, E - 1);
        const float *rowp = Wp + (size_t)e * d;
#pragma unroll
        for (int i = 0; i < NST; ++i) wr[i] = *reinterpret_cast<const v4f *>(rowp + 32 * i + 4 * l8);
    };
    float scale;
    {
        float ss = 0.0f;
#pragma unroll
        for (uint32_t u = 0; u < XB; ++u) {
            const uint32_t i = tid + u * nthr;
            if (i < d) {
                if (EXACT) ps[i] = xv[u] * xv[u];
                else ss += xv[u] * xv[u];
            }
        }
        for (uint32_t i = tid + XB * nthr; i < d; i += nthr) {   // d > XB * nthr only
            const float v = x[i];
            if (EXACT) ps[i] = v * v;
            else ss += v * v;
        }
        if (EXACT) {
            if (tid == 0) xs.sync = 0;
            __syncthreads();
            if (rows) fetch_rows();   // arrives during the sum
            if (d % 4 == 0) {         // (the squares are 16-byte aligned)
                if (tid < 256) {
                    const float r = block_seq_sum<4, 4>(ps, d, xs, tid >> 6, lane);   // ss += v * v in index order
                    if (tid == 0) s_ss = r;
                }
            } else if (tid == 0) {
                s_ss = seq_sum_lds(ps, d, 0.0f);
            }
        } else {
            for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
            if (lane == 0) red[tid >> 6] = ss;
            __syncthreads();
            if (rows) fetch_rows();
            if (tid == 0) {
                float t = 0.0f;
                for (int i = 0; i < nthr / 64; ++i) t += red[i];
                s_ss = t;
            }
        }
        __syncthreads();
        scale = 1.0f / sqrtf(s_ss / (float)d + eps);
        auto put = [&](uint32_t i, float v) {
            hs[i] = v;
            if (pre) hp[router_perm(i)] = v;
        };
#pragma unroll
        for (uint32_t u = 0; u < XB; ++u) {
            const uint32_t i = tid + u * nthr;
            if (i < d) put(i, xv[u] * scale * wv[u]);
        }
        for (uint32_t i = tid + XB * nthr; i < d; i += nthr) put(i, x[i] * scale * w[i]);
    }
    __syncthreads();
    // router logits: lane l8 of expert e8 runs chains l8 + 8 a, a = 0..3; after the butterfly
    // every lane of the 8 holds the logit (each add pairs the same two operands in every lane)
    float myv = 0.0f;
    for (uint32_t e0 = 0; rows && e0 < E; e0 += nrt / 8) {   // (uniform per wave)
        const uint32_t e = e0 + e8;
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (e < E) {
            if (pre) {
#pragma unroll
                for (int i = 0; i < NST; ++i) {
                    const v4f hv = *reinterpret_cast<const v4f *>(hp + 32 * i + 4 * l8);
                    a[0] = fmaf(wr[i].x, hv.x, a[0]);
                    a[1] = fmaf(wr[i].y, hv.y, a[1]);
                    a[2] = fmaf(wr[i].z, hv.z, a[2]);
                    a[3] = fmaf(wr[i].w, hv.w, a[3]);
                }
            } else {
                const float *row = Wr + (size_t)e * d;
                uint32_t i = 0;
                for (; i < main; i += 32) {
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c) a[c] = fmaf(row[i + 8 * c + l8], hs[i + 8 * c + l8], a[c]);
                }
                for (; i + 8 <= d; i += 8)      // 8-wide tail into accumulator 0
                    a[0] = fmaf(row[i + l8], hs[i + l8], a[0]);
            }
        }
        float v = (a[0] + a[1]) + (a[2] + a[3]);
        {   // both moves in every lane, then the select (a move under a branch would read
            // lanes the branch switched off)
            const float dn = dpp_f<0x124>(v), up = dpp_f<0x12C>(v);
            v = v + ((l8 & 4) ? dn : up);   // lane ^ 4
        }
        v = v + dpp_f<0x4E>(v);   // lane ^ 2
        v = v + dpp_f<0xB1>(v);   // lane ^ 1
        if (e0 == 0) myv = v;     // (d is a multiple of 32: no scalar tail)
        if (e < E && l8 == 0) lg[e] = v;
    }
    // quantization of h for the expert matvecs (quant.rs:111-123), by waves 1.. after the last
    // barrier (a barrier after global stores waits for them to complete)
    auto quantize_h = [&] {
        const uint32_t nb = d / QK, nc = div_up(nb, 4);
        const int j = tid & 7, qt = tid - 64, nq = nthr - 64;
        for (uint32_t b0 = 0; b0 < nb; b0 += nq / 8) {
            const uint32_t b = b0 + (qt >> 3);
            if (b < nb) {
                const v4f hv = *reinterpret_cast<const v4f *>(hs + b * QK + j * 4);
                const float v[4] = {hv.x, hv.y, hv.z, hv.w};
                quant_block_lane(v, j, b, q_out, d_out);
            }
        }
        zero_pad(nb, nc, q_out, d_out, qt, nq);
    };
    auto rlf = [](float v, uint32_t l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)l));
    };
    auto rlu = [](uint32_t v, uint32_t l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l); };
    if (gating_sigmoid && E * 8 <= nrt && E <= ROUTER_MAXE && top_k <= 64) {
        // every row's 8 lanes form its gate and key; the rank of expert e is
        // #{e' : key_e' > key_e or (key_e' == key_e and e' < e)}, one unsigned 64-bit compare
        // (high word the key's order-preserving bits with -0 made +0, as the float compare has
        // -0 == +0; low word ~e), lane l8 counting the experts l8, l8 + 8, ...
        __shared__ uint64_t K[ROUTER_MAXE];
        const float g = hg_sigmoid_l(myv, tab);   // (wave 0: unused)
        const float key = (g + bv8) + 0.0f;
        const uint32_t mb = __builtin_bit_cast(uint32_t, key);
        const uint64_t mk = ((uint64_t)((mb & 0x80000000u) ? ~mb : (mb | 0x80000000u)) << 32) | (uint32_t)~e8;
        if (rows && l8 == 0 && e8 < E) K[e8] = mk;
        __syncthreads();
        if (rows) {
            uint64_t kk[ROUTER_MAXE / 8];
#pragma unroll
            for (uint32_t q = 0; q < ROUTER_MAXE / 8; ++q) kk[q] = K[min(l8 + 8 * q, E - 1)];
            uint32_t cnt = 0;
#pragma unroll
            for (uint32_t q = 0; q < ROUTER_MAXE / 8; ++q) cnt += (l8 + 8 * q < E) && (kk[q] > mk);
            {
                const uint32_t dn = dpp_u<0x124>(cnt), up = dpp_u<0x12C>(cnt);
                cnt += (l8 & 4) ? dn : up;
            }
            cnt += dpp_u<0x4E>(cnt);
            cnt += dpp_u<0xB1>(cnt);
            if (l8 == 0 && e8 < E && cnt < top_k) { tk[cnt] = e8; tw[cnt] = g; }
        }
        __syncthreads();
        if (tid >= 64) {
            quantize_h();
            return;
        }
        const uint32_t rl = min((uint32_t)lane, top_k - 1);
        const uint32_t ei = tk[rl];
        const float twl = tw[rl];
        float s = 0.0f;   // every lane forms the same sequential sum (f32 iterator sum + 1e-9)
        if (weights_norm) {
            for (uint32_t r = 0; r < top_k; ++r) s = s + rlf(twl, r);
            s = s + 1e-9f;
        }
        uint32_t rk = 0;   // slot order by ascending expert id (the prompt path's accumulation order)
        for (uint32_t q = 0; q < top_k; ++q) rk += rlu(ei, q) < ei;
        if ((uint32_t)lane < top_k) {
            const uint32_t r = lane;
            const float wr_ = (weights_norm ? twl / s : twl) * weights_scale;
            topk_idx[r] = ei;
            topk_w[r] = wr_;
            rec_idx[r] = ei;
            rec_w[r] = wr_;
            order[rk] = r;
        }
        return;
    }
    if ((uint32_t)tid < E) sel[tid] = bv;   // bias, combined below
    __syncthreads();
    if (tid >= 64) {
        quantize_h();
        return;
    }
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // general path: lane owns experts lane, lane + 64, ...
    const uint32_t KE = div_up(E, 64);
    if (gating_sigmoid) {
        for (uint32_t k = 0; k < KE; ++k) {
            const uint32_t e = lane + 64 * k;
            const float sg = hg_sigmoid_l(lg[min(e, E - 1)], tab);
            if (e < E) scr[e] = sg;
        }
    } else {   // softmax (ops.rs:112-128): max, exp, sequential sum, scale by 1/sum
        float mx = -__builtin_huge_valf();
        for (uint32_t k = 0; k < KE; ++k)
            if (lane + 64 * k < E) mx = fmaxf(mx, lg[lane + 64 * k]);
        for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, shfl_xor(mx, m));
        for (uint32_t k = 0; k < KE; ++k) {
            const uint32_t e = lane + 64 * k;
            const float ex = hg_expf_l(lg[min(e, E - 1)] - mx, tab);
            if (e < E) scr[e] = ex;
        }
        wave_sync();
        float sum = 0.0f;
        for (uint32_t e = 0; e < E; ++e) sum = sum + scr[e];
        const float inv = 1.0f / sum;
        wave_sync();
        for (uint32_t k = 0; k < KE; ++k)
            if (lane + 64 * k < E) scr[lane + 64 * k] = scr[lane + 64 * k] * inv;
    }
    for (uint32_t k = 0; k < KE; ++k)
        if (lane + 64 * k < E) sel[lane + 64 * k] = scr[lane + 64 * k] + sel[lane + 64 * k];
    wave_sync();
    for (uint32_t k = 0; k < KE; ++k) {
        const uint32_t me_e = lane + 64 * k;
        if (me_e < E) {
            const float me = sel[me_e];
            uint32_t rank = 0;
            for (uint32_t e = 0; e < E; ++e) rank += (sel[e] > me) || (sel[e] == me && e < me_e);
            if (rank < top_k) { tk[rank] = me_e; tw[rank] = scr[me_e]; }
        }
    }
    wave_sync();
    float s = 0.0f;   // every lane forms the same sequential sum (f32 iterator sum + 1e-9)
    if (weights_norm) {
        for (uint32_t r = 0; r < top_k; ++r) s = s + tw[r];
        s = s + 1e-9f;
    }
    if ((uint32_t)lane < top_k) {
        const uint32_t r = lane, ei = tk[r];
        const float wr_ = (weights_norm ? tw[r] / s : tw[r]) * weights_scale;
        topk_idx[r] = ei;
        topk_w[r] = wr_;
        rec_idx[r] = ei;
        rec_w[r] = wr_;
        uint32_t rk = 0;   // slot order by ascending expert id (the prompt path's accumulation order)
        for (uint32_t q = 0; q < top_k; ++q) rk += tk[q] < ei;
        order[rk] = r;
    }
}

// ffn_norm RMSNorm, the F32 router and the gate/up rows of one expert slot in one launch (the
// router of k_ffn_router and the rows of k_ffn_gateup; model.rs:170-172, 270-305, 314-318).
// Workgroup (bx, slot) owns rows 16 bx .. 16 bx + 15 of the slot's expert: the routed pick
// `slot` (slot < top_k) or the shared expert; with E == 0 slot 0 is the dense FFN
// (model.rs:247-251).  Every workgroup forms the norm, the router logits and the ranking itself
// (the same deterministic arithmetic, so every workgroup picks the same experts) and quantizes h
// into its LDS, so the expert rows are fetched without a kernel boundary and without a round
// trip through memory; workgroup (0, 0) also writes the picks for the down projection.
// Threads: waves 0-1 form the index-order sum of squares while threads 128 + 8 e .. + 7 own
// router row e (prefetched meanwhile in the 16-byte-step layout of k_ffn_router); waves 0-1 then
// own the 16 gate/up rows.  Few
// rows per workgroup spread the expert rows, which cannot be fetched before the ranking, over
// many CUs (one CU issues about 64 bytes a clock).
constexpr uint32_t FF_NT = 512, FF_ROWS = 16;   // gate/up rows per workgroup: waves 0-1
constexpr uint32_t FF_MAXE = (FF_NT - 128) / 8;   // 48 experts
template <bool EXACT, int ORDER, bool SCF32, int NCT, int NST>
__global__ __launch_bounds__(512) void k_ffn_front(const float *__restrict__ x, const float *__restrict__ w, float eps,
                                                   uint32_t d, const float *__restrict__ Wp,
                                                   const float *__restrict__ bias, uint32_t E, uint32_t top_k,
                                                   int weights_norm, float weights_scale, Q8Mat Wg, Q8Mat Wu,
                                                   Q8Mat Sg, Q8Mat Su, uint32_t f, uint32_t *topk_idx,
                                                   float *topk_w, uint32_t *order, uint32_t *rec_idx,
                                                   float *rec_w, float *a_out) {
    static_assert(NST >= 1 && NST <= 32, "router steps held in registers");
    extern __shared__ __align__(16) float hs[];   // h, h permuted, squares (3 d), then sq / sd
    float *hp = hs + d, *ps = hs + 2 * d;
    uint8_t *sq = reinterpret_cast<uint8_t *>(hs + 3 * d);
    float *sd = reinterpret_cast<float *>(sq + Wg.nc * CHUNK_BYTES);
    __shared__ float red[FF_NT / 64];
    __shared__ float s_ss;
    __shared__ xsum::Scratch xs;
    __shared__ uint64_t K[64];
    __shared__ __align__(16) uint32_t tk[64];
    __shared__ __align__(16) float tw[64];
    const int tid = threadIdx.x, lane = tid & 63, j = tid & 7;
    const bool rows = tid >= 128;   // waves 2..7: the router rows (waves 0, 1 sum the squares)
    const uint32_t e8 = rows ? (uint32_t)(tid - 128) >> 3 : 0u, l8 = (uint32_t)tid & 7;
    const bool router = E > 0;
    const uint32_t slot = blockIdx.y, row = blockIdx.x * FF_ROWS + ((uint32_t)tid >> 3);
    const uint32_t lrow = min(row, f - 1);
    // loads in issue order: x and the norm gain (needed first), the exp table, the bias of this
    // thread's router row
    constexpr uint32_t XB = 2;   // d <= 1024 in registers
    float xv[XB], wv[XB];
#pragma unroll
    for (uint32_t u = 0; u < XB; ++u) {
        const uint32_t i = min(tid + u * FF_NT, d - 1);
        xv[u] = x[i];
        wv[u] = w[i];
    }
    const WaveExpTab tab = WaveExpTab::load(lane);
    const float bv8 = router ? bias[min(e8, E - 1)] : 0.0f;
    v4f wr[NST];
    auto fetch_rows = [&] {
        const float *rowp = Wp + (size_t)min(e8, E - 1) * d;
#pragma unroll
        for (int i = 0; i < NST; ++i) wr[i] = *reinterpret_cast<const v4f *>(rowp + 32 * i + 4 * l8);
    };
    float ss = 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < XB; ++u) {
        const uint32_t i = tid + u * FF_NT;
        if (i < d) {
            if (EXACT) ps[i] = xv[u] * xv[u];
            else ss += xv[u] * xv[u];
        }
    }
    if (EXACT) {
        if (tid == 0) xs.sync = 0;
        __syncthreads();
        if (router && rows && e8 < E) fetch_rows();   // arrives during the sum
        if (tid < 128) {
            const float r = block_seq_sum<2, 8>(ps, d, xs, tid >> 6, lane);   // ss += v * v in index order
            if (tid == 0) s_ss = r;
        }
    } else {
        for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor(ss, m);
        if (lane == 0) red[tid >> 6] = ss;
        __syncthreads();
        if (router && rows && e8 < E) fetch_rows();
        if (tid == 0) {
            float t = 0.0f;
            for (int i = 0; i < (int)(FF_NT / 64); ++i) t += red[i];
            s_ss = t;
        }
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf(s_ss / (float)d + eps);
#pragma unroll
    for (uint32_t u = 0; u < XB; ++u) {
        const uint32_t i = tid + u * FF_NT;
        if (i < d) {
            const float v = xv[u] * scale * wv[u];
            hs[i] = v;
            hp[router_perm(i)] = v;
        }
    }
    __syncthreads();
    if (tid < 128) {   // quantization of h for the expert rows (quant.rs:111-123), into this
                       // workgroup's LDS, by waves 0-1 while the router waves form the logits
        const uint32_t nb = d / QK;
        for (uint32_t b0 = 0; b0 < nb; b0 += 16) {
            const uint32_t b = b0 + ((uint32_t)tid >> 3);
            const v4f hv = *reinterpret_cast<const v4f *>(hs + min(b, nb - 1) * QK + j * 4);
            const float v[4] = {hv.x, hv.y, hv.z, hv.w};
            quant_block_lane(v, j, min(b, nb - 1), sq, sd, b < nb);
        }
        zero_pad(nb, Wg.nc, sq, sd, tid, 128);
    }
    float g = 0.0f;   // the gate of this thread's router row
    if (router) {
        if (rows) {   // logits: lane l8 of row e8 runs the ops::dot chains l8 + 8 a (uniform per wave)
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (e8 < E) {
#pragma unroll
                for (int i = 0; i < NST; ++i) {
                    const v4f hv = *reinterpret_cast<const v4f *>(hp + 32 * i + 4 * l8);
                    a[0] = fmaf(wr[i].x, hv.x, a[0]);
                    a[1] = fmaf(wr[i].y, hv.y, a[1]);
                    a[2] = fmaf(wr[i].z, hv.z, a[2]);
                    a[3] = fmaf(wr[i].w, hv.w, a[3]);
                }
            }
            float v = (a[0] + a[1]) + (a[2] + a[3]);
            {
                const float dn = dpp_f<0x124>(v), up = dpp_f<0x12C>(v);
                v = v + ((l8 & 4) ? dn : up);   // lane ^ 4
            }
            v = v + dpp_f<0x4E>(v);   // lane ^ 2
            v = v + dpp_f<0xB1>(v);   // lane ^ 1
            g = hg_sigmoid_l(v, tab);
            const float key = (g + bv8) + 0.0f;   // -0 made +0 (the float compare has -0 == +0)
            const uint32_t mb = __builtin_bit_cast(uint32_t, key);
            const uint64_t mk = ((uint64_t)((mb & 0x80000000u) ? ~mb : (mb | 0x80000000u)) << 32) | (uint32_t)~e8;
            if (l8 == 0 && e8 < E) K[e8] = mk;
        }
        __syncthreads();
        if (rows) {   // rank = #{e' : key_e' > key_e or equal with e' < e}: lane l8 counts e' = l8 + 8 q
            const float key = (g + bv8) + 0.0f;
            const uint32_t mb = __builtin_bit_cast(uint32_t, key);
            const uint64_t mk = ((uint64_t)((mb & 0x80000000u) ? ~mb : (mb | 0x80000000u)) << 32) | (uint32_t)~e8;
            uint64_t kk[8];
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q) kk[q] = K[min(l8 + 8 * q, E - 1)];
            uint32_t cnt = 0;
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q) cnt += (l8 + 8 * q < E) && (kk[q] > mk);
            {
                const uint32_t dn = dpp_u<0x124>(cnt), up = dpp_u<0x12C>(cnt);
                cnt += (l8 & 4) ? dn : up;
            }
            cnt += dpp_u<0x4E>(cnt);
            cnt += dpp_u<0xB1>(cnt);
            if (l8 == 0 && e8 < E && cnt < top_k) { tk[cnt] = e8; tw[cnt] = g; }
        }
    }
    __syncthreads();
    if (tid >= (int)(8 * FF_ROWS)) return;   // the router needed every wave, the rows need two
    // the slot's rows
    const bool routed = router && slot < top_k;
    const Q8Mat &G = routed ? Wg : Sg;
    const Q8Mat &U = routed ? Wu : Su;
    const uint32_t r = routed ? tk[slot] * f + lrow : lrow;
    Q8Row<ORDER, SCF32, NCT> rg, ru;
    rg.begin(row_qs(G, r), row_sc<SCF32>(G, r), G.nb, G.nc, j);
    ru.begin(row_qs(U, r), row_sc<SCF32>(U, r), U.nb, U.nc, j);
    if (router && blockIdx.x == 0 && slot == 0 && tid < 64) {   // the picks for the down projection
        auto rlf = [](float v, uint32_t l) {
            return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)l));
        };
        auto rlu = [](uint32_t v, uint32_t l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l); };
        const uint32_t rl = min((uint32_t)lane, top_k - 1);
        const uint32_t ei = tk[rl];
        const float twl = tw[rl];
        float sw = 0.0f;   // every lane forms the same sequential sum (f32 iterator sum + 1e-9)
        if (weights_norm) {
            for (uint32_t q = 0; q < top_k; ++q) sw = sw + rlf(twl, q);
            sw = sw + 1e-9f;
        }
        uint32_t rk = 0;   // slot order by ascending expert id (the prompt path's accumulation order)
        for (uint32_t q = 0; q < top_k; ++q) rk += rlu(ei, q) < ei;
        if ((uint32_t)lane < top_k) {
            const float wr_ = (weights_norm ? twl / sw : twl) * weights_scale;
            topk_idx[lane] = ei;
            topk_w[lane] = wr_;
            rec_idx[lane] = ei;
            rec_w[lane] = wr_;
            order[rk] = (uint32_t)lane;
        }
    }
    const float gv = rg.finish(sq, sd);
    const float uv = ru.finish(sq, sd);
    const float av = hg_silu_l(gv, tab) * uv;   // every lane: the table lookup is a lane exchange
    if (row < f && j == 0) a_out[(size_t)slot * f + row] = av;
}

// ------------------------------------------------------------------ experts
// Gate and up rows of every active expert slot and a = silu(g)*u (model.rs:301-305,
// 314-318; dense: 247-251).  blockIdx.y = slot: slots < top_k are routed experts
// (topk_idx), the next one the shared expert (or the dense FFN).  8 rows per workgroup.
template <int ORDER, bool SCF32, int NCT>
__global__ __launch_bounds__(64) void k_ffn_gateup(Q8Mat Wg, Q8Mat Wu, Q8Mat Sg, Q8Mat Su,
                                                   const uint32_t *__restrict__ topk_idx, uint32_t top_k,
                                                   uint32_t f, const uint8_t *__restrict__ gq,
                                                   const float *__restrict__ gd, float *a_out) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *sq = smem;
    float *sd = reinterpret_cast<float *>(smem + Wg.nc * CHUNK_BYTES);
    const int tid = threadIdx.x;
    const uint32_t slot = blockIdx.y;
    const uint32_t i = blockIdx.x * 8 + (tid >> 3);
    const uint32_t li = min(i, f - 1);
    const int j = tid & 7;
    const bool routed = slot < top_k;
    const Q8Mat &G = routed ? Wg : Sg;
    const Q8Mat &U = routed ? Wu : Su;
    // loads in issue order: the router's pick, the activation (first 2 x 64 chunks in
    // registers) and the exp table, then the rows the pick selects
    const uint32_t e = routed ? topk_idx[slot] : 0u;
    const uint32_t nc = Wg.nc;
    v4i qv[2];
#pragma unroll
    for (uint32_t u = 0; u < 2; ++u) qv[u] = reinterpret_cast<const v4i *>(gq)[min(u * 64 + (uint32_t)tid, nc * 8 - 1)];
    const float dv = gd[min((uint32_t)tid, nc * 4 - 1)];
    const WaveExpTab tab = WaveExpTab::load(tid);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t r = routed ? e * f + li : li;
    Q8Row<ORDER, SCF32, NCT> rg, ru;
    rg.begin(row_qs(G, r), row_sc<SCF32>(G, r), G.nb, G.nc, j);
    ru.begin(row_qs(U, r), row_sc<SCF32>(U, r), U.nb, U.nc, j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t u = 0; u < 2; ++u)   // (clamped slots rewrite the value they already hold)
        reinterpret_cast<v4i *>(sq)[min(u * 64 + (uint32_t)tid, nc * 8 - 1)] = qv[u];
    for (uint32_t q = 128 + (uint32_t)tid; q < nc * 8; q += 64)
        reinterpret_cast<v4i *>(sq)[q] = reinterpret_cast<const v4i *>(gq)[q];
    sd[min((uint32_t)tid, nc * 4 - 1)] = dv;
    for (uint32_t q = (uint32_t)tid + 64; q < nc * 4; q += 64) sd[q] = gd[q];
    __syncthreads();
    const float g = rg.finish(sq, sd);
    const float u = ru.finish(sq, sd);
    const float a = hg_silu_l(g, tab) * u;   // every lane: the table lookup is a lane exchange
    if (i < f && j == 0) a_out[(size_t)slot * f + i] = a;
}

// Down rows of every slot and the fixed-order combination (model.rs:306-323; dense:
// 253-254), then the residual add x += ffn (model.rs:173-176).  One wave per slot; each
// wave quantizes its slot's activation a[slot] (quant.rs:111-123) into LDS.
//   decode:  out = ((0 + w_0 y_0) + w_1 y_1 ...) + y_shared    (rank order)
//   prefill: the same sum in ascending expert-id order (model.rs:707-731)
//   dense:   x += y
template <int ORDER, bool SCF32, int NCT>
__global__ __launch_bounds__(1024) void k_ffn_down(Q8Mat Wd, Q8Mat Sd, const uint32_t *__restrict__ topk_idx,
                                                   const float *__restrict__ topk_w,
                                                   const uint32_t *__restrict__ order, uint32_t top_k,
                                                   uint32_t n_slots, int dense, uint32_t d, uint32_t f,
                                                   const float *__restrict__ a, float *x) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t nc = Sd.nc, nb = Sd.nb;
    const size_t per = (size_t)nc * CHUNK_BYTES + (size_t)nc * 4 * sizeof(float);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *ys = reinterpret_cast<float *>(smem + per * n_slots);  // [n_slots][8]
    const uint32_t slot = wave;
    uint8_t *sq = smem + per * slot;
    float *sd = reinterpret_cast<float *>(sq + (size_t)nc * CHUNK_BYTES);
    const uint32_t r = blockIdx.x * 8 + (lane >> 3);
    const uint32_t lr = min(r, d - 1);
    const int j = lane & 7;
    __shared__ float wsl[64];   // combine weights topk_w[0..top_k)
    const bool routed = slot < top_k;
    const Q8Mat &D = routed ? Wd : Sd;
    // loads in issue order: the slot's activation (lane j of blocks b = 8u + lane/8) and the
    // combine weights, then the down row, whose index waits for the router's pick
    const float *as = a + (size_t)slot * f;
    constexpr uint32_t AB = 4;
    v4f av[AB];
#pragma unroll
    for (uint32_t u = 0; u < AB; ++u) {
        const uint32_t b = min(u * 8 + (lane >> 3), nb - 1);
        av[u] = *reinterpret_cast<const v4f *>(as + b * QK + j * 4);
    }
    const float wsel = (!dense && top_k) ? topk_w[min((uint32_t)lane, top_k - 1)] : 0.0f;
    const float xold = x[min(blockIdx.x * 8 + (uint32_t)(tid & 7), d - 1)];   // the residual, used by tid < 8
    const uint32_t row = routed ? topk_idx[slot] * d + lr : lr;
    Q8Row<ORDER, SCF32, NCT> rd;
    rd.begin(row_qs(D, row), row_sc<SCF32>(D, row), nb, nc, j);
#pragma unroll
    for (uint32_t u = 0; u < AB; ++u) {   // a block's 8 lanes are all in or all out
        const uint32_t b = u * 8 + (lane >> 3);
        const float v[4] = {av[u].x, av[u].y, av[u].z, av[u].w};
        quant_block_lane(v, j, min(b, nb - 1), sq, sd, b < nb);
    }
    for (uint32_t b0 = AB * 8; b0 < nb; b0 += 8) {
        const uint32_t b = b0 + (lane >> 3);
        if (b < nb) {
            float v[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) v[m] = as[b * QK + j * 4 + m];
            quant_block_lane(v, j, b, sq, sd);
        }
    }
    zero_pad(nb, nc, sq, sd, lane, 64);
    __syncthreads();
    const float y = rd.finish(sq, sd);
    if (j == 0) ys[slot * 8 + (lane >> 3)] = y;
    if (wave == 0 && (uint32_t)lane < top_k) wsl[lane] = wsel;
    __syncthreads();
    if (tid < 8) {
        const uint32_t rr = blockIdx.x * 8 + tid;
        if (rr < d) {
            if (dense) {
                x[rr] = xold + ys[tid];
            } else {
                float acc = 0.0f;
                for (uint32_t q = 0; q < top_k; ++q) {
                    const uint32_t s = (ORDER == ORDER_PREFILL) ? order[q] : q;
                    acc = acc + wsl[s] * ys[s * 8 + tid];
                }
                if (n_slots > top_k) acc = acc + ys[top_k * 8 + tid];
                x[rr] = xold + acc;
            }
        }
    }
}

// ====================================================================== launchers
// While a LaunchTimer is installed on this thread, every launch carries a start/stop event
// pair recorded by its own dispatch (hipExtLaunchKernelGGL): the kernel's execution time.
thread_local LaunchTimer *g_timer = nullptr;
void set_launch_timer(LaunchTimer *t) { g_timer = t; }
LaunchTimer *launch_timer() { return g_timer; }

// The first launch error since the last take: a launch HIP rejected (its error code) or one
// the launch helpers refused on the host (hipErrorInvalidConfiguration).
thread_local hipError_t g_launch_err = hipSuccess;
thread_local std::string g_launch_msg;
void note_launch_error(hipError_t e, const std::string &what) {
    if (g_launch_err != hipSuccess) return;
    g_launch_err = e;
    g_launch_msg = what + ": " + hipGetErrorString(e);
}
hipError_t take_launch_error(std::string &msg) {
    const hipError_t e = g_launch_err;
    msg = g_launch_msg;
    g_launch_err = hipSuccess;
    g_launch_msg.clear();
    return e;
}
hipError_t take_launch_error_reset() {
    std::string m;
    return take_launch_error(m);
}

#define LAUNCH(kern, grid, block, shm, st, ...)                                                              \
    do {                                                                                                     \
        if (g_timer) {                                                                                       \
            hipEvent_t a_ = nullptr, b_ = nullptr;                                                           \
            (void)hipEventCreate(&a_);                                                                       \
            (void)hipEventCreate(&b_);                                                                       \
            hipExtLaunchKernelGGL(kern, grid, block, shm, st, a_, b_, 0, __VA_ARGS__);                       \
            g_timer->add(a_, b_);                                                                            \
        } else {                                                                                             \
            hipLaunchKernelGGL(kern, grid, block, shm, st, __VA_ARGS__);                                     \
        }                                                                                                    \
        const hipError_t le_ = hipGetLastError();                                                            \
        if (le_ != hipSuccess) note_launch_error(le_, #kern);                                                \
    } while (0)

// Kernels whose LDS exceeds the 64 KiB default opt in to the larger gfx950 allocation.
hipError_t init_kernel_attributes() {
    hipError_t e = hipSuccess;
#define PV_ATTR(HD)                                                                                         \
    if (e == hipSuccess)                                                                                    \
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attn_softmax_pv<HD>),                     \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)PV_LDS_BUDGET);
    PV_ATTR(32) PV_ATTR(64) PV_ATTR(128)
#undef PV_ATTR
#define PVR_ATTR(HD)                                                                                        \
    if (e == hipSuccess)                                                                                    \
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attn_softmax_pv_res<HD, false>),          \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)PV_LDS_BUDGET);            \
    if (e == hipSuccess)                                                                                    \
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attn_softmax_pv_res<HD, true>),           \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)PV_LDS_BUDGET);
    PVR_ATTR(32) PVR_ATTR(64) PVR_ATTR(128)
#undef PVR_ATTR
#define QKS_ATTR(O, S, N)                                                                                    \
    if (e == hipSuccess)                                                                                     \
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_qkv_head<true, O, S, N, 64, true>),        \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)PV_LDS_BUDGET);
#define QKS_ATTR_N(O, S) QKS_ATTR(O, S, 1) QKS_ATTR(O, S, 2) QKS_ATTR(O, S, 4) QKS_ATTR(O, S, 8)
    QKS_ATTR_N(ORDER_DECODE, false) QKS_ATTR_N(ORDER_DECODE, true) QKS_ATTR_N(ORDER_PREFILL, false)
    QKS_ATTR_N(ORDER_PREFILL, true)
#undef QKS_ATTR_N
#undef QKS_ATTR
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attn_softmax_pv_res<64, false, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)PV_LDS_BUDGET);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attn_softmax_pv_res<64, true, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)PV_LDS_BUDGET);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_seq_sum), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)((SEQSUM_MAX + 4) * sizeof(float)));
    return e;
}

// Chunks per load batch of a row of nc chunks.
static int nct_of(uint32_t nc) { return nc >= 8 ? 8 : nc >= 4 ? 4 : nc >= 2 ? 2 : 1; }

// Instantiate F<NCT> for the runtime batch size.
#define DISPATCH_NCT(nc, F)                  \
    switch (nct_of(nc)) {                    \
    case 8: F(8); break;                     \
    case 4: F(4); break;                     \
    case 2: F(2); break;                     \
    default: F(1); break;                    \
    }

void launch_embed(hipStream_t st, const float *emb, uint32_t d, const StepParams *p, float *x) {
    LAUNCH(k_embed, dim3(div_up(d, 256)), dim3(256), 0, st, emb, d, p, x);
}
void launch_load_row(hipStream_t st, const float *inputs, uint32_t d, const StepParams *p, float *x) {
    LAUNCH(k_load_row, dim3(div_up(d, 256)), dim3(256), 0, st, inputs, d, p, x);
}
void launch_advance(hipStream_t st, StepParams *p) { LAUNCH(k_advance, dim3(1), dim3(64), 0, st, p); }

void launch_seq_sum(hipStream_t st, const float *x, uint32_t n, int method, float *out) {
    const size_t shm = ((method == 7 ? SEQSUM_MAX : 4096) + 4) * sizeof(float);
    LAUNCH(k_seq_sum, dim3(1), dim3(512), shm, st, x, n, method, out);
}

void launch_rmsnorm_quant(hipStream_t st, bool exact, const float *x, const float *w, float eps, uint32_t d,
                          float *h, uint8_t *q, float *dq) {
    launch_rmsnorm_quant_rows(st, exact, 1, x, w, eps, d, h, q, dq);
}

void launch_rmsnorm_quant_rows(hipStream_t st, bool exact, uint32_t rows, const float *x, const float *w, float eps,
                               uint32_t d, float *h, uint8_t *q, float *dq) {
    const size_t shm = 2 * d * sizeof(float);
    const uint32_t nc = div_up(d / QK, 4);
    const RowStrides rs{d, nc * CHUNK_BYTES, nc * 4, 0, 0};
    if (exact) LAUNCH(k_rmsnorm_quant<true>, dim3(rows), dim3(256), shm, st, x, w, eps, d, h, q, dq, rs);
    else LAUNCH(k_rmsnorm_quant<false>, dim3(rows), dim3(256), shm, st, x, w, eps, d, h, q, dq, rs);
}

void launch_quant_vec(hipStream_t st, const float *x, uint32_t n, uint8_t *q, float *dq) {
    LAUNCH(k_quant_vec, dim3(div_up(n / QK, 32)), dim3(256), 0, st, x, n, q, dq);
}

uint32_t matvec_blocks(uint32_t N, uint32_t threads) { return div_up(N, threads / 8); }

template <int ORDER, int EPI, bool SCF32>
static void mv_launch(hipStream_t st, const Q8Mat &W, const uint8_t *q, const float *dq, float *y, uint32_t threads,
                      uint32_t valid, float *pv, uint32_t *pi) {
    const dim3 grid(matvec_blocks(W.N, threads)), block(threads);
    const size_t shm = (size_t)W.nc * CHUNK_BYTES + (size_t)W.nc * 4 * sizeof(float);
    if (dq == nullptr) {  // q holds an f32 activation, quantized by each workgroup
#define MVKF(N) LAUNCH((k_matvec<ORDER, EPI, SCF32, N, true>), grid, block, shm, st, W, q, dq, y, valid, pv, pi)
        DISPATCH_NCT(W.nc, MVKF)
#undef MVKF
        return;
    }
#define MVK(N) LAUNCH((k_matvec<ORDER, EPI, SCF32, N>), grid, block, shm, st, W, q, dq, y, valid, pv, pi)
    DISPATCH_NCT(W.nc, MVK)
#undef MVK
}

void launch_matvec(hipStream_t st, int order, int epi, const Q8Mat &W, const uint8_t *q, const float *dq, float *y,
                   uint32_t threads, uint32_t valid, float *pv, uint32_t *pi) {
    if (threads < 64 || threads > 256 || threads % 64) {   // k_matvec: __launch_bounds__(256), whole waves
        note_launch_error(hipErrorInvalidConfiguration, "k_matvec with " + std::to_string(threads) + " threads");
        return;
    }
#define MV(O, E)                                                                   \
    do {                                                                           \
        if (W.sc_f32) mv_launch<O, E, true>(st, W, q, dq, y, threads, valid, pv, pi);  \
        else mv_launch<O, E, false>(st, W, q, dq, y, threads, valid, pv, pi);          \
    } while (0)
    if (order == ORDER_DECODE) {
        if (epi == EPI_STORE) MV(ORDER_DECODE, EPI_STORE);
        else if (epi == EPI_RESID) MV(ORDER_DECODE, EPI_RESID);
        else MV(ORDER_DECODE, EPI_LOGITS);
    } else {
        if (epi == EPI_STORE) MV(ORDER_PREFILL, EPI_STORE);
        else if (epi == EPI_RESID) MV(ORDER_PREFILL, EPI_RESID);
        else MV(ORDER_PREFILL, EPI_LOGITS);
    }
#undef MV
}

bool launch_qkv_head(hipStream_t st, bool exact, int order, uint32_t hd, const Q8Mat &W, const float *x,
                     const float *w, float eps, const float *qn, const float *kn, const float *cs, const float *sn,
                     const StepParams *p, uint32_t n_heads, uint32_t n_kv, float *kc, float *vc, uint32_t cap,
                     float *out) {
    const dim3 grid(n_heads + 2 * n_kv);
    const size_t shm = (size_t)W.nc * CHUNK_BYTES + (size_t)W.nc * 4 * sizeof(float) + (size_t)W.K * sizeof(float);
#define QKH(E, O, S, N, HD)                                                                                     \
    LAUNCH((k_qkv_head<E, O, S, N, HD>), grid, dim3(QkvCfg<HD>::NT), shm, st, W, x, w, eps, qn, kn, cs, sn, p, \
           n_heads, n_kv, kc, vc, cap, out, 0u, 0u, nullptr, nullptr)
#define QKH_S(E, O, N, HD)                  \
    do {                                    \
        if (W.sc_f32) QKH(E, O, true, N, HD);  \
        else QKH(E, O, false, N, HD);          \
    } while (0)
#define QKH_O(N, HD)                                      \
    do {                                                  \
        if (order == ORDER_DECODE) {                      \
            if (exact) QKH_S(true, ORDER_DECODE, N, HD);  \
            else QKH_S(false, ORDER_DECODE, N, HD);       \
        } else {                                          \
            if (exact) QKH_S(true, ORDER_PREFILL, N, HD); \
            else QKH_S(false, ORDER_PREFILL, N, HD);      \
        }                                                 \
    } while (0)
#define QKH_N(HD)                    \
    switch (nct_of(W.nc)) {          \
    case 8: QKH_O(8, HD); break;     \
    case 4: QKH_O(4, HD); break;     \
    case 2: QKH_O(2, HD); break;     \
    default: QKH_O(1, HD); break;    \
    }
    switch (hd) {
    case 32: QKH_N(32); break;
    case 64: QKH_N(64); break;
    case 128: QKH_N(128); break;
    default: return false;
    }
#undef QKH_N
#undef QKH_O
#undef QKH_S
#undef QKH
    return true;
}

// Score splits of a window: at most QKV_SCORE_POS positions each, and as many more (down to 64
// positions each) as keep the launch within one workgroup per CU; a multiple of the XCDs per kv
// group.
uint32_t qkv_score_splits(uint32_t win, uint32_t n_heads, uint32_t n_kv) {
    static const uint32_t n_cu = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            v = 0;
        return (uint32_t)v;
    }();
    const uint32_t xq = n_kv && n_kv <= 8 && 8 % n_kv == 0 ? 8 / n_kv : 1;
    const uint32_t need = div_up(div_up(win, QKV_SCORE_POS), xq) * xq;
    const uint32_t fill = n_heads && n_cu > 2 * n_kv ? (n_cu - 2 * n_kv) / n_heads / xq * xq : 0;
    const uint32_t most = div_up(div_up(win, 64), xq) * xq;
    return std::max(need, std::min(fill, most));
}
// k_qkv_head's dynamic LDS with SC: the activation, its scales, the squares, the split's K rows
static size_t qkv_scores_lds(uint32_t d, uint32_t win, uint32_t n_heads, uint32_t n_kv) {
    const size_t nc = div_up(d / 32, 4), c = div_up(win, qkv_score_splits(win, n_heads, n_kv));
    return nc * CHUNK_BYTES + nc * 4 * sizeof(float) + (size_t)d * sizeof(float) + div_up(c, 4) * 4 * 64 * sizeof(float);
}
bool qkv_scores_ok(bool exact, uint32_t hd, uint32_t win, uint32_t n_heads, uint32_t n_kv, uint32_t d) {
    // (the split maxima fit the attention partials buffer, attn_splits(cap) (hd + 2) floats a head)
    return exact && hd == 64 && n_kv && n_heads % n_kv == 0 && pv_res_fits(win) && d % 32 == 0 &&
           qkv_scores_lds(d, win, n_heads, n_kv) <= PV_LDS_BUDGET &&
           qkv_score_splits(win, n_heads, n_kv) <= attn_splits(win) * (hd + 2);
}

bool launch_qkv_scores(hipStream_t st, int order, const Q8Mat &W, const float *x, const float *w, float eps,
                       const float *qn, const float *kn, const float *cs, const float *sn, const StepParams *p,
                       uint32_t n_heads, uint32_t n_kv, float *kc, float *vc, uint32_t cap, uint32_t win, float *out,
                       float *scores, float *pmax) {
    if (!qkv_scores_ok(true, 64, win, n_heads, n_kv, W.K) || win > cap || W.nc != div_up(W.K / 32, 4)) return false;
    const uint32_t S2 = qkv_score_splits(win, n_heads, n_kv);
    static_assert(QKV_SCORE_POS <= 8 * 64, "one position per row thread");
    const dim3 grid(n_heads * S2 + 2 * n_kv);
    const size_t shm = qkv_scores_lds(W.K, win, n_heads, n_kv);
#define QKS(O, S, N)                                                                                               \
    LAUNCH((k_qkv_head<true, O, S, N, 64, true>), grid, dim3(QkvCfg<64>::NT), shm, st, W, x, w, eps, qn, kn, cs, sn, \
           p, n_heads, n_kv, kc, vc, cap, out, win, S2, scores, pmax)
#define QKS_S(O, N)                  \
    do {                             \
        if (W.sc_f32) QKS(O, true, N);  \
        else QKS(O, false, N);          \
    } while (0)
#define QKS_O(N)                                          \
    do {                                                  \
        if (order == ORDER_DECODE) QKS_S(ORDER_DECODE, N); \
        else QKS_S(ORDER_PREFILL, N);                      \
    } while (0)
    switch (nct_of(W.nc)) {
    case 8: QKS_O(8); break;
    case 4: QKS_O(4); break;
    case 2: QKS_O(2); break;
    default: QKS_O(1); break;
    }
#undef QKS_O
#undef QKS_S
#undef QKS
    return true;
}

bool launch_qk_rope_append(hipStream_t st, uint32_t hd, float *qkv, const float *qn, const float *kn, float eps,
                           const float *cs, const float *sn, const StepParams *p, uint32_t n_heads, uint32_t n_kv,
                           float *kc, float *vc, uint32_t cap) {
    const dim3 grid(n_heads + 2 * n_kv);
    switch (hd) {
    case 32: LAUNCH(k_qk_rope_append<32>, grid, dim3(64), 0, st, qkv, qn, kn, eps, cs, sn, p, n_heads, n_kv, kc, vc, cap); break;
    case 64: LAUNCH(k_qk_rope_append<64>, grid, dim3(64), 0, st, qkv, qn, kn, eps, cs, sn, p, n_heads, n_kv, kc, vc, cap); break;
    case 128: LAUNCH(k_qk_rope_append<128>, grid, dim3(64), 0, st, qkv, qn, kn, eps, cs, sn, p, n_heads, n_kv, kc, vc, cap); break;
    default: return false;
    }
    return true;
}

void launch_matvec_gather(hipStream_t st, const Q8Mat &W, uint32_t rows_per_mat, const uint32_t *ids, uint32_t n_ids,
                          const uint8_t *q, const float *dq, float *y) {
    const dim3 grid(div_up(rows_per_mat, 32), n_ids);
    const size_t shm = (size_t)W.nc * CHUNK_BYTES + (size_t)W.nc * 4 * sizeof(float);
#define MGK(N)                                                                                               \
    do {                                                                                                     \
        if (W.sc_f32) LAUNCH((k_matvec_gather<true, N>), grid, dim3(256), shm, st, W, rows_per_mat, ids, q, dq, y);   \
        else LAUNCH((k_matvec_gather<false, N>), grid, dim3(256), shm, st, W, rows_per_mat, ids, q, dq, y);           \
    } while (0)
    DISPATCH_NCT(W.nc, MGK)
#undef MGK
}

void launch_argmax_final(hipStream_t st, const float *pv, const uint32_t *pi, uint32_t n, StepParams *p,
                         uint32_t *out_ids) {
    LAUNCH(k_argmax_final, dim3(1), dim3(1024), 0, st, pv, pi, n, p, out_ids);
}

size_t attn_fast_shm(uint32_t hd, uint32_t rep, uint32_t cap, uint32_t S) {
    const uint32_t tok = 256 / (hd / 4);
    const size_t floats = (size_t)(rep + 2) * hd + (size_t)(rep + 1) * hd + 4 * hd + (size_t)rep * attn_maxchunk(cap, S) +
                          (size_t)tok * rep * hd + 2 * rep;
    return floats * sizeof(float);
}

template <int HD>
static void attn_exact_launch(hipStream_t st, int which, const float *qkv, const float *qn, const float *kn,
                              float eps, const float *cs, const float *sn, const StepParams *p, float *kc, float *vc,
                              uint32_t cap, uint32_t win, uint32_t n_heads, uint32_t n_kv, uint32_t S, float *part,
                              float *scratch, float *o_out, uint8_t *q_out, float *d_out) {
    const bool fuse_quant = q_out == nullptr;  // the consumer quantizes o itself
    if (which == 0) {
        LAUNCH(k_attn_scores<HD>, dim3(n_kv, S), dim3(256), 0, st, qkv, p, kc, cap, win, n_heads, n_kv, S,
               scratch, part);
        return;
    }
    if (pv_res_fits(win)) {
        if (pv_res_rows(win) <= PvResCfg::SHORT)
            LAUNCH((k_attn_softmax_pv_res<HD, false>), dim3(n_heads * (HD / PvResCfg::D)), dim3(512), pv_res_lds(win),
                   st, scratch, part, qkv, p, vc, cap, win, S, n_heads, n_kv, o_out);
        else
            LAUNCH((k_attn_softmax_pv_res<HD, true>), dim3(n_heads * (HD / PvResCfg::D)), dim3(512), pv_res_lds(win),
                   st, scratch, part, qkv, p, vc, cap, win, S, n_heads, n_kv, o_out);
    } else {
        const size_t shm = (size_t)div_up(win, 4) * 16 + (size_t)pv_ring_slots(win) * PvCfg::SLOT * 4 + XSUM_FLOATS * 4;
        LAUNCH(k_attn_softmax_pv<HD>, dim3(n_heads * (HD / PvCfg::D)), dim3(PvCfg::NW * 64), shm, st, scratch, part, qkv,
               p, vc, cap, win, S, n_heads, n_kv, o_out, q_out, d_out);
    }
    if (!fuse_quant) LAUNCH(k_quant_o, dim3(1), dim3(256), 0, st, o_out, n_heads * HD, q_out, d_out);
}

template <int HD>
static void attn_fast_launch(hipStream_t st, int which, const float *qkv, const float *qn, const float *kn, float eps,
                             const float *cs, const float *sn, const StepParams *p, float *kc, float *vc,
                             uint32_t cap, uint32_t win, uint32_t n_heads, uint32_t n_kv, uint32_t S, float *part,
                             float *o_out, uint8_t *q_out, float *d_out) {
    if (which == 0) {
        const size_t shm = attn_fast_shm(HD, n_heads / n_kv, win, S);
        LAUNCH(k_attn_fast<HD>, dim3(n_kv, S), dim3(256), shm, st, qkv, qn, kn, eps, cs, sn, p, kc, vc, cap, win,
               n_heads, n_kv, S, part);
        return;
    }
    LAUNCH(k_attn_combine<HD>, dim3(n_heads), dim3(256), 0, st, part, n_heads, S, o_out, q_out, d_out);
}

void launch_attn_pv_self(hipStream_t st, const float *qkv, const StepParams *p, float *vc, uint32_t cap, uint32_t win,
                         uint32_t n_heads, uint32_t n_kv, float *part, float *scratch, float *o_out) {
    constexpr int HD = 64;
    const uint32_t S2 = qkv_score_splits(win, n_heads, n_kv);
    if (pv_res_rows(win) <= PvResCfg::SHORT)
        LAUNCH((k_attn_softmax_pv_res<HD, false, true>), dim3(n_heads * (HD / PvResCfg::D)), dim3(512), pv_res_lds(win),
               st, scratch, part, qkv, p, vc, cap, win, S2, n_heads, n_kv, o_out);
    else
        LAUNCH((k_attn_softmax_pv_res<HD, true, true>), dim3(n_heads * (HD / PvResCfg::D)), dim3(512), pv_res_lds(win),
               st, scratch, part, qkv, p, vc, cap, win, S2, n_heads, n_kv, o_out);
}

bool launch_attn(hipStream_t st, bool exact, int which, uint32_t hd, const float *qkv, const float *qn,
                 const float *kn, float eps, const float *cs, const float *sn, const StepParams *p, float *kc,
                 float *vc, uint32_t cap, uint32_t win, uint32_t n_heads, uint32_t n_kv, uint32_t S, float *part,
                 float *scratch, float *o_out, uint8_t *q_out, float *d_out) {
#define ATTN(HD)                                                                                                    \
    do {                                                                                                            \
        if (exact)                                                                                                  \
            attn_exact_launch<HD>(st, which, qkv, qn, kn, eps, cs, sn, p, kc, vc, cap, win, n_heads, n_kv, S, part, \
                                  scratch, o_out, q_out, d_out);                                                    \
        else                                                                                                        \
            attn_fast_launch<HD>(st, which, qkv, qn, kn, eps, cs, sn, p, kc, vc, cap, win, n_heads, n_kv, S, part,  \
                                 o_out, q_out, d_out);                                                              \
    } while (0)
    if (hd == 64) ATTN(64);
    else if (hd == 128) ATTN(128);
    else if (hd == 32) ATTN(32);
    else return false;
#undef ATTN
    return true;
}

void launch_ffn_router(hipStream_t st, bool exact, const float *x, const float *w, float eps, uint32_t d,
                       const float *Wr, const float *Wp, const float *bias, uint32_t E, uint32_t top_k,
                       int gating_sigmoid, int weights_norm, float weights_scale, uint8_t *q, float *dq,
                       uint32_t *topk_idx, float *topk_w, uint32_t *order, uint32_t *rec_idx, float *rec_w) {
    launch_ffn_router_rows(st, exact, 1, RowStrides{}, x, w, eps, d, Wr, Wp, bias, E, top_k, gating_sigmoid,
                           weights_norm, weights_scale, q, dq, topk_idx, topk_w, order, rec_idx, rec_w);
}

void launch_ffn_router_rows(hipStream_t st, bool exact, uint32_t rows, RowStrides rs, const float *x, const float *w,
                            float eps, uint32_t d, const float *Wr, const float *Wp, const float *bias, uint32_t E,
                            uint32_t top_k, int gating_sigmoid, int weights_norm, float weights_scale, uint8_t *q,
                            float *dq, uint32_t *topk_idx, float *topk_w, uint32_t *order, uint32_t *rec_idx,
                            float *rec_w) {
    const size_t shm = 3 * d * sizeof(float);
    const uint32_t nt = router_threads(E);
    // up to 512 threads (E <= 64) the kernel may hold 256 VGPRs (the prefetched weights)
#define RTK(EX, MT, NS) LAUNCH((k_ffn_router<EX, MT, NS>), dim3(rows), dim3(nt), shm, st, x, w, eps, d, Wr, Wp, bias, \
                               E, top_k, gating_sigmoid, weights_norm, weights_scale, q, dq, topk_idx, topk_w,   \
                               order, rec_idx, rec_w, rs)
#define RTK_E(MT, NS)               \
    do {                            \
        if (exact) RTK(true, MT, NS);  \
        else RTK(false, MT, NS);       \
    } while (0)
    if (nt <= 512) {
        switch (d) {
        case 1024: RTK_E(512, 32); break;
        case 768: RTK_E(512, 24); break;
        case 512: RTK_E(512, 16); break;
        case 256: RTK_E(512, 8); break;
        case 128: RTK_E(512, 4); break;
        default: RTK_E(512, 0); break;
        }
    } else {
        RTK_E(1024, 0);
    }
#undef RTK_E
#undef RTK
}

template <int ORDER, bool SCF32>
static void gateup_launch(hipStream_t st, const Q8Mat &Wg, const Q8Mat &Wu, const Q8Mat &Sg, const Q8Mat &Su,
                          const uint32_t *topk_idx, uint32_t top_k, uint32_t n_slots, uint32_t f, const uint8_t *q,
                          const float *dq, float *a) {
    const dim3 grid(div_up(f, 8), n_slots);
    const size_t shm = (size_t)Wg.nc * CHUNK_BYTES + (size_t)Wg.nc * 4 * sizeof(float);
#define GUK(N) LAUNCH((k_ffn_gateup<ORDER, SCF32, N>), grid, dim3(64), shm, st, Wg, Wu, Sg, Su, topk_idx, top_k, f, q, dq, a)
    DISPATCH_NCT(Wg.nc, GUK)
#undef GUK
}

void launch_ffn_gateup(hipStream_t st, int order, const Q8Mat &Wg, const Q8Mat &Wu, const Q8Mat &Sg,
                       const Q8Mat &Su, const uint32_t *topk_idx, uint32_t top_k, uint32_t n_slots, uint32_t f,
                       const uint8_t *q, const float *dq, float *a) {
    if (order == ORDER_DECODE) {
        if (Wg.sc_f32) gateup_launch<ORDER_DECODE, true>(st, Wg, Wu, Sg, Su, topk_idx, top_k, n_slots, f, q, dq, a);
        else gateup_launch<ORDER_DECODE, false>(st, Wg, Wu, Sg, Su, topk_idx, top_k, n_slots, f, q, dq, a);
    } else {
        if (Wg.sc_f32) gateup_launch<ORDER_PREFILL, true>(st, Wg, Wu, Sg, Su, topk_idx, top_k, n_slots, f, q, dq, a);
        else gateup_launch<ORDER_PREFILL, false>(st, Wg, Wu, Sg, Su, topk_idx, top_k, n_slots, f, q, dq, a);
    }
}

bool launch_ffn_front(hipStream_t st, bool exact, int order, const float *x, const float *w, float eps, uint32_t d,
                      const float *Wp, const float *bias, uint32_t E, uint32_t top_k, int gating_sigmoid,
                      int weights_norm, float weights_scale, const Q8Mat &Wg, const Q8Mat &Wu, const Q8Mat &Sg,
                      const Q8Mat &Su, uint32_t n_slots, uint32_t f, uint32_t *topk_idx, float *topk_w,
                      uint32_t *ord, uint32_t *rec_idx, float *rec_w, float *a) {
    if (d % 32 || d > 1024 || (E && (!gating_sigmoid || E > FF_MAXE || top_k > 64 || top_k > E)) ||
        Wg.nc != Sg.nc || Wg.sc_f32 != Sg.sc_f32)
        return false;
    const dim3 grid(div_up(f, FF_ROWS), E ? n_slots : 1);
    const size_t shm = 3 * (size_t)d * sizeof(float) + (size_t)Wg.nc * CHUNK_BYTES + (size_t)Wg.nc * 4 * sizeof(float);
    if (!Wp) Wp = x;      // (not read without a router)
    if (!bias) bias = x;
#define FFK(EX, O, S, N, NS)                                                                                      \
    LAUNCH((k_ffn_front<EX, O, S, N, NS>), grid, dim3(FF_NT), shm, st, x, w, eps, d, Wp, bias, E, top_k,          \
           weights_norm, weights_scale, Wg, Wu, Sg, Su, f, topk_idx, topk_w, ord, rec_idx, rec_w, a)
#define FFK_S(EX, O, N, NS)                 \
    do {                                    \
        if (Wg.sc_f32) FFK(EX, O, true, N, NS);  \
        else FFK(EX, O, false, N, NS);           \
    } while (0)
#define FFK_O(N, NS)                                      \
    do {                                                  \
        if (order == ORDER_DECODE) {                      \
            if (exact) FFK_S(true, ORDER_DECODE, N, NS);  \
            else FFK_S(false, ORDER_DECODE, N, NS);       \
        } else {                                          \
            if (exact) FFK_S(true, ORDER_PREFILL, N, NS); \
            else FFK_S(false, ORDER_PREFILL, N, NS);      \
        }                                                 \
    } while (0)
    // one instantiation per model width: the chunk batch and the router steps both follow d
    if (nct_of(Wg.nc) != nct_of(div_up(d, 128))) return false;
    switch (d) {
    case 1024: FFK_O(8, 32); break;
    case 768: FFK_O(4, 24); break;
    case 512: FFK_O(4, 16); break;
    case 256: FFK_O(2, 8); break;
    case 128: FFK_O(1, 4); break;
    case 64: FFK_O(1, 2); break;
    default: return false;
    }
#undef FFK_O
#undef FFK_S
#undef FFK
    return true;
}

template <int ORDER, bool SCF32>
static void down_launch(hipStream_t st, const Q8Mat &Wd, const Q8Mat &Sd, const uint32_t *topk_idx,
                        const float *topk_w, const uint32_t *ord, uint32_t top_k, uint32_t n_slots, int dense,
                        uint32_t d, uint32_t f, const float *a, float *x) {
    const size_t per = (size_t)Sd.nc * CHUNK_BYTES + (size_t)Sd.nc * 4 * sizeof(float);
    const size_t shm = per * n_slots + (size_t)n_slots * 8 * sizeof(float);
    const dim3 grid(div_up(d, 8)), block(64 * n_slots);
#define DNK(N) LAUNCH((k_ffn_down<ORDER, SCF32, N>), grid, block, shm, st, Wd, Sd, topk_idx, topk_w, ord, top_k, n_slots, dense, d, f, a, x)
    DISPATCH_NCT(Sd.nc, DNK)
#undef DNK
}

void launch_ffn_down(hipStream_t st, int order, const Q8Mat &Wd, const Q8Mat &Sd, const uint32_t *topk_idx,
                     const float *topk_w, const uint32_t *ord, uint32_t top_k, uint32_t n_slots, int dense,
                     uint32_t d, uint32_t f, const float *a, float *x) {
    if (order == ORDER_DECODE) {
        if (Sd.sc_f32) down_launch<ORDER_DECODE, true>(st, Wd, Sd, topk_idx, topk_w, ord, top_k, n_slots, dense, d, f, a, x);
        else down_launch<ORDER_DECODE, false>(st, Wd, Sd, topk_idx, topk_w, ord, top_k, n_slots, dense, d, f, a, x);
    } else {
        if (Sd.sc_f32) down_launch<ORDER_PREFILL, true>(st, Wd, Sd, topk_idx, topk_w, ord, top_k, n_slots, dense, d, f, a, x);
        else down_launch<ORDER_PREFILL, false>(st, Wd, Sd, topk_idx, topk_w, ord, top_k, n_slots, dense, d, f, a, x);
    }
}

}  // namespace hg
