// hg_batch_kernels.hip -- gfx950 kernels of the batched decode step: many sequences, one token
// each, every sequence's arithmetic identical to its own single-sequence step.
//
// The Q8 matrix products of the step run as int8 MFMA GEMMs (v_mfma_i32_32x32x32_i8) that keep
// the per-sequence operation order of the reference:
//   decode order, qrow_dot_avx2 (quant.rs:44-67): lane j of a row's 8 accumulators takes
//     acc_j = fma(sw[b] * dx[b], isum_{b,j}, acc_j) over blocks b, where isum_{b,j} is the int8
//     dot of the 4 elements 32b + 4j .. 32b + 4j + 3 only.  An MFMA sums over all 32 K slots
//     of its block, so the activation operand is masked: column (token, j) holds token's 4
//     elements of lane j and zeros elsewhere, and C[row][(token, j)] is exactly isum_{b,j}.
//     One MFMA covers 32 rows x 4 tokens x 8 lanes; the 8 lane accumulators are then reduced
//     ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) across lanes, as the reference's hsum.
// MFMA operand layout (probed on gfx950): lane l supplies row (A) / column (B) l % 32, K half
// l / 32 (16 bytes, the same K slots in A and B); C register v of lane l is row
// 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32.  K slot (h, i) here carries block element
// 16 h + i: in the device row layout (hg_common.h) that is lanes j = 4h .. 4h + 3 of the chunk,
// so a lane's A operand for the 4 blocks of a chunk is the chunk's contiguous 64 bytes at 64 h
// (4 x 16 bytes, word t of each piece = block t).
//
// KV rows live in pages of PAGE positions (a pool per layer, [page][kv head][PAGE][hd]); each
// sequence's block table maps position t to page bt[t / PAGE].
#include <hip/hip_ext.h>

#include "hg_batch.h"
#include "hg_common.h"
#include "hg_device.h"
#include "hg_expf.h"

namespace hg {

typedef int v16i __attribute__((ext_vector_type(16)));

__device__ inline v16i mfma_i8(v4i a, v4i b) {
    const v16i z = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

// A bounded wait: the flag protocol of a kernel guarantees progress, and the cap turns a
// protocol slip into an error report (*err = 1 and the wait ends) instead of a hang.
constexpr uint32_t SPIN_CAP = 1u << 22;

// ------------------------------------------------------------------ embedding
// x[s] = token_embd[tokens[s]] (model.rs:152-154).  grid (d / 256, n).
__global__ void k_b_embed(const float *__restrict__ emb, uint32_t d, const uint32_t *__restrict__ tokens, float *x) {
    const uint32_t s = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < d) x[(size_t)s * d + i] = emb[(size_t)tokens[s] * d + i];
}

// ------------------------------------------------------------------ activation quantization
// Rows of an f32 matrix quantized for the matvec that consumes them (quant.rs:111-123):
// row r = blockIdx.y of n floats at x + r xs into q + r qs (chunks) and dq + r ds (scales).
__global__ __launch_bounds__(256) void k_b_quant_rows(const float *__restrict__ x, uint32_t xs, uint32_t n,
                                                      uint8_t *q, uint32_t qs, float *dq, uint32_t ds) {
    const int tid = threadIdx.x, j = tid & 7;
    const uint32_t r = blockIdx.y, nb = n / QK, nc = div_up(nb, 4);
    const float *xr = x + (size_t)r * xs;
    uint8_t *qr = q + (size_t)r * qs;
    float *dr = dq + (size_t)r * ds;
    for (uint32_t b0 = blockIdx.x * 32; b0 < nb; b0 += gridDim.x * 32) {
        const uint32_t b = b0 + (tid >> 3);
        if (b < nb) {   // a block's 8 lanes are all in or all out
            const v4f x4 = *reinterpret_cast<const v4f *>(xr + b * QK + j * 4);
            const float v[4] = {x4.x, x4.y, x4.z, x4.w};
            quant_block_lane(v, j, b, qr, dr);
        }
    }
    if (blockIdx.x == 0) zero_pad(nb, nc, qr, dr, tid, 256);
}

// ------------------------------------------------------------------ MFMA GEMM, decode order
// y[out_row[e]][row] (+)= (W x_{act_row[e]})[row] for the entries e of each column tile and the
// rows of its matrix group, in qrow_dot_avx2's order (see the file comment).  Workgroup =
// 4 waves; blockIdx.y = column tile (tiles past *n_tiles exit), blockIdx.x = a block of rows.
//   GM_STORE / GM_RESID: waves = WR row tiles of 32 rows x 4 / WR column groups of 4 entries.
//   GM_GATEUP: wave w = (matrix w & 1: gate / up) x (column group w >> 1), 32 rows; the up
//     wave hands its sums to the gate wave, which stores silu(g) * u (model.rs:301-305).
// Per chunk, lanes 0..31 fetch the 4 block scales of row rbase + lane with the weights and
// stage them in LDS (double-buffered by chunk parity; within one wave LDS accesses complete in
// program order), from where every lane reads those of its 16 output rows.

template <bool SCF32, int MODE, int WR>
__global__ __launch_bounds__(256) void k_gemm_dec(GemmArgs g) {
    static_assert(MODE != GM_GATEUP || WR == 1, "gate/up: one row tile per workgroup");
    __shared__ __align__(16) float scl_all[4][2][32][4];
    __shared__ float up_sum[2][16][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (blockIdx.y >= *g.n_tiles) return;   // (uniform)
    const GemmTile tile = g.tiles[blockIdx.y];
    const int mat = MODE == GM_GATEUP ? (wave & 1) : 0;
    const int rt = MODE == GM_GATEUP ? 0 : wave % WR;
    const int cg = MODE == GM_GATEUP ? (wave >> 1) : wave / WR;
    const Q8Mat &M = MODE == GM_GATEUP && mat == 1 ? g.U[tile.mat] : g.W[tile.mat];
    const uint32_t r0 = blockIdx.x * 32 * WR + rt * 32;   // first row of the wave within the group
    const uint32_t gbase = tile.grp * g.rows, rbase = gbase + r0, rlim = gbase + g.rows - 1;
    const uint32_t nc = M.nc, nb = M.nb;
    const WaveExpTab tab = WaveExpTab::load(lane);
    // this lane's operands: A row rbase + lane % 32 (K half lane / 32); B column lane % 32 =
    // (entry k = (lane % 32) / 8 of the column group, lane j = lane % 8)
    const uint32_t h = (uint32_t)lane >> 5, j = (uint32_t)lane & 7, k = ((uint32_t)lane & 31) >> 3;
    const uint32_t arow = min(rbase + ((uint32_t)lane & 31), rlim);
    const uint32_t ent = (uint32_t)cg * 4 + k;
    const bool valid = ent < tile.count;
    const uint32_t e = tile.entry0 + min(ent, tile.count - 1);
    const uint32_t xr = g.act_row[e];
    const bool bact = valid && h == (j >> 2);   // the lane whose 16 B hold the column's 4 elements
    const uint8_t *wrow = M.qs + (size_t)arow * nc * CHUNK_BYTES + 64 * h;
    typedef typename ScaleVec<SCF32>::T SV;
    const SV *srow = reinterpret_cast<const SV *>(row_sc<SCF32>(M, arow));   // (lanes 0..31: its row's)
    const uint8_t *xq = g.aq + (size_t)xr * g.aqs + j * 16;
    const float *xd = g.ad + (size_t)xr * g.ads;
    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    v4i P[4], Pn[4], bp, bpn;
    v4f dx, dxn;
    SV sv, svn;
    auto load = [&](uint32_t c, v4i (&p)[4], v4i &b, v4f &d, SV &sc) {
        const v4i *wp = reinterpret_cast<const v4i *>(wrow + (size_t)c * CHUNK_BYTES);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = __builtin_nontemporal_load(wp + i);
        sc = srow[c];
        b = *reinterpret_cast<const v4i *>(xq + (size_t)c * CHUNK_BYTES);
        d = *reinterpret_cast<const v4f *>(xd + 4 * c);
    };
    load(0, P, bp, dx, sv);
    for (uint32_t c = 0; c < nc; ++c) {
        if (c + 1 < nc) load(c + 1, Pn, bpn, dxn, svn);
        // the 4 block scales of this wave's 32 rows through LDS; lane reads its 16 rows'
        // (C register v is row 8 (v / 4) + 4 h + v % 4)
        float (*scl)[4] = scl_all[wave][c & 1];
        if (lane < 32) {
            float f[4];
            unpack_scales(sv, f);
            *reinterpret_cast<v4f *>(scl[lane]) = v4f{f[0], f[1], f[2], f[3]};
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        v4f s16[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) s16[v] = *reinterpret_cast<const v4f *>(scl[8 * (v / 4) + 4 * h + v % 4]);
        const int pa[4] = {P[0].x, P[1].x, P[2].x, P[3].x}, pb[4] = {P[0].y, P[1].y, P[2].y, P[3].y},
                  pc[4] = {P[0].z, P[1].z, P[2].z, P[3].z}, pd[4] = {P[0].w, P[1].w, P[2].w, P[3].w};
        const int bw[4] = {bp.x, bp.y, bp.z, bp.w};
        const float dxs[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int *pt = t == 0 ? pa : t == 1 ? pb : t == 2 ? pc : pd;
            const v4i A = {pt[0], pt[1], pt[2], pt[3]};
            const int w = bact ? bw[t] : 0;
            const uint32_t jj = j & 3;
            const v4i B = {jj == 0 ? w : 0, jj == 1 ? w : 0, jj == 2 ? w : 0, jj == 3 ? w : 0};
            const v16i C = mfma_i8(A, B);
            if (4 * c + t < nb) {   // (padding blocks of a partial last chunk: no add)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float sw = t == 0 ? s16[v].x : t == 1 ? s16[v].y : t == 2 ? s16[v].z : s16[v].w;
                    acc[v] = fmaf(sw * dxs[t], (float)C[v], acc[v]);
                }
            }
        }
        if (c + 1 < nc) {
#pragma unroll
            for (int i = 0; i < 4; ++i) P[i] = Pn[i];
            bp = bpn;
            dx = dxn;
            sv = svn;
        }
    }
    // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) over the 8 lanes j of each (row, entry)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        float a = acc[v];
        {
            const float dn = dpp_f<0x124>(a), up = dpp_f<0x12C>(a);
            a = a + ((j & 4) ? dn : up);
        }
        a = a + dpp_f<0x4E>(a);
        a = a + dpp_f<0xB1>(a);
        acc[v] = a;
    }
    if constexpr (MODE == GM_GATEUP) {
        if (mat == 1) {
#pragma unroll
            for (int v = 0; v < 16; ++v) up_sum[cg][v][lane] = acc[v];
        }
        __syncthreads();
        if (mat == 1) return;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float a = hg_silu_l(acc[v], tab) * up_sum[cg][v][lane];   // every lane (a lane exchange)
            const uint32_t rl = r0 + 8 * (v / 4) + 4 * h + v % 4;
            if (j == 0 && valid && rl < g.rows) g.y[(size_t)g.out_row[e] * g.ys + rl] = a;
        }
        return;
    }
    if (j == 0 && valid) {
        float *yo = g.y + (size_t)g.out_row[e] * g.ys;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t rl = r0 + 8 * (v / 4) + 4 * h + v % 4;
            if (rl < g.rows) {
                if (MODE == GM_RESID) yo[rl] = yo[rl] + acc[v];
                else yo[rl] = acc[v];
            }
        }
    }
}

// ------------------------------------------------------------------ QK-norm, RoPE, paged append
// For each sequence s (blockIdx.y) and head hh (blockIdx.x, q | k | v as the QKV rows): q and k
// heads normed (model.rs:753-763) and rotated at pos[s] (ops.rs:155-166) in place; k and v rows
// appended to the layer's page of position pos[s] (model.rs:210-211).  64 threads.
template <int HD>
__global__ __launch_bounds__(64) void k_b_qk_rope_append(float *qkv, uint32_t qkv_stride, const float *__restrict__ qn,
                                                         const float *__restrict__ kn, float eps,
                                                         const float *__restrict__ cs, const float *__restrict__ sn,
                                                         const uint32_t *__restrict__ pos, PagedKV kv) {
    __shared__ __align__(16) float u[HD], o[HD], tmp[HD];
    const int lane = threadIdx.x;
    const uint32_t hh = blockIdx.x, s = blockIdx.y, p = pos[s];
    const uint32_t n_heads = kv.n_heads, n_kv = kv.n_kv;
    float *src = qkv + (size_t)s * qkv_stride + (size_t)hh * HD;
    HeadConst<HD> hc;
    hc.load(qn, kn, cs, sn, p, lane);
    for (uint32_t i = lane; i < HD; i += 64) u[i] = src[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t page = kv.bt[(size_t)s * kv.bt_stride + p / PAGE];
    if (hh >= n_heads + n_kv) {
        float *vr = kv.v + kv_row_off(page, hh - n_heads - n_kv, p % PAGE, n_kv, HD);
        for (uint32_t i = lane; i < HD; i += 64) vr[i] = u[i];
        return;
    }
    norm_rope_head<HD>(u, o, hc, hh < n_heads, eps, tmp, lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (uint32_t i = lane; i < HD; i += 64) src[i] = o[i];
    if (hh >= n_heads) {
        float *kr = kv.k + kv_row_off(page, hh - n_heads, p % PAGE, n_kv, HD);
        for (uint32_t i = lane; i < HD; i += 64) kr[i] = o[i];
    }
}

// ------------------------------------------------------------------ paged attention: scores
// s_t = dot(q_h, K_t) * (1/sqrt(hd)) (model.rs:213-218, ops::dot's order) for the rep query
// heads of kv head g (blockIdx.y) of sequence s (blockIdx.z) over positions
// [256 c, 256 c + 256) of its context (c = blockIdx.x; chunks past the context exit), and each
// head's chunk maximum.  Lanes as k_attn_scores: R lanes (rep rounded up to a power of two)
// share a position, one K row fetch per position.
template <int HD>
__global__ __launch_bounds__(256) void k_b_scores(const float *__restrict__ qkv, uint32_t qkv_stride,
                                                  const uint32_t *__restrict__ pos, PagedKV kv, float *scores,
                                                  uint32_t sc_stride, float *pmax, uint32_t pm_stride) {
    constexpr int MAXREP = 8;
    __shared__ __align__(16) float qs[MAXREP * HD];
    __shared__ float wm[4][MAXREP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t c = blockIdx.x, g = blockIdx.y, s = blockIdx.z;
    const uint32_t n = pos[s] + 1, t0 = c * ACH;
    if (t0 >= n) return;   // (uniform)
    const uint32_t n_heads = kv.n_heads, rep = n_heads / kv.n_kv;
    const uint32_t R = rep <= 1 ? 1u : rep <= 2 ? 2u : rep <= 4 ? 4u : 8u;
    const uint32_t r = (uint32_t)tid % R, pp = 256 / R, t1 = min(n, t0 + ACH);
    const uint32_t *bts = kv.bt + (size_t)s * kv.bt_stride;
    auto krow = [&](uint32_t t) { return kv.k + kv_row_off(bts[t / PAGE], g, t % PAGE, kv.n_kv, HD); };
    float kt[HD];
    {
        const float *kp = krow(min(t0 + (uint32_t)tid / R, n - 1));
#pragma unroll
        for (int i = 0; i < HD; i += 4) *reinterpret_cast<v4f *>(kt + i) = *reinterpret_cast<const v4f *>(kp + i);
    }
    const float *qsrc = qkv + (size_t)s * qkv_stride + (size_t)g * rep * HD;
    for (uint32_t i = tid; i < rep * HD; i += 256) qs[i] = qsrc[i];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    float mx = -__builtin_huge_valf();
    const float *qr = qs + min(r, rep - 1) * HD;
    float *sc = scores + ((size_t)s * n_heads + g * rep + r) * sc_stride;
    for (uint32_t tb = t0; tb < t1; tb += pp) {
        const uint32_t t = tb + (uint32_t)tid / R;
        if (tb != t0) {
            const float *kp = krow(min(t, n - 1));
#pragma unroll
            for (int i = 0; i < HD; i += 4) *reinterpret_cast<v4f *>(kt + i) = *reinterpret_cast<const v4f *>(kp + i);
        }
        if (r < rep && t < t1) {
            const float v = dot_wide_serial(qr, kt, HD) * scale;
            sc[t] = v;
            mx = fmaxf(mx, v);
        }
    }
    for (uint32_t o = R; o < 64; o <<= 1) mx = fmaxf(mx, shfl_xor(mx, (int)o));
    if ((uint32_t)lane < R) wm[wave][lane] = mx;
    __syncthreads();
    if ((uint32_t)tid < rep)
        pmax[((size_t)s * n_heads + g * rep + tid) * pm_stride + c] =
            fmaxf(fmaxf(wm[0][tid], wm[1][tid]), fmaxf(wm[2][tid], wm[3][tid]));
}

// ------------------------------------------------------------------ paged attention: softmax + P.V
// One workgroup per (sequence, query head) (ops.rs:112-128, model.rs:226-232):
//   m = max of the chunk maxima; e_t = exp(s_t - m) (the reference expf) into LDS; sum = the
//   index-order sum of e_t (block_seq_sum up to 3072 terms, else one lane); p_t = e_t (1/sum);
//   o[di] = ((0 + p_0 v_0[di]) + p_1 v_1[di]) + ..., one chain per element di.
// P.V: the chain wave(s) (lane = di; HD / 64 waves) add the products in position order;
// producer waves (not on a chain wave's SIMD) read the V rows of 64-position groups from the
// pages, form the rounded products p_t v_t[di] and store them [di][t] into a ring of LDS slots
// (positions past the context: -0, the exact identity of the adds).  Slot hand-offs are LDS
// flags with bounded waits.  Workgroups of one (sequence, kv head) get ids equal mod 8, so the
// query heads sharing V rows run on one XCD's L2.
struct PvCfgB {
    static constexpr uint32_t G = 64;        // positions per ring slot
    static constexpr uint32_t GP = G + 4;    // padded row of a slot
    static constexpr uint32_t NW = 8;        // waves
    static constexpr uint32_t RMAX = 8;
};

uint32_t bpv_slots(uint32_t max_ctx, uint32_t hd) {
    const size_t e_bytes = (size_t)div_up(max_ctx, 4) * 16 + 64 * 4;
    const size_t slot = (size_t)hd * PvCfgB::GP * 4;
    const size_t budget = BPV_LDS_BUDGET - sizeof(xsum::Scratch) - 64;
    const size_t r = budget > e_bytes ? (budget - e_bytes) / slot : 0;
    return (uint32_t)(r > PvCfgB::RMAX ? PvCfgB::RMAX : r);
}
static size_t bpv_lds(uint32_t max_ctx, uint32_t hd, uint32_t slots) {
    return (size_t)div_up(max_ctx, 4) * 16 + 64 * 4 + (size_t)slots * hd * PvCfgB::GP * 4;
}

template <int HD>
__global__ __launch_bounds__(512) void k_b_attn_pv(const float *__restrict__ scores, uint32_t sc_stride,
                                                   const float *__restrict__ pmax, uint32_t pm_stride,
                                                   const uint32_t *__restrict__ pos, PagedKV kv, uint32_t n_seq,
                                                   uint32_t max_ctx, uint32_t R, float *o_out, uint32_t *err) {
    using C = PvCfgB;
    constexpr uint32_t NCW = HD / 64;   // chain waves
    static_assert(HD % 64 == 0 && NCW <= 2, "head_dim 64 or 128");
    extern __shared__ __align__(16) float lds[];
    __shared__ xsum::Scratch xs;
    __shared__ uint32_t ready[C::RMAX], done[NCW];
    __shared__ float s_inv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n_heads = kv.n_heads, n_kv = kv.n_kv, rep = n_heads / n_kv;
    // workgroup -> (sequence, head): the rep heads of a (sequence, kv head) key get ids equal mod 8
    uint32_t s, h;
    {
        const uint32_t L = blockIdx.x, nkeys = n_seq * n_kv;
        if (nkeys % 8 == 0) {
            const uint32_t slot = L / 8, key = L % 8 + 8 * (slot / rep), r = slot % rep;
            s = key / n_kv;
            h = (key % n_kv) * rep + r;
        } else {
            s = L / n_heads;
            h = L % n_heads;
        }
    }
    const uint32_t g = h / rep, n = pos[s] + 1, nch = div_up(n, ACH);
    float *e = lds;                                                        // [max_ctx] e_t
    float *ring = lds + (size_t)div_up(max_ctx, 4) * 4 + 64;               // [R][HD][GP]
    const float *sc = scores + ((size_t)s * n_heads + h) * sc_stride;
    const float *pm = pmax + ((size_t)s * n_heads + h) * pm_stride;
    const uint32_t *bts = kv.bt + (size_t)s * kv.bt_stride;
    const WaveExpTab tab = WaveExpTab::load(lane);
    float m = -__builtin_huge_valf();
    for (uint32_t c = lane; c < nch; c += 64) m = fmaxf(m, pm[c]);
    for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, shfl_xor(m, k));   // max is order-free
    if (tid < (int)C::RMAX) ready[tid] = 0;
    if (tid < (int)NCW) done[tid] = 0;
    if (tid == 0) xs.sync = 0;
    for (uint32_t t0 = 0; t0 < n; t0 += 512) {   // (uniform: every lane calls the exp)
        const uint32_t t = t0 + (uint32_t)tid;
        const float ev = hg_expf_l(sc[min(t, n - 1)] - m, tab);
        if (t < n) e[t] = ev;
    }
    if (tid < 4) e[n + tid] = 0.0f;   // readable up to a multiple of 4 past n
    __syncthreads();
    if (n <= 3072) {   // sum += e_t in index order (ops.rs:119-122)
        if (wave < 4) {
            const float r = n <= 2048 ? block_seq_sum<4, 8>(e, n, xs, wave, lane) : block_seq_sum<4, 12>(e, n, xs, wave, lane);
            if (tid == 0) s_inv = 1.0f / r;
        }
    } else if (tid == 0) {
        s_inv = 1.0f / seq_sum_lds(e, n, 0.0f);
    }
    __syncthreads();
    const float inv = s_inv;
    const uint32_t ngr = div_up(n, C::G);
    // waves on SIMD wave % 4: the chain waves 0 .. NCW - 1 run alone on their SIMDs
    const bool chain = (uint32_t)wave < NCW;
    const bool idle = !chain && (uint32_t)(wave % 4) < NCW;
    if (!chain && !idle) {
        // producer index among the producer waves
        uint32_t pw = 0, np = 0;
        for (uint32_t w = 0; w < C::NW; ++w) {
            const bool pr = w >= NCW && (w % 4) >= NCW;
            if (pr && w < (uint32_t)wave) ++pw;
            if (pr) ++np;
        }
        // lane -> (position sub within a pass, 4 elements): HD / 4 lanes per row
        constexpr uint32_t LPR = HD / 4, PPI = 64 / LPR;
        const uint32_t sub = (uint32_t)lane / LPR, d4 = ((uint32_t)lane % LPR) * 4;
        for (uint32_t k = pw; k < ngr; k += np) {
            if (k >= R) {   // slot k % R is free once every chain wave finished group k - R
                uint32_t it = 0;
                for (;;) {
                    uint32_t dmin = __hip_atomic_load(&done[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
                    if (NCW > 1) dmin = min(dmin, __hip_atomic_load(&done[NCW - 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP));
                    if (dmin >= k - R + 1) break;
                    if (++it > SPIN_CAP) { if (lane == 0) atomicOr(err, 1u); break; }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            float *slot = ring + (size_t)(k % R) * HD * C::GP;
            v4f vr[C::G / PPI];
#pragma unroll
            for (uint32_t i = 0; i < C::G / PPI; ++i) {
                const uint32_t t = min(k * C::G + i * PPI + sub, n - 1);
                vr[i] = *reinterpret_cast<const v4f *>(kv.v + kv_row_off(bts[t / PAGE], g, t % PAGE, n_kv, HD) + d4);
            }
#pragma unroll
            for (uint32_t i = 0; i < C::G / PPI; ++i) {
                const uint32_t tt = i * PPI + sub, t = k * C::G + tt;
                const bool in = t < n;
                const float pt = in ? e[t] * inv : 0.0f;
                slot[(d4 + 0) * C::GP + tt] = in ? pt * vr[i].x : -0.0f;
                slot[(d4 + 1) * C::GP + tt] = in ? pt * vr[i].y : -0.0f;
                slot[(d4 + 2) * C::GP + tt] = in ? pt * vr[i].z : -0.0f;
                slot[(d4 + 3) * C::GP + tt] = in ? pt * vr[i].w : -0.0f;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_store(&ready[k % R], k + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    } else if (chain) {
        const uint32_t di = (uint32_t)wave * 64 + (uint32_t)lane;
        float o = 0.0f;
        for (uint32_t k = 0; k < ngr; ++k) {
            uint32_t it = 0;
            while (__hip_atomic_load(&ready[k % R], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != k + 1) {
                if (++it > SPIN_CAP) { if (lane == 0) atomicOr(err, 1u); break; }
                __builtin_amdgcn_s_sleep(1);
            }
            const v4f *row = reinterpret_cast<const v4f *>(ring + (size_t)(k % R) * HD * C::GP + (size_t)di * C::GP);
            v4f a[C::G / 4];
#pragma unroll
            for (uint32_t u = 0; u < C::G / 4; ++u) a[u] = row[u];
#pragma unroll
            for (uint32_t u = 0; u < C::G / 4; ++u) {
                o = o + a[u].x;
                o = o + a[u].y;
                o = o + a[u].z;
                o = o + a[u].w;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_store(&done[wave], k + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        o_out[((size_t)s * n_heads + h) * HD + di] = o;
    }
}

// ------------------------------------------------------------------ expert grouping
// The ffn_prefill grouping (model.rs:676-731) for one decode step of n sequences: for every
// expert e (ascending), the (sequence, rank) pairs that picked it (sequences ascending), then
// the shared expert with every sequence (slot top_k).  Entry i of the table: act_row = the
// sequence (its quantized h), out_row = sequence * n_slots + slot (its row of a and y).
// Column tiles of at most TT entries cover each expert's entries (matrix group e of set 0; the
// shared expert's tiles use group 0 of set 1).  One workgroup.
__global__ __launch_bounds__(256) void k_b_group(const uint32_t *__restrict__ topk_idx, uint32_t n, uint32_t top_k,
                                                 uint32_t E, uint32_t n_slots, uint32_t TT,
                                                 uint32_t *act_row, uint32_t *out_row, GemmTile *tiles,
                                                 uint32_t *n_tiles) {
    __shared__ uint32_t cnt[MAX_GROUPS + 1], off[MAX_GROUPS + 1], toff[MAX_GROUPS + 1];
    const uint32_t tid = threadIdx.x;
    const uint32_t NG = E + (n_slots > top_k ? 1 : 0);
    for (uint32_t e = tid; e < NG; e += 256) {
        uint32_t c = 0;
        if (e < E) {
            for (uint32_t s = 0; s < n; ++s)
                for (uint32_t r = 0; r < top_k; ++r) c += topk_idx[s * top_k + r] == e;
        } else {
            c = n;
        }
        cnt[e] = c;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t a = 0, t = 0;
        for (uint32_t e = 0; e < NG; ++e) {
            off[e] = a;
            toff[e] = t;
            a += cnt[e];
            t += div_up(cnt[e], TT);
        }
        *n_tiles = t;
    }
    __syncthreads();
    for (uint32_t e = tid; e < NG; e += 256) {
        uint32_t i = off[e];
        if (e < E) {
            for (uint32_t s = 0; s < n; ++s)
                for (uint32_t r = 0; r < top_k; ++r)
                    if (topk_idx[s * top_k + r] == e) {
                        act_row[i] = s;
                        out_row[i] = s * n_slots + r;
                        ++i;
                    }
        } else {
            for (uint32_t s = 0; s < n; ++s, ++i) {
                act_row[i] = s;
                out_row[i] = s * n_slots + top_k;
            }
        }
        for (uint32_t q = 0; q < div_up(cnt[e], TT); ++q) {
            GemmTile tl;
            tl.grp = e < E ? e : 0u;
            tl.entry0 = off[e] + q * TT;
            tl.count = min(TT, cnt[e] - q * TT);
            tl.mat = e < E ? 0u : 1u;
            tiles[toff[e] + q] = tl;
        }
    }
}

// ------------------------------------------------------------------ expert combine + residual
// x[s] += ((0 + w_0 y_0) + w_1 y_1 + ...) + y_shared (rank order; model.rs:306-323 and
// 173-176 as k_ffn_down's decode combine).  grid (d / 256, n).
__global__ void k_b_combine(const float *__restrict__ y, const float *__restrict__ topk_w, uint32_t top_k,
                            uint32_t n_slots, uint32_t d, float *x) {
    const uint32_t s = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d) return;
    const float *ys = y + (size_t)s * n_slots * d + i;
    float acc = 0.0f;
    for (uint32_t q = 0; q < top_k; ++q) acc = acc + topk_w[s * top_k + q] * ys[(size_t)q * d];
    if (n_slots > top_k) acc = acc + ys[(size_t)top_k * d];
    x[(size_t)s * d + i] = x[(size_t)s * d + i] + acc;
}

// ------------------------------------------------------------------ greedy argmax per sequence
// sample::argmax (sample.rs:53-63) of logits[s][0..valid) (ids >= valid masked, lib.rs:132-134):
// the first maximum; 0 when nothing exceeds -inf.  Writes out[step][s]; then advances the
// sequence: pos[s] += 1 and, in feedback mode, tokens[s] = the pick.  grid n, 1024 threads.
__global__ __launch_bounds__(1024) void k_b_argmax(const float *__restrict__ logits, uint32_t V, uint32_t valid,
                                                   uint32_t *pos, uint32_t *tokens, uint32_t *out_ids,
                                                   const uint32_t *step, uint32_t n, uint32_t feedback) {
    __shared__ float bv[16];
    __shared__ uint32_t bi[16];
    const int tid = threadIdx.x;
    const uint32_t s = blockIdx.x;
    const float *lg = logits + (size_t)s * V;
    float mv = -__builtin_huge_valf();
    uint32_t mi = 0xffffffffu;
    for (uint32_t i = tid; i < valid; i += 1024) {
        const float v = lg[i];
        if (v > mv) { mv = v; mi = i; }   // (per thread: ascending i, strict >)
    }
    for (int m = 1; m < 64; m <<= 1) {
        const float ov = shfl_xor(mv, m);
        const uint32_t oi = (uint32_t)shfl_xor_i((int)mi, m);
        if (ov > mv || (ov == mv && oi < mi)) { mv = ov; mi = oi; }
    }
    if ((tid & 63) == 0) { bv[tid >> 6] = mv; bi[tid >> 6] = mi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; ++w)
            if (bv[w] > mv || (bv[w] == mv && bi[w] < mi)) { mv = bv[w]; mi = bi[w]; }
        const uint32_t next = mi == 0xffffffffu ? 0u : mi;
        out_ids[(size_t)(*step) * n + s] = next;
        pos[s] += 1;
        if (feedback) tokens[s] = next;
    }
}

__global__ void k_b_step_advance(uint32_t *step) {
    if (threadIdx.x == 0) *step += 1;
}

// ====================================================================== launchers
#define BLAUNCH(kern, grid, block, shm, st, ...)                                                             \
    do {                                                                                                     \
        hipLaunchKernelGGL(kern, grid, block, shm, st, __VA_ARGS__);                                         \
        const hipError_t le_ = hipGetLastError();                                                            \
        if (le_ != hipSuccess) note_launch_error(le_, #kern);                                                \
    } while (0)

hipError_t init_batch_kernel_attributes() {
    hipError_t e = hipSuccess;
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_b_attn_pv<64>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)BPV_LDS_BUDGET);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_b_attn_pv<128>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)BPV_LDS_BUDGET);
    return e;
}

void launch_b_embed(hipStream_t st, const float *emb, uint32_t d, const uint32_t *tokens, uint32_t n, float *x) {
    BLAUNCH(k_b_embed, dim3(div_up(d, 256), n), dim3(256), 0, st, emb, d, tokens, x);
}

void launch_b_quant_rows(hipStream_t st, const float *x, uint32_t xs, uint32_t n_elems, uint32_t rows, uint8_t *q,
                         uint32_t qs, float *dq, uint32_t ds) {
    BLAUNCH(k_b_quant_rows, dim3(div_up(n_elems / QK, 32), rows), dim3(256), 0, st, x, xs, n_elems, q, qs, dq, ds);
}

// Column tiles of tt entries: 8 (two row tiles per workgroup; gate/up: both matrices) or 16.
bool launch_b_gemm(hipStream_t st, int mode, uint32_t tt, const GemmArgs &a, uint32_t max_tiles) {
    const Q8Mat &M = a.W[0];
    if (a.W[1].qs && a.W[1].sc_f32 != M.sc_f32) return false;
    const bool f32s = M.sc_f32 != 0;
#define GEMM_L(S, MD, WR)                                                                                     \
    BLAUNCH((k_gemm_dec<S, MD, WR>), dim3(div_up(a.rows, 32 * (WR)), max_tiles), dim3(256), 0, st, a)
    if (mode == GM_GATEUP) {
        if (tt != 8) return false;
        if (f32s) GEMM_L(true, GM_GATEUP, 1);
        else GEMM_L(false, GM_GATEUP, 1);
        return true;
    }
    if (tt != 8 && tt != 16) return false;
    if (mode == GM_STORE) {
        if (tt == 8) {
            if (f32s) GEMM_L(true, GM_STORE, 2);
            else GEMM_L(false, GM_STORE, 2);
        } else {
            if (f32s) GEMM_L(true, GM_STORE, 1);
            else GEMM_L(false, GM_STORE, 1);
        }
    } else {
        if (tt == 8) {
            if (f32s) GEMM_L(true, GM_RESID, 2);
            else GEMM_L(false, GM_RESID, 2);
        } else {
            if (f32s) GEMM_L(true, GM_RESID, 1);
            else GEMM_L(false, GM_RESID, 1);
        }
    }
#undef GEMM_L
    return true;
}

bool launch_b_qk_rope_append(hipStream_t st, uint32_t hd, float *qkv, uint32_t qkv_stride, const float *qn,
                             const float *kn, float eps, const float *cs, const float *sn, const uint32_t *pos,
                             const PagedKV &kv, uint32_t n) {
    const dim3 grid(kv.n_heads + 2 * kv.n_kv, n);
    switch (hd) {
    case 64: BLAUNCH(k_b_qk_rope_append<64>, grid, dim3(64), 0, st, qkv, qkv_stride, qn, kn, eps, cs, sn, pos, kv); break;
    case 128: BLAUNCH(k_b_qk_rope_append<128>, grid, dim3(64), 0, st, qkv, qkv_stride, qn, kn, eps, cs, sn, pos, kv); break;
    default: return false;
    }
    return true;
}

bool launch_b_attention(hipStream_t st, uint32_t hd, const float *qkv, uint32_t qkv_stride, const uint32_t *pos,
                        const PagedKV &kv, uint32_t n, uint32_t max_ctx, float *scores, float *pmax, float *o,
                        uint32_t *err) {
    const uint32_t nch = div_up(max_ctx, ACH), R = bpv_slots(max_ctx, hd);
    if (R < 2) return false;
    const size_t shm = bpv_lds(max_ctx, hd, R);
    const dim3 gs(nch, kv.n_kv, n), gp(n * kv.n_heads);
    switch (hd) {
    case 64:
        BLAUNCH(k_b_scores<64>, gs, dim3(256), 0, st, qkv, qkv_stride, pos, kv, scores, max_ctx, pmax, nch);
        BLAUNCH(k_b_attn_pv<64>, gp, dim3(512), shm, st, scores, max_ctx, pmax, nch, pos, kv, n, max_ctx, R, o, err);
        break;
    case 128:
        BLAUNCH(k_b_scores<128>, gs, dim3(256), 0, st, qkv, qkv_stride, pos, kv, scores, max_ctx, pmax, nch);
        BLAUNCH(k_b_attn_pv<128>, gp, dim3(512), shm, st, scores, max_ctx, pmax, nch, pos, kv, n, max_ctx, R, o, err);
        break;
    default: return false;
    }
    return true;
}

void launch_b_group(hipStream_t st, const uint32_t *topk_idx, uint32_t n, uint32_t top_k, uint32_t E,
                    uint32_t n_slots, uint32_t tt, uint32_t *act_row, uint32_t *out_row, GemmTile *tiles,
                    uint32_t *n_tiles) {
    BLAUNCH(k_b_group, dim3(1), dim3(256), 0, st, topk_idx, n, top_k, E, n_slots, tt, act_row, out_row, tiles,
            n_tiles);
}

// Pages of one sequence between a contiguous buffer [i][page_floats] and the pool (page bt[i]):
// dir 0 writes the pool, dir 1 reads it.  grid npg.
__global__ void k_b_page_copy(float *flat, float *pool, const uint32_t *__restrict__ bt, uint32_t page_floats,
                              int dir) {
    const uint32_t i = blockIdx.x;
    float *f = flat + (size_t)i * page_floats, *p = pool + (size_t)bt[i] * page_floats;
    for (uint32_t q = threadIdx.x; q < page_floats; q += blockDim.x) {
        if (dir == 0) p[q] = f[q];
        else f[q] = p[q];
    }
}

void launch_b_page_copy(hipStream_t st, float *flat, float *pool, const uint32_t *bt, uint32_t npg,
                        uint32_t page_floats, int dir) {
    if (npg) BLAUNCH(k_b_page_copy, dim3(npg), dim3(256), 0, st, flat, pool, bt, page_floats, dir);
}

void launch_b_combine(hipStream_t st, const float *y, const float *topk_w, uint32_t top_k, uint32_t n_slots,
                      uint32_t d, uint32_t n, float *x) {
    BLAUNCH(k_b_combine, dim3(div_up(d, 256), n), dim3(256), 0, st, y, topk_w, top_k, n_slots, d, x);
}

void launch_b_argmax(hipStream_t st, const float *logits, uint32_t V, uint32_t valid, uint32_t *pos, uint32_t *tokens,
                     uint32_t *out_ids, const uint32_t *step, uint32_t n, uint32_t feedback) {
    BLAUNCH(k_b_argmax, dim3(n), dim3(1024), 0, st, logits, V, valid, pos, tokens, out_ids, step, n, feedback);
}

void launch_b_step_advance(hipStream_t st, uint32_t *step) {
    BLAUNCH(k_b_step_advance, dim3(1), dim3(64), 0, st, step);
}

}  // namespace hg
