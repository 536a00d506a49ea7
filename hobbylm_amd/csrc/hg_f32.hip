// hg_f32.hip -- kernels of the F32 matrix mode: ops::matvec (ops.rs:40-53) in ops::dot's
// order (ops.rs:7-36) for the whole-matrix products, the expert gate/up (silu * up) and down
// products of one token's slots.  The other parts of the step (norms, QK-norm + RoPE + append,
// attention, router, combine) are the Q8 mode's kernels.
#include "hg_f32.h"

#include <hip/hip_ext.h>

#include <string>

#include "hg_common.h"
#include "hg_device.h"
#include "hg_expf.h"
#include "hg_kernels.h"

namespace hg {

void permute_f32_rows(const float *src, uint32_t N, uint32_t K, std::vector<float> &dst) {
    dst.resize((size_t)N * K);
    for (size_t r = 0; r < N; ++r)
        for (uint32_t k = 0; k < K; ++k) dst[r * K + router_perm(k)] = src[r * K + k];
}

namespace {

// ops::dot(w, x) over K elements (K a multiple of 32) for the 8 lanes j of a row: lane j runs
// the four chains acc_a = fma(w[32 i + 8 a + j], x[32 i + 8 a + j], acc_a) over the 32-element
// steps i (f32x8::mul_add of accumulator a, lane j), forms (acc0 + acc1) + (acc2 + acc3), and the
// row's 8 lanes add ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)) (f32x8::reduce_add as the
// oracle restates it).  wr: the row in F32Mat's permuted layout (global), xs: the activation in
// the same layout (LDS).  Every lane of the row returns the sum.
__device__ inline float dot_row_f32(const float *__restrict__ wr, const float *xs, uint32_t K, int j) {
    const v4f *w4 = reinterpret_cast<const v4f *>(wr) + j;
    const v4f *x4 = reinterpret_cast<const v4f *>(xs) + j;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 8
    for (uint32_t i = 0; i < K / 32; ++i) {
        const v4f w = __builtin_nontemporal_load(w4 + 8 * i);
        const v4f x = x4[8 * i];
        a0 = fmaf(w.x, x.x, a0);
        a1 = fmaf(w.y, x.y, a1);
        a2 = fmaf(w.z, x.z, a2);
        a3 = fmaf(w.w, x.w, a3);
    }
    float v = (a0 + a1) + (a2 + a3);
    v = v + shfl_xor(v, 4);
    v = v + shfl_xor(v, 2);
    v = v + shfl_xor(v, 1);
    return v;
}

// x[0 .. K) (global) into xs (LDS) in the permuted layout.
__device__ inline void stage_perm(const float *__restrict__ x, uint32_t K, float *xs) {
    for (uint32_t k = threadIdx.x; k < K; k += blockDim.x) xs[router_perm(k)] = x[k];
}

// 32 rows per workgroup of 256 threads (8 lanes a row).
template <int EPI>
__global__ __launch_bounds__(256) void k_f32_matvec(F32Mat W, const float *__restrict__ x, float *y, uint32_t valid,
                                                    float *part_v, uint32_t *part_i) {
    extern __shared__ __align__(16) float xs[];
    const int tid = threadIdx.x, j = tid & 7;
    const uint32_t row = blockIdx.x * 32 + (uint32_t)(tid >> 3), lrow = min(row, W.N - 1);
    stage_perm(x, W.K, xs);
    __syncthreads();
    const float v = dot_row_f32(W.w + (size_t)lrow * W.K, xs, W.K, j);
    if (row < W.N && j == 0) {
        if (EPI == EPI_RESID) y[row] = y[row] + v;
        else y[row] = v;
    }
    if (EPI == EPI_LOGITS) {   // the greedy argmax's partials (sample.rs:53-63): first maximum wins
        __shared__ float bv[4];
        __shared__ uint32_t bi[4];
        float mv = -__builtin_huge_valf();
        uint32_t mi = 0xffffffffu;
        if (j == 0 && row < W.N && row < valid && v > mv) {
            mv = v;
            mi = row;
        }
        for (int m = 8; m < 64; m <<= 1) {
            const float ov = shfl_xor(mv, m);
            const uint32_t oi = (uint32_t)shfl_xor_i((int)mi, m);
            if (ov > mv || (ov == mv && oi < mi)) {
                mv = ov;
                mi = oi;
            }
        }
        if ((tid & 63) == 0) {
            bv[tid >> 6] = mv;
            bi[tid >> 6] = mi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int wv = 1; wv < 4; ++wv)
                if (bv[wv] > mv || (bv[wv] == mv && bi[wv] < mi)) {
                    mv = bv[wv];
                    mi = bi[wv];
                }
            part_v[blockIdx.x] = mv;
            part_i[blockIdx.x] = mi;
        }
    }
}

// grid (ceil(f / 32), n_slots).  The slot's matrices: expert ids[s] of the stacked G / U (rows
// ids[s] f ..), the shared G_sh / U_sh for s = top_k, the dense G / U when ids is null.
__global__ __launch_bounds__(256) void k_f32_gateup(F32Mat G, F32Mat U, F32Mat Gs, F32Mat Us,
                                                    const uint32_t *__restrict__ ids, uint32_t top_k, uint32_t f,
                                                    const float *__restrict__ h, float *a) {
    extern __shared__ __align__(16) float xs[];
    const int tid = threadIdx.x, j = tid & 7;
    const uint32_t s = blockIdx.y;
    const bool sh = ids != nullptr && s >= top_k;   // (uniform)
    const F32Mat g = sh ? Gs : G, u = sh ? Us : U;
    const uint32_t base = (ids != nullptr && !sh) ? ids[s] * f : 0u;
    const uint32_t row = blockIdx.x * 32 + (uint32_t)(tid >> 3), lrow = base + min(row, f - 1);
    stage_perm(h, g.K, xs);
    __syncthreads();
    const float gv = dot_row_f32(g.w + (size_t)lrow * g.K, xs, g.K, j);
    const float uv = dot_row_f32(u.w + (size_t)lrow * u.K, xs, u.K, j);
    if (row < f && j == 0) a[(size_t)s * f + row] = hg_silu(gv) * uv;
}

// grid (ceil(d / 32), n_slots): y[s][r] = dot(D_s[r], a[s]).
__global__ __launch_bounds__(256) void k_f32_down(F32Mat D, F32Mat Ds, const uint32_t *__restrict__ ids,
                                                  uint32_t top_k, uint32_t d, uint32_t f, const float *__restrict__ a,
                                                  float *y) {
    extern __shared__ __align__(16) float xs[];
    const int tid = threadIdx.x, j = tid & 7;
    const uint32_t s = blockIdx.y;
    const bool sh = ids != nullptr && s >= top_k;   // (uniform)
    const F32Mat m = sh ? Ds : D;
    const uint32_t base = (ids != nullptr && !sh) ? ids[s] * d : 0u;
    const uint32_t row = blockIdx.x * 32 + (uint32_t)(tid >> 3), lrow = base + min(row, d - 1);
    stage_perm(a + (size_t)s * f, f, xs);
    __syncthreads();
    const float v = dot_row_f32(m.w + (size_t)lrow * m.K, xs, m.K, j);
    if (row < d && j == 0) y[(size_t)s * d + row] = v;
}

#define FLAUNCH(kern, grid, block, shm, st, ...)                                                             \
    do {                                                                                                     \
        if (LaunchTimer *t_ = launch_timer()) {                                                              \
            hipEvent_t a_ = nullptr, b_ = nullptr;                                                           \
            (void)hipEventCreate(&a_);                                                                       \
            (void)hipEventCreate(&b_);                                                                       \
            hipExtLaunchKernelGGL(kern, grid, block, shm, st, a_, b_, 0, __VA_ARGS__);                       \
            t_->add(a_, b_);                                                                                 \
        } else {                                                                                             \
            hipLaunchKernelGGL(kern, grid, block, shm, st, __VA_ARGS__);                                     \
        }                                                                                                    \
        const hipError_t le_ = hipGetLastError();                                                            \
        if (le_ != hipSuccess) note_launch_error(le_, #kern);                                                \
    } while (0)

bool shape_ok(const F32Mat &W, const char *what) {
    if (W.w && W.N && W.K && W.K % 32 == 0) return true;
    note_launch_error(hipErrorInvalidValue, std::string(what) + ": F32 matrix without rows or with K % 32 != 0");
    return false;
}

}  // namespace

void launch_f32_matvec(hipStream_t st, int epi, const F32Mat &W, const float *x, float *y, uint32_t valid,
                       float *part_v, uint32_t *part_i) {
    if (!shape_ok(W, "k_f32_matvec")) return;
    const dim3 grid(f32_matvec_blocks(W.N));
    const size_t shm = (size_t)W.K * 4;
    if (epi == EPI_RESID) FLAUNCH(k_f32_matvec<EPI_RESID>, grid, dim3(256), shm, st, W, x, y, valid, part_v, part_i);
    else if (epi == EPI_LOGITS)
        FLAUNCH(k_f32_matvec<EPI_LOGITS>, grid, dim3(256), shm, st, W, x, y, valid, part_v, part_i);
    else FLAUNCH(k_f32_matvec<EPI_STORE>, grid, dim3(256), shm, st, W, x, y, valid, part_v, part_i);
}

void launch_f32_gateup(hipStream_t st, const F32Mat &G, const F32Mat &U, const F32Mat &Gs, const F32Mat &Us,
                       const uint32_t *ids, uint32_t top_k, uint32_t n_slots, uint32_t f, const float *h, float *a) {
    if (!shape_ok(G, "k_f32_gateup") || !shape_ok(U, "k_f32_gateup") || U.K != G.K) return;
    if (ids && top_k < n_slots && (!shape_ok(Gs, "k_f32_gateup") || !shape_ok(Us, "k_f32_gateup") || Gs.K != G.K))
        return;
    FLAUNCH(k_f32_gateup, dim3(f32_matvec_blocks(f), n_slots), dim3(256), (size_t)G.K * 4, st, G, U, Gs, Us, ids, top_k,
            f, h, a);
}

void launch_f32_down(hipStream_t st, const F32Mat &D, const F32Mat &Ds, const uint32_t *ids, uint32_t top_k,
                     uint32_t n_slots, uint32_t d, uint32_t f, const float *a, float *y) {
    if (!shape_ok(D, "k_f32_down") || D.K != f) return;
    if (ids && top_k < n_slots && (!shape_ok(Ds, "k_f32_down") || Ds.K != f)) return;
    FLAUNCH(k_f32_down, dim3(f32_matvec_blocks(d), n_slots), dim3(256), (size_t)f * 4, st, D, Ds, ids, top_k, d, f, a,
            y);
}

}  // namespace hg
