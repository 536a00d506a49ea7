// hg_f32.h -- the F32 matrix mode (Engine::load(path, quant = false), lib.rs:85-92): every weight
// matrix kept as f32 (Mat::Owned, quant.rs:198-222) and applied with ops::matvec / ops::matmul
// (ops.rs:40-71), whose per-output arithmetic is ops::dot (ops.rs:7-36) for decode and prompt
// rows alike.  Kernels in hg_f32.hip.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace hg {

// A row-major f32 matrix [N][K] on the device, K a multiple of 32, each row stored with
// router_perm applied within every 32-element step (element k of a row at 32 (k / 32) +
// 4 (k % 8) + (k % 32) / 8): the four accumulator chains of ops::dot's lane l (elements
// 32 i + l, + 8, + 16, + 24) are one 16-byte load.
struct F32Mat {
    const float *w = nullptr;
    uint32_t N = 0, K = 0;
};

// Row permutation of a host [N][K] matrix into F32Mat's layout.
void permute_f32_rows(const float *src, uint32_t N, uint32_t K, std::vector<float> &dst);

// y[r] = dot(W[r], x) (ops::matvec): EPI_STORE y[r] = v, EPI_RESID y[r] += v, EPI_LOGITS y[r] = v
// and per-workgroup (max, first index) partials over rows < valid into part_v / part_i (one
// per 32 rows).  x: device, K floats.
void launch_f32_matvec(hipStream_t st, int epi, const F32Mat &W, const float *x, float *y, uint32_t valid,
                       float *part_v, uint32_t *part_i);
inline uint32_t f32_matvec_blocks(uint32_t N) { return (N + 31) / 32; }

// a[s][i] = silu(dot(G_s[i], h)) * dot(U_s[i], h) for the slots s < n_slots (model.rs:301-305,
// 314-318, 243-255): slot s < top_k uses expert ids[s] of the stacked G / U ([E f][K]), slot top_k
// the shared G_sh / U_sh; with ids == nullptr slot 0 is the dense G / U.  a: [n_slots][f].
void launch_f32_gateup(hipStream_t st, const F32Mat &G, const F32Mat &U, const F32Mat &Gs, const F32Mat &Us,
                       const uint32_t *ids, uint32_t top_k, uint32_t n_slots, uint32_t f, const float *h, float *a);

// y[s][r] = dot(D_s[r], a[s]) for every slot (the routed experts' down rows of ids[s], the shared
// expert's for slot top_k).  y: [n_slots][d].
void launch_f32_down(hipStream_t st, const F32Mat &D, const F32Mat &Ds, const uint32_t *ids, uint32_t top_k,
                     uint32_t n_slots, uint32_t d, uint32_t f, const float *a, float *y);

}  // namespace hg
