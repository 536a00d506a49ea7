// hg_batch_kernels.hip -- gfx950 kernels of the batched decode step: many sequences, one token
// each, every sequence's arithmetic identical to its own single-sequence step.
//
// The Q8 matrix products of the step run as int8 MFMA GEMMs (v_mfma_i32_16x16x32_i8) that keep
// the per-sequence operation order of the reference:
//   decode order, qrow_dot_avx2 (quant.rs:44-67): lane j of a row's 8 accumulators takes
//     acc_j = fma(sw[b] * dx[b], isum_{b,j}, acc_j) over blocks b, where isum_{b,j} is the int8
//     dot of the 4 elements 32b + 4j .. 32b + 4j + 3 only.  An MFMA sums over all 32 K slots
//     of its block, so the activation operand is masked: column (token, j) holds token's 4
//     elements of lane j and zeros elsewhere, and C[row][(token, j)] is exactly isum_{b,j}.
//     One MFMA covers 16 rows x 2 tokens x 8 lanes; the 8 lane accumulators are then reduced
//     ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) across lanes, as the reference's hsum.
// The operand layout is given at k_gemm16.
//
// KV rows live in pages of PAGE positions (a pool per layer; per page and kv head a K tile and a
// V tile laid out for 16-byte loads, see PagedKV); each sequence's block table maps position t
// to page bt[t / PAGE].
#include <hip/hip_ext.h>

#include "hg_batch.h"
#include "hg_common.h"
#include "hg_device.h"
#include "hg_expf.h"

namespace hg {

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
// y[out_row[e]][row] (+)= (W x_{act_row[e]})[row] for the entries e of each column tile (at most
// 8) and the rows of its matrix group, in qrow_dot_avx2's order (see the file comment).
// Workgroup = 4 waves over 16 PPW rows (blockIdx.x) of one column tile (blockIdx.y; tiles past
// *n_tiles exit); a wave owns 16 rows and PPW of the tile's 4 entry pairs (4 / PPW waves share a
// row tile through L1), so with PPW = 4 its weight loads are its own and each serves all the
// tile's entries, and smaller PPW spread small GEMMs over more waves.  The tile's activations
// (quants and block scales of its <= 8 entries) are staged in LDS first; the wave streams its
// rows' chunks through a register ring of D chunks.  One
// v_mfma_i32_16x16x32_i8 per (block, entry pair): lane l supplies A row l % 16 and B column
// l % 16 = (entry 2p + (l % 16) / 8, lane j = l % 8) for K group g = l / 16 (8 bytes: block
// elements 8g .. 8g + 7, i.e. the reference lanes 2g and 2g + 1 -- in the device row layout the
// chunk's 32 bytes at 32 g, word t of each 16-byte half = block t); C register v of lane l is
// row 4 g + v, column l % 16 (probed on gfx950).  The B operand is masked to the 4 elements of
// lane j (only group g = j / 2 is nonzero), so C[v] = isum_{b,j} exactly, and each lane runs
// acc = fma(sw * dx, isum, acc) over the blocks in order for its (row, entry, lane-j)
// accumulators.  GM_GATEUP: each wave runs the gate and the up matrices and stores silu(g) * u
// (model.rs:301-305).  D divides nc; FULLK: every chunk has 4 blocks (else D = 1 and the last
// chunk's padding blocks are skipped).
__host__ __device__ inline size_t gemm_lds(uint32_t nc) { return (size_t)8 * nc * (CHUNK_BYTES + 16); }

template <bool SCF32, int MODE, int D, bool FULLK, int PPW>
__global__ __launch_bounds__(256) void k_gemm16(GemmArgs g) {
    static_assert(FULLK || D == 1, "a partial last chunk: one chunk per group");
    static_assert(PPW == 1 || PPW == 2 || PPW == 4, "entry pairs per wave");
    constexpr uint32_t WPR = 4 / PPW;   // waves per row tile
    constexpr int NM = MODE == GM_GATEUP ? 2 : 1;   // matrices per wave
    typedef typename ScaleVec<SCF32>::T SV;
    extern __shared__ __align__(16) uint8_t xs[];   // [8 entries][nc][128] quants, then [8][nc][4] scales
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t ntl = *g.n_tiles;
    const GemmTile tile = g.tiles[blockIdx.y];   // (read with the count: the table has gridDim.y entries)
    if (blockIdx.y >= ntl) return;   // (uniform)
    Q8Mat M[NM];
    M[0] = g.W[tile.mat];
    if constexpr (NM == 2) M[1] = g.U[tile.mat];
    const uint32_t nc = M[0].nc, nb = M[0].nb, ne = tile.count;
    float *xds = reinterpret_cast<float *>(xs + (size_t)8 * nc * CHUNK_BYTES);
    // the tile's activations (entries past the count: zeros)
    for (uint32_t i = tid; i < 8 * nc * 8; i += 256) {   // 16-byte pieces: entry i / (8 nc)
        const uint32_t e = i / (nc * 8), p = i % (nc * 8);
        v4i v = {0, 0, 0, 0};
        if (e < ne) v = *reinterpret_cast<const v4i *>(g.aq + (size_t)g.act_row[tile.entry0 + e] * g.aqs + p * 16);
        *reinterpret_cast<v4i *>(xs + (size_t)i * 16) = v;
    }
    for (uint32_t i = tid; i < 8 * nc; i += 256) {   // block scales: entry i / nc, chunk i % nc
        const uint32_t e = i / nc, c = i % nc;
        v4f v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (e < ne) v = *reinterpret_cast<const v4f *>(g.ad + (size_t)g.act_row[tile.entry0 + e] * g.ads + 4 * c);
        *reinterpret_cast<v4f *>(xds + 4 * i) = v;
    }
    __syncthreads();
    const uint32_t r0 = blockIdx.x * 16 * PPW + ((uint32_t)wave / WPR) * 16;   // this wave's rows within the group
    const uint32_t p0 = ((uint32_t)wave % WPR) * PPW;                           // and its first entry pair
    if (r0 >= g.rows) return;   // (uniform per wave; after the workgroup's only barrier)
    const WaveExpTab tab = WaveExpTab::load(lane);
    const uint32_t gq = (uint32_t)lane >> 4, cc = (uint32_t)lane & 15, k = cc >> 3, j = cc & 7;
    const uint32_t gbase = tile.grp * g.rows, rlim = gbase + g.rows - 1, np = div_up(ne, 2);
    const bool bact = gq == (j >> 1);   // the lane whose K group holds lane j's 4 elements
    const uint8_t *wrow[NM];
    const SV *srow[NM][4];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        wrow[m] = M[m].qs + (size_t)min(gbase + r0 + cc, rlim) * nc * CHUNK_BYTES + 32 * gq;
#pragma unroll
        for (int v = 0; v < 4; ++v)
            srow[m][v] = reinterpret_cast<const SV *>(row_sc<SCF32>(M[m], min(gbase + r0 + 4 * gq + v, rlim)));
    }
    struct Ch {
        v4i w[NM][2];
        SV s[NM][4];
    };
    auto load = [&](Ch &d, uint32_t c) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const v4i *wp = reinterpret_cast<const v4i *>(wrow[m] + (size_t)c * CHUNK_BYTES);
            d.w[m][0] = __builtin_nontemporal_load(wp);
            d.w[m][1] = __builtin_nontemporal_load(wp + 1);
#pragma unroll
            for (int v = 0; v < 4; ++v) d.s[m][v] = srow[m][v][c];
        }
    };
    float acc[NM][PPW][4];   // [matrix][entry pair][row v]
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int p = 0; p < PPW; ++p)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[m][p][v] = 0.0f;
    auto compute = [&](const Ch &d, uint32_t c) {
        float sw[NM][4][4];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) unpack_scales(d.s[m][v], sw[m][v]);
#pragma unroll
        for (uint32_t p = 0; p < PPW; ++p) {
            if (p0 + p < np) {   // (uniform)
                const uint32_t ei = 2 * (p0 + p) + k;   // this lane's entry of the pair
                const v4i b4 = *reinterpret_cast<const v4i *>(xs + ((size_t)ei * nc + c) * CHUNK_BYTES + j * 16);
                const v4f dx4 = *reinterpret_cast<const v4f *>(xds + ((size_t)ei * nc + c) * 4);
                const int bw[4] = {b4.x, b4.y, b4.z, b4.w};
                const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    if (FULLK || 4 * c + t < nb) {   // (uniform; padding blocks of a partial last chunk: no add)
                        const uint32_t w = bact ? (uint32_t)bw[t] : 0u;
                        const long B = (long)((j & 1) ? (uint64_t)w << 32 : (uint64_t)w);
#pragma unroll
                        for (int m = 0; m < NM; ++m) {
                            const int lo = t == 0 ? d.w[m][0].x : t == 1 ? d.w[m][0].y : t == 2 ? d.w[m][0].z : d.w[m][0].w;
                            const int hi = t == 0 ? d.w[m][1].x : t == 1 ? d.w[m][1].y : t == 2 ? d.w[m][1].z : d.w[m][1].w;
                            const long A = (long)((uint64_t)(uint32_t)lo | (uint64_t)(uint32_t)hi << 32);
                            const v4i z = {0, 0, 0, 0};
                            const v4i C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, z, 0, 0, 0);
#pragma unroll
                            for (int v = 0; v < 4; ++v)
                                acc[m][p][v] = fmaf(sw[m][v][t] * dxs[t], (float)C[v], acc[m][p][v]);
                        }
                    }
                }
            }
        }
    };
    Ch ring[D];
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
        load(ring[u], min(u, nc - 1));
        __builtin_amdgcn_sched_barrier(0);   // (slot order as in the loop: the loop's waits hold for its first pass)
    }
    // groups of D chunks; each group refills its slots with the chunks D ahead (the last group's
    // refills re-read the last chunk: cache hits, issued without a branch so that each chunk's
    // wait counts only the loads after its own)
    for (uint32_t c0 = 0; c0 < nc; c0 += D) {
#pragma unroll
        for (uint32_t u = 0; u < D; ++u) {
            compute(ring[u], c0 + u);
            load(ring[u], min(c0 + D + u, nc - 1));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) over the 8 lanes j of each (row, entry), then the stores
#pragma unroll
    for (uint32_t p = 0; p < PPW; ++p) {
        if (p0 + p >= np) break;   // (uniform)
        float out[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            float r[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                float a = acc[m][p][v];
                {
                    const float dn = dpp_f<0x124>(a), up = dpp_f<0x12C>(a);
                    a = a + ((j & 4) ? dn : up);
                }
                a = a + dpp_f<0x4E>(a);
                a = a + dpp_f<0xB1>(a);
                r[m] = a;
            }
            out[v] = MODE == GM_GATEUP ? hg_silu_l(r[0], tab) * r[NM - 1] : r[0];   // (every lane)
        }
        const uint32_t ei = 2 * (p0 + p) + k;
        if (j == 0 && ei < ne) {
            float *yo = g.y + (size_t)g.out_row[tile.entry0 + ei] * g.ys;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t rl = r0 + 4 * gq + v;
                if (rl < g.rows) {
                    if (MODE == GM_RESID) yo[rl] = yo[rl] + out[v];
                    else yo[rl] = out[v];
                }
            }
        }
    }
}

// ------------------------------------------------------------------ MFMA GEMM, prompt order
// y[out_row[e]][row] (+)= (W x_{act_row[e]})[row] in Q8Tensor::matmul's order (quant.rs:164-184):
// acc = acc + (sw[b] * dx[b]) * isum_b over the blocks b in order from 0, isum_b the int8 dot of
// the whole block (exact in any order).  One v_mfma_i32_16x16x32_i8 yields isum_b for 16 rows x
// 16 entries with no masking: lane l supplies A row l % 16 and B column (entry) l % 16 for K
// group g = l / 16 (block elements 8g .. 8g + 7: word t of the 16-byte halves at 32 g and
// 32 g + 16 of a chunk, t the block within the chunk); C register v of lane l is row 4 g + v,
// column l % 16.  Workgroup = PG_WAVES waves over 16 PG_WAVES rows (blockIdx.x) of one column
// tile of at most 16 NG entries (blockIdx.y; tiles past *n_tiles exit).  The tile's activations are staged in
// LDS with entry strides of an odd number of 16-byte units, so the 16 entries read at one chunk
// offset fall in distinct banks; each wave owns 16 rows and all of the tile's entries and streams
// its rows' chunks through a register ring of D chunks.  The epilogue is 4 VALU operations per
// (row, entry, block) against one MFMA per 256 of them, so the kernel is VALU-bound.
constexpr uint32_t PG_WAVES = 8;   // waves (of 16 rows each) per workgroup: 128 rows share a staged tile
__host__ __device__ inline uint32_t pgemm_qstride(uint32_t nc) { return nc * CHUNK_BYTES + 16; }
__host__ __device__ inline uint32_t pgemm_sstride(uint32_t nc) { return nc * 4 + 4; }
__host__ __device__ inline size_t pgemm_lds(uint32_t nc, uint32_t tt) {
    return (size_t)tt * (pgemm_qstride(nc) + 4 * pgemm_sstride(nc));
}

template <bool SCF32, int MODE, int D, bool FULLK, int NG>
__global__ __launch_bounds__(64 * PG_WAVES) void k_gemm_p(GemmArgs g) {
    static_assert(FULLK || D == 1, "a partial last chunk: one chunk per group");
    constexpr int NM = MODE == GM_GATEUP ? 2 : 1;   // matrices per wave
    constexpr uint32_t TT = 16 * NG;                // entries per column tile
    typedef typename ScaleVec<SCF32>::T SV;
    extern __shared__ __align__(16) uint8_t xs[];   // [TT][qstride] quants, then [TT][sstride] scales
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t ntl = *g.n_tiles;
    const GemmTile tile = g.tiles[blockIdx.y];   // (read with the count: the table has gridDim.y entries)
    if (blockIdx.y >= ntl) return;   // (uniform)
    Q8Mat M[NM];
    M[0] = g.W[tile.mat];
    if constexpr (NM == 2) M[1] = g.U[tile.mat];
    const uint32_t nc = M[0].nc, nb = M[0].nb, ne = tile.count;
    const uint32_t qst = pgemm_qstride(nc), sst = pgemm_sstride(nc);
    float *xds = reinterpret_cast<float *>(xs + (size_t)TT * qst);
    // 32-byte groups (a chunk's K group g: the lanes 2g and 2g + 1 of its 4 blocks), stored with
    // each block's two words side by side, so that the B operand of block t is one aligned pair
    for (uint32_t i = tid; i < TT * nc * 4; i += 64 * PG_WAVES) {   // entry i / (4 nc)
        const uint32_t e = i / (nc * 4), p = i % (nc * 4);
        v4i a = {0, 0, 0, 0}, b = {0, 0, 0, 0};
        if (e < ne) {
            const v4i *src = reinterpret_cast<const v4i *>(g.aq + (size_t)g.act_row[tile.entry0 + e] * g.aqs + p * 32);
            a = src[0];
            b = src[1];
        }
        v4i *dst = reinterpret_cast<v4i *>(xs + (size_t)e * qst + p * 32);
        dst[0] = v4i{a.x, b.x, a.y, b.y};
        dst[1] = v4i{a.z, b.z, a.w, b.w};
    }
    for (uint32_t i = tid; i < TT * nc; i += 64 * PG_WAVES) {   // block scales: entry i / nc, chunk i % nc
        const uint32_t e = i / nc, c = i % nc;
        v4f v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (e < ne) v = *reinterpret_cast<const v4f *>(g.ad + (size_t)g.act_row[tile.entry0 + e] * g.ads + 4 * c);
        *reinterpret_cast<v4f *>(xds + (size_t)e * sst + 4 * c) = v;
    }
    __syncthreads();
    const uint32_t r0 = blockIdx.x * 16 * PG_WAVES + (uint32_t)wave * 16;   // this wave's rows within the group
    if (r0 >= g.rows) return;   // (uniform per wave; after the workgroup's only barrier)
    const WaveExpTab tab = WaveExpTab::load(lane);
    const uint32_t gq = (uint32_t)lane >> 4, cc = (uint32_t)lane & 15;
    const uint32_t gbase = tile.grp * g.rows, rlim = gbase + g.rows - 1, ngr = div_up(ne, 16);
    const uint8_t *wrow[NM];
    const SV *srow[NM][4];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        wrow[m] = M[m].qs + (size_t)min(gbase + r0 + cc, rlim) * nc * CHUNK_BYTES + 32 * gq;
#pragma unroll
        for (int v = 0; v < 4; ++v)
            srow[m][v] = reinterpret_cast<const SV *>(row_sc<SCF32>(M[m], min(gbase + r0 + 4 * gq + v, rlim)));
    }
    struct Ch {
        long A[NM][4];   // the A operand of each block of the chunk (paired at load time)
        SV s[NM][4];
    };
    auto load = [&](Ch &d, uint32_t c) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const v4i *wp = reinterpret_cast<const v4i *>(wrow[m] + (size_t)c * CHUNK_BYTES);
            const v4i w0 = wp[0], w1 = wp[1];
            d.A[m][0] = (long)((uint64_t)(uint32_t)w0.x | (uint64_t)(uint32_t)w1.x << 32);
            d.A[m][1] = (long)((uint64_t)(uint32_t)w0.y | (uint64_t)(uint32_t)w1.y << 32);
            d.A[m][2] = (long)((uint64_t)(uint32_t)w0.z | (uint64_t)(uint32_t)w1.z << 32);
            d.A[m][3] = (long)((uint64_t)(uint32_t)w0.w | (uint64_t)(uint32_t)w1.w << 32);
#pragma unroll
            for (int v = 0; v < 4; ++v) d.s[m][v] = srow[m][v][c];
        }
    };
    const uint8_t *xb = xs + (size_t)cc * qst + 32 * gq;   // this lane's entry of group 0, its K group
    const float *xd = xds + (size_t)cc * sst;
    float acc[NM][NG][4];   // [matrix][entry group][row v]
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int q = 0; q < NG; ++q)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[m][q][v] = 0.0f;
    auto compute = [&](const Ch &d, uint32_t c) {
        float sw[NM][4][4];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) unpack_scales(d.s[m][v], sw[m][v]);
#pragma unroll
        for (int q = 0; q < NG; ++q) {
            if ((uint32_t)q < ngr) {   // (uniform)
                const uint8_t *bp = xb + (size_t)q * 16 * qst + (size_t)c * CHUNK_BYTES;
                const v2l b0 = *reinterpret_cast<const v2l *>(bp), b1 = *reinterpret_cast<const v2l *>(bp + 16);
                const v4f dx4 = *reinterpret_cast<const v4f *>(xd + (size_t)q * 16 * sst + 4 * c);
                const long Bt[4] = {b0.x, b0.y, b1.x, b1.y};
                const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    if (FULLK || 4 * c + t < nb) {   // (uniform; padding blocks of a partial last chunk: no add)
#pragma unroll
                        for (int m = 0; m < NM; ++m) {
                            const v4i z = {0, 0, 0, 0};
                            const v4i C = __builtin_amdgcn_mfma_i32_16x16x32_i8(d.A[m][t], Bt[t], z, 0, 0, 0);
#pragma unroll
                            for (int v = 0; v < 4; ++v) {
                                const float dd = sw[m][v][t] * dxs[t];
                                acc[m][q][v] = acc[m][q][v] + dd * (float)C[v];
                            }
                        }
                    }
                }
            }
        }
    };
    Ch ring[D];
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
        load(ring[u], min(u, nc - 1));
        __builtin_amdgcn_sched_barrier(0);
    }
    for (uint32_t c0 = 0; c0 < nc; c0 += D) {
#pragma unroll
        for (uint32_t u = 0; u < D; ++u) {
            compute(ring[u], c0 + u);
            load(ring[u], min(c0 + D + u, nc - 1));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int q = 0; q < NG; ++q) {
        if ((uint32_t)q >= ngr) break;   // (uniform)
        float out[4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
            out[v] = MODE == GM_GATEUP ? hg_silu_l(acc[0][q][v], tab) * acc[NM - 1][q][v] : acc[0][q][v];   // (every lane)
        const uint32_t ei = (uint32_t)q * 16 + cc;
        if (ei < ne) {
            float *yo = g.y + (size_t)g.out_row[tile.entry0 + ei] * g.ys;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t rl = r0 + 4 * gq + v;
                if (rl < g.rows) {
                    if (MODE == GM_RESID) yo[rl] = yo[rl] + out[v];
                    else yo[rl] = out[v];
                }
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
        float *vr = kv.v + kv_tile(page, hh - n_heads - n_kv, n_kv, HD);
        for (uint32_t i = lane; i < HD; i += 64) vr[v_el(i, p % PAGE, HD)] = u[i];
        return;
    }
    norm_rope_head<HD>(u, o, hc, hh < n_heads, eps, tmp, lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (uint32_t i = lane; i < HD; i += 64) src[i] = o[i];
    if (hh >= n_heads) {
        float *kr = kv.k + kv_tile(page, hh - n_heads, n_kv, HD);
        for (uint32_t i = lane; i < HD; i += 64) kr[k_el(i, p % PAGE)] = o[i];
    }
}

// ------------------------------------------------------------------ paged attention: scores
// s_t = dot(q_h, K_t) * (1/sqrt(hd)) (model.rs:213-218, ops::dot's order) for the rep query
// heads of kv head g (blockIdx.y) of sequence s (blockIdx.z) over positions
// [256 c, 256 c + 256) of its context (c = blockIdx.x; chunks past the context exit), and each
// head's chunk maximum.  Lane = position: its K row is read once (hd/4 16-byte loads, k_el) and
// dotted with every query head of the group (q broadcast from LDS).
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
    const uint32_t t = t0 + 64 * (uint32_t)wave + (uint32_t)lane;
    const bool live = t0 + 64 * (uint32_t)wave < n;   // (uniform per wave)
    v4f kt[HD / 4];
    if (live) {
        const uint32_t tc = min(t, n - 1);
        const v4f *kp = reinterpret_cast<const v4f *>(kv.k + kv_tile(kv.bt[(size_t)s * kv.bt_stride + tc / PAGE], g,
                                                                     kv.n_kv, HD)) + tc % PAGE;
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) kt[i] = kp[i * PAGE];
    }
    const float *qsrc = qkv + (size_t)s * qkv_stride + (size_t)g * rep * HD;
    for (uint32_t i = tid; i < rep * HD; i += 256) qs[i] = qsrc[i];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    float *scb = scores + ((size_t)s * n_heads + g * rep) * sc_stride;
    for (uint32_t r = 0; r < rep; ++r) {
        float mx = -__builtin_huge_valf();
        if (live) {
            const float *qr = qs + r * HD;
            float acc[4][8];   // ops::dot: four 8-lane FMA accumulators over 32-wide steps
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int l = 0; l < 8; ++l) acc[a][l] = 0.0f;
#pragma unroll
            for (int i = 0; i < HD; i += 32)
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int l = 0; l < 8; ++l) {
                        const int e = i + 8 * a + l;
                        acc[a][l] = fmaf(qr[e], kt[e / 4][e % 4], acc[a][l]);
                    }
            float v[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
            const float sv = (((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]))) * scale;
            if (t < n) {
                scb[(size_t)r * sc_stride + t] = sv;
                mx = sv;
            }
        }
        mx = wave_max_f(mx);
        if (lane == 0) wm[wave][r] = mx;
    }
    __syncthreads();
    if ((uint32_t)tid < rep)
        pmax[((size_t)s * n_heads + g * rep + tid) * pm_stride + c] =
            fmaxf(fmaxf(wm[0][tid], wm[1][tid]), fmaxf(wm[2][tid], wm[3][tid]));
}

// ------------------------------------------------------------------ paged attention: softmax
// The softmax of one (sequence, query head) row of scores (ops.rs:112-128): m = max of the
// chunk maxima, or with pmax == nullptr the max of the row itself (the scores staged in LDS
// first; the max is order-free); e_t = exp(s_t - m) with the reference expf, into LDS; sum = the
// index-order sum of e_t (block_seq_sum: 4 waves up to 3072 terms, 8 waves x 32 up to 16384,
// else one lane); p_t = e_t * (1 / sum) written over the scores.  Workgroups are dealt longest
// sequence first (order[] ranks the sequences by length).  NT = 512 threads, or 256 / 128 for
// contexts of at most 3072 positions (4- or 2-wave sums; more workgroups per CU).
__host__ __device__ inline size_t bsm_lds(uint32_t max_ctx) { return ((size_t)div_up(max_ctx, 4) * 4 + 64) * 4; }

template <int NT>
__global__ __launch_bounds__(NT) void k_b_softmax(float *scores, uint32_t sc_stride, const float *__restrict__ pmax,
                                                  uint32_t pm_stride, const uint32_t *__restrict__ pos,
                                                  const uint32_t *__restrict__ order, uint32_t n_heads) {
    extern __shared__ __align__(16) float e[];   // [max_ctx + 64]
    __shared__ xsum::Scratch xs;
    __shared__ float s_inv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t s = order[blockIdx.x / n_heads], h = blockIdx.x % n_heads;
    const uint32_t n = pos[s] + 1, nch = div_up(n, ACH);
    float *sc = scores + ((size_t)s * n_heads + h) * sc_stride;
    const float *pm = pmax + ((size_t)s * n_heads + h) * pm_stride;
    const WaveExpTab tab = WaveExpTab::load(lane);
    float m = -__builtin_huge_valf();
    constexpr uint32_t EB = 8;   // score loads in flight per thread
    if (pmax) {
        for (uint32_t c = lane; c < nch; c += 64) m = fmaxf(m, pm[c]);
        for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, shfl_xor(m, k));
    } else {   // the row into LDS and its max
        __shared__ float wmax[NT / 64];
        for (uint32_t t0 = 0; t0 < n; t0 += EB * NT) {
            float sv[EB];
#pragma unroll
            for (uint32_t u = 0; u < EB; ++u) sv[u] = sc[min(t0 + u * NT + (uint32_t)tid, n - 1)];
#pragma unroll
            for (uint32_t u = 0; u < EB; ++u) {
                const uint32_t t = t0 + u * NT + (uint32_t)tid;
                m = fmaxf(m, sv[u]);   // (clamped lanes repeat s_{n-1})
                if (t < n) e[t] = sv[u];
            }
        }
        m = wave_max_f(m);
        if (lane == 0) wmax[wave] = m;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) m = fmaxf(m, wmax[w]);
    }
    if (tid == 0) xs.sync = 0;
    for (uint32_t t0 = 0; t0 < n; t0 += EB * NT) {   // (uniform: every lane calls the exp)
        float sv[EB];
#pragma unroll
        for (uint32_t u = 0; u < EB; ++u) {
            const uint32_t t = min(t0 + u * NT + (uint32_t)tid, n - 1);
            sv[u] = pmax ? sc[t] : e[t];   // (each thread reads back only the entries it wrote)
        }
#pragma unroll
        for (uint32_t u = 0; u < EB; ++u) {
            const uint32_t t = t0 + u * NT + (uint32_t)tid;
            if (t0 + u * NT < n) {
                const float ev = hg_expf_l(sv[u] - m, tab);
                if (t < n) e[t] = ev;
            }
        }
    }
    if (tid < 4) e[n + tid] = 0.0f;   // readable up to a multiple of 4 past n
    __syncthreads();
    if (n <= 3072) {   // sum += e_t in index order (ops.rs:119-122)
        if constexpr (NT >= 256) {
            if (wave < 4) {
                const float r = n <= 2048 ? block_seq_sum<4, 8>(e, n, xs, wave, lane) : block_seq_sum<4, 12>(e, n, xs, wave, lane);
                if (tid == 0) s_inv = 1.0f / r;
            }
        } else {   // two waves, 16 or 24 terms per lane
            const float r = n <= 2048 ? block_seq_sum<2, 16>(e, n, xs, wave, lane) : block_seq_sum<2, 24>(e, n, xs, wave, lane);
            if (tid == 0) s_inv = 1.0f / r;
        }
    } else if (NT == 512 && n <= 16384) {
        const float r = block_seq_sum<8, 32>(e, n, xs, wave, lane);
        if (tid == 0) s_inv = 1.0f / r;
    } else if (tid == 0) {
        s_inv = 1.0f / seq_sum_lds(e, n, 0.0f);
    }
    __syncthreads();
    const float inv = s_inv;
    for (uint32_t t = tid; t < n; t += NT) sc[t] = e[t] * inv;   // p_t (x *= inv, ops.rs:124-126)
}

// ------------------------------------------------------------------ paged attention: P.V
// o[di] = ((0 + p_0 v_0[di]) + p_1 v_1[di]) + ... (model.rs:227-232): every (head, element) is a
// one-lane chain of rounded products added in position order, and the products are formed by
// other waves than the chain's: workgroup = a chain wave and PV2_NP producer waves for one
// (sequence, kv head, group of 4 query heads, slice of 16 elements).  A
// producer (lane = (slot quad q, element e)) loads each page's V slice (one 16-byte load:
// 4 positions of element e) and the 4 heads' probabilities of those positions, and writes the
// 16 products p * v (+0 past the context) into an LDS ring of PV2_NS slots of PV2_G pages, laid
// out [q][head][element][4 positions]; the chain wave (lane = (head, element)) reads 16
// positions of its chain per page with 4 conflict-free 16-byte reads and only adds.  Hand-offs:
// ready[slot] = group + 1 (producer), done = groups consumed (chain), both plain LDS words --
// the LDS executes one wave's operations in order, so a flag written after the data (and read
// before it) orders them without waits; only the compiler is fenced.  Every wait is bounded and
// reports *err.  Workgroups are dealt longest sequence first; the slices of one (sequence,
// kv head) get ids equal mod 8.  Positions past the context contribute +0, which leaves the
// chain unchanged: it never holds -0 (it starts at +0, and x + (-x) rounds to +0).
constexpr uint32_t PV2_G = 4, PV2_NS = 4, PV2_R = 24;   // pages per slot, ring slots, producer V ring (pages)
constexpr uint32_t PV2_NP = 3;                          // producer waves
constexpr size_t PV2_LDS_MAX = 96 * 1024;
constexpr uint32_t PV_SPIN_CAP = 1u << 22;
constexpr uint32_t PV2_PROB_FLOATS = PV2_NP * 2 * 4 * (PV2_G * PAGE + 4);   // the producers' probability rows
__host__ __device__ inline size_t pv2_lds(uint32_t max_ctx) {
    return (size_t)PV2_NS * PV2_G * 4096 + (size_t)div_up(div_up(max_ctx, PAGE), 4) * 16 + PV2_PROB_FLOATS * 4;
}
#define PV2_COMPILER_FENCE() asm volatile("" ::: "memory")

template <int HD>
__global__ __launch_bounds__(64 * (PV2_NP + 1)) void k_b_pv2(const float *__restrict__ probs, uint32_t sc_stride,
                                               const uint32_t *__restrict__ pos, const uint32_t *__restrict__ order,
                                               PagedKV kv, uint32_t n_seq, float *o_out, uint32_t *err,
                                               uint32_t flip) {
    constexpr uint32_t EW = 16, WPE = HD / EW, G = PV2_G, NS = PV2_NS, R = PV2_R;
    static_assert(R % G == 0, "whole slots per register ring");
    extern __shared__ __align__(16) float lds[];
    v4f *ring = reinterpret_cast<v4f *>(lds);   // [NS][G][q 4][head 4][element 16] x 4 positions
    float *pw_base = lds + NS * G * 1024;                                   // the producer's probability rows
    uint32_t *btl = reinterpret_cast<uint32_t *>(pw_base + PV2_PROB_FLOATS);   // the block table
    __shared__ uint32_t ready[NS], done;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n_heads = kv.n_heads, n_kv = kv.n_kv, rep = n_heads / n_kv;
    const uint32_t wpk = div_up(rep, 4) * WPE;   // workgroups per (sequence, kv head)
    uint32_t key, w;
    {
        // second round of the dispatch (ids >= flip) in reverse rank order, so the CU that holds
        // a long sequence's workgroup also holds a short one
        const uint32_t W = gridDim.x, L0 = blockIdx.x;
        const uint32_t L = (flip && L0 >= flip && W <= 2 * flip) ? flip + (W - 1 - L0) : L0;
        const uint32_t nkeys = n_seq * n_kv;
        if (nkeys % 8 == 0) {
            const uint32_t slot = L / 8;
            key = L % 8 + 8 * (slot / wpk);
            w = slot % wpk;
        } else {
            key = L / wpk;
            w = L % wpk;
        }
    }
    const uint32_t s = order[key / n_kv], g = key % n_kv, n = pos[s] + 1, npg = div_up(n, PAGE), ngr = div_up(npg, G);
    const uint32_t *bts = kv.bt + (size_t)s * kv.bt_stride;
    for (uint32_t i = threadIdx.x; i < npg; i += 64 * (PV2_NP + 1)) btl[i] = bts[i];
    if (threadIdx.x < NS) ready[threadIdx.x] = 0;
    if (threadIdx.x == 0) done = 0;
    __syncthreads();
    const uint32_t hb = (w / WPE) * 4, es = (w % WPE) * EW;   // head group, element slice
    if (wave >= 1) {
        // ---------------- producers: wave 1 + pp (pp < NP) writes the groups gi = pp, pp + NP, ...
        // lane = (slot quad q, element e).  A producer's local page k is page k % G of its
        // local group m = k / G (global group NP m + pp).  V: one 16-byte load per page through a
        // register ring of R local pages.  Probabilities: per local group (G pages, 16 G
        // positions), each lane loading 4 of its 4 x 16 G values two groups ahead, staged into an
        // LDS row per head (double buffered) at the end of the group before, and read back one
        // page ahead (4 broadcast 16-byte reads).
        constexpr uint32_t PB = G * PAGE, PLS = PB + 4;   // positions per group, padded row
        constexpr uint32_t NP = PV2_NP;
        static_assert(PB == 64 && NP * 2 * 4 * PLS == PV2_PROB_FLOATS, "probability rows");
        static_assert(R % (2 * G) == 0, "group parity constant across ring passes");
        const uint32_t pp = (uint32_t)wave - 1;
        float *pw = pw_base + pp * 2 * 4 * PLS;   // [2][4 heads][PLS]
        const uint32_t q = (uint32_t)lane >> 4, e = (uint32_t)lane & 15;
        const float *prb = probs + ((size_t)s * n_heads + g * rep) * sc_stride;
        const float *vg = kv.v + kv_tile(0, g, n_kv, HD) + (size_t)(q * HD + es + e) * 4;
        const size_t pstride = (size_t)n_kv * HD * PAGE;
        auto gpage = [&](uint32_t k) { return (NP * (k / G) + pp) * G + k % G; };   // local page -> page
        v4f vr[R];
        float pn[2][4];
        auto load_probs = [&](float (&d)[4], uint32_t m) {   // local group m; value i: head i, position lane
            const uint32_t t = min((NP * m + pp) * PB + (uint32_t)lane, n - 1);
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) d[i] = prb[(size_t)min(hb + i, rep - 1) * sc_stride + t];
        };
        auto stage_probs = [&](const float (&d)[4], uint32_t buf) {
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) pw[(buf * 4 + i) * PLS + lane] = d[i];
        };
        auto read_probs = [&](v4f (&d)[4], uint32_t k) {   // local page k's 4 positions 4q .. of each head
            const float *src = pw + ((k / G) % 2) * 4 * PLS + (k % G) * 16 + 4 * q;
#pragma unroll
            for (uint32_t h = 0; h < 4; ++h) d[h] = *reinterpret_cast<const v4f *>(src + h * PLS);
        };
        auto id_of = [&](uint32_t k) { return btl[min(gpage(k), npg - 1)]; };   // (clamped to the context's pages)
        // (issue order as in the loop: the loop's waits hold for its first pass)
        load_probs(pn[0], 0);
        load_probs(pn[1], 1);
        const uint32_t ids0 = id_of(lane);   // local pages 0 .. R - 1
#pragma unroll
        for (uint32_t u = 0; u < R; ++u) {
            vr[u] = *reinterpret_cast<const v4f *>(vg + (size_t)__builtin_amdgcn_readlane(ids0, u) * pstride);
            __builtin_amdgcn_sched_barrier(0);
        }
        uint32_t ids_nx = id_of(R + lane);
        stage_probs(pn[0], 0);
        load_probs(pn[0], 2);
        v4f pc[4], pn4[4], pr[G][4];   // (pr: the current group's products)
        read_probs(pc, 0);
        // local pages in blocks of R (the ring's loads run past the producer's last group; those
        // pages are not written)
        const uint32_t npr = (ngr > pp ? div_up(ngr - pp, NP) : 0u) * G;
        uint32_t dc = 0;
        for (uint32_t k0 = 0; k0 < npr; k0 += R) {
            const uint32_t ids = ids_nx;
            ids_nx = id_of(k0 + 2 * R + lane);
#pragma unroll
            for (uint32_t u = 0; u < R; ++u) {
                const uint32_t k = k0 + u, gi = NP * (k / G) + pp, sl = gi % NS, kg = gpage(k);
                if (u % G == G - 1) {   // the next local page starts local group m: stage it, load m + 2
                    const uint32_t m = (k + 1) / G;
                    stage_probs(pn[(u / G + 1) % 2], (u / G + 1) % 2);
                    load_probs(pn[(u / G + 1) % 2], m + 2);
                }
                read_probs(pn4, k + 1);
                if (gi < ngr) {   // (uniform; pages of groups past the last one are only loaded)
                    // the page's 16 products into registers; the group's G pages go to its ring
                    // slot together once the slot is free, so the wait for the chain overlaps
                    // the group's V waits and multiplies
                    const v4f vv = vr[u];
                    if (16 * kg + 16 <= n) {   // (uniform) a full page
#pragma unroll
                        for (uint32_t h = 0; h < 4; ++h)
                            pr[u % G][h] = v4f{pc[h].x * vv.x, pc[h].y * vv.y, pc[h].z * vv.z, pc[h].w * vv.w};
                    } else {   // positions t = 16 k + 4 q + c < n only
                        const uint32_t t = 16 * kg + 4 * q;
#pragma unroll
                        for (uint32_t h = 0; h < 4; ++h)
                            pr[u % G][h] = v4f{t < n ? pc[h].x * vv.x : 0.0f, t + 1 < n ? pc[h].y * vv.y : 0.0f,
                                               t + 2 < n ? pc[h].z * vv.z : 0.0f, t + 3 < n ? pc[h].w * vv.w : 0.0f};
                    }
                    if (u % G == G - 1) {
                        if (gi >= NS && dc < gi - NS + 1) {   // the slot's previous group consumed
                            uint32_t it = 0;   // (dc: the last count read; read again only when it is too low)
                            while ((dc = __hip_atomic_load(&done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < gi - NS + 1) {
                                if (++it > PV_SPIN_CAP) {
                                    if (lane == 0) atomicOr(err, 1u);
                                    break;
                                }
                                __builtin_amdgcn_s_sleep(1);
                            }
                            PV2_COMPILER_FENCE();
                        }
                        v4f *dst = ring + (size_t)sl * G * 256 + q * 64 + e;
#pragma unroll
                        for (uint32_t pg = 0; pg < G; ++pg)
#pragma unroll
                            for (uint32_t h = 0; h < 4; ++h) dst[pg * 256 + h * 16] = pr[pg][h];
                        PV2_COMPILER_FENCE();   // (the slot's data written before its flag)
                        if (lane == 0)
                            __hip_atomic_store(&ready[sl], gi + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    }
                }
                vr[u] = *reinterpret_cast<const v4f *>(vg + (size_t)__builtin_amdgcn_readlane(ids, u) * pstride);
#pragma unroll
                for (uint32_t h = 0; h < 4; ++h) pc[h] = pn4[h];
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        return;
    }
    // ---------------- chain
    const uint32_t hl = (uint32_t)lane >> 4;
    float o = 0.0f;
    auto poll = [&](uint32_t gi) {
        return __hip_atomic_load(&ready[gi % NS], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    auto wait_from = [&](uint32_t f, uint32_t gi) {   // f: the flag read early; spin only if not yet set
        uint32_t it = 0;
        while (f != gi + 1) {
            if (++it > PV_SPIN_CAP) {
                if (lane == 0) atomicOr(err, 1u);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            f = poll(gi);
        }
        PV2_COMPILER_FENCE();
    };
    auto read_group = [&](v4f (&a)[G * 4], uint32_t gi) {
        const v4f *src = ring + (size_t)(gi % NS) * G * 256 + lane;
#pragma unroll
        for (uint32_t i = 0; i < G * 4; ++i) a[i] = src[i * 64];   // page i / 4, quad i % 4
    };
    auto adds = [&](const v4f (&a)[G * 4], uint32_t i0, uint32_t i1) {
#pragma unroll
        for (uint32_t i = i0; i < i1; ++i) {
            o = o + a[i].x;
            o = o + a[i].y;
            o = o + a[i].z;
            o = o + a[i].w;
        }
    };
    v4f A[G * 4], B[G * 4];
    wait_from(poll(0), 0);
    read_group(A, 0);
    // two groups per iteration (A, B alternate): the next group's flag is read before the current
    // group's adds and its data read half-way through them; done is raised once a group's reads
    // are issued (the LDS executes them before the store)
    for (uint32_t gi = 0; gi < ngr; gi += 2) {
        const bool m1 = gi + 1 < ngr, m2 = gi + 2 < ngr;
        const uint32_t f1 = poll(gi + 1);
        __builtin_amdgcn_sched_barrier(0);
        adds(A, 0, G * 2);
        if (m1) {
            wait_from(f1, gi + 1);
            read_group(B, gi + 1);
        }
        PV2_COMPILER_FENCE();
        if (lane == 0) __hip_atomic_store(&done, gi + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        adds(A, G * 2, G * 4);
        if (!m1) break;
        const uint32_t f2 = poll(gi + 2);
        __builtin_amdgcn_sched_barrier(0);
        adds(B, 0, G * 2);
        if (m2) {
            wait_from(f2, gi + 2);
            read_group(A, gi + 2);
        }
        PV2_COMPILER_FENCE();
        if (lane == 0) __hip_atomic_store(&done, gi + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        adds(B, G * 2, G * 4);
    }
    if (hb + hl < rep) o_out[((size_t)s * n_heads + g * rep + hb + hl) * HD + es + (uint32_t)lane % 16] = o;
}

// Sequences ranked by length, longest first (equal lengths: lower index first).  One workgroup.
__global__ void k_b_order(const uint32_t *__restrict__ pos, uint32_t n, uint32_t *order) {
    for (uint32_t s = threadIdx.x; s < n; s += blockDim.x) {
        const uint32_t p = pos[s];
        uint32_t r = 0;
        for (uint32_t q = 0; q < n; ++q) {
            const uint32_t pq = pos[q];
            r += pq > p || (pq == p && q < s);
        }
        order[r] = s;
    }
}

// ------------------------------------------------------------------ expert grouping
// The ffn_prefill grouping (model.rs:676-731) for one step of n rows (sequences, or prompt
// rows): for every expert e (ascending), the (row, rank) pairs that picked it, then the shared
// expert with every row (slot top_k).  Entry i of the table: act_row = the
// sequence (its quantized h), out_row = sequence * n_slots + slot (its row of a and y).
// Column tiles of at most TT entries cover each expert's entries (matrix group e of set 0; the
// shared expert's tiles use group 0 of set 1).  One workgroup.
__global__ __launch_bounds__(1024) void k_b_group(const uint32_t *__restrict__ topk_idx, uint32_t n, uint32_t top_k,
                                                  uint32_t E, uint32_t n_slots, uint32_t TT,
                                                  uint32_t *act_row, uint32_t *out_row, GemmTile *tiles,
                                                  uint32_t *n_tiles) {
    __shared__ uint32_t cnt[MAX_GROUPS], base[MAX_GROUPS], wa[4], wt[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, NP = n * top_k;
    const uint32_t NG = E + (n_slots > top_k ? 1 : 0);
    if (tid < MAX_GROUPS) cnt[tid] = 0;
    __syncthreads();
#pragma unroll 4
    for (uint32_t i = tid; i < NP; i += 1024) {
        const uint32_t e = topk_idx[i];   // (< E: the router's output; anything else is dropped)
        if (e < E) atomicAdd(&cnt[e], 1u);
    }
    __syncthreads();
    // exclusive scans of the entry and tile counts over the groups (threads 0 .. 255 = groups)
    uint32_t c = 0, tc = 0, ia = 0, it = 0;
    if (tid < MAX_GROUPS) {   // (whole waves)
        c = tid < E ? cnt[tid] : tid < NG ? n : 0u;
        tc = div_up(c, TT);
        ia = wave_scan_u(c);
        it = wave_scan_u(tc);
        if (lane == 63) {
            wa[wave] = ia;
            wt[wave] = it;
        }
    }
    __syncthreads();
    if (tid < MAX_GROUPS) {
        uint32_t ba = 0, bt = 0;
        for (uint32_t w = 0; w < wave; ++w) {
            ba += wa[w];
            bt += wt[w];
        }
        const uint32_t off = ba + ia - c, toff = bt + it - tc;
        base[tid] = off;
        cnt[tid] = 0;   // (now the fill count of the placement below)
        if (tid == MAX_GROUPS - 1) *n_tiles = bt + it;
        if (tid < NG) {
            for (uint32_t q = 0; q < tc; ++q) {
                GemmTile tl;
                tl.grp = tid < E ? tid : 0u;
                tl.entry0 = off + q * TT;
                tl.count = min(TT, c - q * TT);
                tl.mat = tid < E ? 0u : 1u;
                tiles[toff + q] = tl;
            }
        }
    }
    __syncthreads();
    if (NG > E) {   // the shared expert: every row, slot top_k
        const uint32_t sb = base[E];
        for (uint32_t sq = tid; sq < n; sq += 1024) {
            act_row[sb + sq] = sq;
            out_row[sb + sq] = sq * n_slots + top_k;
        }
    }
    // the routed picks: a pick's entry is its expert's base + a slot taken with an LDS atomic
    // (the order of an expert's entries is arbitrary: each entry's GEMM column is its own)
#pragma unroll 4
    for (uint32_t i = tid; i < NP; i += 1024) {
        const uint32_t e = topk_idx[i];
        if (e < E) {
            const uint32_t at = base[e] + atomicAdd(&cnt[e], 1u);
            const uint32_t sq = i / top_k;
            act_row[at] = sq;
            out_row[at] = sq * n_slots + (i - sq * top_k);
        }
    }
}

// ------------------------------------------------------------------ expert combine + residual
// x[s] += ((0 + w_0 y_0) + w_1 y_1 + ...) + y_shared: rank order (model.rs:306-323 and 173-176,
// as k_ffn_down's decode combine), or with `order` (the router's ranks in ascending expert id)
// the prompt path's expert-id order (model.rs:707-731).  grid (d / 256, n).
__global__ void k_b_combine(const float *__restrict__ y, const float *__restrict__ topk_w,
                            const uint32_t *__restrict__ order, uint32_t top_k, uint32_t n_slots, uint32_t d,
                            float *x) {
    const uint32_t s = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d) return;
    const float *ys = y + (size_t)s * n_slots * d + i;
    float acc = 0.0f;
    for (uint32_t q = 0; q < top_k; ++q) {
        const uint32_t r = order ? order[s * top_k + q] : q;
        acc = acc + topk_w[s * top_k + r] * ys[(size_t)r * d];
    }
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

bool batch_ctx_ok(uint32_t max_ctx) { return bsm_lds(max_ctx) <= BSM_LDS_MAX && pv2_lds(max_ctx) <= PV2_LDS_MAX; }

hipError_t init_batch_kernel_attributes() {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_b_softmax<512>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)BSM_LDS_MAX);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_b_pv2<64>), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)PV2_LDS_MAX);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_b_pv2<128>), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)PV2_LDS_MAX);
    return e;
}

void launch_b_embed(hipStream_t st, const float *emb, uint32_t d, const uint32_t *tokens, uint32_t n, float *x) {
    BLAUNCH(k_b_embed, dim3(div_up(d, 256), n), dim3(256), 0, st, emb, d, tokens, x);
}

void launch_b_quant_rows(hipStream_t st, const float *x, uint32_t xs, uint32_t n_elems, uint32_t rows, uint8_t *q,
                         uint32_t qs, float *dq, uint32_t ds) {
    BLAUNCH(k_b_quant_rows, dim3(div_up(n_elems / QK, 32), rows), dim3(256), 0, st, x, xs, n_elems, q, qs, dq, ds);
}

bool launch_b_gemm(hipStream_t st, int mode, const GemmArgs &a, uint32_t max_tiles) {
    const Q8Mat &M = a.W[0];
    if (a.W[1].qs && a.W[1].sc_f32 != M.sc_f32) return false;
    if (mode == GM_GATEUP && (a.U[0].sc_f32 != M.sc_f32 || (a.U[1].qs && a.U[1].sc_f32 != M.sc_f32))) return false;
    const size_t lds = gemm_lds(M.nc);
    if (lds > 64 * 1024) return false;
    // entry pairs per wave: 4 (each weight load serves the whole tile) unless that leaves fewer
    // than 1024 waves, then 2; a ring of 2 chunks (occupancy over depth: measured on the 500M
    // shapes, 2 beats 4 and 8 for every GEMM of the step)
    const uint32_t nrt = div_up(a.rows, 16), cap = max_tiles * nrt;
    const uint32_t ppw = cap >= 1024 ? 4u : 2u;
    const dim3 grid(div_up(a.rows, 16 * ppw), max_tiles);
#define GEMM_L(S, MD, DD, FK)                                                                                \
    do {                                                                                                     \
        if (ppw == 4) BLAUNCH((k_gemm16<S, MD, DD, FK, 4>), grid, dim3(256), lds, st, a);                    \
        else BLAUNCH((k_gemm16<S, MD, DD, FK, 2>), grid, dim3(256), lds, st, a);                             \
    } while (0)
#define GEMM_D(S, MD)                                                                                        \
    if (M.nb % 4 != 0) GEMM_L(S, MD, 1, false);                                                              \
    else if (M.nc % 2 == 0) GEMM_L(S, MD, 2, true);                                                          \
    else GEMM_L(S, MD, 1, true);
    const bool f32s = M.sc_f32 != 0;
    switch (mode) {
    case GM_GATEUP:
        if (f32s) { GEMM_D(true, GM_GATEUP) } else { GEMM_D(false, GM_GATEUP) }
        break;
    case GM_STORE:
        if (f32s) { GEMM_D(true, GM_STORE) } else { GEMM_D(false, GM_STORE) }
        break;
    case GM_RESID:
        if (f32s) { GEMM_D(true, GM_RESID) } else { GEMM_D(false, GM_RESID) }
        break;
    default: return false;
    }
#undef GEMM_D
#undef GEMM_L
    return true;
}

bool launch_b_qk_rope_append(hipStream_t st, uint32_t hd, float *qkv, uint32_t qkv_stride, const float *qn,
                             const float *kn, float eps, const float *cs, const float *sn, const uint32_t *pos,
                             const PagedKV &kv, uint32_t n) {
    const dim3 grid(kv.n_heads + 2 * kv.n_kv, n);
    switch (hd) {
    case 32: BLAUNCH(k_b_qk_rope_append<32>, grid, dim3(64), 0, st, qkv, qkv_stride, qn, kn, eps, cs, sn, pos, kv); break;
    case 64: BLAUNCH(k_b_qk_rope_append<64>, grid, dim3(64), 0, st, qkv, qkv_stride, qn, kn, eps, cs, sn, pos, kv); break;
    case 128: BLAUNCH(k_b_qk_rope_append<128>, grid, dim3(64), 0, st, qkv, qkv_stride, qn, kn, eps, cs, sn, pos, kv); break;
    default: return false;
    }
    return true;
}

void launch_b_order(hipStream_t st, const uint32_t *pos, uint32_t n, uint32_t *order) {
    BLAUNCH(k_b_order, dim3(1), dim3(256), 0, st, pos, n, order);
}

bool launch_b_attention(hipStream_t st, uint32_t hd, const float *qkv, uint32_t qkv_stride, const uint32_t *pos,
                        const uint32_t *order, const PagedKV &kv, uint32_t n, uint32_t max_ctx, float *scores,
                        float *pmax, float *o, uint32_t *err) {
    if (!batch_ctx_ok(max_ctx) || (hd != 64 && hd != 128)) return false;
    const uint32_t nch = div_up(max_ctx, ACH), rep = kv.n_heads / kv.n_kv;
    const uint32_t wpk = div_up(rep, 4) * (hd / 16);
    const dim3 gs(nch, kv.n_kv, n), gm(n * kv.n_heads), gp(n * kv.n_kv * wpk);
    const uint32_t ss = b_sc_stride(max_ctx);
    if (hd == 64)
        BLAUNCH(k_b_scores<64>, gs, dim3(256), 0, st, qkv, qkv_stride, pos, kv, scores, ss, pmax, nch);
    else
        BLAUNCH(k_b_scores<128>, gs, dim3(256), 0, st, qkv, qkv_stride, pos, kv, scores, ss, pmax, nch);
    BLAUNCH(k_b_softmax<512>, gm, dim3(512), bsm_lds(max_ctx), st, scores, ss, pmax, nch, pos, order, kv.n_heads);
    // workgroups of the first dispatch round: one per CU
    static const uint32_t n_cu = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            v = 0;
        return (uint32_t)v;
    }();
    const uint32_t flip = n_cu;
    if (hd == 64)
        BLAUNCH(k_b_pv2<64>, gp, dim3(64 * (PV2_NP + 1)), pv2_lds(max_ctx), st, scores, ss, pos, order, kv, n, o, err,
                flip);
    else
        BLAUNCH(k_b_pv2<128>, gp, dim3(64 * (PV2_NP + 1)), pv2_lds(max_ctx), st, scores, ss, pos, order, kv, n, o, err,
                flip);
    return true;
}

void launch_b_group(hipStream_t st, const uint32_t *topk_idx, uint32_t n, uint32_t top_k, uint32_t E,
                    uint32_t n_slots, uint32_t tt, uint32_t *act_row, uint32_t *out_row, GemmTile *tiles,
                    uint32_t *n_tiles) {
    BLAUNCH(k_b_group, dim3(1), dim3(1024), 0, st, topk_idx, n, top_k, E, n_slots, tt, act_row, out_row, tiles,
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

// Seeded pseudo-random rows for positions [0, len) of one sequence in every layer's K and V
// pages (timing workloads): element value = a hash of (seed, layer, which, position, element)
// mapped to [-sqrt 3, sqrt 3) (unit variance).  grid (npg, n_layers, 2).
__global__ void k_b_page_fill(float *kpool, float *vpool, const uint32_t *__restrict__ bt, uint32_t len,
                              uint32_t n_kv, uint32_t hd, size_t layer_floats, uint64_t seed) {
    const uint32_t i = blockIdx.x, l = blockIdx.y, which = blockIdx.z, pf = n_kv * PAGE * hd;
    float *p = (which ? vpool : kpool) + layer_floats * l + (size_t)bt[i] * pf;
    for (uint32_t q = threadIdx.x; q < pf; q += blockDim.x) {
        // the inverse of k_el / v_el within the kv head's tile
        const uint32_t g = q / (PAGE * hd), r = q % (PAGE * hd);
        const uint32_t slot = which ? (r / 4 / hd) * 4 + r % 4 : (r / 4) % PAGE;
        const uint32_t e = which ? (r / 4) % hd : (r / (4 * PAGE)) * 4 + r % 4, t = i * PAGE + slot;
        uint64_t z = seed ^ ((uint64_t)l << 40) ^ ((uint64_t)which << 39) ^ ((uint64_t)t << 12) ^ (uint64_t)(g * hd + e);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;   // splitmix64 finalizer
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        const float u = (float)(z >> 40) * 0x1p-24f;
        p[q] = t < len ? (u * 2.0f - 1.0f) * 1.7320508f : 0.0f;
    }
}

void launch_b_page_fill(hipStream_t st, float *kpool, float *vpool, const uint32_t *bt, uint32_t len, uint32_t n_layers,
                        uint32_t n_kv, uint32_t hd, size_t layer_floats, uint64_t seed) {
    const uint32_t npg = div_up(len, PAGE);
    if (npg) BLAUNCH(k_b_page_fill, dim3(npg, n_layers, 2), dim3(256), 0, st, kpool, vpool, bt, len, n_kv, hd,
                     layer_floats, seed);
}

void launch_b_page_copy(hipStream_t st, float *flat, float *pool, const uint32_t *bt, uint32_t npg,
                        uint32_t page_floats, int dir) {
    if (npg) BLAUNCH(k_b_page_copy, dim3(npg), dim3(256), 0, st, flat, pool, bt, page_floats, dir);
}

void launch_b_combine(hipStream_t st, const float *y, const float *topk_w, const uint32_t *order, uint32_t top_k,
                      uint32_t n_slots, uint32_t d, uint32_t n, float *x) {
    BLAUNCH(k_b_combine, dim3(div_up(d, 256), n), dim3(256), 0, st, y, topk_w, order, top_k, n_slots, d, x);
}

// ====================================================================== prompt path
// Prompt rows r = blockIdx.y at positions base + r, their k (normed and rotated) and v rows from
// the QKV output, into a single-sequence cache layer: K [n_kv][cap][hd], V [n_kv][cap][hd] and
// V's transposed copy [n_kv][hd][vt_stride(cap)] after it (the appends of model.rs:384-389).
__global__ void k_p_kv_store(const float *__restrict__ qkv, uint32_t qw, uint32_t qd, uint32_t kvd, uint32_t hd,
                             uint32_t n_kv, uint32_t base, uint32_t cap, float *kc, float *vc) {
    const uint32_t r = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= kvd) return;
    const uint32_t g = i / hd, e = i % hd, p = base + r;
    const float *row = qkv + (size_t)r * qw + qd;
    const size_t at = ((size_t)g * cap + p) * hd + e;
    kc[at] = row[i];
    const float v = row[kvd + i];
    vc[at] = v;
    vc[(size_t)n_kv * cap * hd + ((size_t)g * hd + e) * vt_stride(cap) + p] = v;
}

// Positions [0, npos) of a single-sequence cache layer into pages 0, 1, ... of PAGE positions
// (the identity block table).  grid (div_up(npos hd, 256), n_kv).
__global__ void k_p_kv_pages(const float *__restrict__ kc, const float *__restrict__ vc, uint32_t cap, uint32_t n_kv,
                             uint32_t hd, uint32_t npos, float *kpg, float *vpg) {
    const uint32_t g = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npos * hd) return;
    const uint32_t p = i / hd, e = i % hd;
    const size_t src = ((size_t)g * cap + p) * hd + e, t = kv_tile(p / PAGE, g, n_kv, hd);
    kpg[t + k_el(e, p % PAGE)] = kc[src];
    vpg[t + v_el(e, p % PAGE, hd)] = vc[src];
}

// order[i] = n - 1 - i: prompt rows by context length, longest first.
__global__ void k_p_rev(uint32_t n, uint32_t *order) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) order[i] = n - 1 - i;
}

// Scores of prompt rows (model.rs:386-391): s_t = dot(q_{r,h}, K_t) * (1/sqrt(hd)) in ops::dot's
// order, as k_b_scores, for a block of PRB consecutive rows (blockIdx.z, longest block first)
// and the rep query heads of kv head g (blockIdx.y) over positions [256 c, 256 c + 256)
// (c = blockIdx.x; chunks past the block's longest row exit).  Lane = position: its K row is
// read once and dotted with the block's rep PRB query heads (scalar operands), so K is read once
// per block of rows instead of once per row.  The row maxima are left to the softmax, which
// reads every score anyway (a wave maximum per row and head here cost ~15 % of this kernel).
constexpr uint32_t PRB = 16;
template <int HD>
__global__ __launch_bounds__(256) void k_p_scores(const float *__restrict__ qkv, uint32_t qkv_stride,
                                                  const uint32_t *__restrict__ pos, uint32_t R, PagedKV kv,
                                                  float *scores, uint32_t sc_stride) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t c = blockIdx.x, g = blockIdx.y, rb0 = (gridDim.z - 1 - blockIdx.z) * PRB;
    const uint32_t nrow = min(PRB, R - rb0), nlast = pos[rb0 + nrow - 1] + 1, t0 = c * ACH;
    if (t0 >= nlast) return;   // (uniform)
    const uint32_t n_heads = kv.n_heads, rep = n_heads / kv.n_kv;
    const uint32_t t = t0 + 64 * (uint32_t)wave + (uint32_t)lane, tw = t0 + 64 * (uint32_t)wave;
    if (tw >= nlast) return;   // (uniform per wave: a wave past every row of the block)
    v4f kt[HD / 4];
    {
        const uint32_t tc = min(t, nlast - 1);
        const v4f *kp = reinterpret_cast<const v4f *>(kv.k + kv_tile(kv.bt[tc / PAGE], g, kv.n_kv, HD)) + tc % PAGE;
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) kt[i] = kp[i * PAGE];
    }
    const float scale = 1.0f / sqrtf((float)HD);
    for (uint32_t k = 0; k < nrow; ++k) {
        const uint32_t n = pos[rb0 + k] + 1;
        if (tw >= n) continue;   // (uniform per wave)
        float *scb = scores + ((size_t)(rb0 + k) * n_heads + g * rep) * sc_stride;
        for (uint32_t r = 0; r < rep; ++r) {
            // (a wave-uniform address of read-only memory: the query comes in scalar loads)
            const float *qr = qkv + (size_t)(rb0 + k) * qkv_stride + (size_t)(g * rep + r) * HD;
            float acc[4][8];   // ops::dot: four 8-lane FMA accumulators over 32-wide steps
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int l = 0; l < 8; ++l) acc[a][l] = 0.0f;
#pragma unroll
            for (int i = 0; i < HD; i += 32)
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int l = 0; l < 8; ++l) {
                        const int e = i + 8 * a + l;
                        acc[a][l] = fmaf(qr[e], kt[e / 4][e % 4], acc[a][l]);
                    }
            float v[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
            const float sv = (((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]))) * scale;
            if (t < n) scb[(size_t)r * sc_stride + t] = sv;
        }
    }
}

// P.V of prompt rows (model.rs:392-397): o[r][h][e] = ((0 + p_0 v_0[e]) + p_1 v_1[e]) + ... over
// positions 0 .. n_r - 1 (n_r = pos[r] + 1), every (row, head, element) its own chain: a rounded
// product, then the add.  A wave takes one row and the REP query heads of kv head g
// (blockIdx.y): lane = element (HD / 64 of them per lane), REP chains per element sharing each V
// load (16-byte loads of a page tile: 4 positions).  The probabilities are scalar operands
// (wave-uniform loads of read-only memory), PB = 64 / REP positions of every chain per block
// (64 scalar registers).  Workgroups of 4 waves (4 rows) are dealt longest rows first.
template <int HD, int REP>
__global__ __launch_bounds__(256) void k_p_pv(const float *__restrict__ probs, uint32_t ss,
                                              const uint32_t *__restrict__ pos, uint32_t R, PagedKV kv, float *o) {
    constexpr int EPL = HD >= 64 ? HD / 64 : 1, PB = 64 / REP;   // (heads of 32: lanes 32 .. 63 idle)
    const int lane_ = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool act = HD >= 64 || lane_ < HD;
    const int lane = act ? lane_ : HD - 1;   // (idle lanes load in bounds and store nothing)
    const uint32_t ngrp = div_up(R, 4u), g = blockIdx.y;
    const uint32_t r = (ngrp - 1 - blockIdx.x) * 4 + (uint32_t)wave;
    if (r >= R) return;   // (uniform per wave)
    const uint32_t n_heads = kv.n_heads, n = pos[r] + 1;
    const float *pb[REP];
#pragma unroll
    for (int c = 0; c < REP; ++c) pb[c] = probs + ((size_t)r * n_heads + g * REP + c) * ss;
    float acc[REP][EPL];
#pragma unroll
    for (int c = 0; c < REP; ++c)
#pragma unroll
        for (int q = 0; q < EPL; ++q) acc[c][q] = 0.0f;
    uint32_t t0 = 0;
    for (; t0 + PB <= n; t0 += PB) {   // blocks of PB positions
        v4f vv[PB / 4][EPL];
#pragma unroll
        for (int j = 0; j < PB / 4; ++j) {
            const uint32_t t = t0 + 4 * j;
            const float *vt = kv.v + kv_tile(kv.bt[t / PAGE], g, kv.n_kv, HD) + (size_t)((t % PAGE) / 4) * HD * 4;
#pragma unroll
            for (int q = 0; q < EPL; ++q) vv[j][q] = *reinterpret_cast<const v4f *>(vt + (size_t)(lane + 64 * q) * 4);
        }
        v4f pp[REP][PB / 4];
#pragma unroll
        for (int c = 0; c < REP; ++c)
#pragma unroll
            for (int j = 0; j < PB / 4; ++j) pp[c][j] = *reinterpret_cast<const v4f *>(pb[c] + t0 + 4 * j);
#pragma unroll
        for (int c = 0; c < REP; ++c)
#pragma unroll
            for (int j = 0; j < PB / 4; ++j)
#pragma unroll
                for (int q = 0; q < EPL; ++q) {
                    float a = acc[c][q];
                    a = a + pp[c][j].x * vv[j][q].x;
                    a = a + pp[c][j].y * vv[j][q].y;
                    a = a + pp[c][j].z * vv[j][q].z;
                    a = a + pp[c][j].w * vv[j][q].w;
                    acc[c][q] = a;
                }
    }
    for (; t0 < n; t0 += 4) {   // the rest, 4 positions at a time
        const float *vt = kv.v + kv_tile(kv.bt[t0 / PAGE], g, kv.n_kv, HD) + (size_t)((t0 % PAGE) / 4) * HD * 4;
        v4f vv[EPL];
#pragma unroll
        for (int q = 0; q < EPL; ++q) vv[q] = *reinterpret_cast<const v4f *>(vt + (size_t)(lane + 64 * q) * 4);
#pragma unroll
        for (int c = 0; c < REP; ++c) {
            const v4f pp = *reinterpret_cast<const v4f *>(pb[c] + t0);   // (t0 + 3 < ss)
#pragma unroll
            for (int q = 0; q < EPL; ++q) {
                float a = acc[c][q];
                a = a + pp.x * vv[q].x;
                if (t0 + 1 < n) a = a + pp.y * vv[q].y;
                if (t0 + 2 < n) a = a + pp.z * vv[q].z;
                if (t0 + 3 < n) a = a + pp.w * vv[q].w;
                acc[c][q] = a;
            }
        }
    }
    if (act)
#pragma unroll
        for (int c = 0; c < REP; ++c)
#pragma unroll
            for (int q = 0; q < EPL; ++q) o[((size_t)r * n_heads + g * REP + c) * HD + lane + 64 * q] = acc[c][q];
}

bool launch_p_attention(hipStream_t st, uint32_t hd, const float *qkv, uint32_t qkv_stride, const uint32_t *pos,
                        const uint32_t *order, const PagedKV &kv, uint32_t n, uint32_t max_ctx, float *scores,
                        float *pmax, float *o, uint32_t *err) {
    if (!batch_ctx_ok(max_ctx) || (hd != 32 && hd != 64 && hd != 128)) return false;
    const uint32_t rep = kv.n_heads / kv.n_kv;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8)   // other groupings: the decode step's P.V kernel
        return hd != 32 && launch_b_attention(st, hd, qkv, qkv_stride, pos, order, kv, n, max_ctx, scores, pmax, o, err);
    const uint32_t nch = div_up(max_ctx, ACH);
    const dim3 gs(nch, kv.n_kv, div_up(n, PRB)), gm(n * kv.n_heads);
    const uint32_t ss = b_sc_stride(max_ctx);
    if (hd == 32)
        BLAUNCH(k_p_scores<32>, gs, dim3(256), 0, st, qkv, qkv_stride, pos, n, kv, scores, ss);
    else if (hd == 64)
        BLAUNCH(k_p_scores<64>, gs, dim3(256), 0, st, qkv, qkv_stride, pos, n, kv, scores, ss);
    else
        BLAUNCH(k_p_scores<128>, gs, dim3(256), 0, st, qkv, qkv_stride, pos, n, kv, scores, ss);
    // (the softmax forms each row's maximum itself: pmax = nullptr)
    if (max_ctx <= 3072)   // (a prompt chunk's window: bsm_lds fits the default limit)
        BLAUNCH(k_b_softmax<128>, gm, dim3(128), bsm_lds(max_ctx), st, scores, ss, nullptr, nch, pos, order,
                kv.n_heads);
    else
        BLAUNCH(k_b_softmax<512>, gm, dim3(512), bsm_lds(max_ctx), st, scores, ss, nullptr, nch, pos, order,
                kv.n_heads);
    const dim3 gp(div_up(n, 4u), kv.n_kv);
#define PPV(H, P) BLAUNCH((k_p_pv<H, P>), gp, dim3(256), 0, st, scores, ss, pos, n, kv, o)
    if (hd == 32) {
        if (rep == 1) PPV(32, 1);
        else if (rep == 2) PPV(32, 2);
        else if (rep == 4) PPV(32, 4);
        else PPV(32, 8);
    } else if (hd == 64) {
        if (rep == 1) PPV(64, 1);
        else if (rep == 2) PPV(64, 2);
        else if (rep == 4) PPV(64, 4);
        else PPV(64, 8);
    } else {
        if (rep == 1) PPV(128, 1);
        else if (rep == 2) PPV(128, 2);
        else if (rep == 4) PPV(128, 4);
        else PPV(128, 8);
    }
#undef PPV
    return true;
}

void launch_p_kv_store(hipStream_t st, const float *qkv, uint32_t qw, uint32_t qd, uint32_t kvd, uint32_t hd,
                       uint32_t n_kv, uint32_t base, uint32_t rows, uint32_t cap, float *kc, float *vc) {
    BLAUNCH(k_p_kv_store, dim3(div_up(kvd, 256), rows), dim3(256), 0, st, qkv, qw, qd, kvd, hd, n_kv, base, cap, kc, vc);
}

void launch_p_kv_pages(hipStream_t st, const float *kc, const float *vc, uint32_t cap, uint32_t n_kv, uint32_t hd,
                       uint32_t npos, float *kpg, float *vpg) {
    if (npos == 0) return;
    BLAUNCH(k_p_kv_pages, dim3(div_up(npos * hd, 256), n_kv), dim3(256), 0, st, kc, vc, cap, n_kv, hd, npos, kpg, vpg);
}

void launch_p_rev(hipStream_t st, uint32_t n, uint32_t *order) {
    BLAUNCH(k_p_rev, dim3(div_up(n, 256)), dim3(256), 0, st, n, order);
}

uint32_t pgemm_tile(uint32_t nc) {
    for (uint32_t tt = 64; tt >= 16; tt /= 2)
        if (pgemm_lds(nc, tt) <= PGEMM_LDS_MAX) return tt;
    return 0;
}

bool launch_p_gemm(hipStream_t st, int mode, const GemmArgs &a, uint32_t max_tiles, uint32_t tt) {
    const Q8Mat &M = a.W[0];
    if (a.W[1].qs && a.W[1].sc_f32 != M.sc_f32) return false;
    if (mode == GM_GATEUP && (a.U[0].sc_f32 != M.sc_f32 || (a.U[1].qs && a.U[1].sc_f32 != M.sc_f32))) return false;
    if (tt != 16 && tt != 32 && tt != 64) return false;
    const size_t lds = pgemm_lds(M.nc, tt);
    if (lds > PGEMM_LDS_MAX || max_tiles == 0) return false;
    const dim3 grid(div_up(a.rows, 16 * PG_WAVES), max_tiles);
    // (each instantiation raises its dynamic LDS limit on first use)
#define PG_L(S, MD, DD, FK, N)                                                                               \
    do {                                                                                                     \
        auto kf_ = k_gemm_p<S, MD, DD, FK, N>;                                                               \
        static const hipError_t ae_ = hipFuncSetAttribute(reinterpret_cast<const void *>(kf_),               \
                                                          hipFuncAttributeMaxDynamicSharedMemorySize,        \
                                                          (int)PGEMM_LDS_MAX);                               \
        if (ae_ != hipSuccess) {                                                                             \
            note_launch_error(ae_, "k_gemm_p LDS limit");                                                    \
            return false;                                                                                    \
        }                                                                                                    \
        BLAUNCH(kf_, grid, dim3(64 * PG_WAVES), lds, st, a);                                                 \
    } while (0)
#define PG_N(S, MD, DD, FK)                                                                                  \
    if (tt == 64) PG_L(S, MD, DD, FK, 4);                                                                    \
    else if (tt == 32) PG_L(S, MD, DD, FK, 2);                                                               \
    else PG_L(S, MD, DD, FK, 1);
#define PG_D(S, MD)                                                                                          \
    if (M.nb % 4 == 0 && M.nc % 2 == 0) { PG_N(S, MD, 2, true) }                                             \
    else { PG_N(S, MD, 1, false) }
    const bool f32s = M.sc_f32 != 0;
    switch (mode) {
    case GM_GATEUP:
        if (f32s) { PG_D(true, GM_GATEUP) } else { PG_D(false, GM_GATEUP) }
        break;
    case GM_STORE:
        if (f32s) { PG_D(true, GM_STORE) } else { PG_D(false, GM_STORE) }
        break;
    case GM_RESID:
        if (f32s) { PG_D(true, GM_RESID) } else { PG_D(false, GM_RESID) }
        break;
    default: return false;
    }
#undef PG_D
#undef PG_N
#undef PG_L
    return true;
}

void launch_b_argmax(hipStream_t st, const float *logits, uint32_t V, uint32_t valid, uint32_t *pos, uint32_t *tokens,
                     uint32_t *out_ids, const uint32_t *step, uint32_t n, uint32_t feedback) {
    BLAUNCH(k_b_argmax, dim3(n), dim3(1024), 0, st, logits, V, valid, pos, tokens, out_ids, step, n, feedback);
}

void launch_b_step_advance(hipStream_t st, uint32_t *step) {
    BLAUNCH(k_b_step_advance, dim3(1), dim3(64), 0, st, step);
}

}  // namespace hg
