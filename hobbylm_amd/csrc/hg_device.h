// hg_device.h -- device helpers shared by the gfx950 kernels: lane moves, activation
// quantization, the Q8 row dot in the reference's lane order, exact sequential sums,
// QK-norm + RoPE of one head and ops::dot's order.  Every function restates a piece of
// hobby-rs's arithmetic in the same floating-point operation order (file:line at each).
#pragma once
#include <hip/hip_runtime.h>

#include "hg_common.h"
#include "hg_expf.h"

namespace hg {

// ------------------------------------------------------------------ small helpers
__device__ inline float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ inline int shfl_xor_i(int v, int m) { return __shfl_xor(v, m, 64); }

__device__ inline int sdot4(int a, int b) { return __builtin_amdgcn_sdot4(a, b, 0, false); }

// The 32-entry exp table held by the lanes of a wave (lane l: entry l mod 32) and read by
// lane shuffles, so an exp costs no dependent memory load.  load() is issued at kernel
// start; the lookup must be reached by every lane of the wave (hg_expf_l guarantees that
// within one call, the caller that the call itself is uniform).
struct WaveExpTab {
    int lo, hi;
    __device__ static WaveExpTab load(int lane) {
        const uint64_t b = hg_exp2_bits((uint32_t)lane & 31);
        return {(int)(uint32_t)b, (int)(uint32_t)(b >> 32)};
    }
    __device__ uint64_t operator()(uint32_t i) const {
        const uint32_t l = (uint32_t)__shfl(lo, (int)i, 64), h = (uint32_t)__shfl(hi, (int)i, 64);
        return ((uint64_t)h << 32) | l;
    }
};

// Lane moves within rows of 16 lanes (DPP): no LDS round trip.  quad_perm [1,0,3,2] and
// [2,3,0,1] exchange with lane^1 and lane^2; row_ror:12 reads lane+4 and row_ror:4 lane-4
// (mod 16), so lane^4 is the one or the other by bit 2 of the lane.
template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v),
                                                                 CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ inline uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xf, 0xf, false);
}
// The maximum over the 64 lanes, in every lane: within each row of 16 by DPP (lane ^ 1, lane ^ 2,
// then rotations by 4 and 8), then the four rows' maxima read as scalars.  No LDS round trip.
// Every lane must be active.
__device__ inline float wave_max_f(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x128>(v));
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// max over the 8 aligned lanes of a quantization block (lane j = lane & 7); every lane of the
// group must be active.
__device__ inline float max8_lanes(float m, int j) {
    m = fmaxf(m, dpp_f<0xB1>(m));
    m = fmaxf(m, dpp_f<0x4E>(m));
    const float up = dpp_f<0x12C>(m), dn = dpp_f<0x124>(m);
    return fmaxf(m, (j & 4) ? dn : up);
}

// One 32-block of activation quantization (quant.rs:114-122), lanes j = 0..7 of 8 adjacent
// threads each holding v[0..3] = x[32b + 4j + 0..3].  d = amax/127, id = 1/d (0 if d == 0),
// q = clamp(round_half_away(x*id), +-127).  Writes q into the lane-major chunk layout.
// `store` = false computes without writing: callers run the lane exchanges with every lane
// active and keep the loads that feed them unconditional (a load used only under a branch is
// moved into it by the compiler, behind later loads).
__device__ inline void quant_block_lane(const float v[4], int j, uint32_t b, uint8_t *q, float *d,
                                        bool store = true) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = max8_lanes(amax, j);
    const float dd = amax / 127.0f;
    const float id = dd > 0.0f ? 1.0f / dd : 0.0f;
    uint32_t packed = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        float r = roundf(v[m] * id);
        if (r != r) r = 0.0f;
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        packed |= (uint32_t)(uint8_t)(int8_t)(int)r << (8 * m);
    }
    if (store) {
        *reinterpret_cast<uint32_t *>(q + (b / 4) * CHUNK_BYTES + j * 16 + (b % 4) * 4) = packed;
        if (j == 0) d[b] = dd;
    }
}

// Zero the padding blocks of a partial last chunk so padded lanes contribute 0.
__device__ inline void zero_pad(uint32_t nb, uint32_t nc, uint8_t *q, float *d, int tid, int nthr) {
    for (uint32_t b = nb + tid; b < nc * 4; b += nthr) {
        for (int j = 0; j < 8; ++j)
            *reinterpret_cast<uint32_t *>(q + (b / 4) * CHUNK_BYTES + j * 16 + (b % 4) * 4) = 0;
        d[b] = 0.0f;
    }
}

// Stage a quantized activation (nc chunks + scales) from global into LDS.
__device__ inline void stage_act(const uint8_t *gq, const float *gd, uint32_t nc, uint8_t *sq,
                                 float *sd, int tid, int nthr) {
    const int4 *src = reinterpret_cast<const int4 *>(gq);
    int4 *dst = reinterpret_cast<int4 *>(sq);
    for (uint32_t i = tid; i < nc * 8; i += nthr) dst[i] = src[i];
    for (uint32_t i = tid; i < nc * 4; i += nthr) sd[i] = gd[i];
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef long v2l __attribute__((ext_vector_type(2)));

// Storage vector of the four scales of one chunk: f32 (16 B) or f16 (8 B).
template <bool SCF32> struct ScaleVec { typedef v2u T; };
template <> struct ScaleVec<true> { typedef v4f T; };

__device__ inline void unpack_scales(v4f s, float o[4]) { o[0] = s.x; o[1] = s.y; o[2] = s.z; o[3] = s.w; }
__device__ inline void unpack_scales(v2u h, float o[4]) {
    o[0] = (float)__builtin_bit_cast(_Float16, (unsigned short)(h.x & 0xffffu));
    o[1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(h.x >> 16));
    o[2] = (float)__builtin_bit_cast(_Float16, (unsigned short)(h.y & 0xffffu));
    o[3] = (float)__builtin_bit_cast(_Float16, (unsigned short)(h.y >> 16));
}

// Row dot of the Q8 matvec, lane j of the 8 lanes owning the row.
//   ORDER_DECODE: qrow_dot_avx2 (quant.rs:44-67).  Lane j keeps accumulator lane j:
//     acc_j = fma(sw[b]*dx[b], (float)sum_{m<4} w[32b+4j+m]*x[32b+4j+m], acc_j) over b,
//     then ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) (the hsum of quant.rs:61-65) by xor 4/2/1.
//   ORDER_PREFILL: Q8Tensor::matmul (quant.rs:171-184).  isum over the whole block (exact),
//     acc += (sw[b]*dx[b]) * isum in block order, one accumulator.
// begin() issues the first NCT chunks' weight and scale loads (branch free, the index
// clamped into the row), so a kernel can start them before staging its activation; finish()
// consumes them and streams the rest of the row NCT chunks at a time.
template <int ORDER, bool SCF32, int NCT>
struct Q8Row {
    const uint8_t *w;
    const void *s;
    uint32_t nb, nc;
    int j;
    v4i wq[NCT];
    typename ScaleVec<SCF32>::T sq[NCT];

    // A row of exactly 8 full chunks (the single-batch case with NCT = 8) loads its scales once:
    // lane j takes chunk j's, and chunk u's reach the row's lanes by an LDS-free swizzle
    // (lane i reads lane (i & ~7) | u), which halves the row's load instructions.
    __device__ inline bool bcast() const { return NCT == 8 && nc == 8 && nb == 32; }
    __device__ inline void load(uint32_t c0) {
        const bool bc = bcast() && c0 == 0;
#pragma unroll
        for (int u = 0; u < NCT; ++u) {
            const uint32_t c = min(c0 + (uint32_t)u, nc - 1);
            wq[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(w + c * CHUNK_BYTES + j * 16));
            if (!bc)
                sq[u] = __builtin_nontemporal_load(reinterpret_cast<const typename ScaleVec<SCF32>::T *>(s) + c);
        }
        if (bc) sq[0] = __builtin_nontemporal_load(reinterpret_cast<const typename ScaleVec<SCF32>::T *>(s) + j);
    }
    template <int U>
    __device__ inline typename ScaleVec<SCF32>::T row_scales() const {   // chunk U's, from lane U of the row
        constexpr int pat = 0x18 | (U << 5);   // and_mask 0x18, or_mask U
        // (the elements go through scalars: a bit cast of a vector element expression reads
        // element 0 with this compiler)
        typename ScaleVec<SCF32>::T r;
        if constexpr (SCF32) {
            const float s0 = sq[0].x, s1 = sq[0].y, s2 = sq[0].z, s3 = sq[0].w;
            r.x = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, s0), pat));
            r.y = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, s1), pat));
            r.z = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, s2), pat));
            r.w = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, s3), pat));
        } else {
            const uint32_t h0 = sq[0].x, h1 = sq[0].y;
            r.x = (uint32_t)__builtin_amdgcn_ds_swizzle((int)h0, pat);
            r.y = (uint32_t)__builtin_amdgcn_ds_swizzle((int)h1, pat);
        }
        return r;
    }
    __device__ inline void begin(const uint8_t *w_, const void *s_, uint32_t nb_, uint32_t nc_, int j_) {
        w = w_;
        s = s_;
        nb = nb_;
        nc = nc_;
        j = j_;
        load(0);
    }
    // One chunk c (batch slot u) against the activation chunk x and its scales.
    __device__ inline void chunk(int u, uint32_t c, const v4i x, const v4f dxc, bool guard, float &acc) const {
        chunk_s(u, c, x, dxc, guard, acc, sq[u]);
    }
    __device__ inline void chunk_s(int u, uint32_t c, const v4i x, const v4f dxc, bool guard, float &acc,
                                   const typename ScaleVec<SCF32>::T scl) const {
        const int p[4] = {sdot4(wq[u].x, x.x), sdot4(wq[u].y, x.y), sdot4(wq[u].z, x.z), sdot4(wq[u].w, x.w)};
        float sv[4];
        unpack_scales(scl, sv);
        const float dv[4] = {dxc.x, dxc.y, dxc.z, dxc.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t b = c * 4 + t;
            const float d = sv[t] * dv[t];
            if (ORDER == ORDER_DECODE) {
                if (!guard || b < nb) acc = fmaf(d, (float)p[t], acc);
            } else {   // the block's integer sum over the 8 lanes (exact in any order)
                int is = p[t];
                is += (int)dpp_u<0xB1>((uint32_t)is);
                is += (int)dpp_u<0x4E>((uint32_t)is);
                {
                    const int dn = (int)dpp_u<0x124>((uint32_t)is), up = (int)dpp_u<0x12C>((uint32_t)is);
                    is += (j & 4) ? dn : up;
                }
                if (!guard || b < nb) acc = acc + d * (float)is;
            }
        }
    }
    // Every lane of the row's 8 must be active.
    __device__ inline float finish(const uint8_t *qx, const float *dx) {
        float acc = 0.0f;
        if (nc == (uint32_t)NCT && nb == 4 * (uint32_t)NCT) {
            // one batch and no padding blocks: straight-line code
            v4i xa[NCT];
            v4f xs[NCT];
#pragma unroll
            for (int u = 0; u < NCT; ++u) {
                xa[u] = *reinterpret_cast<const v4i *>(qx + u * CHUNK_BYTES + j * 16);
                xs[u] = *reinterpret_cast<const v4f *>(dx + u * 4);
            }
            if constexpr (NCT == 8) {
                if (bcast()) {
                    typename ScaleVec<SCF32>::T sc[8];
                    sc[0] = row_scales<0>();
                    sc[1] = row_scales<1>();
                    sc[2] = row_scales<2>();
                    sc[3] = row_scales<3>();
                    sc[4] = row_scales<4>();
                    sc[5] = row_scales<5>();
                    sc[6] = row_scales<6>();
                    sc[7] = row_scales<7>();
#pragma unroll
                    for (int u = 0; u < NCT; ++u) chunk_s(u, (uint32_t)u, xa[u], xs[u], false, acc, sc[u]);
                    goto reduce;
                }
            }
#pragma unroll
            for (int u = 0; u < NCT; ++u) chunk(u, (uint32_t)u, xa[u], xs[u], false, acc);
        } else {
            uint32_t c0 = 0;
            while (true) {
                // the batch's activation chunks and scales, read from LDS together (addresses
                // clamped into the row) before any of them is used
                v4i xa[NCT];
                v4f xs[NCT];
#pragma unroll
                for (int u = 0; u < NCT; ++u) {
                    const uint32_t c = min(c0 + (uint32_t)u, nc - 1);
                    xa[u] = *reinterpret_cast<const v4i *>(qx + c * CHUNK_BYTES + j * 16);
                    xs[u] = *reinterpret_cast<const v4f *>(dx + c * 4);
                }
#pragma unroll
                for (int u = 0; u < NCT; ++u)
                    if (c0 + u < nc) chunk(u, c0 + u, xa[u], xs[u], true, acc);
                c0 += NCT;
                if (c0 >= nc) break;
                load(c0);
            }
        }
    reduce:
        if (ORDER == ORDER_DECODE) {   // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) in lane 0 (quant.rs:61-65)
            {
                const float dn = dpp_f<0x124>(acc), up = dpp_f<0x12C>(acc);
                acc = acc + ((j & 4) ? dn : up);
            }
            acc = acc + dpp_f<0x4E>(acc);
            acc = acc + dpp_f<0xB1>(acc);
        }
        return acc;
    }
};

__device__ inline const uint8_t *row_qs(const Q8Mat &W, uint32_t r) {
    return W.qs + (size_t)r * W.nc * CHUNK_BYTES;
}
template <bool SCF32>
__device__ inline const void *row_sc(const Q8Mat &W, uint32_t r) {
    return reinterpret_cast<const uint8_t *>(W.sc) + (size_t)r * W.nc * 4 * (SCF32 ? 4 : 2);
}

// s + a[0] + a[1] + ... + a[n-1] in index order (binary32), by one lane over LDS `a`
// (16-byte aligned).  Batches of 32 values (eight 16-byte reads) alternate between two
// register sets; each batch's reads are issued before the previous batch's adds and the
// instruction order is pinned, so the reads stay ahead of the dependent adds.
__device__ inline float seq_sum_lds(const float *a, uint32_t n, float s) {
    constexpr uint32_t B = 32;
    const uint32_t nb = n / B;
    const v4f *a4 = reinterpret_cast<const v4f *>(a);
    if (nb) {
        v4f ra[B / 4], rb[B / 4];
        auto ld = [&](v4f(&r)[B / 4], uint32_t b) {
#pragma unroll
            for (uint32_t u = 0; u < B / 4; ++u) r[u] = a4[b * (B / 4) + u];
        };
        auto add = [&](const v4f(&r)[B / 4]) {
#pragma unroll
            for (uint32_t u = 0; u < B / 4; ++u) {
                s = s + r[u].x;
                s = s + r[u].y;
                s = s + r[u].z;
                s = s + r[u].w;
            }
        };
        ld(ra, 0);
        ld(rb, min(1u, nb - 1));
        uint32_t b = 0;
        for (; b + 2 <= nb; b += 2) {
            __builtin_amdgcn_sched_barrier(0);
            add(ra);
            __builtin_amdgcn_sched_barrier(0);
            ld(ra, min(b + 2, nb - 1));
            __builtin_amdgcn_sched_barrier(0);
            add(rb);
            __builtin_amdgcn_sched_barrier(0);
            ld(rb, min(b + 3, nb - 1));
        }
        if (b < nb) add(ra);
    }
    for (uint32_t i = nb * B; i < n; ++i) s = s + a[i];
    return s;
}

// ------------------------------------------------------------------ exact parallel sum
// The same sequential binary32 sum 0 + a[0] + ... + a[n-1] of non-negative terms (the
// reference's `ss += v * v` of rmsnorm, ops.rs:101-104, and `sum += *v` of softmax,
// ops.rs:119-122), formed by a few waves with identical result bits.
//
// Why it can be parallel.  While the running sum s stays in one binade [2^e, 2^(e+1)) (binade
// -126 also holds zero and the subnormals; the quantum is u = 2^(e-23) in both) it is an
// integer number of quanta, and each add rounds to the quantum grid, so what a stretch of adds
// contributes depends only on the terms and on the parity of s at its start (round half to
// even is the only place s enters).  A lane that holds EPT consecutive terms and knows their
// adds stay in binade e replays them from the anchors c = 2^e (even; 0 for binade -126) and
// c + u (odd): both chains stay in the binade, so each reproduces the true adds for a start of
// its parity.  If the two increments agree, the lane adds that many quanta whatever s is; they
// differ exactly when one of its adds is a tie.
//
// Certification.  Each add errs by at most 2^-24 of its result (results below 2^-125 are
// exact) and s never decreases, so with T_k = a[0] + ... + a[k-1] (real numbers)
// |s_k - T_k| <= k 2^-24 (T_k + |s_k - T_k|), i.e. <= 1.001 k 2^-24 T_k for k <= 2^14.  Lanes
// form T_k in binary32 from their partial sums, a wave scan and the previous waves' terms: a
// sum of non-negative terms D roundings deep errs by at most D 2^-24 relative, with
// D <= (NPW - 1) 3 EPT / 4 (the previous waves' terms at the lane's position) + 6 (the scan of
// those) + EPT + 6 (the lane's own terms and their scan) + 2.  A margin R covers that and the
// rounding of the bound products: 2^-16 while D <= 64 (relative error below 2^-18), else
// 2^-13 (D <= 512).  s_k then lies in [T~_k (1 - R - C k), T~_k (1 + R + C k)] with
// C = 1.01 2^-24.  A lane whose bracket from its first sum to its
// last lies in one binade is "clean"; two consecutive clean lanes always share their binade
// (the brackets at their common boundary both hold s).
//
// Schedule.  Every participant wave, without waiting for the others: lane l of wave p holds
// terms (64 p + l) EPT .. + EPT - 1 and sums the previous waves' terms at its own position
// (their wave total is the wave's offset); brackets classify the lanes; clean lanes with
// agreeing chains contribute their quanta to a wave scan, every other lane (binade crossings,
// ties) is an "event lane" whose terms stay real float adds; the wave records its event lanes
// (quanta prefix, position, the binade of the lane before) and totals in LDS.  After one
// meeting, lane j of wave 0 takes event lane j's terms and incr_j, the clean quanta between
// event lanes j - 1 and j as one exact float of the run's binade; the ordered adds incr_0, the
// terms of event lane 0, incr_1, ..., incr_M then run lane by lane, each lane receiving the
// sum so far from the one before.  Negative, NaN or infinite terms, a total that may overflow,
// n > NPW 64 EPT, more than EVCAP event lanes in a wave or more than 64 in all fall back to
// adding every term.
namespace xsum {
constexpr uint32_t EVCAP = 32;    // event lanes recorded per wave
struct Scratch {
    uint32_t sync;   // participant arrivals (zeroed by the caller before a workgroup barrier)
    uint32_t wbad[8], wm[8], wq[8];
    int32_t wtail[8], efin;
    uint32_t evip[8][EVCAP];   // quanta before the event lane (wave-local prefix, mod 2^32)
    uint32_t evk[8][EVCAP];    // lane | (binade of the lane before + 127) << 8 (0: the wave's first lane)
};
}   // namespace xsum

template <int CTRL, int RM>
__device__ inline uint32_t dpp_zero(uint32_t v) {   // lanes without a source (or masked rows) read 0
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, RM, 0xf, true);
}
// Pins a value computed by lane exchanges to where it is written, so that the compiler cannot
// move the exchange under a lane-dependent branch (source lanes outside it would read 0).
__device__ inline uint32_t pin_u(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ inline float pin_f(float v) {
    asm volatile("" : "+v"(v));
    return v;
}
// Inclusive scans over the 64 lanes: row_shr 1, 2, 4, 8 within rows of 16, then row_bcast 15
// (rows 1, 3) and row_bcast 31 (rows 2, 3).
__device__ inline uint32_t wave_scan_u(uint32_t v) {
    v += dpp_zero<0x111, 0xf>(v);
    v += dpp_zero<0x112, 0xf>(v);
    v += dpp_zero<0x114, 0xf>(v);
    v += dpp_zero<0x118, 0xf>(v);
    v += dpp_zero<0x142, 0xa>(v);
    v += dpp_zero<0x143, 0xc>(v);
    return pin_u(v);
}
template <int CTRL, int RM>
__device__ inline float dpp_zero_f(float v) {
    return __builtin_bit_cast(float, dpp_zero<CTRL, RM>(__builtin_bit_cast(uint32_t, v)));
}
__device__ inline float wave_incl_scan_f(float v) {
    v += dpp_zero_f<0x111, 0xf>(v);
    v += dpp_zero_f<0x112, 0xf>(v);
    v += dpp_zero_f<0x114, 0xf>(v);
    v += dpp_zero_f<0x118, 0xf>(v);
    v += dpp_zero_f<0x142, 0xa>(v);
    v += dpp_zero_f<0x143, 0xc>(v);
    return pin_f(v);
}
// exclusive scan: wave_shr 1 (lane 0 reads 0), then the inclusive scan
__device__ inline float wave_excl_scan_f(float v) {
    return wave_incl_scan_f(dpp_zero_f<0x138, 0xf>(v));
}
// binade exponent of x >= 0 (x < 2^-126: -126)
__device__ inline int binade_of(float x) {
    return x >= 0x1p-126f ? (int)((__builtin_bit_cast(uint32_t, x) >> 23) & 0xff) - 127 : -126;
}
__device__ inline float rlane_f(float v, uint32_t l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)l));
}

// Meeting point of the NPW participant waves only (the other waves of the workgroup are not
// waited for): arrival count in LDS, phase ph = 1, 2, ...
template <int NPW>
__device__ inline void part_sync(xsum::Scratch &L, uint32_t ph) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(&L.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(&L.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < NPW * ph)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// a: LDS, 16-byte aligned, readable up to a multiple of 4 terms past n.  The waves with
// p = 0 .. NPW - 1 call (p uniform per wave; p = 0 is the wave that receives the result); they
// meet once among themselves, so the other waves of the workgroup keep working.  L.sync must be
// 0 on entry (zeroed before a workgroup barrier).
template <int NPW, int EPT>
__device__ __forceinline__ float block_seq_sum(const float *a, uint32_t n, xsum::Scratch &L, int p_, int lane) {
    static_assert(NPW >= 1 && NPW <= 8 && EPT % 4 == 0 && EPT <= 32 && NPW * 64 * EPT <= (1 << 14),
                  "wave tables, offsets depth, terms within the certified count");
    constexpr int D = (NPW - 1) * 3 * EPT / 4 + EPT + 14;   // rounding depth of the lanes' T~
    static_assert(D <= 512, "margin");
    constexpr float C = 1.01f * 0x1p-24f, R = D <= 64 ? 0x1p-16f : 0x1p-13f;
    constexpr uint32_t WT = 64 * EPT;   // terms per wave
    const int p = __builtin_amdgcn_readfirstlane(p_);
    const uint32_t k0 = (uint32_t)(64 * p + lane) * EPT;
    const bool fits = n <= WT * NPW;                      // (uniform)
    const bool act = fits && WT * (uint32_t)p < n;        // (uniform per wave)
    const v4f *a4 = reinterpret_cast<const v4f *>(a);
    if (act) {
        float v[EPT];
#pragma unroll
        for (int u = 0; u < EPT / 4; ++u) {
            v4f r = {0.0f, 0.0f, 0.0f, 0.0f};
            if (k0 + 4 * u < n) r = a4[k0 / 4 + u];
            v[4 * u] = r.x;
            v[4 * u + 1] = r.y;
            v[4 * u + 2] = r.z;
            v[4 * u + 3] = r.w;
        }
        uint32_t mx = 0;   // largest bit pattern: above 0x7f7fffff is negative, -0, inf or NaN
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            v[i] = k0 + i < n ? v[i] : 0.0f;
            mx = max(mx, __builtin_bit_cast(uint32_t, v[i]));
            t = t + v[i];
        }
        float x = 0.0f;   // the previous waves' terms at this lane's position (all below n)
#pragma unroll
        for (int w = 0; w < NPW - 1; ++w)
            if (w < p) {
#pragma unroll
                for (int u = 0; u < EPT / 4; ++u) {
                    const v4f r = a4[(uint32_t)(64 * w + lane) * (EPT / 4) + u];
                    x = ((x + r.x) + (r.y + r.z)) + r.w;
                }
            }
        const float before = p > 0 ? rlane_f(wave_incl_scan_f(x), 63) : 0.0f;
        const float off = before + wave_excl_scan_f(t);
        const float lo = off * (1.0f - R - C * (float)k0), hi = (off + t) * (1.0f + R + C * (float)(k0 + EPT));
        const bool bad = mx > 0x7f7fffffu || !(hi < 0x1p126f);
        const int el = binade_of(lo), eh = binade_of(hi);
        const bool in = k0 < n;
        // both parity chains from the anchors of binade el (meaningful for clean lanes)
        const float cA = el == -126 ? 0.0f : __builtin_bit_cast(float, (uint32_t)(el + 127) << 23);
        const float cB = cA + ldexpf(1.0f, el - 23);
        float A = cA, B = cB;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            A = A + v[i];
            B = B + v[i];
        }
        const uint32_t qA = (uint32_t)ldexpf(A - cA, 23 - el), qB = (uint32_t)ldexpf(B - cB, 23 - el);
        const bool ev = in && (el != eh || qA != qB);
        const uint32_t q = in && !ev ? qA : 0u;
        const uint32_t qi = wave_scan_u(q);
        const uint64_t em = __builtin_amdgcn_ballot_w64(ev);
        const bool anyb = __builtin_amdgcn_ballot_w64(bad) != 0;
        const uint32_t idx = __builtin_amdgcn_mbcnt_hi((uint32_t)(em >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)em, 0u));
        const uint32_t ep = pin_u(dpp_zero<0x138, 0xf>((uint32_t)(el + 127)));   // the lane before (lane 0: 0)
        const uint32_t nev = (uint32_t)__builtin_popcountll(em);
        if (ev && idx < xsum::EVCAP) {
            L.evip[p][idx] = qi - q;
            L.evk[p][idx] = (uint32_t)lane | ep << 8;
        }
        if (lane == 63) {
            L.wq[p] = qi;
            L.wtail[p] = el;
        }
        if (lane == 0) {
            L.wm[p] = min(nev, xsum::EVCAP);
            L.wbad[p] = anyb || nev > xsum::EVCAP;
        }
        if (in && k0 + EPT >= n) L.efin = el;   // the last lane: binade of the final run
    }
    part_sync<NPW>(L, 1);
    if (p != 0) return 0.0f;
    // wave 0: the event lanes' offsets in the list, the quanta before each wave
    uint32_t mb[NPW], qb[NPW], M = 0, Q = 0, anybad = 0;
#pragma unroll
    for (int w = 0; w < NPW; ++w) {
        const bool has = WT * (uint32_t)w < n;
        mb[w] = M;
        qb[w] = Q;
        M += has ? L.wm[w] : 0u;
        Q += has ? L.wq[w] : 0u;
        anybad |= has ? L.wbad[w] : 0u;
    }
    if (!fits || anybad || M > 64) return rlane_f(lane == 0 ? seq_sum_lds(a, n, 0.0f) : 0.0f, 0);
    // lane j < M: event lane j's terms, the quanta before it (mod 2^32) and its run's binade
    uint32_t ip = 0;
    int e = -126;
    float tv[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) tv[i] = 0.0f;
    if ((uint32_t)lane < M) {
        uint32_t w = 0, mw = 0, qw = 0;
#pragma unroll
        for (int q = 1; q < NPW; ++q)
            if (mb[q] <= (uint32_t)lane && WT * (uint32_t)q < n) {
                w = q;
                mw = mb[q];
                qw = qb[q];
            }
        const uint32_t ix = (uint32_t)lane - mw;
        ip = L.evip[w][ix] + qw;
        const uint32_t kw = L.evk[w][ix];
        const int ep = (int)(kw >> 8) - 127;
        e = ep == -127 ? (w > 0 ? L.wtail[w - 1] : -126) : ep;
        const uint32_t kj = (64 * w + (kw & 63)) * EPT;
#pragma unroll
        for (int u = 0; u < EPT / 4; ++u) {
            const v4f r = a4[kj / 4 + u];
            tv[4 * u] = kj + 4 * u < n ? r.x : 0.0f;
            tv[4 * u + 1] = kj + 4 * u + 1 < n ? r.y : 0.0f;
            tv[4 * u + 2] = kj + 4 * u + 2 < n ? r.z : 0.0f;
            tv[4 * u + 3] = kj + 4 * u + 3 < n ? r.w : 0.0f;
        }
    }
    const uint32_t ipp = pin_u(dpp_zero<0x138, 0xf>(ip));   // event lane j - 1's (lane 0: 0)
    const uint32_t dI = ip - ipp;   // < 2^24 quanta: the run stays in its binade
    const float inc = (uint32_t)lane < M && dI ? ldexpf((float)dI, min(max(e, -126), 127) - 23) : 0.0f;
    const uint32_t dF = Q - (M ? (uint32_t)__builtin_amdgcn_readlane((int)ip, (int)(M - 1)) : 0u);
    const float incF = dF ? ldexpf((float)dF, min(max(L.efin, -126), 127) - 23) : 0.0f;   // the final run
    // the ordered adds: step j runs in lane j, which receives the sum so far from lane j - 1
    float x = 0.0f;
    for (uint32_t j = 0; j < M; ++j) {
        x = dpp_zero_f<0x138, 0xf>(x) + inc;
#pragma unroll
        for (int i = 0; i < EPT; ++i) x = x + tv[i];
    }
    return (M ? rlane_f(x, M - 1) : 0.0f) + incF;
}


// ------------------------------------------------------------------ QK-norm + RoPE
// Per-lane constants of norm_rope_head for one step, fetched at kernel start: the q and k
// norm gains of elements lane + 64k and the RoPE cos/sin row at pos for pairs lane + 64k.
template <int HD>
struct HeadConst {
    static constexpr int NW = (HD + 63) / 64, NR = (HD / 2 + 63) / 64;
    float qn[NW], kn[NW], c[NR], s[NR];
    __device__ inline void load(const float *__restrict__ qnw, const float *__restrict__ knw,
                                const float *__restrict__ cs, const float *__restrict__ sn, uint32_t pos,
                                int lane) {
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            const uint32_t i = min((uint32_t)(lane + 64 * k), (uint32_t)HD - 1);
            qn[k] = qnw[i];
            kn[k] = knw[i];
        }
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const uint32_t i = min((uint32_t)(lane + 64 * k), (uint32_t)HD / 2 - 1);
            c[k] = cs[(size_t)pos * (HD / 2) + i];
            s[k] = sn[(size_t)pos * (HD / 2) + i];
        }
    }
};

// norm_head (model.rs:753-763) then Rope::apply (ops.rs:155-166) of one head vector held in
// LDS `u` (HD floats); result in `o`.  The sum of squares is sequential (as the reference);
// called by one wave, lane 0 doing the sum.
template <int HD>
__device__ inline void norm_rope_head(const float *u, float *o, const HeadConst<HD> &hc, bool is_q, float eps,
                                      float *tmp, int lane) {
    float scale = 0.0f;
    if (lane == 0) {   // ss += x * x in index order; the reads are issued together first
        v4f r[HD / 4];
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) r[i] = reinterpret_cast<const v4f *>(u)[i];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) {
            ss = ss + r[i].x * r[i].x;
            ss = ss + r[i].y * r[i].y;
            ss = ss + r[i].z * r[i].z;
            ss = ss + r[i].w * r[i].w;
        }
        scale = 1.0f / sqrtf(ss / (float)HD + eps);
    }
    scale = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, scale), 0));
#pragma unroll
    for (int k = 0; k < HeadConst<HD>::NW; ++k) {
        const uint32_t i = lane + 64 * k;
        if (i < HD) tmp[i] = u[i] * scale * (is_q ? hc.qn[k] : hc.kn[k]);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    constexpr uint32_t half = HD / 2;
#pragma unroll
    for (int k = 0; k < HeadConst<HD>::NR; ++k) {
        const uint32_t i = lane + 64 * k;
        if (i < half) {
            const float c = hc.c[k], s = hc.s[k];
            const float x1 = tmp[i], x2 = tmp[half + i];
            o[i] = x1 * c - x2 * s;
            o[half + i] = x2 * c + x1 * s;
        }
    }
}


// dot_wide_serial(a, b, 64) by the lanes of one wave: lane 8 r + l (and its mirror 32 + 8 r + l)
// holds accumulator (r, l), fmaf(a[32 + e], b[32 + e], fmaf(a[e], b[e], 0)); the butterflies
// then form (acc0 + acc1) + (acc2 + acc3) and ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)),
// the same additions as the serial form (each IEEE addition is commutative).  Every lane
// returns the sum.
// (a0, b0, a1, b1: lane e's elements e % 32 and 32 + e % 32 of a and b)
__device__ inline float dot64_lanes(float a0, float b0, float a1, float b1) {
    float acc = fmaf(a0, b0, 0.0f);
    acc = fmaf(a1, b1, acc);
    acc = acc + shfl_xor(acc, 8);
    acc = acc + shfl_xor(acc, 16);
    acc = acc + shfl_xor(acc, 4);
    acc = acc + shfl_xor(acc, 2);
    acc = acc + shfl_xor(acc, 1);
    return acc;
}

// ops::dot (ops.rs:7-36) of two hd-vectors in the reference order: four 8-lane FMA
// accumulators over 32-wide steps, 8-wide tail on accumulator 0, then
// ((a0+a1)+(a2+a3)) reduced as ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)), then a scalar tail.
__device__ inline float dot_wide_serial(const float *a, const float *b, uint32_t n) {
    float acc[4][8];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[r][l] = 0.0f;
    uint32_t i = 0;
    const uint32_t main = n - n % 32;
    for (; i < main; i += 32)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[r][l] = fmaf(a[i + 8 * r + l], b[i + 8 * r + l], acc[r][l]);
    for (; i + 8 <= n; i += 8)
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[0][l] = fmaf(a[i + l], b[i + l], acc[0][l]);
    float v[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    float s = ((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7]));
    for (; i < n; ++i) s = s + a[i] * b[i];
    return s;
}

}  // namespace hg
