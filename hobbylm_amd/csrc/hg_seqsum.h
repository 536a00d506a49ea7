// hg_seqsum.h -- the sequential binary32 sum ((0 + a_0) + a_1) + ... + a_{n-1} of
// non-negative terms (the reference's `ss += v * v` of rmsnorm, ops.rs:101-104, and `sum += *v`
// of softmax, ops.rs:119-122), computed by a whole workgroup with the same result bits.
//
// Why it can be parallel.  Every add rounds to nearest-even at the quantum u = 2^(e-23) of the
// binade [2^e, 2^(e+1)) its result lies in (binade -126 also holds the subnormals, same u).
// While the running sum s stays in one binade it is an integer S in units of u, and adding a
// term contributes the integer inc = round(a / u) -- independent of S -- unless a / u has a
// fraction of exactly 1/2 (a tie, resolved to even by S's parity).  So between two "events"
// (an add whose result leaves the binade, or a tie) the partial sums are S plus prefix sums of
// inc, and each event is one real float add.  With non-negative terms s never decreases, so it
// crosses each binade boundary at most once.
//
// Schedule (NT threads):
//   A. a tree total T of the terms bounds the sequential sum: s_n <= hi = T (1 + 2^-9) for
//      n <= 4096, so after it reaches e_lo = binade(hi) - KB + 1 the sum only visits the KB
//      candidate binades e_lo .. binade(hi);
//   B. every thread rounds its terms for each candidate binade, and a block scan writes the
//      inclusive prefix P_k[i] of inc (mod 2^32) and the tie bits of every term to LDS;
//   C. wave 0 walks: serial float adds while s < 2^e_lo (the head), then event to event: a
//      ballot over 64-term block ends finds the block holding the next event, a ballot over
//      that block's 64 terms finds the event, and one float add resolves it.
// NaN/inf terms, a bound above 1e38, or n > 4096 fall back to one lane adding every term.
#pragma once
#include <stdint.h>

namespace hg {

typedef float sq_v4f __attribute__((ext_vector_type(4)));

// s + a[0] + a[1] + ... + a[n-1] in index order (binary32), by one lane over LDS `a`
// (16-byte aligned).  Batches of 32 values (eight 16-byte reads) alternate between two
// register sets; each batch's reads are issued before the previous batch's adds and the
// instruction order is pinned, so the reads stay ahead of the dependent adds.
__device__ inline float seq_sum_lds(const float *a, uint32_t n, float s) {
    constexpr uint32_t B = 32;
    const uint32_t nb = n / B;
    const sq_v4f *a4 = reinterpret_cast<const sq_v4f *>(a);
    if (nb) {
        sq_v4f ra[B / 4], rb[B / 4];
        auto ld = [&](sq_v4f(&r)[B / 4], uint32_t b) {
#pragma unroll
            for (uint32_t u = 0; u < B / 4; ++u) r[u] = a4[b * (B / 4) + u];
        };
        auto add = [&](const sq_v4f(&r)[B / 4]) {
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

constexpr uint32_t SEQSUM_MAXN = 4096;   // 64 blocks of 64 terms: one block per lane

__device__ inline int seqsum_binade(float s) {
    const int eb = (int)(__builtin_bit_cast(uint32_t, s) >> 23) - 127;
    return eb < -126 ? -126 : eb;
}

// LDS words the caller provides for block_seq_sum<NT, KB, ...> over n terms (8-byte aligned).
__host__ __device__ constexpr uint32_t seqsum_lds_words(uint32_t n, int KB, int NT) {
    return (uint32_t)KB * ((n + 63) / 64 * 64)   // P[k][i]: inclusive prefix of the increments
           + (uint32_t)KB * 64 * 2               // TM[k][b]: tie positions of block b (64 bits)
           + (uint32_t)KB * 64                   // BE[k][b]: P[k][64 b + 63]
           + (uint32_t)(NT / 64) * KB            // per-wave increment totals
           + 2;                                  // result
}

template <int CTRL, int ROW_MASK>
__device__ inline uint32_t seqsum_dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, true);
}
// Inclusive scan over the 64 lanes of a wave (unsigned, wrapping).
__device__ inline uint32_t seqsum_wave_scan(uint32_t v) {
    v += seqsum_dpp<0x111, 0xf>(v);   // row_shr:1
    v += seqsum_dpp<0x112, 0xf>(v);   // row_shr:2
    v += seqsum_dpp<0x114, 0xf>(v);   // row_shr:4
    v += seqsum_dpp<0x118, 0xf>(v);   // row_shr:8
    v += seqsum_dpp<0x142, 0xa>(v);   // row_bcast:15 into rows 1, 3
    v += seqsum_dpp<0x143, 0xc>(v);   // row_bcast:31 into rows 2, 3
    return v;
}
// A fixed-order tree total of a wave's values (deterministic; used only for the bound).
__device__ inline float seqsum_wave_total(float v) {
#define SQ_FDPP(C, M) __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), C, M, 0xf, true))
    v += SQ_FDPP(0x111, 0xf);
    v += SQ_FDPP(0x112, 0xf);
    v += SQ_FDPP(0x114, 0xf);
    v += SQ_FDPP(0x118, 0xf);
    v += SQ_FDPP(0x142, 0xa);
    v += SQ_FDPP(0x143, 0xc);
#undef SQ_FDPP
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ inline uint32_t seqsum_rl(uint32_t v, uint32_t lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)lane);
}
__device__ inline float seqsum_rlf(float v, uint32_t lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)lane));
}

// One lane: s += a[i] for i = *i0 .. while s < lo and i < lim, in batches of 32 (the check
// is made per batch; adding past the point where s reaches lo is harmless).
__device__ inline float seqsum_head(const float *a, uint32_t lim, float s, float lo, uint32_t *i0) {
    uint32_t i = *i0;
    while (i < lim && s < lo) {
        if (i % 4 == 0 && i + 32 <= lim) {
            const sq_v4f *a4 = reinterpret_cast<const sq_v4f *>(a + i);
            sq_v4f r[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) r[u] = a4[u];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                s = s + r[u].x;
                s = s + r[u].y;
                s = s + r[u].z;
                s = s + r[u].w;
            }
            i += 32;
        } else {
            s = s + a[i];
            ++i;
        }
    }
    *i0 = i;
    return s;
}

// All NT threads call (NT = 128 .. 1024, a multiple of 64); `a` holds the n terms in LDS
// (16-byte aligned), `w` the scratch of seqsum_lds_words(n, KB, NT) words (8-byte aligned).
// Returns the sum in every thread.  Contains barriers.
// Wave 0 runs the head and the walk; waves 1.. build the tables, thread t of them owning the c
// consecutive terms [t c, t c + c) (c odd, so the prefix writes of a wave hit distinct banks).
template <int NT, int KB, int CMAX>
__device__ float block_seq_sum(const float *a, uint32_t n, uint32_t *w, int tid) {
    constexpr int NW = NT / 64, NWK = NW - 1;
    static_assert(NT % 64 == 0 && NW >= 2 && NW <= 16, "2..16 waves");
    static_assert(KB >= 2 && KB <= 8, "2..8 candidate binades");
    constexpr uint32_t HEAD1 = 512;   // head terms before the first barrier
    const uint32_t nblk = (n + 63) / 64, nbp = nblk * 64;
    uint32_t *P = w;                                                      // [KB][nbp]
    uint32_t *TM = w + (size_t)KB * nbp;                                  // [KB][64] x 2 words
    uint32_t *BE = TM + KB * 128;                                         // [KB][64]
    uint32_t *wrun = BE + KB * 64;                                        // [NW][KB]
    float *res = reinterpret_cast<float *>(wrun + NW * KB);
    const int lane = tid & 63, wave = tid >> 6;

    // ---- A (every wave for itself): a fixed-order total bounds the sequential sum
    float part = 0.0f;
    {
        const sq_v4f *a4 = reinterpret_cast<const sq_v4f *>(a);
        const uint32_t n4 = n / 4;
        for (uint32_t q = (uint32_t)lane; q < n4; q += 64) {
            const sq_v4f x = a4[q];
            part += (x.x + x.y) + (x.z + x.w);
        }
        for (uint32_t q = n4 * 4 + (uint32_t)lane; q < n; q += 64) part += a[q];
    }
    const float tot = seqsum_wave_total(part);
    const float hi = tot * (1.0f + 0x1p-9f);
    const bool serial = !(hi <= 1.0e38f) || n > SEQSUM_MAXN;
    const int e_max = seqsum_binade(hi);
    const int e_lo = e_max - KB + 1 < -126 ? -126 : e_max - KB + 1;
    const float lo = e_lo > -126 ? ldexpf(1.0f, e_lo) : 0.0f;   // -126: every sum is in the window
    uint32_t c = (nbp + NWK * 64 - 1) / (NWK * 64);
    c |= 1u;
    const bool fits = c <= (uint32_t)CMAX;

    float s = 0.0f;   // wave 0: the running sum, terms [0, i) added
    uint32_t i = 0;
    uint32_t run[KB], incl[KB];
    float v[CMAX];
    const uint32_t wt = (uint32_t)(tid - 64), i0 = wt * c;
    if (wave == 0) {
        if (lane == 0) {
            if (serial || !fits) s = seq_sum_lds(a, n, 0.0f), i = n;
            else s = seqsum_head(a, min(n, HEAD1), 0.0f, lo, &i);
        }
    } else if (!serial && fits) {
        // ---- B1: increments of this thread's terms per candidate binade, wave scans
        for (uint32_t q = wt; q < (uint32_t)KB * 128; q += NWK * 64) TM[q] = 0;
#pragma unroll
        for (int m = 0; m < CMAX; ++m) {
            const uint32_t idx = i0 + m;
            v[m] = ((uint32_t)m < c && idx < n) ? a[idx] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            uint32_t r = 0;
#pragma unroll
            for (int m = 0; m < CMAX; ++m) {
                const float y = fminf(ldexpf(v[m], 23 - (e_lo + k)), 16777216.0f);
                r += (uint32_t)y + (y - floorf(y) > 0.5f ? 1u : 0u);
            }
            run[k] = r;
            incl[k] = seqsum_wave_scan(r);
            if (lane == 63) wrun[wave * KB + k] = incl[k];
        }
    }
    __syncthreads();
    if (wave == 0) {
        if (lane == 0 && i < n && s < lo) s = seqsum_head(a, n, s, lo, &i);
    } else if (!serial && fits) {
        // ---- B2: prefixes of every term, block ends and tie masks
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            uint32_t off = incl[k] - run[k];
            for (int q = 1; q < wave; ++q) off += wrun[q * KB + k];
#pragma unroll
            for (int m = 0; m < CMAX; ++m) {
                const uint32_t idx = i0 + m;
                const float y = fminf(ldexpf(v[m], 23 - (e_lo + k)), 16777216.0f);
                const float fr = y - floorf(y);
                off += (uint32_t)y + (fr > 0.5f ? 1u : 0u);
                if ((uint32_t)m < c && idx < nbp) {
                    P[k * nbp + idx] = off;
                    if (idx % 64 == 63) BE[k * 64 + idx / 64] = off;
                    if (fr == 0.5f && idx < n)
                        atomicOr(&TM[(k * 64 + idx / 64) * 2 + (idx % 64) / 32], 1u << (idx % 32));
                }
            }
        }
    }
    __syncthreads();

    // ---- C: the walk, wave 0 (uniform control; the state lives in lane 0 until here)
    if (wave == 0) {
        s = seqsum_rlf(s, 0);
        i = seqsum_rl(i, 0);
        if (i < n) {
            int k = seqsum_binade(s) - e_lo;
            uint32_t base = (i > 0 && k >= 0 && k < KB) ? P[k * nbp + i - 1] : 0u;
            uint32_t guard = 0;
            while (i < n) {
                if (k < 0 || k >= KB || ++guard > n + 64) {   // outside the window: not expected
                    if (lane == 0)
                        for (; i < n; ++i) s = s + a[i];
                    s = seqsum_rlf(s, 0);
                    break;
                }
                const int ek = e_lo + k;
                const uint32_t S = (uint32_t)ldexpf(s, 23 - ek);
                const uint32_t lim = 16777216u - S;
                const uint32_t bi = i / 64;
                // level 1: the first block (from i's) whose end crosses, or with a tie at >= i
                const uint32_t bl = min((uint32_t)lane, nblk - 1);
                const uint32_t be = BE[k * 64 + bl];
                const uint64_t tm = *reinterpret_cast<const uint64_t *>(TM + (k * 64 + bl) * 2);
                const uint64_t keep = (uint32_t)lane > bi ? ~0ull : ((uint32_t)lane == bi ? (~0ull << (i % 64)) : 0ull);
                const uint64_t b1 = __ballot((uint32_t)lane >= bi && (uint32_t)lane < nblk &&
                                             (be - base >= lim || (tm & keep) != 0));
                if (!b1) {   // no event left: the rest is one integer sum
                    const uint32_t fin = seqsum_rl(be, nblk - 1) - base;
                    s = ldexpf((float)(S + fin), ek - 23);
                    break;
                }
                const uint32_t bs = (uint32_t)__builtin_ctzll(b1);
                // level 2: the event within block bs
                const uint32_t idx = bs * 64 + (uint32_t)lane;
                const uint32_t pk = P[k * nbp + idx];
                const uint32_t pk1 = k + 1 < KB ? P[(k + 1) * nbp + idx] : 0u;
                const float x = a[min(idx, n - 1)];
                const uint64_t tmb = ((uint64_t)seqsum_rl((uint32_t)(tm >> 32), bs) << 32) | seqsum_rl((uint32_t)tm, bs);
                const uint64_t b2 = __ballot(idx >= i && idx < n && (pk - base >= lim || ((tmb >> lane) & 1u)));
                if (!b2) {   // (a flagged block always holds its event; kept as a guard)
                    k = -1;
                    continue;
                }
                const uint32_t jl = (uint32_t)__builtin_ctzll(b2), j = bs * 64 + jl;
                uint32_t pre = 0;   // increments of the terms i .. j-1
                if (j > i) pre = (jl ? seqsum_rl(pk, jl - 1) : seqsum_rl(be, bs - 1)) - base;
                s = ldexpf((float)(S + pre), ek - 23) + seqsum_rlf(x, jl);
                i = j + 1;
                const int k2 = seqsum_binade(s) - e_lo;
                if (k2 == k) base = seqsum_rl(pk, jl);
                else if (k2 == k + 1) base = seqsum_rl(pk1, jl);
                else if (k2 >= 0 && k2 < KB) base = P[k2 * nbp + j];
                k = k2;
            }
        }
        if (lane == 0) *res = s;
    }
    __syncthreads();
    return *res;
}

}  // namespace hg
