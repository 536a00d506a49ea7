// hg_sample.hip -- sample::sample (sample.rs:66-112) of a generation step on the device, bit for
// bit: the masked and penalized logits (lib.rs:132-141) divided by the temperature, their
// maximum, e_i = exp(l_i / temp - m) with the reference expf, the sum of the e_i in id order,
// p_i = e_i / sum; with 0 < top_p < 1 the ids sorted by descending p (equal p: ascending id;
// rocPRIM's radix sort is stable), the cumulative sum in that order up to the first entry that
// reaches top_p, the kept p divided by their sum; then one uniform draw r of the xorshift64*
// RNG and the first entry whose cumulative probability exceeds r (else the last kept).
//
// Every cumulative sum is the reference's sequential binary32 sum.  Sums run over segments of
// up to SEG - 1 terms, each formed exactly in parallel (block_seq_sum) with the running sum of
// the earlier segments as its first term (0 + s = s, so the chain of segment sums is the one
// sequential sum); the segment where a running sum crosses a threshold is then replayed by one
// lane from its exact start.
#include <math.h>

#include <mutex>
#include <vector>

#include <rocprim/device/device_radix_sort.hpp>

#include "hg_common.h"
#include "hg_device.h"
#include "hg_expf.h"
#include "hg_sample.h"

namespace hg {
namespace {

constexpr uint32_t SEG = 8 * 64 * 32;   // terms of one exact parallel sum (8 waves x 64 lanes x 32)
constexpr uint32_t NT = 512;

struct SegLds {
    __align__(16) float a[SEG + 8];   // a[0] = the running sum before the segment, then its terms
    xsum::Scratch xs;
    float red[NT / 64];
    uint32_t redi[NT / 64];
    float val;
    uint32_t idx;
};

// The ordered sum a[0] + ... + a[n-1] of the segment in LDS (the 8 waves of the workgroup).
__device__ float seg_sum(SegLds &L, uint32_t n, int wave, int lane) {
    if (threadIdx.x < 4) L.a[n + threadIdx.x] = 0.0f;   // readable up to a multiple of 4 past n
    if (threadIdx.x == 0) L.xs.sync = 0;
    __syncthreads();
    const float r = block_seq_sum<8, 32>(L.a, n, L.xs, wave, lane);
    if (threadIdx.x == 0) L.val = r;
    __syncthreads();
    return L.val;
}

// One lane: from s = a[0], s = s + a[k] for k = 1, 2, ... until s >= thr (strict: s > thr);
// returns that k (n if none) and the sum there in *cum.  The sums never decrease, so a block of
// 32 adds whose end fails the test holds no crossing.
__device__ uint32_t scan_first(const float *a, uint32_t n, float thr, bool strict, float *cum) {
    float s = a[0];
    uint32_t k = 1;
    for (; k + 32 <= n; k += 32) {
        float t = s;
#pragma unroll
        for (uint32_t u = 0; u < 32; ++u) t = t + a[k + u];
        if (strict ? t > thr : t >= thr) break;
        s = t;
    }
    for (; k < n; ++k) {
        s = s + a[k];
        if (strict ? s > thr : s >= thr) {
            *cum = s;
            return k;
        }
    }
    *cum = s;
    return n;
}

__device__ inline float penalized(const float *logits, const uint32_t *counts, uint32_t i, uint32_t valid, float rp) {
    float l = i < valid ? logits[i] : -__builtin_huge_valf();
    if (counts) {
        const uint32_t c = counts[i];
        for (uint32_t k = 0; k < c; ++k) l = l > 0.0f ? l / rp : l * rp;
    }
    return l;
}

// sample::argmax (sample.rs:53-63) of the masked, penalized logits: the first maximum, 0 when
// nothing exceeds -inf.  One workgroup.
__global__ __launch_bounds__(NT) void k_s_argmax(const float *__restrict__ logits, uint32_t V, uint32_t valid,
                                                 uint32_t *counts, float rp, uint32_t *pick, StepParams *p) {
    __shared__ float bv[NT / 64];
    __shared__ uint32_t bi[NT / 64];
    const uint32_t tid = threadIdx.x;
    float mv = -__builtin_huge_valf();
    uint32_t mi = 0xffffffffu;
    for (uint32_t i = tid; i < V; i += NT) {
        const float v = penalized(logits, counts, i, valid, rp);
        if (v > mv) {
            mv = v;
            mi = i;
        }
    }
    for (int m = 1; m < 64; m <<= 1) {
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
        for (uint32_t w = 1; w < NT / 64; ++w)
            if (bv[w] > mv || (bv[w] == mv && bi[w] < mi)) {
                mv = bv[w];
                mi = bi[w];
            }
        const uint32_t next = mi == 0xffffffffu ? 0u : mi;
        *pick = next;
        if (p) p->token = next;
        if (counts) counts[next] += 1;
    }
}

// p_i = exp(l_i / temp - m) / sum (sample.rs:71-83) of the masked, penalized logits, with the
// sort keys (the bits of p_i: non-negative floats order as their bit patterns) and ids.  One
// workgroup.
__global__ __launch_bounds__(NT) void k_s_probs(const float *__restrict__ logits, uint32_t V, uint32_t valid,
                                                const uint32_t *__restrict__ counts, float rp, float temp, float *p,
                                                uint32_t *keys, uint32_t *ids) {
    __shared__ SegLds L;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const WaveExpTab tab = WaveExpTab::load(lane);
    float mx = -__builtin_huge_valf();
    for (uint32_t i = tid; i < V; i += NT) {
        const float v = penalized(logits, counts, i, valid, rp) / temp;
        p[i] = v;
        mx = fmaxf(mx, v);
    }
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, shfl_xor(mx, m));
    if (lane == 0) L.red[wave] = mx;
    __syncthreads();
    float m = L.red[0];
    for (uint32_t w = 1; w < NT / 64; ++w) m = fmaxf(m, L.red[w]);
    for (uint32_t b = 0; b < V; b += NT) {   // (uniform: every lane calls the exp)
        const uint32_t i = b + tid;
        const float v = i < V ? p[i] : -__builtin_huge_valf();
        const float e = hg_expf_l(v - m, tab);
        if (i < V) p[i] = e;
    }
    __syncthreads();
    float sum = 0.0f;
    for (uint32_t s0 = 0; s0 < V; s0 += SEG - 1) {   // sum += e_i in id order, a segment at a time
        const uint32_t cnt = min(SEG - 1, V - s0);
        if (tid == 0) L.a[0] = sum;
        for (uint32_t k = tid; k < cnt; k += NT) L.a[1 + k] = p[s0 + k];
        sum = seg_sum(L, cnt + 1, wave, lane);
    }
    for (uint32_t i = tid; i < V; i += NT) {
        const float q = p[i] / sum;
        p[i] = q;
        keys[i] = __builtin_bit_cast(uint32_t, q);
        ids[i] = i;
    }
}

// The draw (sample.rs:84-111) over q[0 .. V) in scan order (ids[k]: the id of entry k; nullptr:
// entry k is id k): with TOPP the nucleus cut and its renormalization, then r = next_f32() and
// the first entry whose cumulative probability exceeds r.  One workgroup.
template <bool TOPP>
__global__ __launch_bounds__(NT) void k_s_pick(const float *__restrict__ q, const uint32_t *__restrict__ ids, uint32_t V,
                                               float top_p, uint64_t *rng, uint32_t *counts, uint32_t *pick,
                                               StepParams *p) {
    __shared__ SegLds L;
    __shared__ uint32_t s_cut, s_found;
    __shared__ float s_s, s_r;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t cut = V;
    float s = 1.0f;
    if (TOPP) {   // cum += p in descending order until cum >= top_p (sample.rs:85-97)
        float run = 0.0f;
        if (tid == 0) s_found = 0;
        for (uint32_t s0 = 0; s0 < V; s0 += SEG - 1) {
            const uint32_t cnt = min(SEG - 1, V - s0);
            if (tid == 0) L.a[0] = run;
            for (uint32_t k = tid; k < cnt; k += NT) L.a[1 + k] = q[s0 + k];
            const float nxt = seg_sum(L, cnt + 1, wave, lane);
            if (nxt >= top_p) {   // (uniform) the crossing is in this segment
                if (tid == 0) {
                    float c;
                    const uint32_t k = scan_first(L.a, cnt + 1, top_p, false, &c);
                    s_cut = s0 + k;   // entries 0 .. s0 + k - 1 (k >= 1: the k-th term of the segment)
                    s_s = c;          // (the kept sum is the cumulative sum at the cut, sample.rs:98)
                    s_found = 1;
                }
                __syncthreads();
                break;
            }
            run = nxt;
        }
        __syncthreads();
        if (s_found) {
            cut = s_cut;
            s = s_s;
        } else {
            cut = V;
            s = run;
        }
    }
    if (tid == 0) {   // Rng::next_f32 (sample.rs:10-20)
        uint64_t x = *rng;
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        *rng = x;
        s_r = (float)((x * 0x2545F4914F6CDD1DULL) >> 40) / (float)(1u << 24);
        s_found = 0;
    }
    __syncthreads();
    const float r = s_r;
    float run = 0.0f;
    uint32_t k_pick = cut - 1;   // none exceeds r: the last kept entry (sample.rs:111)
    for (uint32_t s0 = 0; s0 < cut; s0 += SEG - 1) {
        const uint32_t cnt = min(SEG - 1, cut - s0);
        if (tid == 0) L.a[0] = run;
        for (uint32_t k = tid; k < cnt; k += NT) L.a[1 + k] = TOPP ? q[s0 + k] / s : q[s0 + k];
        const float nxt = seg_sum(L, cnt + 1, wave, lane);
        if (nxt > r) {   // (uniform)
            if (tid == 0) {
                float c;
                s_cut = s0 + scan_first(L.a, cnt + 1, r, true, &c) - 1;
                s_found = 1;
            }
            __syncthreads();
            break;
        }
        run = nxt;
    }
    __syncthreads();
    if (s_found) k_pick = s_cut;
    if (tid == 0) {
        const uint32_t id = ids ? ids[k_pick] : k_pick;
        *pick = id;
        if (p) p->token = id;
        if (counts) counts[id] += 1;
    }
}

// Engine::score_block at temp 0 (lib.rs:226-262): row r = blockIdx.x of logits [rows][V] with the
// ids >= valid masked and, when present != nullptr, the presence penalty once per present id;
// pred = the argmax (gumbel_argmax at temp 0, sample.rs:36-38), then ops::softmax of the row
// (ops.rs:112-128: m, e = exp(v - m), the id-order sum, x * (1 / sum)) read at pred and at the
// row's current id.  One workgroup per row.
// The xorshift64* state after n steps (sample.rs:10-17): the state step is linear over GF(2), so
// n steps are the product of the matrices T^(2^j) of n's set bits (M: [32][64] columns).
__device__ inline uint64_t rng_jump(uint64_t s, uint64_t n, const uint64_t *M) {
    for (uint32_t j = 0; n; ++j, n >>= 1)
        if (n & 1) {
            uint64_t r = 0;
            for (uint32_t i = 0; i < 64; ++i)
                if ((s >> i) & 1) r ^= M[j * 64 + i];
            s = r;
        }
    return s;
}

__device__ inline uint64_t rng_step(uint64_t x) {
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    return x;
}

__device__ inline float pen_logit(const float *row, uint32_t i, uint32_t valid, const uint8_t *present, float rp) {
    float l = i < valid ? row[i] : -__builtin_huge_valf();
    if (present && i < valid && present[i]) l = l > 0.0f ? l / rp : l * rp;
    return l;
}

// Finite (drawn) entries per row of the masked, penalized logits.  One workgroup per row.
__global__ __launch_bounds__(NT) void k_d_count(const float *__restrict__ logits, uint32_t V, uint32_t valid,
                                                const uint8_t *__restrict__ present, float rp, uint32_t *count) {
    __shared__ uint32_t red[NT / 64];
    const uint32_t tid = threadIdx.x, r = blockIdx.x;
    const float *row = logits + (size_t)r * V;
    uint32_t c = 0;
    for (uint32_t i = tid; i < V; i += NT) c += __builtin_isfinite(pen_logit(row, i, valid, present, rp)) ? 1u : 0u;
    for (int m = 32; m >= 1; m >>= 1) c += (uint32_t)shfl_xor_i((int)c, m);
    if ((tid & 63) == 0) red[tid >> 6] = c;
    __syncthreads();
    if (tid == 0) {
        uint32_t t = 0;
        for (uint32_t w = 0; w < NT / 64; ++w) t += red[w];
        count[r] = t;
    }
}

// Engine::score_block (lib.rs:226-262): row r = blockIdx.x of logits [rows][V] with the ids >=
// valid masked and, when present != nullptr, the presence penalty once per present id; the pick
// (GUMBEL: sample::gumbel_argmax, sample.rs:32-50 -- one draw per finite entry in id order, the
// rows' draws consecutive from state s0, g = -ln(-ln(u)) read from the table G of the 2^24
// possible u; else the argmax), then ops::softmax of the row (ops.rs:112-128: m, e = exp(v - m),
// the id-order sum, x * (1 / sum)) read at the pick and at the row's current id.  One
// workgroup per row; a thread's draws start from s0 advanced past the earlier rows' and threads'
// finite entries (rng_jump).
template <bool GUMBEL>
__global__ __launch_bounds__(NT) void k_d_score(const float *__restrict__ logits, uint32_t V, uint32_t valid,
                                                const uint8_t *__restrict__ present, float rp,
                                                const uint32_t *__restrict__ cur, uint32_t *pred, float *pconf,
                                                float *cconf, float temp, uint64_t s0,
                                                const uint64_t *__restrict__ M, const float *__restrict__ G,
                                                const uint32_t *__restrict__ count) {
    __shared__ SegLds L;
    __shared__ uint64_t Ms[GUMBEL ? 32 * 64 : 1];
    __shared__ uint32_t tcnt[NT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t r = blockIdx.x;
    const float *row = logits + (size_t)r * V;
    auto pen = [&](uint32_t i) { return pen_logit(row, i, valid, present, rp); };
    const WaveExpTab tab = WaveExpTab::load(lane);
    float mv = -__builtin_huge_valf();
    uint32_t mi = 0xffffffffu;
    if constexpr (GUMBEL) {   // a contiguous run of ids per thread, its draws in id order
        for (uint32_t i = tid; i < 32 * 64; i += NT) Ms[i] = M[i];
        const uint32_t K = div_up(V, NT), i0 = min(tid * K, V), i1 = min(i0 + K, V);
        uint32_t c = 0;
        for (uint32_t i = i0; i < i1; ++i) c += __builtin_isfinite(pen(i)) ? 1u : 0u;
        tcnt[tid] = c;
        __syncthreads();
        uint64_t off = 0;   // draws before this thread's: the earlier rows', then the earlier threads'
        for (uint32_t q = 0; q < r; ++q) off += count[q];
        for (uint32_t t = 0; t < (uint32_t)tid; ++t) off += tcnt[t];
        uint64_t st = rng_jump(s0, off, Ms);
        for (uint32_t i = i0; i < i1; ++i) {
            const float l = pen(i);
            if (!__builtin_isfinite(l)) continue;
            st = rng_step(st);
            const uint32_t k = (uint32_t)((st * 0x2545F4914F6CDD1DULL) >> 40);   // u = k / 2^24 (next_f32)
            const float val = l / temp + G[k];
            if (val > mv) {
                mv = val;
                mi = i;
            }
        }
    } else {
        for (uint32_t i = tid; i < V; i += NT) {
            const float v = pen(i);
            if (v > mv) {
                mv = v;
                mi = i;
            }
        }
    }
    for (int m = 1; m < 64; m <<= 1) {
        const float ov = shfl_xor(mv, m);
        const uint32_t oi = (uint32_t)shfl_xor_i((int)mi, m);
        if (ov > mv || (ov == mv && oi < mi)) {
            mv = ov;
            mi = oi;
        }
    }
    if (lane == 0) {
        L.red[wave] = mv;
        L.redi[wave] = mi;
    }
    __syncthreads();
    float m = L.red[0];
    uint32_t pk = L.redi[0];
    for (uint32_t w = 1; w < NT / 64; ++w)
        if (L.red[w] > m || (L.red[w] == m && L.redi[w] < pk)) {
            m = L.red[w];
            pk = L.redi[w];
        }
    if (pk == 0xffffffffu) pk = 0;   // no finite candidate: sample.rs's best = 0
    if constexpr (GUMBEL) {   // the softmax's maximum is the penalized row's own
        __syncthreads();
        float mx = -__builtin_huge_valf();
        for (uint32_t i = tid; i < V; i += NT) mx = fmaxf(mx, pen(i));
        for (int q = 32; q >= 1; q >>= 1) mx = fmaxf(mx, shfl_xor(mx, q));
        if (lane == 0) L.red[wave] = mx;
        __syncthreads();
        m = L.red[0];
        for (uint32_t w = 1; w < NT / 64; ++w) m = fmaxf(m, L.red[w]);
    }
    float sum = 0.0f;
    for (uint32_t s0 = 0; s0 < V; s0 += SEG - 1) {   // sum += exp(v - m) in id order
        const uint32_t cnt = min(SEG - 1, V - s0);
        if (tid == 0) L.a[0] = sum;
        for (uint32_t k0 = 0; k0 < cnt; k0 += NT) {   // (uniform: every lane calls the exp)
            const uint32_t k = k0 + tid;
            const float e = hg_expf_l((k < cnt ? pen(s0 + k) : m) - m, tab);
            if (k < cnt) L.a[1 + k] = e;
        }
        sum = seg_sum(L, cnt + 1, wave, lane);
    }
    if (tid == 0) {
        const float inv = 1.0f / sum;
        pred[r] = pk;
        pconf[r] = hg_expf(pen(pk) - m) * inv;
        cconf[r] = hg_expf(pen(cur[r]) - m) * inv;
    }
}

}  // namespace

bool enqueue_score_rows(hipStream_t st, const float *logits, uint32_t rows, uint32_t V, uint32_t valid,
                        const uint8_t *present, float rp, const uint32_t *cur, uint32_t *pred, float *pconf,
                        float *cconf, const GumbelDraws *gd) {
    if (!gd) {
        hipLaunchKernelGGL(k_d_score<false>, dim3(rows), dim3(NT), 0, st, logits, V, valid, present, rp, cur, pred, pconf,
                           cconf, 1.0f, (uint64_t)1, nullptr, nullptr, nullptr);
        return hipGetLastError() == hipSuccess;
    }
    hipLaunchKernelGGL(k_d_count, dim3(rows), dim3(NT), 0, st, logits, V, valid, present, rp, gd->count);
    if (hipGetLastError() != hipSuccess) return false;
    hipLaunchKernelGGL(k_d_score<true>, dim3(rows), dim3(NT), 0, st, logits, V, valid, present, rp, cur, pred, pconf,
                       cconf, gd->temp, gd->state, gd->M, gd->G, gd->count);
    return hipGetLastError() == hipSuccess;
}

// The xorshift state step as GF(2) matrices T^(2^j), j < 32, column i = the image of bit i.
void rng_jump_matrices(uint64_t *M) {
    for (uint32_t i = 0; i < 64; ++i) {
        uint64_t x = 1ull << i;
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        M[i] = x;
    }
    for (uint32_t j = 1; j < 32; ++j)
        for (uint32_t i = 0; i < 64; ++i) {
            uint64_t s = M[(j - 1) * 64 + i], r = 0;
            for (uint32_t b = 0; b < 64; ++b)
                if ((s >> b) & 1) r ^= M[(j - 1) * 64 + b];
            M[j * 64 + i] = r;
        }
}

uint64_t rng_jump_host(uint64_t s, uint64_t n, const uint64_t *M) {
    for (uint32_t j = 0; n; ++j, n >>= 1)
        if (n & 1) {
            uint64_t r = 0;
            for (uint32_t i = 0; i < 64; ++i)
                if ((s >> i) & 1) r ^= M[j * 64 + i];
            s = r;
        }
    return s;
}

// g(k) = -ln(-ln(u)) for u = k / 2^24 clamped to [1e-9, 1 - 1e-9] (sample.rs:42-43), with the
// host libm's logf -- the function Rust's f32::ln calls.  Computed once per process.
const std::vector<float> &gumbel_table() {
    static std::vector<float> t;
    static std::once_flag once;
    std::call_once(once, [] {
        t.resize((size_t)1 << 24);
        const float lo = 1e-9f, hi = 1.0f - 1e-9f;
        for (uint32_t k = 0; k < (1u << 24); ++k) {
            float u = (float)k / (float)(1u << 24);
            u = u < lo ? lo : u > hi ? hi : u;
            t[k] = -logf(-logf(u));
        }
    });
    return t;
}

int sample_init(SampleWork &w, uint32_t V) {
    int rc;
    if (w.V != V) {
        size_t bytes = 0;
        uint32_t *none = nullptr;
        HIP_TRY(rocprim::radix_sort_pairs_desc(nullptr, bytes, none, none, none, none, V, 0, 31));
        if ((rc = w.p.alloc((size_t)V * 4)) || (rc = w.keys.alloc((size_t)V * 4)) || (rc = w.ids.alloc((size_t)V * 4)) ||
            (rc = w.keys_out.alloc((size_t)V * 4)) || (rc = w.ids_out.alloc((size_t)V * 4)) ||
            (rc = w.sort_tmp.alloc(bytes)) || (rc = w.counts.alloc((size_t)V * 4)) || (rc = w.rng.alloc(8)))
            return rc;
        w.sort_bytes = bytes;
        w.V = V;
    }
    HIP_TRY(hipMemset(w.counts.p, 0, w.counts.n));
    return HG_OK;
}

bool enqueue_sample(hipStream_t st, SampleWork &w, const float *logits, uint32_t valid, float temp, float top_p,
                    float rep_penalty, uint32_t *pick, StepParams *p) {
    const uint32_t V = w.V;
    uint32_t *counts = w.counts.as<uint32_t>();
    const uint32_t *pen = rep_penalty != 1.0f ? counts : nullptr;
    if (!(temp > 0.0f)) {
        hipLaunchKernelGGL(k_s_argmax, dim3(1), dim3(NT), 0, st, logits, V, valid, rep_penalty != 1.0f ? counts : nullptr,
                           rep_penalty, pick, p);
        if (hipGetLastError() != hipSuccess) return false;
        // (occurrences are counted only when the penalty reads them)
        return true;
    }
    hipLaunchKernelGGL(k_s_probs, dim3(1), dim3(NT), 0, st, logits, V, valid, pen, rep_penalty, temp, w.p.as<float>(),
                       w.keys.as<uint32_t>(), w.ids.as<uint32_t>());
    if (hipGetLastError() != hipSuccess) return false;
    uint32_t *cnt_upd = rep_penalty != 1.0f ? counts : nullptr;
    if (top_p > 0.0f && top_p < 1.0f) {
        size_t bytes = w.sort_bytes;
        if (rocprim::radix_sort_pairs_desc(w.sort_tmp.p, bytes, w.keys.as<uint32_t>(), w.keys_out.as<uint32_t>(),
                                           w.ids.as<uint32_t>(), w.ids_out.as<uint32_t>(), V, 0, 31, st) != hipSuccess)
            return false;
        hipLaunchKernelGGL(k_s_pick<true>, dim3(1), dim3(NT), 0, st, w.keys_out.as<float>(), w.ids_out.as<uint32_t>(), V,
                           top_p, w.rng.as<uint64_t>(), cnt_upd, pick, p);
    } else {
        hipLaunchKernelGGL(k_s_pick<false>, dim3(1), dim3(NT), 0, st, w.p.as<float>(), nullptr, V, top_p,
                           w.rng.as<uint64_t>(), cnt_upd, pick, p);
    }
    return hipGetLastError() == hipSuccess;
}

}  // namespace hg
