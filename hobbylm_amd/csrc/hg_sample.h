// hg_sample.h -- sample::sample (sample.rs:66-112) on the device (hg_sample.hip): the token of a
// generation step is drawn from logits that never leave the GPU.
#pragma once
#include <vector>

#include "hg_model.h"

namespace hg {

// Device buffers of the sampler for a vocabulary of V ids, and its RNG state.
struct SampleWork {
    uint32_t V = 0;
    size_t sort_bytes = 0;
    DevBuf p, keys, ids, keys_out, ids_out, sort_tmp, counts, rng;
};

// Allocates w for V ids (keeps it when V is unchanged) and zeroes the occurrence counts.
int sample_init(SampleWork &w, uint32_t V);

// One draw of Engine::generate's sampling step (lib.rs:132-142): logits[0 .. V) (device) with
// ids >= valid masked to -inf and, when rep_penalty != 1, the repetition penalty applied once
// per earlier occurrence (w.counts), then sample::sample with temperature temp and nucleus
// top_p using the device RNG state w.rng (xorshift64*, sample.rs:3-29).  The pick goes to
// *pick; with p, p->token = pick; its occurrence count is incremented.  false if a launch was
// refused.  Equal probabilities in the nucleus order by ascending id.
bool enqueue_sample(hipStream_t st, SampleWork &w, const float *logits, uint32_t valid, float temp, float top_p,
                    float rep_penalty, uint32_t *pick, StepParams *p);

// Engine::score_block at temperature 0 (lib.rs:226-262) of `rows` logit rows [rows][V] (device):
// per row the ids >= valid masked, the presence penalty (present: valid bytes, nonzero = present;
// nullptr = off), pred = the argmax, pconf / cconf = the row's softmax at pred and at cur[row].
// With Gumbel draws (temp > 0): the picks are sample::gumbel_argmax's (sample.rs:32-50) over
// the rows in order, drawing from RNG state `state`; count[row] receives each row's number of
// draws (the caller advances the state by their total).
struct GumbelDraws {
    float temp;
    uint64_t state;
    const uint64_t *M;   // device: rng_jump_matrices
    const float *G;      // device: gumbel_table()
    uint32_t *count;     // device: [rows]
};
bool enqueue_score_rows(hipStream_t st, const float *logits, uint32_t rows, uint32_t V, uint32_t valid,
                        const uint8_t *present, float rp, const uint32_t *cur, uint32_t *pred, float *pconf,
                        float *cconf, const GumbelDraws *gd = nullptr);
// GF(2) matrices of the xorshift64* state step: M[j][i] = T^(2^j) e_i (32 x 64 words).
void rng_jump_matrices(uint64_t *M);
uint64_t rng_jump_host(uint64_t s, uint64_t n, const uint64_t *M);
// -ln(-ln(u)) of every u the Rng draws (2^24 values), with the host libm's logf.
const std::vector<float> &gumbel_table();

}  // namespace hg
