// hg_common.h -- device data layouts shared by the host engine and the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hg {

constexpr int QK = 32;          // Q8_0 block (quant.rs:9)
constexpr int CHUNK_BLOCKS = 4; // blocks per 128-byte chunk of the device row layout
constexpr int CHUNK_BYTES = 128;

// A Q8_0 matrix resident in HBM, after the load-time requantization of
// Q8Tensor::quantize (quant.rs:78-102).
//
// Row layout ("lane-major chunks"): a row of K int8 weights is nb = K/32 blocks; blocks are
// grouped 4 to a 128-byte chunk, and inside a chunk the bytes are ordered
//   [lane j = 0..7][block t = 0..3][byte m = 0..3]  <- weight 32*(4c+t) + 4*j + m
// so that lane j's 16 bytes are the four 4-byte pieces qrow_dot_avx2 folds into its
// accumulator lane j (the madd_epi16 lanes of quant.rs:55-56) for 4 consecutive blocks.
// Eight consecutive threads own a row, each streaming its lane with 16-byte loads; the 8
// loads of one chunk are one contiguous, fully used 128-byte line.  A partial last chunk is
// zero padded.  Scales are a separate [N][nc*4] array, f16 when every requantized scale
// is an f16 value exactly (the GGUF case: 34 bytes per 32 weights, as on disk), else f32.
struct Q8Mat {
    const uint8_t *qs;   // [N][nc*128]
    const void *sc;      // [N][nc*4] f16 or f32
    uint32_t N, K, nb, nc;
    uint32_t sc_f32;
};

// Per-step control block in device memory; graph replays read it and the greedy argmax
// kernel may advance it, so steps chain on the device without host round trips.
struct StepParams {
    uint32_t token;     // token embedded by this step
    uint32_t pos;       // position of this step (KV row written, RoPE angle)
    uint32_t step;      // index of out_ids written by the argmax kernel
    uint32_t feedback;  // 1: argmax writes token = next and pos += 1 for the next replay
    uint32_t embed;     // 1: x = token_embd[token]; 0: x already holds the input row
    uint32_t base;      // first position of the current prefill batch
    uint32_t err;       // set by a bounded wait of the attention kernels that ran out (host: HG_ERR_DEVICE)
    uint32_t spin_cap;  // polls a bounded wait makes before giving up (0: SPIN_CAP_DEFAULT)
};
constexpr uint32_t SPIN_CAP_DEFAULT = 1u << 22;

// Per-row pointer offsets of a batched launch of a one-row kernel (blockIdx.x = row), in
// elements: x / h rows, quantized chunk bytes, scales, top-k entries, routing records.  All
// zero for a single row.
struct RowStrides {
    uint32_t x, q, d, k, rec;
};

// Matvec row order of the activation / weight dot.
enum { ORDER_DECODE = 0, ORDER_PREFILL = 1 };
// Matvec epilogues.
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_LOGITS = 2 };

inline __host__ __device__ uint32_t div_up(uint32_t a, uint32_t b) { return (a + b - 1) / b; }
// The V cache of a layer holds the rows [n_kv][cap][hd] and, after them, the same values
// transposed, [n_kv][hd][vt_stride(cap)], which the resident P.V kernel reads as contiguous
// position runs of one element.
inline __host__ __device__ uint32_t vt_stride(uint32_t cap) { return (cap + 63) / 64 * 64; }
inline __host__ __device__ size_t v_layer_floats(uint32_t cap, uint32_t n_kv, uint32_t hd) {
    return (size_t)n_kv * hd * (cap + vt_stride(cap));
}

}  // namespace hg
