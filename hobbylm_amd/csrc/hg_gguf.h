// hg_gguf.h -- GGUF v3 reader, hobbylm config and the Q8 load path (host side).
#pragma once
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/hobby_gpu.h"

namespace hg {

// A parsed metadata value, typed as Gguf::open keeps it (gguf.rs:16-28, 109-163).
struct Meta {
    enum Kind { U32, I32, F32, U64, BOOL, STR, ARR_STR, ARR_I32, ARR_F32, OTHER } kind = OTHER;
    uint64_t u = 0;
    int32_t i = 0;
    float f = 0.0f;
    std::string s;
};

// ggml tensor types the loader reads (gguf.rs:349-359)
enum : uint32_t { GGML_F32 = 0, GGML_F16 = 1, GGML_Q5_0 = 6, GGML_Q8_0 = 8, GGML_Q4_K = 12, GGML_Q6_K = 14 };

struct TensorInfo {
    std::vector<uint64_t> ne;  // fastest-varying first (gguf.rs:32-34)
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t n_elems() const;
    bool n_elems_checked(uint64_t &n) const;   // false if the product overflows 64 bits
};

class Gguf {
  public:
    ~Gguf();
    // Gguf::open (gguf.rs:166-212).  Returns HG_OK or a negative HG_ERR_* with `err` set.
    int open(const char *path, std::string &err);
    const TensorInfo *info(const std::string &name) const;
    bool get_u32(const std::string &key, uint32_t &v) const;   // gguf.rs:272-279
    bool get_f32(const std::string &key, float &v) const;      // gguf.rs:280-286
    bool get_bool(const std::string &key, bool &v) const;      // gguf.rs:287-292
    bool get_str(const std::string &key, std::string &v) const;
    // Gguf::f32 (gguf.rs:215-235): an F32 tensor, any other type is an error.
    int f32(const std::string &name, std::vector<float> &out, std::string &err) const;
    // Raw bytes of a tensor of a supported ggml type (F32, F16, Q5_0, Q8_0, Q4_K, Q6_K),
    // bounds-checked.
    int raw(const std::string &name, const TensorInfo *&t, const uint8_t *&data, size_t &nbytes,
            std::string &err) const;
    // Gguf::load (gguf.rs:250-269): the tensor as f32, dequantized from any supported type.
    int load(const std::string &name, std::vector<float> &out, std::string &err) const;
    const std::unordered_map<std::string, TensorInfo> &tensors() const { return tensors_; }

  private:
    const uint8_t *map_ = nullptr;
    size_t size_ = 0;
    size_t data_start_ = 0;
    std::unordered_map<std::string, Meta> meta_;
    std::unordered_map<std::string, TensorInfo> tensors_;
};

float half_to_f32(uint16_t h);  // gguf.rs:329-341
// Block dequantizers of the K-quant and 5-bit files (gguf.rs:377-468): n elements into y.
void dequant_q5_0(const uint8_t *b, size_t n, float *y);
void dequant_q4_k(const uint8_t *b, size_t n, float *y);
void dequant_q6_k(const uint8_t *b, size_t n, float *y);

// Config::from_gguf (config.rs:35-97)
int config_from_gguf(const Gguf &g, hg_config &c, std::string &err);

// A Q8_0 matrix after Q8Tensor::quantize (quant.rs:78-102), packed in the device row
// layout of hg_common.h (lane-major 128-byte chunks, scales per row).
struct PackedQ8 {
    uint32_t N = 0, K = 0, nb = 0, nc = 0;
    bool f16_exact = false;    // every scale is a binary16 value exactly
    bool f32sc = true;         // storage chosen by set_scale_storage
    std::vector<uint8_t> qs;   // N * nc * 128
    std::vector<float> sc32;   // N * nc * 4 scales (zero padded)
    std::vector<uint16_t> sc16;
    uint64_t ref_bytes() const { return (uint64_t)N * K + (uint64_t)N * nb * 4; }  // Q8Tensor::bytes
    void set_scale_storage(bool f32);
    const void *sc_bytes() const { return f32sc ? (const void *)sc32.data() : (const void *)sc16.data(); }
    size_t sc_size() const { return f32sc ? sc32.size() * 4 : sc16.size() * 2; }
};

// Requantize f32 rows (Q8Tensor::quantize) and pack them.
void pack_q8_from_f32(const float *w, uint32_t N, uint32_t K, PackedQ8 &out);
// dequant_q8_0 (gguf.rs:365-375) fused with Q8Tensor::quantize, block by block.
void pack_q8_from_q8_0(const uint8_t *blocks, uint32_t N, uint32_t K, PackedQ8 &out);

// Rope::new (ops.rs:139-152): cos/sin[max_pos][hd/2] from f64 angles.
void rope_table(uint32_t head_dim, uint32_t max_pos, float theta, std::vector<float> &cs, std::vector<float> &sn);

}  // namespace hg
