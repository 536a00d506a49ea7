// hg_gguf.cpp -- GGUF v3 reader, hobbylm config, load-time Q8 requantization and packing.
#include "hg_gguf.h"

#include <fcntl.h>
#include <math.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <thread>

#include "hg_common.h"

namespace hg {

uint64_t TensorInfo::n_elems() const {
    uint64_t n = 1;
    for (uint64_t v : ne) n *= v;
    return n;
}

bool TensorInfo::n_elems_checked(uint64_t &n) const {
    n = 1;
    for (uint64_t v : ne)
        if (__builtin_mul_overflow(n, v, &n)) return false;
    return true;
}

namespace {

struct Cursor {
    const uint8_t *b;
    size_t n, p = 0;
    bool bad = false;
    const uint8_t *take(size_t k) {
        if (bad || k > n - p) { bad = true; return nullptr; }
        const uint8_t *r = b + p;
        p += k;
        return r;
    }
    uint64_t le(size_t k) {
        const uint8_t *q = take(k);
        uint64_t v = 0;
        if (q)
            for (size_t i = 0; i < k; ++i) v |= (uint64_t)q[i] << (8 * i);
        return v;
    }
    bool str(std::string &s) {
        const uint64_t len = le(8);
        const uint8_t *q = take((size_t)len);
        if (!q) return false;
        s.assign(reinterpret_cast<const char *>(q), (size_t)len);
        return true;
    }
};

enum { T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 };

// gguf.rs:109-125
bool read_scalar(Cursor &c, uint32_t ty, Meta &m, std::string &err) {
    switch (ty) {
    case T_U8: m.kind = Meta::U32; m.u = c.le(1); break;
    case T_I8: m.kind = Meta::I32; m.i = (int8_t)c.le(1); break;
    case T_U16: m.kind = Meta::U32; m.u = c.le(2); break;
    case T_I16: m.kind = Meta::I32; m.i = (int16_t)c.le(2); break;
    case T_U32: m.kind = Meta::U32; m.u = c.le(4); break;
    case T_I32: m.kind = Meta::I32; m.i = (int32_t)c.le(4); break;
    case T_F32: { const uint32_t u = (uint32_t)c.le(4); m.kind = Meta::F32; memcpy(&m.f, &u, 4); break; }
    case T_BOOL: m.kind = Meta::BOOL; m.u = c.le(1) != 0; break;
    case T_STR: m.kind = Meta::STR; if (!c.str(m.s)) c.bad = true; break;
    case T_U64: m.kind = Meta::U64; m.u = c.le(8); break;
    case T_I64: m.kind = Meta::I32; m.i = (int32_t)c.le(8); break;
    case T_F64: { const uint64_t u = c.le(8); double d; memcpy(&d, &u, 8); m.kind = Meta::F32; m.f = (float)d; break; }
    default: err = "GGUF: unsupported metadata scalar type " + std::to_string(ty); return false;
    }
    if (c.bad) { err = "GGUF: unexpected end of file"; return false; }
    return true;
}

// gguf.rs:127-163
bool read_value(Cursor &c, uint32_t ty, Meta &m, std::string &err) {
    if (ty != T_ARR) return read_scalar(c, ty, m, err);
    const uint32_t at = (uint32_t)c.le(4);
    const uint64_t n = c.le(8);
    if (c.bad) { err = "GGUF: unexpected end of file"; return false; }
    if (at == T_STR) {
        m.kind = Meta::ARR_STR;
        std::string s;
        for (uint64_t k = 0; k < n; ++k)
            if (!c.str(s)) { err = "GGUF: unexpected end of file"; return false; }
    } else if (at == T_I32 || at == T_U32 || at == T_F32) {
        m.kind = at == T_F32 ? Meta::ARR_F32 : Meta::ARR_I32;
        if (n > (c.n - c.p) / 4 || !c.take((size_t)n * 4)) { err = "GGUF: unexpected end of file"; return false; }
    } else {
        m.kind = Meta::OTHER;
        for (uint64_t k = 0; k < n; ++k) {
            Meta t;
            if (!read_scalar(c, at, t, err)) return false;
        }
    }
    return true;
}

// type_nbytes (gguf.rs:349-359): bytes of n elements of ggml type ty (whole blocks; a partial
// block is not stored).  ok = false for another type; an unrepresentable size is reported as
// SIZE_MAX, which no file holds.
size_t type_nbytes(uint32_t ty, uint64_t n, bool &ok) {
    ok = true;
    uint64_t unit, per;   // bytes per `per` elements
    switch (ty) {
    case GGML_F32: unit = 4; per = 1; break;
    case GGML_F16: unit = 2; per = 1; break;
    case GGML_Q5_0: unit = 22; per = 32; break;    // d(2) qh(4) qs(16)
    case GGML_Q8_0: unit = 34; per = 32; break;    // d(2) qs(32)
    case GGML_Q4_K: unit = 144; per = 256; break;  // d(2) dmin(2) scales(12) qs(128)
    case GGML_Q6_K: unit = 210; per = 256; break;  // ql(128) qh(64) scales(16) d(2)
    default: ok = false; return 0;
    }
    uint64_t b;
    if (__builtin_mul_overflow(n / per, unit, &b) || b > (uint64_t)SIZE_MAX) return SIZE_MAX;
    return (size_t)b;
}

inline float rd_half(const uint8_t *b) { return half_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

// scale_min_k4 (gguf.rs:399-408): the 6-bit scale and min of sub-block j of a K-quant super
// block, packed in 12 bytes (j < 4 in the low 6 bits of bytes j and j + 4; j >= 4 split over
// a nibble of byte j + 4 and the top 2 bits of bytes j - 4 and j).
inline void scale_min_k4(uint32_t j, const uint8_t *sc, uint32_t &d, uint32_t &m) {
    if (j < 4) {
        d = sc[j] & 63u;
        m = sc[j + 4] & 63u;
    } else {
        d = (sc[j + 4] & 0x0fu) | ((uint32_t)(sc[j - 4] >> 6) << 4);
        m = (uint32_t)(sc[j + 4] >> 4) | ((uint32_t)(sc[j] >> 6) << 4);
    }
}

}  // namespace

// dequant_q5_0 (gguf.rs:377-397): block {f16 d; u32 qh; u8 qs[16]}; element j < 16 is the low
// nibble of qs[j] with bit j of qh as its fifth bit, element 16 + j the high nibble with bit
// 16 + j of qh, both offset by -16, times d.
void dequant_q5_0(const uint8_t *b, size_t n, float *y) {
    for (size_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t *o = b + blk * 22;
        const float d = rd_half(o);
        const uint32_t qh = (uint32_t)o[2] | (uint32_t)o[3] << 8 | (uint32_t)o[4] << 16 | (uint32_t)o[5] << 24;
        const uint8_t *qs = o + 6;
        for (uint32_t j = 0; j < 16; ++j) {
            const uint32_t lo = (qs[j] & 0x0fu) | (((qh >> j) << 4) & 0x10u);
            const uint32_t hi = (qs[j] >> 4) | ((qh >> (j + 12)) & 0x10u);
            y[blk * 32 + j] = (float)((int)lo - 16) * d;
            y[blk * 32 + 16 + j] = (float)((int)hi - 16) * d;
        }
    }
}

// dequant_q4_k (gguf.rs:410-439): super blocks of 256 = 8 sub-blocks of 32; sub-block pair
// (2i, 2i + 1) uses the low and high nibbles of qs[32 i .. 32 i + 32]:
// y = (d * sc) * q - dmin * m, each product rounded (no fused multiply-add).
void dequant_q4_k(const uint8_t *b, size_t n, float *y) {
    for (size_t blk = 0; blk < n / 256; ++blk) {
        const uint8_t *o = b + blk * 144;
        const float d = rd_half(o), dmin = rd_half(o + 2);
        const uint8_t *scales = o + 4, *qs = o + 16;
        float *yo = y + blk * 256;
        for (uint32_t i = 0; i < 4; ++i) {
            uint32_t sc1, m1, sc2, m2;
            scale_min_k4(2 * i, scales, sc1, m1);
            scale_min_k4(2 * i + 1, scales, sc2, m2);
            const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
            const float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
            for (uint32_t l = 0; l < 32; ++l) yo[64 * i + l] = d1 * (float)(qs[32 * i + l] & 0x0f) - mm1;
            for (uint32_t l = 0; l < 32; ++l) yo[64 * i + 32 + l] = d2 * (float)(qs[32 * i + l] >> 4) - mm2;
        }
    }
}

// dequant_q6_k (gguf.rs:441-468): super blocks of 256 as two halves of 128; element l (< 32)
// of quarter k of a half takes 4 low bits from ql and 2 high bits from qh, offset by -32, and
// the int8 scale of its 16-element group: y = (d * s) * q.
void dequant_q6_k(const uint8_t *b, size_t n, float *y) {
    for (size_t blk = 0; blk < n / 256; ++blk) {
        const uint8_t *o = b + blk * 210;
        const uint8_t *ql = o, *qh = o + 128;
        const int8_t *sc = reinterpret_cast<const int8_t *>(o + 192);
        const float d = rd_half(o + 208);
        for (uint32_t half = 0; half < 2; ++half) {
            float *yb = y + blk * 256 + half * 128;
            const uint8_t *qlb = ql + half * 64, *qhb = qh + half * 32;
            const int8_t *scb = sc + half * 8;
            for (uint32_t l = 0; l < 32; ++l) {
                const uint32_t is = l / 16;
                const int q1 = (int)((qlb[l] & 0x0fu) | (((qhb[l] >> 0) & 3u) << 4)) - 32;
                const int q2 = (int)((qlb[l + 32] & 0x0fu) | (((qhb[l] >> 2) & 3u) << 4)) - 32;
                const int q3 = (int)((uint32_t)(qlb[l] >> 4) | (((qhb[l] >> 4) & 3u) << 4)) - 32;
                const int q4 = (int)((uint32_t)(qlb[l + 32] >> 4) | (((qhb[l] >> 6) & 3u) << 4)) - 32;
                yb[l] = d * (float)scb[is + 0] * (float)q1;
                yb[l + 32] = d * (float)scb[is + 2] * (float)q2;
                yb[l + 64] = d * (float)scb[is + 4] * (float)q3;
                yb[l + 96] = d * (float)scb[is + 6] * (float)q4;
            }
        }
    }
}


Gguf::~Gguf() {
    if (map_) munmap(const_cast<uint8_t *>(map_), size_);
}

int Gguf::open(const char *path, std::string &err) {
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) { err = std::string("opening ") + path; return HG_ERR_IO; }
    struct stat st;
    if (fstat(fd, &st) != 0) { ::close(fd); err = std::string("opening ") + path; return HG_ERR_IO; }
    size_ = (size_t)st.st_size;
    if (size_ == 0) { ::close(fd); err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
    void *p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) { err = std::string("mmap ") + path; return HG_ERR_IO; }
    map_ = static_cast<const uint8_t *>(p);
    Cursor c{map_, size_};
    const uint32_t magic = (uint32_t)c.le(4);
    if (c.bad) { err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
    if (magic != 0x46554747u) { err = "not a GGUF file (bad magic)"; return HG_ERR_FORMAT; }
    const uint32_t version = (uint32_t)c.le(4);
    if (c.bad) { err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
    if (version != 3) { err = "unsupported GGUF version " + std::to_string(version) + " (expected 3)"; return HG_ERR_FORMAT; }
    const uint64_t n_t = c.le(8), n_m = c.le(8);
    if (c.bad) { err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
    for (uint64_t k = 0; k < n_m; ++k) {
        std::string key;
        if (!c.str(key)) { err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
        const uint32_t ty = (uint32_t)c.le(4);
        if (c.bad) { err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
        Meta m;
        if (!read_value(c, ty, m, err)) return HG_ERR_FORMAT;
        meta_[key] = std::move(m);
    }
    for (uint64_t k = 0; k < n_t; ++k) {
        std::string name;
        if (!c.str(name)) { err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
        const uint32_t nd = (uint32_t)c.le(4);
        if (c.bad || nd > 8) { err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
        TensorInfo t;
        for (uint32_t d = 0; d < nd; ++d) t.ne.push_back(c.le(8));
        t.type = (uint32_t)c.le(4);
        t.offset = c.le(8);
        if (c.bad) { err = "GGUF: unexpected end of file"; return HG_ERR_FORMAT; }
        tensors_[name] = std::move(t);
    }
    size_t align = 32;
    auto it = meta_.find("general.alignment");
    if (it != meta_.end() && it->second.kind == Meta::U32) align = (size_t)it->second.u;
    if (align == 0) { err = "GGUF: general.alignment is 0"; return HG_ERR_FORMAT; }
    data_start_ = (c.p + align - 1) / align * align;
    return HG_OK;
}

const TensorInfo *Gguf::info(const std::string &name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

bool Gguf::get_u32(const std::string &key, uint32_t &v) const {
    auto it = meta_.find(key);
    if (it == meta_.end()) return false;
    const Meta &m = it->second;
    if (m.kind == Meta::U32 || m.kind == Meta::U64) { v = (uint32_t)m.u; return true; }
    if (m.kind == Meta::I32) { v = (uint32_t)m.i; return true; }
    return false;
}

bool Gguf::get_f32(const std::string &key, float &v) const {
    auto it = meta_.find(key);
    if (it == meta_.end()) return false;
    if (it->second.kind == Meta::F32) { v = it->second.f; return true; }
    if (it->second.kind == Meta::U32) { v = (float)(uint32_t)it->second.u; return true; }
    return false;
}

bool Gguf::get_bool(const std::string &key, bool &v) const {
    auto it = meta_.find(key);
    if (it == meta_.end() || it->second.kind != Meta::BOOL) return false;
    v = it->second.u != 0;
    return true;
}

bool Gguf::get_str(const std::string &key, std::string &v) const {
    auto it = meta_.find(key);
    if (it == meta_.end() || it->second.kind != Meta::STR) return false;
    v = it->second.s;
    return true;
}

int Gguf::raw(const std::string &name, const TensorInfo *&t, const uint8_t *&data, size_t &nbytes,
              std::string &err) const {
    t = info(name);
    if (!t) { err = "tensor `" + name + "` not found"; return HG_ERR_FORMAT; }
    uint64_t n;
    if (!t->n_elems_checked(n) || n > (uint64_t)SIZE_MAX / 4) {
        err = "tensor `" + name + "`: element count overflows";
        return HG_ERR_FORMAT;
    }
    bool ok;
    nbytes = type_nbytes(t->type, n, ok);
    if (!ok) {   // gguf.rs:358 (Gguf::raw adds no context)
        err = "type_nbytes: unsupported ggml_type " + std::to_string(t->type);
        return HG_ERR_UNSUPPORTED;
    }
    if (t->offset > size_ || data_start_ > size_ - t->offset) {
        err = "tensor `" + name + "` data out of bounds";
        return HG_ERR_FORMAT;
    }
    const size_t off = data_start_ + (size_t)t->offset;
    if (nbytes > size_ - off) { err = "tensor `" + name + "` data out of bounds"; return HG_ERR_FORMAT; }
    data = map_ + off;
    return HG_OK;
}

int Gguf::f32(const std::string &name, std::vector<float> &out, std::string &err) const {
    const TensorInfo *t = info(name);
    if (!t) { err = "tensor `" + name + "` not found in GGUF"; return HG_ERR_FORMAT; }
    if (t->type != 0) {
        err = "tensor `" + name + "` is ggml_type " + std::to_string(t->type) +
              " (expected F32=0); this engine is F32-only for now";
        return HG_ERR_FORMAT;
    }
    const uint8_t *d;
    size_t nb;
    int rc = raw(name, t, d, nb, err);
    if (rc) return rc;
    if ((d - map_) % 4) { err = "tensor `" + name + "` is not 4-byte aligned"; return HG_ERR_FORMAT; }
    out.resize(nb / 4);
    memcpy(out.data(), d, nb);
    return HG_OK;
}

int Gguf::load(const std::string &name, std::vector<float> &out, std::string &err) const {
    const TensorInfo *t;
    const uint8_t *d;
    size_t nb;
    int rc = raw(name, t, d, nb, err);
    if (rc) return rc;
    if (t->type == GGML_F32) return f32(name, out, err);
    const size_t n = (size_t)t->n_elems();
    out.assign(n, 0.0f);   // (elements of a partial last block stay 0, as in gguf.rs)
    switch (t->type) {
    case GGML_F16:   // dequant_f16, gguf.rs:361-363
        for (size_t i = 0; i < n; ++i) out[i] = rd_half(d + 2 * i);
        break;
    case GGML_Q8_0:  // dequant_q8_0, gguf.rs:365-375
        for (size_t b = 0; b < n / 32; ++b) {
            const float s = rd_half(d + 34 * b);
            for (int j = 0; j < 32; ++j) out[32 * b + j] = (float)(int8_t)d[34 * b + 2 + j] * s;
        }
        break;
    case GGML_Q5_0: dequant_q5_0(d, n, out.data()); break;
    case GGML_Q4_K: dequant_q4_k(d, n, out.data()); break;
    case GGML_Q6_K: dequant_q6_k(d, n, out.data()); break;
    }
    return HG_OK;
}

// gguf.rs:329-341: sign, 5-bit exponent, 10-bit mantissa; subnormals mant * 2^-24.
float half_to_f32(uint16_t h) {
    const uint32_t sign = (h >> 15) & 1;
    const int exp = (h >> 10) & 0x1f;
    const float mant = (float)(h & 0x3ff);
    float val;
    if (exp == 0) val = mant * ldexpf(1.0f, -24);
    else if (exp == 0x1f) val = (h & 0x3ff) == 0 ? INFINITY : NAN;
    else val = (1.0f + mant / 1024.0f) * ldexpf(1.0f, exp - 15);
    return sign ? -val : val;
}

int config_from_gguf(const Gguf &g, hg_config &c, std::string &err) {
    memset(&c, 0, sizeof c);
    std::string arch;
    if (!g.get_str("general.architecture", arch)) { err = "missing general.architecture"; return HG_ERR_FORMAT; }
    auto key = [&](const char *s) { return arch + "." + s; };
    auto req = [&](const char *s, uint32_t &v) -> bool {
        if (g.get_u32(key(s), v)) return true;
        err = "missing metadata `" + arch + "." + s + "`";
        return false;
    };
    auto opt = [&](const char *s, uint32_t dflt) {
        uint32_t v;
        return g.get_u32(key(s), v) ? v : dflt;
    };
    uint32_t hd;
    if (g.get_u32(key("attention.key_length"), hd)) c.head_dim = hd;
    else {
        uint32_t d = 0, h = 1;
        g.get_u32(key("embedding_length"), d);
        g.get_u32(key("attention.head_count"), h);
        c.head_dim = d / (h ? h : 1);
    }
    const TensorInfo *te = g.info("token_embd.weight");
    uint32_t vs;
    if (te && te->ne.size() > 1) c.vocab_size = (uint32_t)te->ne[1];
    else if (g.get_u32(key("vocab_size"), vs)) c.vocab_size = vs;
    else { err = "cannot determine vocab_size"; return HG_ERR_FORMAT; }
    uint32_t gf;
    c.gating_sigmoid = g.get_u32(key("expert_gating_func"), gf) ? (gf == 1 ? 0 : 1) : 1;
    if (!req("embedding_length", c.d_model) || !req("block_count", c.n_layers)) return HG_ERR_FORMAT;
    c.n_dense = opt("leading_dense_block_count", 1);
    if (!req("attention.head_count", c.n_heads) || !req("attention.head_count_kv", c.n_kv_heads) ||
        !req("feed_forward_length", c.dense_ffn) || !req("expert_feed_forward_length", c.expert_ffn) ||
        !req("expert_count", c.n_experts) || !req("expert_used_count", c.top_k))
        return HG_ERR_FORMAT;
    c.n_shared = opt("expert_shared_count", 0);
    c.context_length = opt("context_length", 8192);
    if (!g.get_f32(key("attention.layer_norm_rms_epsilon"), c.rms_eps)) c.rms_eps = 1e-5f;
    if (!g.get_f32(key("rope.freq_base"), c.rope_theta)) c.rope_theta = 1e6f;
    if (!g.get_f32(key("expert_weights_scale"), c.expert_weights_scale)) c.expert_weights_scale = 1.0f;
    bool b;
    c.expert_weights_norm = g.get_bool(key("expert_weights_norm"), b) ? b : 0;
    if (!g.get_u32("diffusion.mask_token_id", c.mask_token_id)) c.mask_token_id = 50257;   // config.rs:93
    return HG_OK;
}

namespace {

// One block of Q8Tensor::quantize (quant.rs:90-99): d = amax/127, id = 1/d (0 if d == 0),
// q = clamp(round(v*id), -127, 127) with round half away from zero.
inline float quant_block(const float *v, int8_t *q) {
    float amax = 0.0f;
    for (int j = 0; j < QK; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    for (int j = 0; j < QK; ++j) {
        float r = roundf(v[j] * id);
        if (r != r) r = 0.0f;
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        q[j] = (int8_t)r;
    }
    return d;
}

// Lane-major chunk position of weight k of a row (hg_common.h).
inline size_t chunk_pos(uint32_t k) {
    const uint32_t b = k / 32, e = k % 32, j = e / 4, m = e % 4;
    return (size_t)(b / 4) * CHUNK_BYTES + j * 16 + (b % 4) * 4 + m;
}

template <class F>
void parallel_rows(uint32_t N, F fn) {
    unsigned nt = std::max(1u, std::min(std::thread::hardware_concurrency(), 32u));
    if (N < 256) nt = 1;
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; ++t)
        th.emplace_back([=, &fn] {
            for (uint32_t r = (uint32_t)((uint64_t)N * t / nt); r < (uint32_t)((uint64_t)N * (t + 1) / nt); ++r) fn(r);
        });
    for (auto &x : th) x.join();
}

// Requantize rows given a row reader (f32 values of row r into buf), then pack.
template <class Reader>
void pack_rows(uint32_t N, uint32_t K, PackedQ8 &out, Reader read_row) {
    out.N = N;
    out.K = K;
    out.nb = K / QK;
    out.nc = div_up(out.nb, CHUNK_BLOCKS);
    const size_t pitch = (size_t)out.nc * CHUNK_BYTES;
    out.qs.assign((size_t)N * pitch, 0);
    std::vector<float> scales((size_t)N * out.nc * 4, 0.0f);
    parallel_rows(N, [&](uint32_t r) {
        std::vector<float> buf(K);
        int8_t q[QK];
        read_row(r, buf.data());
        uint8_t *dst = out.qs.data() + (size_t)r * pitch;
        for (uint32_t b = 0; b < out.nb; ++b) {
            scales[(size_t)r * out.nc * 4 + b] = quant_block(buf.data() + (size_t)b * QK, q);
            for (int e = 0; e < QK; ++e) dst[chunk_pos(b * QK + e)] = (uint8_t)q[e];
        }
    });
    bool f16_ok = true;
    for (float s : scales) {
        const _Float16 h = (_Float16)s;
        if ((float)h != s) { f16_ok = false; break; }
    }
    out.f16_exact = f16_ok;
    out.sc32 = std::move(scales);
}

}  // namespace

void PackedQ8::set_scale_storage(bool f32) {
    f32sc = f32;
    sc16.clear();
    if (!f32) {
        sc16.resize(sc32.size());
        for (size_t i = 0; i < sc32.size(); ++i) sc16[i] = __builtin_bit_cast(uint16_t, (_Float16)sc32[i]);
    }
}

void pack_q8_from_f32(const float *w, uint32_t N, uint32_t K, PackedQ8 &out) {
    pack_rows(N, K, out, [&](uint32_t r, float *buf) { memcpy(buf, w + (size_t)r * K, (size_t)K * 4); });
}

void pack_q8_from_q8_0(const uint8_t *blocks, uint32_t N, uint32_t K, PackedQ8 &out) {
    const uint32_t nb = K / QK;
    pack_rows(N, K, out, [&](uint32_t r, float *buf) {
        for (uint32_t b = 0; b < nb; ++b) {
            const uint8_t *blk = blocks + ((size_t)r * nb + b) * 34;
            const float s = half_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            for (int j = 0; j < QK; ++j) buf[b * QK + j] = (float)(int8_t)blk[2 + j] * s;
        }
    });
}

void rope_table(uint32_t head_dim, uint32_t max_pos, float theta, std::vector<float> &cs, std::vector<float> &sn) {
    const uint32_t half = head_dim / 2;
    cs.resize((size_t)max_pos * half);
    sn.resize((size_t)max_pos * half);
    for (uint32_t p = 0; p < max_pos; ++p)
        for (uint32_t i = 0; i < half; ++i) {
            const double inv_freq = pow((double)theta, -(2.0 * (double)i) / (double)head_dim);
            const double ang = (double)p * inv_freq;
            cs[(size_t)p * half + i] = (float)cos(ang);
            sn[(size_t)p * half + i] = (float)sin(ang);
        }
}

}  // namespace hg
