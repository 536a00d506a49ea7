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

size_t type_nbytes(uint32_t ty, uint64_t n, bool &ok) {
    ok = true;
    switch (ty) {
    case 0: return (size_t)n * 4;
    case 1: return (size_t)n * 2;
    case 8: return (size_t)(n / 32) * 34;
    default: ok = false; return 0;
    }
}

}  // namespace

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
    bool ok;
    nbytes = type_nbytes(t->type, t->n_elems(), ok);
    if (!ok) {
        err = "tensor `" + name + "`: unsupported ggml_type " + std::to_string(t->type);
        return HG_ERR_UNSUPPORTED;
    }
    const size_t off = data_start_ + (size_t)t->offset;
    if (off > size_ || nbytes > size_ - off) { err = "tensor `" + name + "` data out of bounds"; return HG_ERR_FORMAT; }
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
    if (t->type == 0) return f32(name, out, err);
    const size_t n = (size_t)t->n_elems();
    out.resize(n);
    if (t->type == 1) {
        for (size_t i = 0; i < n; ++i) out[i] = half_to_f32((uint16_t)(d[2 * i] | (d[2 * i + 1] << 8)));
    } else {  // Q8_0, gguf.rs:365-375
        for (size_t b = 0; b < n / 32; ++b) {
            const float s = half_to_f32((uint16_t)(d[34 * b] | (d[34 * b + 1] << 8)));
            for (int j = 0; j < 32; ++j) out[32 * b + j] = (float)(int8_t)d[34 * b + 2 + j] * s;
        }
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
