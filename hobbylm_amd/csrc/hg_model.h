// hg_model.h -- host-side state shared by the engine's translation units: the error
// convention of the C ABI, device buffers, and the loaded model.
#pragma once
#include <hip/hip_runtime.h>

#include <memory>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/hobby_gpu.h"
#include "hg_common.h"
#include "hg_f32.h"
#include "hg_gguf.h"

namespace hg {

// The message of the last failing C-ABI call on this thread.
extern thread_local std::string g_err;

inline int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

#define HIP_TRY(expr)                                                                              \
    do {                                                                                           \
        hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess)                                                                      \
            return ::hg::fail(e_ == hipErrorOutOfMemory ? HG_ERR_NOMEM : HG_ERR_DEVICE,            \
                              std::string(#expr) + ": " + hipGetErrorString(e_));                  \
    } while (0)

// Device allocation that frees itself.
struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    int alloc(size_t bytes) {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = bytes;
        if (bytes == 0) return HG_OK;
        HIP_TRY(hipMalloc(&p, bytes));
        return HG_OK;
    }
    int upload(const void *src, size_t bytes) {
        int rc = alloc(bytes);
        if (rc) return rc;
        if (bytes) HIP_TRY(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice));
        return HG_OK;
    }
    template <class T>
    T *as() const { return static_cast<T *>(p); }
};

struct DevQ8 {
    DevBuf qs, sc;
    Q8Mat m{};
    uint64_t ref_bytes = 0;
    int upload(const PackedQ8 &p) {
        int rc = qs.upload(p.qs.data(), p.qs.size());
        if (!rc) rc = sc.upload(p.sc_bytes(), p.sc_size());
        if (rc) return rc;
        m.qs = qs.as<uint8_t>();
        m.sc = sc.p;
        m.N = p.N;
        m.K = p.K;
        m.nb = p.nb;
        m.nc = p.nc;
        m.sc_f32 = p.f32sc ? 1u : 0u;
        ref_bytes = p.ref_bytes();
        return HG_OK;
    }
    uint64_t dev_bytes() const { return qs.n + sc.n; }
};

// An F32 matrix (the F32 mode's Mat::Owned) in F32Mat's permuted row layout.
struct DevF32 {
    DevBuf w;
    F32Mat m{};
    int upload(const std::vector<float> &perm, uint32_t N, uint32_t K) {
        int rc = w.upload(perm.data(), perm.size() * 4);
        if (rc) return rc;
        m.w = w.as<float>();
        m.N = N;
        m.K = K;
        return HG_OK;
    }
};

struct Layer {
    bool moe = false;
    DevBuf attn_norm, q_norm, k_norm, ffn_norm, router, router_p, bias;
    DevQ8 qkv, o, gate, up, down, gate_e, up_e, down_e, gate_sh, up_sh, down_sh;
    // the F32 mode's matrices (loaded with quant = false; the Q8 ones are then empty)
    DevF32 fqkv, fo, fgate, fup, fdown, fgate_e, fup_e, fdown_e, fgate_sh, fup_sh, fdown_sh;
};

}  // namespace hg

struct hg_model {
    hg_config c{};
    std::vector<std::unique_ptr<hg::Layer>> layers;
    hg::DevBuf token_embd, output_norm, rope_cos, rope_sin;
    hg::DevQ8 output;
    hg::DevF32 foutput;
    bool f32 = false;   // loaded with quant = false: F32 matrices, ops::dot arithmetic
    uint64_t ref_bytes = 0, dev_bytes = 0;
    uint32_t n_slots = 0;  // routed top-k + shared expert slot
};

namespace hg {

inline uint32_t slots_of(const hg_config &c) { return c.top_k + (c.n_shared > 0 ? 1 : 0); }

// Every extern "C" body runs inside guard(): a C++ exception (host allocation failure, a
// container length error) becomes an error code instead of crossing the C boundary.
template <class F>
int guard(F &&body) {
    try {
        return body();
    } catch (const std::bad_alloc &) {
        return fail(HG_ERR_NOMEM, "host allocation failed");
    } catch (const std::length_error &e) {
        return fail(HG_ERR_NOMEM, std::string("host allocation failed: ") + e.what());
    } catch (const std::exception &e) {
        return fail(HG_ERR_DEVICE, std::string("internal error: ") + e.what());
    } catch (...) {
        return fail(HG_ERR_DEVICE, "internal error");
    }
}

// One-time device check (a gfx950 device, kernel attributes set); HG_OK or HG_ERR_DEVICE.
int check_device();

}  // namespace hg
