"""ctypes bindings for the CPU oracle (liboracle.so, built from oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py's cpu_baseline leg.  The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")   # (ORACLE_LIB: a sanitizer build)

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


class OrcConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "d_model", "n_layers", "n_dense", "n_heads", "n_kv_heads", "head_dim", "dense_ffn",
        "expert_ffn", "n_experts", "top_k", "n_shared", "vocab_size", "context_length")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("expert_weights_scale", C.c_float),
        ("expert_weights_norm", C.c_int32), ("gating_sigmoid", C.c_int32), ("mask_token_id", C.c_uint32)]


class DiffOpts(C.Structure):
    """orc_diff_opts: DiffOpts (lib.rs:45-65); defaults as DiffOpts::default (lib.rs:59-64)."""
    _fields_ = [("gen_len", C.c_uint32), ("block", C.c_uint32), ("steps", C.c_uint32), ("temp", C.c_float),
                ("rep_penalty", C.c_float), ("remask_steps", C.c_uint32), ("remask_frac", C.c_float),
                ("seed", C.c_uint64), ("cached", C.c_uint32), ("threshold", C.c_float)]

    @classmethod
    def make(cls, gen_len=128, block=32, steps=32, temp=0.0, rep_penalty=1.4, remask_steps=0, remask_frac=0.3,
             seed=1234, cached=True, threshold=0.0):
        return cls(gen_len, block, steps, temp, rep_penalty, remask_steps, remask_frac, seed, int(cached), threshold)


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        sig = {
            "orc_last_error": (C.c_char_p, []),
            "orc_set_threads": (None, [C.c_int]),
            "orc_get_threads": (C.c_int, []),
            "orc_half_to_f32": (C.c_float, [C.c_uint16]),
            "orc_dequant_q8_0": (None, [_u8p, C.c_size_t, _f32p]),
            "orc_dequant_f16": (None, [_u8p, C.c_size_t, _f32p]),
            "orc_dequant_q5_0": (None, [_u8p, C.c_size_t, _f32p]),
            "orc_dequant_q4_k": (None, [_u8p, C.c_size_t, _f32p]),
            "orc_dequant_q6_k": (None, [_u8p, C.c_size_t, _f32p]),
            "orc_gguf_load_tensor": (C.c_int, [C.c_char_p, C.c_char_p, C.c_void_p, C.c_uint64,
                                               C.POINTER(C.c_uint64)]),
            "orc_q8_quantize": (None, [_f32p, C.c_size_t, C.c_size_t, _f32p, _i8p]),
            "orc_quantize_act": (None, [_f32p, C.c_size_t, _i8p, _f32p]),
            "orc_qrow_dot": (C.c_float, [_i8p, _i8p, _f32p, _f32p, C.c_size_t]),
            "orc_q8_matvec": (None, [_f32p, _i8p, C.c_size_t, C.c_size_t, _f32p, _f32p]),
            "orc_q8_matmul": (None, [_f32p, _i8p, C.c_size_t, C.c_size_t, _f32p, _f32p, C.c_size_t]),
            "orc_dot": (C.c_float, [_f32p, _f32p, C.c_size_t]),
            "orc_matvec_f32": (None, [_f32p, _f32p, _f32p, C.c_size_t, C.c_size_t]),
            "orc_sigmoid": (C.c_float, [C.c_float]),
            "orc_silu": (C.c_float, [C.c_float]),
            "orc_expf": (C.c_float, [C.c_float]),
            "orc_rmsnorm": (None, [_f32p, _f32p, C.c_float, _f32p, C.c_size_t]),
            "orc_softmax": (None, [_f32p, C.c_size_t]),
            "orc_norm_head": (None, [_f32p, _f32p, C.c_float, C.c_size_t]),
            "orc_rope_table": (None, [C.c_size_t, C.c_size_t, C.c_float, _f32p, _f32p]),
            "orc_rope_apply": (None, [_f32p, _f32p, C.c_size_t, _f32p, C.c_size_t]),
            "orc_argmax": (C.c_uint32, [_f32p, C.c_size_t]),
            "orc_route": (C.c_int, [_f32p, _f32p, C.c_uint32, C.c_uint32, C.c_int, C.c_int, _u32p, _f32p,
                                    C.POINTER(C.c_float)]),
            "orc_attention_decode": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                            C.c_float, C.c_uint32, C.c_uint32, C.c_uint32,
                                            C.c_uint32, _f32p, _f32p, _f32p]),
            "orc_model_load": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_void_p)]),
            "orc_model_free": (None, [C.c_void_p]),
            "orc_model_config": (C.c_int, [C.c_void_p, C.POINTER(OrcConfig)]),
            "orc_weight_bytes": (C.c_uint64, [C.c_void_p]),
            "orc_kv_new": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
            "orc_kv_free": (None, [C.c_void_p]),
            "orc_kv_len": (C.c_uint32, [C.c_void_p]),
            "orc_kv_read": (C.c_int, [C.c_void_p, C.c_uint32, _f32p, _f32p]),
            "orc_kv_load": (C.c_int, [C.c_void_p, C.c_uint32, _f32p, _f32p]),
            "orc_token_embedding": (C.c_int, [C.c_void_p, C.c_uint32, _f32p]),
            "orc_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, _f32p]),
            "orc_forward_x": (C.c_int, [C.c_void_p, C.c_void_p, _f32p, C.c_uint32, _f32p]),
            "orc_prefill": (C.c_int, [C.c_void_p, C.c_void_p, _f32p, C.c_uint32, _f32p]),
            "orc_last_routing": (C.c_int, [C.c_void_p, _u32p, _f32p, _f32p]),
            "orc_generate_greedy": (C.c_int, [C.c_void_p, C.c_void_p, _u32p, C.c_uint32, C.c_uint32,
                                              C.c_float, C.c_uint32, _u32p, C.POINTER(C.c_uint32)]),
            "orc_generate": (C.c_int, [C.c_void_p, C.c_void_p, _u32p, C.c_uint32, C.c_uint32, C.c_float,
                                       C.c_float, C.c_uint64, C.c_float, C.c_uint32, _u32p,
                                       C.POINTER(C.c_uint32)]),
            "orc_run_block": (C.c_int, [C.c_void_p, C.c_void_p, _f32p, C.c_uint32, C.c_uint32, C.c_void_p,
                                        C.c_void_p, C.c_void_p]),
            "orc_forward_bidir": (C.c_int, [C.c_void_p, _f32p, C.c_uint32, _f32p]),
            "orc_generate_diffusion": (C.c_int, [C.c_void_p, _u32p, C.c_uint32, C.c_void_p, C.c_uint32, _u32p,
                                                 C.POINTER(C.c_uint32)]),
            "orc_gumbel_argmax": (C.c_uint32, [_f32p, C.c_size_t, C.c_float, C.POINTER(C.c_uint64)]),
            "orc_rng_next_u64": (C.c_uint64, [C.POINTER(C.c_uint64)]),
            "orc_rng_next_f32": (C.c_float, [C.POINTER(C.c_uint64)]),
            "orc_sample": (C.c_uint32, [_f32p, C.c_size_t, C.c_float, C.c_float, C.POINTER(C.c_uint64)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class OracleError(RuntimeError):
    pass


def _check(rc):
    if rc != 0:
        raise OracleError(lib().orc_last_error().decode())


def set_threads(n: int):
    lib().orc_set_threads(int(n))


def threads() -> int:
    return int(lib().orc_get_threads())


# ---- op level ----
class Rng:
    """sample::Rng (sample.rs:3-29): xorshift64*, the seed clamped to at least 1."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(max(int(seed), 1))

    def next_u64(self) -> int:
        return int(lib().orc_rng_next_u64(C.byref(self.state)))

    def next_f32(self) -> float:
        return float(lib().orc_rng_next_f32(C.byref(self.state)))


def gumbel_argmax(logits: np.ndarray, temp: float, rng: Rng) -> int:
    """sample::gumbel_argmax (sample.rs:32-50)."""
    lg = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_gumbel_argmax(lg, lg.size, temp, C.byref(rng.state)))


def sample(logits: np.ndarray, temp: float, top_p: float, rng: Rng) -> int:
    """sample::sample (sample.rs:66-112); ties in the nucleus order by ascending token id."""
    lg = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_sample(lg, lg.size, temp, top_p, C.byref(rng.state)))


def half_to_f32(h: int) -> float:
    return float(lib().orc_half_to_f32(h))


def dequant_q8_0(raw: np.ndarray, n: int) -> np.ndarray:
    y = np.empty(n, np.float32)
    lib().orc_dequant_q8_0(np.ascontiguousarray(raw, np.uint8), n, y)
    return y


def dequant(ggml_type: int, raw: np.ndarray, n: int) -> np.ndarray:
    """Gguf::load's dequantization of n elements of a Q5_0 (6), Q8_0 (8), Q4_K (12) or Q6_K (14)
    tensor (gguf.rs:365-468)."""
    fn = {6: lib().orc_dequant_q5_0, 8: lib().orc_dequant_q8_0, 12: lib().orc_dequant_q4_k,
          14: lib().orc_dequant_q6_k, 1: lib().orc_dequant_f16}[ggml_type]
    y = np.zeros(n, np.float32)
    fn(np.ascontiguousarray(raw, np.uint8).reshape(-1), n, y)
    return y


def gguf_load_tensor(path: str, name: str) -> np.ndarray:
    """Gguf::load (gguf.rs:250-269) of one tensor, as f32."""
    n = C.c_uint64()
    _check(lib().orc_gguf_load_tensor(str(path).encode(), name.encode(), None, 0, C.byref(n)))
    out = np.empty(n.value, np.float32)
    _check(lib().orc_gguf_load_tensor(str(path).encode(), name.encode(), out.ctypes.data_as(C.c_void_p),
                                      out.size, C.byref(n)))
    return out


def q8_quantize(w: np.ndarray):
    out, inn = w.shape
    sc = np.empty(out * (inn // 32), np.float32)
    qs = np.empty(out * inn, np.int8)
    lib().orc_q8_quantize(np.ascontiguousarray(w, np.float32), out, inn, sc, qs)
    return sc.reshape(out, inn // 32), qs.reshape(out, inn)


def quantize_act(x: np.ndarray):
    n = x.size
    qx = np.empty(n, np.int8)
    dx = np.empty(n // 32, np.float32)
    lib().orc_quantize_act(np.ascontiguousarray(x, np.float32), n, qx, dx)
    return qx, dx


def qrow_dot(qw, qa, sw, dx) -> float:
    return float(lib().orc_qrow_dot(np.ascontiguousarray(qw, np.int8), np.ascontiguousarray(qa, np.int8),
                                    np.ascontiguousarray(sw, np.float32),
                                    np.ascontiguousarray(dx, np.float32), len(sw)))


def q8_matvec(scales, qs, x) -> np.ndarray:
    out, inn = qs.shape
    y = np.empty(out, np.float32)
    lib().orc_q8_matvec(np.ascontiguousarray(scales, np.float32).reshape(-1),
                        np.ascontiguousarray(qs, np.int8).reshape(-1), out, inn,
                        np.ascontiguousarray(x, np.float32), y)
    return y


def q8_matmul(scales, qs, x) -> np.ndarray:
    out, inn = qs.shape
    tn = x.shape[0]
    y = np.empty((tn, out), np.float32)
    lib().orc_q8_matmul(np.ascontiguousarray(scales, np.float32).reshape(-1),
                        np.ascontiguousarray(qs, np.int8).reshape(-1), out, inn,
                        np.ascontiguousarray(x, np.float32).reshape(-1), y.reshape(-1), tn)
    return y


def dot(a, b) -> float:
    return float(lib().orc_dot(np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32), a.size))


def matvec_f32(w, x) -> np.ndarray:
    out, inn = w.shape
    y = np.empty(out, np.float32)
    lib().orc_matvec_f32(np.ascontiguousarray(w, np.float32).reshape(-1), np.ascontiguousarray(x, np.float32),
                         y, out, inn)
    return y


def rmsnorm(x, w, eps) -> np.ndarray:
    out = np.empty(x.size, np.float32)
    lib().orc_rmsnorm(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32), eps, out, x.size)
    return out


def softmax(x) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    lib().orc_softmax(y, y.size)
    return y


def norm_head(v, w, eps) -> np.ndarray:
    y = np.array(v, dtype=np.float32, copy=True)
    lib().orc_norm_head(y, np.ascontiguousarray(w, np.float32), eps, y.size)
    return y


def rope_table(head_dim: int, max_pos: int, theta: float):
    c = np.empty(max_pos * (head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_table(head_dim, max_pos, theta, c, s)
    return c.reshape(max_pos, head_dim // 2), s.reshape(max_pos, head_dim // 2)


def rope_apply(cos_t, sin_t, v, pos) -> np.ndarray:
    y = np.array(v, dtype=np.float32, copy=True)
    lib().orc_rope_apply(np.ascontiguousarray(cos_t, np.float32).reshape(-1),
                         np.ascontiguousarray(sin_t, np.float32).reshape(-1), y.size, y, pos)
    return y


def argmax(logits) -> int:
    a = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_argmax(a, a.size))


def route(logits, bias, top_k: int, gating_sigmoid: bool = True, weights_norm: bool = False):
    ne = logits.size
    idx = np.empty(top_k, np.uint32)
    w = np.empty(top_k, np.float32)
    gap = C.c_float()
    _check(lib().orc_route(np.ascontiguousarray(logits, np.float32), np.ascontiguousarray(bias, np.float32),
                           ne, top_k, int(gating_sigmoid), int(weights_norm), idx, w, C.byref(gap)))
    return idx, w, float(gap.value)


def attention_decode(q, k, v, q_norm, k_norm, cos_t, sin_t, eps, n_heads, n_kv, hd, pos, kcache, vcache):
    """One decode-attention layer; updates kcache/vcache in place, returns (out, q_rot, k_rot)."""
    q = np.array(q, np.float32, copy=True)
    k = np.array(k, np.float32, copy=True)
    out = np.empty(n_heads * hd, np.float32)
    lib().orc_attention_decode(q, k, np.ascontiguousarray(v, np.float32), np.ascontiguousarray(q_norm, np.float32),
                               np.ascontiguousarray(k_norm, np.float32),
                               np.ascontiguousarray(cos_t, np.float32).reshape(-1),
                               np.ascontiguousarray(sin_t, np.float32).reshape(-1), eps, n_heads, n_kv, hd,
                               pos, kcache.reshape(-1), vcache.reshape(-1), out)
    return out, q, k


# ---- model level ----
class Model:
    """Model::load / forward / prefill of the CPU restatement."""

    def __init__(self, path: str, quant: bool = True):
        h = C.c_void_p()
        _check(lib().orc_model_load(path.encode(), 1 if quant else 0, C.byref(h)))
        self.h = h
        cfg = OrcConfig()
        lib().orc_model_config(h, C.byref(cfg))
        self.cfg = cfg

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weight_bytes(self) -> int:
        return int(lib().orc_weight_bytes(self.h))

    def new_cache(self) -> "KvCache":
        return KvCache(self)

    def token_embedding(self, tok: int) -> np.ndarray:
        out = np.empty(self.cfg.d_model, np.float32)
        _check(lib().orc_token_embedding(self.h, tok, out))
        return out

    def forward(self, tok: int, pos: int, cache: "KvCache") -> np.ndarray:
        lg = np.empty(self.cfg.vocab_size, np.float32)
        _check(lib().orc_forward(self.h, cache.h, tok, pos, lg))
        return lg

    def forward_x(self, x: np.ndarray, pos: int, cache: "KvCache") -> np.ndarray:
        lg = np.empty(self.cfg.vocab_size, np.float32)
        _check(lib().orc_forward_x(self.h, cache.h, np.ascontiguousarray(x, np.float32), pos, lg))
        return lg

    def prefill(self, inputs: np.ndarray, cache: "KvCache") -> np.ndarray:
        inputs = np.ascontiguousarray(inputs, np.float32)
        lg = np.empty(self.cfg.vocab_size, np.float32)
        _check(lib().orc_prefill(self.h, cache.h, inputs.reshape(-1), inputs.shape[0], lg))
        return lg

    def generate(self, prompt, max_new: int, cache: "KvCache", temp: float = 0.0, top_p: float = 0.95,
                 seed: int = 1234, rep_penalty: float = 1.0, eos: int = 50256) -> np.ndarray:
        """Engine::generate (lib.rs:107-162) with GenOpts {max_new, temp, top_p, seed, rep_penalty}."""
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = C.c_uint32()
        _check(lib().orc_generate(self.h, cache.h, p, p.size, max_new, temp, top_p, seed, rep_penalty, eos, out,
                                  C.byref(n)))
        return out[: n.value].copy()

    def run_block(self, block: np.ndarray, cache: "KvCache", base: int, want_kv: bool = False):
        """Model::run_block (model.rs:471-585): (logits [b][V], bk, bv [L][b][kv_dim] or None)."""
        c = self.cfg
        blk = np.ascontiguousarray(block, np.float32)
        b = blk.shape[0]
        lg = np.empty((b, c.vocab_size), np.float32)
        kvd = c.n_kv_heads * c.head_dim
        bk = np.empty((c.n_layers, b, kvd), np.float32) if want_kv else None
        bv = np.empty((c.n_layers, b, kvd), np.float32) if want_kv else None
        p = lambda a: a.ctypes.data_as(C.c_void_p) if a is not None else None
        _check(lib().orc_run_block(self.h, cache.h, blk.reshape(-1), b, base, p(lg), p(bk), p(bv)))
        return lg, bk, bv

    def forward_bidir(self, inputs: np.ndarray) -> np.ndarray:
        """Model::forward_bidir (model.rs:443-468): logits [tn][V]."""
        x = np.ascontiguousarray(inputs, np.float32)
        lg = np.empty((x.shape[0], self.cfg.vocab_size), np.float32)
        _check(lib().orc_forward_bidir(self.h, x.reshape(-1), x.shape[0], lg.reshape(-1)))
        return lg

    def generate_diffusion(self, prompt, opts: "DiffOpts", eos: int = 50256) -> np.ndarray:
        """Engine::generate_diffusion (lib.rs:214-495) over ids."""
        pr = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(opts.gen_len, 1), np.uint32)
        n = C.c_uint32()
        _check(lib().orc_generate_diffusion(self.h, pr, pr.size, C.cast(C.pointer(opts), C.c_void_p), eos, out,
                                            C.byref(n)))
        return out[: n.value].copy()

    def generate_greedy(self, prompt, max_new: int, cache: "KvCache", rep_penalty: float = 1.0,
                        eos: int = 50256) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = C.c_uint32()
        _check(lib().orc_generate_greedy(self.h, cache.h, p, p.size, max_new, rep_penalty, eos, out, C.byref(n)))
        return out[: n.value].copy()


class KvCache:
    def __init__(self, model: Model):
        self.model = model
        h = C.c_void_p()
        _check(lib().orc_kv_new(model.h, C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().orc_kv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def len(self) -> int:
        return int(lib().orc_kv_len(self.h))

    def read(self, layer: int):
        c = self.model.cfg
        kvd = c.n_kv_heads * c.head_dim
        k = np.empty((self.len, kvd), np.float32)
        v = np.empty((self.len, kvd), np.float32)
        _check(lib().orc_kv_read(self.h, layer, k.reshape(-1), v.reshape(-1)))
        return k, v

    def load(self, k: np.ndarray, v: np.ndarray):
        """k, v: [L, len, kv_dim]"""
        _check(lib().orc_kv_load(self.h, k.shape[1], np.ascontiguousarray(k, np.float32).reshape(-1),
                                 np.ascontiguousarray(v, np.float32).reshape(-1)))

    def routing(self):
        c = self.model.cfg
        idx = np.empty(c.n_layers * c.top_k, np.uint32)
        w = np.empty(c.n_layers * c.top_k, np.float32)
        gap = np.empty(c.n_layers, np.float32)
        lib().orc_last_routing(self.h, idx, w, gap)
        return idx.reshape(c.n_layers, c.top_k), w.reshape(c.n_layers, c.top_k), gap
