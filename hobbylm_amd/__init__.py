"""hobbylm_amd -- MI355X (gfx950) backend for hobby-rs's single-sequence decode step.

Python mirror of the hobby-rs engine API (hobby-rs/src/lib.rs, model.rs, quant.rs) over the
C ABI of include/hobby_gpu.h (libhobby_gpu.so, built in-tree by hobbylm_amd/build.py):

    Engine.load(path, quant)          lib.rs:85-92
    Engine.weight_bytes()             lib.rs:100-102
    Engine.generate_greedy(...)       lib.rs:107-162 at temp 0, over token ids
    Model.forward(token, pos, cache)  model.rs:152-156
    Model.forward_x(x, pos, cache)    model.rs:160-184
    Model.prefill(inputs, cache)      model.rs:340-370
    Model.token_embedding(id)         model.rs:332-335
    KvCache(model) / .len             model.rs:60-75
    Q8Tensor.quantize / .matvec / .matmul   quant.rs:78-194

There is no CPU fallback: every call goes to the HIP library, and importing the module
raises if libhobby_gpu.so has not been built.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhobby_gpu.so")

HG_OK = 0
HG_KV_FAST = 1
GPT2_VALID = 50257

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_vp = C.c_void_p


class GenOpts(C.Structure):
    """hg_gen_opts: GenOpts (lib.rs:29-41)."""
    _fields_ = [("max_new", C.c_uint32), ("temp", C.c_float), ("top_p", C.c_float), ("seed", C.c_uint64),
                ("rep_penalty", C.c_float)]


class DiffOpts(C.Structure):
    """hg_diff_opts: DiffOpts (lib.rs:45-65); defaults as DiffOpts::default (lib.rs:59-64)."""
    _fields_ = [("gen_len", C.c_uint32), ("block", C.c_uint32), ("steps", C.c_uint32), ("temp", C.c_float),
                ("rep_penalty", C.c_float), ("remask_steps", C.c_uint32), ("remask_frac", C.c_float),
                ("seed", C.c_uint64), ("cached", C.c_uint32), ("threshold", C.c_float)]

    @classmethod
    def make(cls, gen_len=128, block=32, steps=32, temp=0.0, rep_penalty=1.4, remask_steps=0, remask_frac=0.3,
             seed=1234, cached=True, threshold=0.0):
        return cls(gen_len, block, steps, temp, rep_penalty, remask_steps, remask_frac, seed, int(cached), threshold)


class HgConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "d_model", "n_layers", "n_dense", "n_heads", "n_kv_heads", "head_dim", "dense_ffn",
        "expert_ffn", "n_experts", "top_k", "n_shared", "vocab_size", "context_length")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("expert_weights_scale", C.c_float),
        ("expert_weights_norm", C.c_int32), ("gating_sigmoid", C.c_int32), ("mask_token_id", C.c_uint32)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


# name -> (restype, argtypes); the complete export list of include/hobby_gpu.h
SIGNATURES = {
    "hg_last_error": (C.c_char_p, []),
    "hg_model_load": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(_vp)]),
    "hg_model_free": (None, [_vp]),
    "hg_gguf_load_tensor": (C.c_int, [C.c_char_p, C.c_char_p, _vp, C.c_uint64, C.POINTER(C.c_uint64)]),
    "hg_model_config": (C.c_int, [_vp, C.POINTER(HgConfig)]),
    "hg_weight_bytes": (C.c_uint64, [_vp]),
    "hg_device_weight_bytes": (C.c_uint64, [_vp]),
    "hg_token_embedding": (C.c_int, [_vp, C.c_uint32, _f32p]),
    "hg_kv_new": (C.c_int, [_vp, C.c_uint32, C.c_uint32, C.POINTER(_vp)]),
    "hg_kv_free": (None, [_vp]),
    "hg_kv_len": (C.c_uint32, [_vp]),
    "hg_kv_truncate": (C.c_int, [_vp, C.c_uint32]),
    "hg_kv_read": (C.c_int, [_vp, C.c_uint32, _f32p, _f32p]),
    "hg_kv_load": (C.c_int, [_vp, C.c_uint32, _f32p, _f32p]),
    "hg_forward": (C.c_int, [_vp, _vp, C.c_uint32, C.c_uint32, _vp, C.POINTER(C.c_uint32)]),
    "hg_forward_x": (C.c_int, [_vp, _vp, _f32p, C.c_uint32, _vp, C.POINTER(C.c_uint32)]),
    "hg_prefill": (C.c_int, [_vp, _vp, _f32p, C.c_uint32, _vp, C.POINTER(C.c_uint32)]),
    "hg_decode_greedy": (C.c_int, [_vp, _vp, C.c_uint32, C.c_uint32, _u32p]),
    "hg_generate_greedy": (C.c_int, [_vp, _vp, _u32p, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32,
                                     _u32p, C.POINTER(C.c_uint32)]),
    "hg_generate": (C.c_int, [_vp, _vp, _u32p, C.c_uint32, _vp, C.c_uint32, _u32p, C.POINTER(C.c_uint32)]),
    "hg_sample": (C.c_int, [_f32p, C.c_uint32, C.c_float, C.c_float, C.POINTER(C.c_uint64),
                            C.POINTER(C.c_uint32)]),
    "hg_run_block": (C.c_int, [_vp, _vp, _f32p, C.c_uint32, C.c_uint32, C.c_int, _vp, _vp, _vp]),
    "hg_forward_bidir": (C.c_int, [_vp, _f32p, C.c_uint32, _f32p]),
    "hg_generate_diffusion": (C.c_int, [_vp, _u32p, C.c_uint32, _vp, C.c_uint32, _u32p, C.POINTER(C.c_uint32)]),
    "hg_last_routing": (C.c_int, [_vp, _u32p, _f32p]),
    "hg_seq_sum": (C.c_int, [_f32p, C.c_uint32, C.c_uint32, _f32p]),
    "hg_profile_step": (C.c_int, [_vp, _vp, C.c_uint32, C.c_uint32, _f32p, _u32p]),
    "hg_profile_class": (C.c_char_p, [C.c_uint32]),
    "hg_q8_tensor_quantize": (C.c_int, [_f32p, C.c_uint32, C.c_uint32, C.POINTER(_vp)]),
    "hg_q8_tensor_from_q8_0": (C.c_int, [_u8p, C.c_uint32, C.c_uint32, C.POINTER(_vp)]),
    "hg_q8_tensor_free": (None, [_vp]),
    "hg_q8_tensor_bytes": (C.c_uint64, [_vp]),
    "hg_q8_tensor_matvec": (C.c_int, [_vp, _f32p, _f32p]),
    "hg_q8_tensor_matmul": (C.c_int, [_vp, _f32p, _f32p, C.c_uint32]),
    "hg_q8_tensor_matvec_noalloc": (C.c_int, [_vp, _vp, _vp, _vp]),
    "hg_q8_tensor_matvec_gather": (C.c_int, [_vp, C.c_uint32, _u32p, C.c_uint32, _f32p, _f32p]),
    "hg_attention_decode": (C.c_int, [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_float, C.c_float, C.c_uint32,
                                      C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _f32p, _f32p, _f32p,
                                      C.c_uint32]),
    "hg_batch_new": (C.c_int, [_vp, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(_vp)]),
    "hg_batch_free": (None, [_vp]),
    "hg_batch_set_pages": (C.c_int, [_vp, C.c_uint32, _u32p, C.c_uint32]),
    "hg_batch_len": (C.c_uint32, [_vp, C.c_uint32]),
    "hg_batch_load": (C.c_int, [_vp, C.c_uint32, C.c_uint32, _f32p, _f32p]),
    "hg_batch_read": (C.c_int, [_vp, C.c_uint32, C.c_uint32, _f32p, _f32p]),
    "hg_batch_fill": (C.c_int, [_vp, C.c_uint32, C.c_uint32, C.c_uint64]),
    "hg_batch_forward": (C.c_int, [_vp, _vp, _u32p, C.c_uint32, _vp, _vp]),
    "hg_batch_decode_greedy": (C.c_int, [_vp, _vp, _u32p, C.c_uint32, C.c_uint32, _u32p]),
    "hg_batch_routing": (C.c_int, [_vp, C.c_uint32, _u32p, _f32p]),
    "hg_q8_tensor_time_matvec": (C.c_int, [_vp, _f32p, C.c_uint32, C.c_uint32, C.c_uint32, _vp, C.c_uint32, _f32p]),
    "hg_attention_time": (C.c_int, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                    _f32p]),
}

_lib = None


def lib():
    """The loaded libhobby_gpu.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m hobbylm_amd.build` "
                              "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class HgError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def _check(rc: int):
    if rc != HG_OK:
        raise HgError(rc, lib().hg_last_error().decode())


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Model:
    """A loaded hobbylm model resident on the GPU (Model::load, model.rs:79-131)."""

    def __init__(self, path: str, quant: bool = True):
        h = _vp()
        _check(lib().hg_model_load(str(path).encode(), 1 if quant else 0, C.byref(h)))
        self.h = h
        cfg = HgConfig()
        _check(lib().hg_model_config(h, C.byref(cfg)))
        self.cfg = cfg

    def close(self):
        if getattr(self, "h", None):
            lib().hg_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weight_bytes(self) -> int:
        return int(lib().hg_weight_bytes(self.h))

    def device_weight_bytes(self) -> int:
        return int(lib().hg_device_weight_bytes(self.h))

    def new_cache(self, max_ctx: int = 0, fast: bool = False) -> "KvCache":
        return KvCache(self, max_ctx, fast)

    def token_embedding(self, tok: int) -> np.ndarray:
        out = np.empty(self.cfg.d_model, np.float32)
        _check(lib().hg_token_embedding(self.h, tok, out))
        return out

    def forward(self, tok: int, pos: int, cache: "KvCache", want_logits: bool = True):
        """Returns (logits or None, greedy next token)."""
        lg = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        nxt = C.c_uint32()
        _check(lib().hg_forward(self.h, cache.h, tok, pos, _ptr(lg), C.byref(nxt)))
        return lg, int(nxt.value)

    def forward_x(self, x: np.ndarray, pos: int, cache: "KvCache", want_logits: bool = True):
        lg = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        nxt = C.c_uint32()
        _check(lib().hg_forward_x(self.h, cache.h, np.ascontiguousarray(x, np.float32), pos, _ptr(lg),
                                  C.byref(nxt)))
        return lg, int(nxt.value)

    def prefill(self, inputs: np.ndarray, cache: "KvCache", want_logits: bool = True):
        inputs = np.ascontiguousarray(inputs, np.float32)
        lg = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        nxt = C.c_uint32()
        _check(lib().hg_prefill(self.h, cache.h, inputs.reshape(-1), inputs.shape[0], _ptr(lg), C.byref(nxt)))
        return lg, int(nxt.value)

    def decode_greedy(self, first_token: int, n_steps: int, cache: "KvCache") -> np.ndarray:
        out = np.empty(max(n_steps, 1), np.uint32)
        _check(lib().hg_decode_greedy(self.h, cache.h, first_token, n_steps, out))
        return out[:n_steps]

    def profile_step(self, token: int, cache: "KvCache", reps: int = 10) -> dict:
        """Per-kernel-class microseconds of one decode step at pos = cache.len (HIP events on the
        cache's stream); returns {class: (us_per_step, launches_per_step)}."""
        n = 12
        us = np.zeros(n, np.float32)
        cnt = np.zeros(n, np.uint32)
        _check(lib().hg_profile_step(self.h, cache.h, token, reps, us, cnt))
        return {lib().hg_profile_class(c).decode(): (float(us[c]), int(cnt[c])) for c in range(n) if cnt[c]}

    def generate(self, prompt, max_new: int, cache: "KvCache", temp: float = 0.0, top_p: float = 0.95,
                 seed: int = 1234, rep_penalty: float = 1.0, eos: int = 50256) -> np.ndarray:
        """Engine::generate (lib.rs:107-162) with GenOpts {max_new, temp, top_p, seed, rep_penalty},
        sampling on the device."""
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = C.c_uint32()
        opts = GenOpts(max_new, temp, top_p, seed, rep_penalty)
        _check(lib().hg_generate(self.h, cache.h, p, p.size, C.cast(C.pointer(opts), _vp), eos, out, C.byref(n)))
        return out[: n.value].copy()

    def run_block(self, block: np.ndarray, cache: "KvCache", base: int, append: bool = False,
                  want_kv: bool = False):
        """Model::run_block (model.rs:471-585): (logits [b][V], bk, bv [L][b][kv_dim] or None)."""
        c = self.cfg
        blk = np.ascontiguousarray(block, np.float32)
        b = blk.shape[0]
        lg = np.empty((b, c.vocab_size), np.float32)
        kvd = c.n_kv_heads * c.head_dim
        bk = np.empty((c.n_layers, b, kvd), np.float32) if want_kv else None
        bv = np.empty((c.n_layers, b, kvd), np.float32) if want_kv else None
        p = lambda a: a.ctypes.data_as(_vp) if a is not None else None
        _check(lib().hg_run_block(self.h, cache.h, blk.reshape(-1), b, base, int(append), p(lg), p(bk), p(bv)))
        return lg, bk, bv

    def forward_bidir(self, inputs: np.ndarray) -> np.ndarray:
        """Model::forward_bidir (model.rs:443-468): logits [tn][V]."""
        x = np.ascontiguousarray(inputs, np.float32)
        lg = np.empty((x.shape[0], self.cfg.vocab_size), np.float32)
        _check(lib().hg_forward_bidir(self.h, x.reshape(-1), x.shape[0], lg.reshape(-1)))
        return lg

    def generate_diffusion(self, prompt, opts: DiffOpts, eos: int = 50256) -> np.ndarray:
        """Engine::generate_diffusion (lib.rs:214-495) over ids, scored on the device."""
        pr = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(opts.gen_len, 1), np.uint32)
        n = C.c_uint32()
        _check(lib().hg_generate_diffusion(self.h, pr, pr.size, C.cast(C.pointer(opts), _vp), eos, out, C.byref(n)))
        return out[: n.value].copy()

    def generate_greedy(self, prompt, max_new: int, cache: "KvCache", rep_penalty: float = 1.0,
                        eos: int = 50256) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = C.c_uint32()
        _check(lib().hg_generate_greedy(self.h, cache.h, p, p.size, max_new, rep_penalty, eos, out, C.byref(n)))
        return out[: n.value].copy()


class KvCache:
    """Device KV cache (KvCache, model.rs:60-75).  fast=True reassociates the RMSNorm and
    attention sums as trees (not bit-identical to the reference; routing may differ)."""

    def __init__(self, model: Model, max_ctx: int = 0, fast: bool = False):
        self.model = model
        h = _vp()
        _check(lib().hg_kv_new(model.h, max_ctx, HG_KV_FAST if fast else 0, C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().hg_kv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def len(self) -> int:
        return int(lib().hg_kv_len(self.h))

    def truncate(self, length: int):
        """cache.len = length (model.rs:63): decode continues from `length`."""
        _check(lib().hg_kv_truncate(self.h, length))

    def read(self, layer: int):
        c = self.model.cfg
        kvd = c.n_kv_heads * c.head_dim
        k = np.empty((self.len, kvd), np.float32)
        v = np.empty((self.len, kvd), np.float32)
        _check(lib().hg_kv_read(self.h, layer, k.reshape(-1), v.reshape(-1)))
        return k, v

    def load(self, k: np.ndarray, v: np.ndarray):
        """KvCache.k / .v / .len = (k, v, k.shape[1]) (model.rs:60-64); k, v [n_layers][len][kv_dim]."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        assert k.shape == v.shape and k.shape[0] == self.model.cfg.n_layers
        _check(lib().hg_kv_load(self.h, k.shape[1], k.reshape(-1), v.reshape(-1)))

    def routing(self):
        c = self.model.cfg
        idx = np.empty(c.n_layers * c.top_k, np.uint32)
        w = np.empty(c.n_layers * c.top_k, np.float32)
        _check(lib().hg_last_routing(self.h, idx, w))
        return idx.reshape(c.n_layers, c.top_k), w.reshape(c.n_layers, c.top_k)


class Batch:
    """Batched decode of many sequences over a paged KV cache (hg_batch_*): each sequence's
    step is Model::forward on its own cache (model.rs:152-184), bit-identical to hg_forward."""

    PAGE = 16

    def __init__(self, model: Model, max_seqs: int, max_ctx: int = 0, n_pages: int = 0):
        self.model = model
        c = model.cfg
        self.max_ctx = max_ctx or c.context_length
        self.n_pages = n_pages or max_seqs * -(-self.max_ctx // self.PAGE)
        h = _vp()
        _check(lib().hg_batch_new(model.h, max_seqs, max_ctx, self.n_pages, C.byref(h)))
        self.h = h
        self.max_seqs = max_seqs

    def close(self):
        if getattr(self, "h", None):
            lib().hg_batch_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_pages(self, seq: int, pages):
        p = np.ascontiguousarray(pages, np.uint32)
        _check(lib().hg_batch_set_pages(self.h, seq, p, p.size))

    def len(self, seq: int) -> int:
        return int(lib().hg_batch_len(self.h, seq))

    def load(self, seq: int, k: np.ndarray, v: np.ndarray):
        """Sequence seq's KvCache.k / .v / .len = (k, v, k.shape[1]); k, v [n_layers][len][kv_dim]."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        _check(lib().hg_batch_load(self.h, seq, k.shape[1], k.reshape(-1), v.reshape(-1)))

    def fill(self, seq: int, length: int, seed: int):
        """Seeded pseudo-random cache rows [0, length) on the device (timing workloads)."""
        _check(lib().hg_batch_fill(self.h, seq, length, seed))

    def read(self, seq: int, layer: int):
        c = self.model.cfg
        kvd = c.n_kv_heads * c.head_dim
        n = self.len(seq)
        k = np.empty((n, kvd), np.float32)
        v = np.empty((n, kvd), np.float32)
        _check(lib().hg_batch_read(self.h, seq, layer, k.reshape(-1), v.reshape(-1)))
        return k, v

    def forward(self, tokens, want_logits: bool = True):
        """One step of sequences 0..len(tokens)-1: (logits [n][vocab] or None, next tokens [n])."""
        t = np.ascontiguousarray(tokens, np.uint32)
        n = t.size
        lg = np.empty((n, self.model.cfg.vocab_size), np.float32) if want_logits else None
        nxt = np.empty(n, np.uint32)
        _check(lib().hg_batch_forward(self.model.h, self.h, t, n, _ptr(lg), _ptr(nxt)))
        return lg, nxt

    def decode_greedy(self, first, n_steps: int) -> np.ndarray:
        f = np.ascontiguousarray(first, np.uint32)
        out = np.empty((max(n_steps, 1), f.size), np.uint32)
        _check(lib().hg_batch_decode_greedy(self.model.h, self.h, f, f.size, n_steps, out.reshape(-1)))
        return out[:n_steps]

    def routing(self, seq: int):
        c = self.model.cfg
        idx = np.empty(c.n_layers * c.top_k, np.uint32)
        w = np.empty(c.n_layers * c.top_k, np.float32)
        _check(lib().hg_batch_routing(self.h, seq, idx, w))
        return idx.reshape(c.n_layers, c.top_k), w.reshape(c.n_layers, c.top_k)


class Engine(Model):
    """Engine::load (lib.rs:85-92): the model without the tokenizer (token ids cross the boundary)."""

    @classmethod
    def load(cls, path: str, quant: bool = True) -> "Engine":
        return cls(path, quant)


class Q8Tensor:
    """Q8Tensor (quant.rs:69-194) resident on the GPU."""

    def __init__(self, h, out: int, inn: int):
        self.h, self.out, self.inn = h, out, inn

    @classmethod
    def quantize(cls, w: np.ndarray) -> "Q8Tensor":
        out, inn = w.shape
        h = _vp()
        _check(lib().hg_q8_tensor_quantize(np.ascontiguousarray(w, np.float32).reshape(-1), out, inn, C.byref(h)))
        return cls(h, out, inn)

    @classmethod
    def from_q8_0(cls, blocks: np.ndarray, out: int, inn: int) -> "Q8Tensor":
        h = _vp()
        _check(lib().hg_q8_tensor_from_q8_0(np.ascontiguousarray(blocks).view(np.uint8).reshape(-1), out, inn,
                                            C.byref(h)))
        return cls(h, out, inn)

    def close(self):
        if getattr(self, "h", None):
            lib().hg_q8_tensor_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def bytes(self) -> int:
        return int(lib().hg_q8_tensor_bytes(self.h))

    def matvec(self, x: np.ndarray) -> np.ndarray:
        y = np.empty(self.out, np.float32)
        _check(lib().hg_q8_tensor_matvec(self.h, np.ascontiguousarray(x, np.float32), y))
        return y

    def time_matvec(self, x: np.ndarray, reps: int = 100, copies: int = 1, rows_per_mat: int = 0,
                    ids=None) -> float:
        """Mean kernel microseconds of a device-resident matvec (or gather over `ids`), rotating
        through `copies` replicas of the weights (measurement only)."""
        us = np.zeros(1, np.float32)
        if ids is None:
            _check(lib().hg_q8_tensor_time_matvec(self.h, np.ascontiguousarray(x, np.float32), reps, copies, 0,
                                                  None, 0, us))
        else:
            idv = np.ascontiguousarray(ids, np.uint32)
            _check(lib().hg_q8_tensor_time_matvec(self.h, np.ascontiguousarray(x, np.float32), reps, copies,
                                                  rows_per_mat, idv.ctypes.data_as(_vp), len(idv), us))
        return float(us[0])

    def matvec_noalloc(self, x_dev_ptr: int, y_dev_ptr: int, stream: int = 0):
        """The allocation-free matvec on device pointers (x[in] -> y[out]) enqueued on a
        hipStream_t handle; the caller synchronizes."""
        _check(lib().hg_q8_tensor_matvec_noalloc(self.h, _vp(x_dev_ptr), _vp(y_dev_ptr), _vp(stream or None)))

    def matmul(self, x: np.ndarray) -> np.ndarray:
        tn = x.shape[0]
        y = np.empty((tn, self.out), np.float32)
        _check(lib().hg_q8_tensor_matmul(self.h, np.ascontiguousarray(x, np.float32).reshape(-1), y.reshape(-1), tn))
        return y

    def matvec_gather(self, rows_per_mat: int, ids, x: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.uint32)
        y = np.empty((ids.size, rows_per_mat), np.float32)
        _check(lib().hg_q8_tensor_matvec_gather(self.h, rows_per_mat, ids, ids.size,
                                                np.ascontiguousarray(x, np.float32), y.reshape(-1)))
        return y


def gguf_load_tensor(path: str, name: str) -> np.ndarray:
    """Gguf::load (gguf.rs:250-269) of one tensor as f32 (host work, no device needed)."""
    n = C.c_uint64()
    _check(lib().hg_gguf_load_tensor(str(path).encode(), name.encode(), None, 0, C.byref(n)))
    out = np.empty(n.value, np.float32)
    _check(lib().hg_gguf_load_tensor(str(path).encode(), name.encode(), _ptr(out), out.size, C.byref(n)))
    return out


def sample(logits, temp: float, top_p: float, state: int):
    """sample::sample (sample.rs:66-112) on the device: (pick, the advanced RNG state)."""
    lg = np.ascontiguousarray(logits, np.float32)
    st = C.c_uint64(state)
    out = C.c_uint32()
    _check(lib().hg_sample(lg, lg.size, temp, top_p, C.byref(st), C.byref(out)))
    return int(out.value), int(st.value)


def seq_sum(x, method: int = 1) -> np.float32:
    """((0 + x[0]) + x[1]) + ... in binary32 on the device (the sums of ops.rs:101-104 and
    ops.rs:119-122): method 1 = the workgroup method of the decode kernels, 0 = one lane."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(1, np.float32)
    _check(lib().hg_seq_sum(x, x.size, method, out))
    return out[0]


def attention_time(n_heads: int, n_kv: int, hd: int, ctx: int, reps: int = 50, fast: bool = False):
    """Mean kernel microseconds (scores, softmax + P.V) of one decode-attention layer at
    context ctx on seeded device-resident data (measurement only)."""
    us = np.zeros(2, np.float32)
    _check(lib().hg_attention_time(n_heads, n_kv, hd, ctx, reps, HG_KV_FAST if fast else 0, us))
    return float(us[0]), float(us[1])


def attention_decode(q, k, v, q_norm, k_norm, eps, theta, rope_len, n_heads, n_kv, hd, pos, kcache, vcache,
                     fast=False):
    """One decode-attention layer (model.rs:199-233); kcache/vcache [pos+1][n_kv*hd] are updated in place."""
    out = np.empty(n_heads * hd, np.float32)
    assert kcache.flags["C_CONTIGUOUS"] and vcache.flags["C_CONTIGUOUS"]
    _check(lib().hg_attention_decode(np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k, np.float32),
                                     np.ascontiguousarray(v, np.float32), np.ascontiguousarray(q_norm, np.float32),
                                     np.ascontiguousarray(k_norm, np.float32), eps, theta, rope_len, n_heads, n_kv,
                                     hd, pos, kcache.reshape(-1), vcache.reshape(-1), out,
                                     HG_KV_FAST if fast else 0))
    return out
