"""Seeded random-init `hobbylm` GGUF v3 writer.

Produces the synthetic models the decode path is measured and checked on:
tensor names, metadata keys and layouts follow the HobbyLM exporter
(export/to_gguf.py:59-129), the init recipe follows hobbylm/model.py:288-313
(N(0, 0.02) everywhere, residual projections x (2L)^-1/2, router x 0.1, unit
norm gains), and matrices are stored as GGML Q8_0 blocks ({f16 d; int8 q[32]},
d = amax/127, q = round-half-away(x/d)), the format llama-quantize writes.

Everything is numpy; the same seed gives the same bytes on every machine
with this numpy version.
"""
from __future__ import annotations

import dataclasses
import hashlib
import os
import struct
import zlib
from typing import Dict, Optional

import numpy as np

GENERATOR_VERSION = 1

GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
_T_U32, _T_I32, _T_F32, _T_BOOL, _T_STR, _T_ARR = 4, 5, 6, 7, 8, 9

Q8_BLOCK = np.dtype([("d", "<f2"), ("qs", "i1", (32,))])
assert Q8_BLOCK.itemsize == 34


@dataclasses.dataclass(frozen=True)
class Shape:
    """Model hyperparameters (hobbylm/config.py ModelConfig fields that reach the GGUF)."""
    d_model: int
    n_layers: int
    n_dense: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    dense_ffn: int
    expert_ffn: int
    n_experts: int
    top_k: int
    n_shared: int
    vocab_size: int
    context_length: int = 8192
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    gating_sigmoid: bool = True
    expert_weights_norm: bool = False
    expert_weights_scale: float = 1.0


PRESETS: Dict[str, Shape] = {
    # hobbylm/config.py:120-124 (the 130M preset), theta = ModelConfig default
    "130M": Shape(512, 12, 1, 8, 2, 64, 1536, 192, 32, 8, 0, 50304),
    # the 500M-shaped sparse-MoE decode workload: d1024 / 24 layers / GQA 16q-4kv hd64 /
    # dense 4096 in layer 0 / 36 experts x 512, top-6 + 1 shared / vocab 50257
    "500M": Shape(1024, 24, 1, 16, 4, 64, 4096, 512, 36, 6, 1, 50257),
    # the published joint12 shape (hobby-rs/README.md:9,35): d768 / 16 layers / 12q-3kv hd128 /
    # 36 x 320 top-6 + 1 shared / vocab 50304 / theta 1e6
    "joint12": Shape(768, 16, 1, 12, 3, 128, 2304, 320, 36, 6, 1, 50304, rope_theta=1e6),
    # small shapes that keep every feature (dense layer, routed + shared experts, GQA,
    # a K that is not a multiple of 128) and run in milliseconds on the CPU oracle
    "tiny": Shape(128, 3, 1, 4, 2, 32, 256, 96, 8, 2, 1, 1000, context_length=512),
    "tiny_noshared": Shape(64, 2, 1, 2, 1, 32, 128, 64, 6, 3, 0, 300, context_length=256,
                           rope_theta=1e6),
    # the other router forms: softmax gating with renormalized weights, and sigmoid gating with
    # renormalized and scaled weights
    "tiny_softmax": Shape(128, 2, 1, 4, 2, 32, 256, 96, 8, 2, 1, 1000, context_length=512,
                          gating_sigmoid=False, expert_weights_norm=True),
    "tiny_wnorm": Shape(256, 2, 1, 4, 2, 64, 256, 96, 12, 4, 1, 1000, context_length=512,
                        expert_weights_norm=True, expert_weights_scale=2.5),
}


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """GGML quantize_row_q8_0: d = amax/127 in f32, id = 1/d, q = roundf(x*id), d stored as f16."""
    b = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 32)
    amax = np.max(np.abs(b), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d > 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (b * idv[:, None]).astype(np.float32)
    # roundf (half away from zero), exact: an f32 plus 0.5 is exact in f64
    q = np.sign(v) * np.floor(np.abs(v).astype(np.float64) + 0.5)
    q = np.clip(q, -127, 127).astype(np.int8)
    out = np.empty(b.shape[0], dtype=Q8_BLOCK)
    out["d"] = d.astype(np.float16)
    out["qs"] = q
    return out


def dequantize_q8_0(blocks: np.ndarray) -> np.ndarray:
    """Q8_0 -> f32 (q * d), the closed form of the format."""
    return (blocks["qs"].astype(np.float32) * blocks["d"].astype(np.float32)[:, None]).reshape(-1)


class _Writer:
    def __init__(self, arch: str):
        self.arch = arch
        self.kv = []
        self.tensors = []  # (name, ne list, type, bytes)

    def _kv(self, key, ty, payload: bytes):
        self.kv.append(_gstr(key) + struct.pack("<I", ty) + payload)

    def u32(self, key, v):
        self._kv(key, _T_U32, struct.pack("<I", int(v)))

    def f32(self, key, v):
        self._kv(key, _T_F32, struct.pack("<f", float(v)))

    def bool(self, key, v):
        self._kv(key, _T_BOOL, struct.pack("<B", 1 if v else 0))

    def str(self, key, v):
        self._kv(key, _T_STR, _gstr(v))

    def arr_str(self, key, vals):
        body = b"".join(_gstr(s) for s in vals)
        self._kv(key, _T_ARR, struct.pack("<IQ", _T_STR, len(vals)) + body)

    def arr_i32(self, key, vals):
        a = np.asarray(vals, dtype="<i4")
        self._kv(key, _T_ARR, struct.pack("<IQ", _T_I32, len(a)) + a.tobytes())

    def tensor(self, name, shape, ggml_type, data: bytes):
        # GGUF dims are fastest-varying first: a torch (out, in) weight has ne = [in, out]
        self.tensors.append((name, list(reversed(shape)), ggml_type, data))

    def write(self, path, alignment=32):
        head = struct.pack("<IIQQ", 0x46554747, 3, len(self.tensors), len(self.kv))
        infos, off = [], 0
        offsets = []
        for name, ne, ty, data in self.tensors:
            off = (off + alignment - 1) // alignment * alignment
            offsets.append(off)
            infos.append(_gstr(name) + struct.pack("<I", len(ne)) +
                         b"".join(struct.pack("<Q", n) for n in ne) + struct.pack("<IQ", ty, off))
            off += len(data)
        meta = head + b"".join(self.kv) + b"".join(infos)
        pad = (-len(meta)) % alignment
        tmp = f"{path}.tmp{os.getpid()}"
        with open(tmp, "wb") as f:
            f.write(meta + b"\0" * pad)
            pos = 0
            for (name, ne, ty, data), o in zip(self.tensors, offsets):
                f.write(b"\0" * (o - pos))
                f.write(data)
                pos = o + len(data)
        os.replace(tmp, path)


def _gstr(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def build_gguf(path: str, shape: Shape, seed: int, *, norm_jitter: float = 0.0,
               bias_std: float = 0.01, init_std: float = 0.02) -> str:
    """Write a random-init hobbylm GGUF with Q8_0 matrices and F32 norms/router/bias."""
    s = shape
    w = _Writer("hobbylm")
    a = "hobbylm"
    w.str("general.architecture", a)
    w.str("general.name", f"HobbyLM synthetic (seed {seed})")
    w.u32("general.alignment", 32)
    w.u32(f"{a}.context_length", s.context_length)
    w.u32(f"{a}.embedding_length", s.d_model)
    w.u32(f"{a}.block_count", s.n_layers)
    w.u32(f"{a}.feed_forward_length", s.dense_ffn)
    w.u32(f"{a}.attention.head_count", s.n_heads)
    w.u32(f"{a}.attention.head_count_kv", s.n_kv_heads)
    w.u32(f"{a}.attention.key_length", s.head_dim)
    w.u32(f"{a}.attention.value_length", s.head_dim)
    w.f32(f"{a}.attention.layer_norm_rms_epsilon", s.rms_eps)
    w.f32(f"{a}.rope.freq_base", s.rope_theta)
    w.u32(f"{a}.expert_count", s.n_experts)
    w.u32(f"{a}.expert_used_count", s.top_k)
    w.u32(f"{a}.expert_feed_forward_length", s.expert_ffn)
    w.u32(f"{a}.expert_shared_count", s.n_shared)
    w.u32(f"{a}.expert_shared_feed_forward_length", s.expert_ffn)
    w.u32(f"{a}.leading_dense_block_count", s.n_dense)
    w.u32(f"{a}.expert_gating_func", 2 if s.gating_sigmoid else 1)
    w.bool(f"{a}.expert_weights_norm", s.expert_weights_norm)
    w.f32(f"{a}.expert_weights_scale", s.expert_weights_scale)
    w.u32(f"{a}.vocab_size", s.vocab_size)
    # tokenizer keys (hobby-rs/src/tokenizer.rs:55-61 requires tokens + merges); synthetic strings
    w.str("tokenizer.ggml.model", "gpt2")
    w.arr_str("tokenizer.ggml.tokens", [f"<|t{i}|>" for i in range(s.vocab_size)])
    w.arr_i32("tokenizer.ggml.token_type", [1] * s.vocab_size)
    w.arr_str("tokenizer.ggml.merges", [])
    w.u32("tokenizer.ggml.bos_token_id", 50256)
    w.u32("tokenizer.ggml.eos_token_id", 50256)

    resid = (2 * s.n_layers) ** -0.5
    q_dim, kv_dim = s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim

    def normal(name, shp, std):
        return (_rng(seed, name).standard_normal(int(np.prod(shp)), dtype=np.float32)
                * np.float32(std)).reshape(shp)

    def q8(name, shp, std):
        w.tensor(name, shp, GGML_Q8_0, quantize_q8_0(normal(name, shp, std)).tobytes())

    def f32(name, arr):
        w.tensor(name, arr.shape, GGML_F32, np.ascontiguousarray(arr, dtype="<f4").tobytes())

    def gain(name, n):
        if norm_jitter:
            return np.float32(1.0) + normal(name, (n,), norm_jitter)
        return np.ones(n, dtype=np.float32)

    emb = quantize_q8_0(normal("token_embd.weight", (s.vocab_size, s.d_model), init_std)).tobytes()
    w.tensor("token_embd.weight", (s.vocab_size, s.d_model), GGML_Q8_0, emb)
    f32("output_norm.weight", gain("output_norm.weight", s.d_model))
    w.tensor("output.weight", (s.vocab_size, s.d_model), GGML_Q8_0, emb)  # tied embeddings
    for i in range(s.n_layers):
        p = f"blk.{i}."
        f32(p + "attn_norm.weight", gain(p + "attn_norm.weight", s.d_model))
        q8(p + "attn_qkv.weight", (q_dim + 2 * kv_dim, s.d_model), init_std)
        f32(p + "attn_q_norm.weight", gain(p + "attn_q_norm.weight", s.head_dim))
        f32(p + "attn_k_norm.weight", gain(p + "attn_k_norm.weight", s.head_dim))
        q8(p + "attn_output.weight", (s.d_model, q_dim), init_std * resid)
        f32(p + "ffn_norm.weight", gain(p + "ffn_norm.weight", s.d_model))
        if i < s.n_dense:
            q8(p + "ffn_gate.weight", (s.dense_ffn, s.d_model), init_std)
            q8(p + "ffn_up.weight", (s.dense_ffn, s.d_model), init_std)
            q8(p + "ffn_down.weight", (s.d_model, s.dense_ffn), init_std * resid)
        else:
            f32(p + "ffn_gate_inp.weight", normal(p + "ffn_gate_inp.weight",
                                                  (s.n_experts, s.d_model), init_std * 0.1))
            f32(p + "exp_probs_b.bias", normal(p + "exp_probs_b.bias", (s.n_experts,), bias_std))
            q8(p + "ffn_gate_exps.weight", (s.n_experts, s.expert_ffn, s.d_model), init_std)
            q8(p + "ffn_up_exps.weight", (s.n_experts, s.expert_ffn, s.d_model), init_std)
            q8(p + "ffn_down_exps.weight", (s.n_experts, s.d_model, s.expert_ffn), init_std * resid)
            if s.n_shared > 0:
                q8(p + "ffn_gate_shexp.weight", (s.expert_ffn, s.d_model), init_std)
                q8(p + "ffn_up_shexp.weight", (s.expert_ffn, s.d_model), init_std)
                q8(p + "ffn_down_shexp.weight", (s.d_model, s.expert_ffn), init_std * resid)
            else:
                # hobby-rs loads the shared-expert tensors unconditionally (model.rs:99-101)
                # and skips them when expert_shared_count is 0 (model.rs:313)
                for nm, shp in (("ffn_gate_shexp.weight", (s.expert_ffn, s.d_model)),
                                ("ffn_up_shexp.weight", (s.expert_ffn, s.d_model)),
                                ("ffn_down_shexp.weight", (s.d_model, s.expert_ffn))):
                    q8(p + nm, shp, init_std)
    w.write(path)
    return path


def cache_dir() -> str:
    d = os.environ.get("HOBBYLM_GGUF_CACHE") or os.path.join(
        os.environ.get("TMPDIR", "/tmp"), "hobbylm_gguf")
    os.makedirs(d, exist_ok=True)
    return d


def synth_path(preset: str, seed: int, *, norm_jitter: float = 0.0,
               directory: Optional[str] = None) -> str:
    """Path of the cached synthetic GGUF for (preset, seed), written on first use."""
    tag = f"{preset}_s{seed}" + (f"_j{norm_jitter:g}" if norm_jitter else "") + f"_v{GENERATOR_VERSION}"
    path = os.path.join(directory or cache_dir(), tag + ".gguf")
    if not os.path.exists(path):
        build_gguf(path, PRESETS[preset], seed, norm_jitter=norm_jitter)
    return path


def file_sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


def prompt_ids(seed: int, n: int = 16, high: int = 50257) -> np.ndarray:
    """Seeded prompt of n token ids drawn uniformly from [0, high)."""
    return np.random.default_rng(seed).integers(0, high, size=n, dtype=np.int64).astype(np.uint32)
