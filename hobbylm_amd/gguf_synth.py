"""Seeded random-init `hobbylm` GGUF v3 writer.

Produces the synthetic models the decode path is measured and checked on:
tensor names, metadata keys and layouts follow the HobbyLM exporter
(export/to_gguf.py:59-129), the init recipe follows hobbylm/model.py:288-313
(N(0, 0.02) everywhere, residual projections x (2L)^-1/2, router x 0.1, unit
norm gains), and matrices are stored as GGML Q8_0 blocks ({f16 d; int8 q[32]},
d = amax/127, q = round-half-away(x/d)), the format llama-quantize writes, or, with
qtype="kquant", as the K-quant / 5-bit mix of a Q4_K_M-style file (Q4_K, Q6_K, Q5_0), whose
block layouts follow ggml's published quantizers (the decoders are gguf.rs:377-468).

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

GGML_F32, GGML_F16, GGML_Q5_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 6, 8, 12, 14
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
    # the 500M shape with room for the batched-decode workload's contexts (up to 16384 + the
    # decoded steps); the same tensors as "500M" for the same seed
    "500M_long": Shape(1024, 24, 1, 16, 4, 64, 4096, 512, 36, 6, 1, 50257, context_length=16896),
    # small shapes that keep every feature (dense layer, routed + shared experts, GQA,
    # a K that is not a multiple of 128) and run in milliseconds on the CPU oracle
    "tiny": Shape(128, 3, 1, 4, 2, 32, 256, 96, 8, 2, 1, 1000, context_length=512),
    # the tiny shape with the GPT-2 vocabulary padded to 50304: the diffusion [MASK] id 50257
    # (config.rs:93's default) is a real row, and ids >= 50257 are masked out of every draw
    "tiny_diff": Shape(128, 3, 1, 4, 2, 32, 256, 96, 8, 2, 1, 50304, context_length=512),
    # the tiny shape with room for prompts of thousands of rows
    "tiny_long": Shape(128, 3, 1, 4, 2, 32, 256, 96, 8, 2, 1, 1000, context_length=4096),
    "tiny_noshared": Shape(64, 2, 1, 2, 1, 32, 128, 64, 6, 3, 0, 300, context_length=256,
                           rope_theta=1e6),
    # one routed expert and no shared one: the decode step's rank-order and the prompt path's
    # expert-id-order accumulations coincide
    "tiny_top1": Shape(64, 2, 1, 2, 1, 32, 128, 64, 6, 1, 0, 300, context_length=256),
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


def _round_away(v):
    return np.sign(v) * np.floor(np.abs(np.asarray(v, np.float64)) + 0.5)


# ---- block packers: logical values -> ggml block bytes (the inverse of the decoders) ----
def pack_q5_0(d: np.ndarray, q: np.ndarray) -> bytes:
    """Q5_0 blocks {f16 d; u32 qh; u8 qs[16]} from f16 scales d[nb] and 5-bit codes q[nb][32]
    (value = (q - 16) * d): code j < 16 in the low nibble of qs[j] with its fifth bit at bit j of
    qh, code 16 + j in the high nibble with its fifth bit at bit 16 + j."""
    q = np.asarray(q, np.uint32).reshape(-1, 32)
    nb = q.shape[0]
    out = np.zeros((nb, 22), np.uint8)
    out[:, 0:2] = np.asarray(d, np.float16).reshape(nb, 1).view(np.uint8)
    lo, hi = q[:, :16], q[:, 16:]
    qh = (((lo >> 4) & 1) << np.arange(16, dtype=np.uint32)).sum(1) + \
         (((hi >> 4) & 1) << (np.arange(16, dtype=np.uint32) + 16)).sum(1)
    out[:, 2:6] = qh.astype("<u4").reshape(nb, 1).view(np.uint8)
    out[:, 6:22] = ((lo & 0xF) | ((hi & 0xF) << 4)).astype(np.uint8)
    return out.tobytes()


def pack_q4_k(d, dmin, ls, lm, q) -> bytes:
    """Q4_K super blocks {f16 d, dmin; u8 scales[12]; u8 qs[128]} from f16 d, dmin [nb], 6-bit
    sub-block scales ls and mins lm [nb][8] and 4-bit codes q [nb][256]
    (value = (d ls) q - dmin lm): ggml's scale packing (sub-blocks j < 4 in the low 6 bits of
    bytes j and j + 4; j >= 4 in a nibble of byte j + 4 plus the top bits of bytes j - 4 and
    j) and codes of sub-blocks 2i / 2i + 1 in the low / high nibbles of qs[32i .. 32i + 32]."""
    ls = np.asarray(ls, np.uint32).reshape(-1, 8)
    lm = np.asarray(lm, np.uint32).reshape(-1, 8)
    q = np.asarray(q, np.uint32).reshape(-1, 256)
    nb = q.shape[0]
    out = np.zeros((nb, 144), np.uint8)
    out[:, 0:2] = np.asarray(d, np.float16).reshape(nb, 1).view(np.uint8)
    out[:, 2:4] = np.asarray(dmin, np.float16).reshape(nb, 1).view(np.uint8)
    sc = np.zeros((nb, 12), np.uint32)
    for j in range(8):
        if j < 4:
            sc[:, j] = ls[:, j]
            sc[:, j + 4] = lm[:, j]
        else:
            sc[:, j + 4] = (ls[:, j] & 0xF) | ((lm[:, j] & 0xF) << 4)
            sc[:, j - 4] |= (ls[:, j] >> 4) << 6
            sc[:, j] |= (lm[:, j] >> 4) << 6
    out[:, 4:16] = sc.astype(np.uint8)
    qs = np.zeros((nb, 128), np.uint32)
    for i in range(4):
        qs[:, 32 * i:32 * i + 32] = q[:, 64 * i:64 * i + 32] | (q[:, 64 * i + 32:64 * i + 64] << 4)
    out[:, 16:144] = qs.astype(np.uint8)
    return out.tobytes()


def pack_q6_k(d, sc, q) -> bytes:
    """Q6_K super blocks {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d} from f16 d [nb], int8
    group scales sc [nb][16] (group = element / 16) and 6-bit codes q [nb][256]
    (value = (d sc) (q - 32)): in half h, element 128 h + 32 k + l (k < 4, l < 32) keeps its low
    nibble in ql[64 h + l + 32 (k & 1)] (high nibble when k >= 2) and its top 2 bits at bit 2 k
    of qh[32 h + l]."""
    sc = np.asarray(sc, np.int8).reshape(-1, 16)
    q = np.asarray(q, np.uint32).reshape(-1, 256)
    nb = q.shape[0]
    out = np.zeros((nb, 210), np.uint8)
    ql = np.zeros((nb, 128), np.uint32)
    qh = np.zeros((nb, 64), np.uint32)
    for h in range(2):
        e = q[:, 128 * h:128 * h + 128].reshape(nb, 4, 32)
        ql[:, 64 * h:64 * h + 32] = (e[:, 0] & 0xF) | ((e[:, 2] & 0xF) << 4)
        ql[:, 64 * h + 32:64 * h + 64] = (e[:, 1] & 0xF) | ((e[:, 3] & 0xF) << 4)
        qh[:, 32 * h:32 * h + 32] = (e[:, 0] >> 4) | ((e[:, 1] >> 4) << 2) | ((e[:, 2] >> 4) << 4) | \
            ((e[:, 3] >> 4) << 6)
    out[:, 0:128] = ql.astype(np.uint8)
    out[:, 128:192] = qh.astype(np.uint8)
    out[:, 192:208] = sc.view(np.uint8)
    out[:, 208:210] = np.asarray(d, np.float16).reshape(nb, 1).view(np.uint8)
    return out.tobytes()


# ---- quantizers: f32 values -> logical codes (any valid encoding; not ggml's error search) ----
def quantize_q5_0(x: np.ndarray) -> bytes:
    """ggml quantize_row_q5_0: d = (the value of largest magnitude) / -16,
    q = min(31, trunc(x / d + 16.5))."""
    b = np.ascontiguousarray(x, np.float32).reshape(-1, 32)
    idx = np.argmax(np.abs(b), axis=1)
    mx = b[np.arange(b.shape[0]), idx]
    d = (mx / np.float32(-16.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.trunc((b * idv[:, None]).astype(np.float32) + np.float32(16.5)), 0, 31).astype(np.uint32)
    return pack_q5_0(d.astype(np.float16), q)


def quantize_q4_k(x: np.ndarray) -> bytes:
    """Per 32-wide sub-block: min and range, 6-bit scale/min relative to the super block's f16
    d and dmin, 4-bit codes."""
    b = np.ascontiguousarray(x, np.float32).reshape(-1, 8, 32).astype(np.float64)
    mn = np.minimum(b.min(2), 0.0)
    sc = (b.max(2) - mn) / 15.0
    d = (sc.max(1) / 63.0).astype(np.float16).astype(np.float64)
    dmin = ((-mn).max(1) / 63.0).astype(np.float16).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        ls = np.clip(np.where(d[:, None] > 0, np.rint(sc / d[:, None]), 0), 0, 63)
        lm = np.clip(np.where(dmin[:, None] > 0, np.rint(-mn / dmin[:, None]), 0), 0, 63)
        step = d[:, None] * ls
        q = np.where(step[:, :, None] > 0, np.rint((b + (dmin[:, None] * lm)[:, :, None]) / step[:, :, None]), 0)
    q = np.clip(q, 0, 15).astype(np.uint32)
    return pack_q4_k(d.astype(np.float16), dmin.astype(np.float16), ls, lm, q.reshape(-1, 256))


def quantize_q6_k(x: np.ndarray) -> bytes:
    """Per 16-element group an int8 scale relative to the super block's f16 d, 6-bit codes."""
    b = np.ascontiguousarray(x, np.float32).reshape(-1, 16, 16).astype(np.float64)
    gs = np.abs(b).max(2) / 31.0
    d = (gs.max(1) / 127.0).astype(np.float16).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.clip(np.where(d[:, None] > 0, np.rint(gs / d[:, None]), 0), -128, 127)
        step = d[:, None] * sc
        q = np.where(step[:, :, None] > 0, np.rint(b / step[:, :, None]), 0)
    q = (np.clip(q, -32, 31) + 32).astype(np.uint32)
    return pack_q6_k(d.astype(np.float16), sc.astype(np.int8), q.reshape(-1, 256))


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


# the tensor types of qtype="kquant" by role (the mix a Q4_K_M file uses: 4-bit K-quants for
# most matrices, 6-bit for the down projections and the embedding, Q5_0 for attn_output)
_KQUANT_ROLE = {"token_embd": GGML_Q6_K, "attn_qkv": GGML_Q4_K, "attn_output": GGML_Q5_0,
                "ffn_gate": GGML_Q4_K, "ffn_up": GGML_Q4_K, "ffn_down": GGML_Q6_K}


def _encode(ggml_type: int, arr: np.ndarray) -> bytes:
    if ggml_type == GGML_Q8_0:
        return quantize_q8_0(arr).tobytes()
    if ggml_type == GGML_Q5_0:
        return quantize_q5_0(arr)
    if ggml_type == GGML_Q4_K:
        return quantize_q4_k(arr)
    return quantize_q6_k(arr)


def build_gguf(path: str, shape: Shape, seed: int, *, norm_jitter: float = 0.0,
               bias_std: float = 0.01, init_std: float = 0.02, qtype: str = "q8_0") -> str:
    """Write a random-init hobbylm GGUF with quantized matrices (qtype "q8_0", or "kquant" for
    the Q4_K / Q6_K / Q5_0 mix) and F32 norms/router/bias."""
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

    def mat_type(name, n):
        if qtype == "q8_0":
            return GGML_Q8_0
        role = name.split(".")[-2] if name.startswith("blk.") else name.split(".")[0]
        for key, ty in _KQUANT_ROLE.items():
            if role.startswith(key):
                # K-quant super blocks need whole 256-element groups
                return ty if ty == GGML_Q5_0 or n % 256 == 0 else GGML_Q5_0
        return GGML_Q8_0

    def q8(name, shp, std):
        ty = mat_type(name, int(np.prod(shp)))
        w.tensor(name, shp, ty, _encode(ty, normal(name, shp, std)))

    def f32(name, arr):
        w.tensor(name, arr.shape, GGML_F32, np.ascontiguousarray(arr, dtype="<f4").tobytes())

    def gain(name, n):
        if norm_jitter:
            return np.float32(1.0) + normal(name, (n,), norm_jitter)
        return np.ones(n, dtype=np.float32)

    ety = mat_type("token_embd.weight", s.vocab_size * s.d_model)
    emb = _encode(ety, normal("token_embd.weight", (s.vocab_size, s.d_model), init_std))
    w.tensor("token_embd.weight", (s.vocab_size, s.d_model), ety, emb)
    f32("output_norm.weight", gain("output_norm.weight", s.d_model))
    w.tensor("output.weight", (s.vocab_size, s.d_model), ety, emb)  # tied embeddings
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
               directory: Optional[str] = None, qtype: str = "q8_0") -> str:
    """Path of the cached synthetic GGUF for (preset, seed, qtype), written on first use."""
    tag = f"{preset}_s{seed}" + (f"_j{norm_jitter:g}" if norm_jitter else "") + \
        ("" if qtype == "q8_0" else f"_{qtype}") + f"_v{GENERATOR_VERSION}"
    path = os.path.join(directory or cache_dir(), tag + ".gguf")
    if not os.path.exists(path):
        tmp = path + f".{os.getpid()}.tmp"
        build_gguf(tmp, PRESETS[preset], seed, norm_jitter=norm_jitter, qtype=qtype)
        os.replace(tmp, path)
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
