"""An independent float64 re-expression of the hobbylm decode step, for checking the oracle.

It reads the GGUF with its own small parser (not the oracle's), dequantizes Q8_0 with
numpy, and evaluates the architecture of hobby-rs/src/model.rs in float64: RMSNorm,
fused QKV, per-head QK-norm, rotate-half RoPE, GQA attention over the cache, sigmoid
router with bias-shifted top-k selection, SwiGLU experts plus the shared expert, and the
tied lm_head.  The only quantization it models is the 32-wide activation quantization
of every Q8 matvec (quant.rs:111-123), done in float64 arithmetic, so its logits agree
with the oracle to the activation-rounding noise, not bit for bit.
"""
from __future__ import annotations

import struct

import numpy as np

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


class GGUF:
    def __init__(self, path):
        self.buf = open(path, "rb").read()
        self.p = 0
        magic, ver, nt, nk = struct.unpack_from("<IIQQ", self.buf, 0)
        assert magic == 0x46554747 and ver == 3
        self.p = 24
        self.meta = {}
        for _ in range(nk):
            k = self._str()
            ty = self._u(4)
            self.meta[k] = self._val(ty)
        self.tensors = {}
        for _ in range(nt):
            name = self._str()
            nd = self._u(4)
            ne = [self._u(8) for _ in range(nd)]
            ty = self._u(4)
            off = self._u(8)
            self.tensors[name] = (ne, ty, off)
        align = self.meta.get("general.alignment", 32)
        self.data = (self.p + align - 1) // align * align

    def _u(self, n):
        v = int.from_bytes(self.buf[self.p:self.p + n], "little")
        self.p += n
        return v

    def _str(self):
        n = self._u(8)
        s = self.buf[self.p:self.p + n].decode("utf-8")
        self.p += n
        return s

    def _val(self, ty):
        if ty == 8:
            return self._str()
        if ty == 9:
            at = self._u(4)
            n = self._u(8)
            return [self._val(at) for _ in range(n)]
        fmt = _SCALAR[ty]
        v = struct.unpack_from(fmt, self.buf, self.p)[0]
        self.p += struct.calcsize(fmt)
        return v

    def tensor(self, name) -> np.ndarray:
        """float64 array in torch (row-major, slowest dim first) order."""
        ne, ty, off = self.tensors[name]
        n = int(np.prod(ne))
        o = self.data + off
        if ty == 0:
            a = np.frombuffer(self.buf, "<f4", n, o).astype(np.float64)
        elif ty == 1:
            a = np.frombuffer(self.buf, "<f2", n, o).astype(np.float64)
        elif ty == 8:
            blk = np.frombuffer(self.buf, np.dtype([("d", "<f2"), ("qs", "i1", (32,))]), n // 32, o)
            a = (blk["qs"].astype(np.float64) * blk["d"].astype(np.float64)[:, None]).reshape(-1)
        else:
            raise ValueError(ty)
        return a.reshape(list(reversed(ne)))


def actq(x: np.ndarray) -> np.ndarray:
    """The 32-block activation quantize->dequantize a Q8 matvec applies to its input."""
    b = x.reshape(-1, 32)
    d = np.abs(b).max(axis=1) / 127.0
    idv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1.0), 0.0)
    v = b * idv[:, None]
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -127, 127)
    return (q * d[:, None]).reshape(x.shape)


class RefModel:
    def __init__(self, path, quant=True):
        g = GGUF(path)
        self.g = g
        self.quant = quant   # False: Mat::Owned, no activation quantization before a product
        a = g.meta["general.architecture"]
        m = lambda k, d=None: g.meta.get(f"{a}.{k}", d)
        self.d = m("embedding_length")
        self.L = m("block_count")
        self.n_dense = m("leading_dense_block_count", 1)
        self.nh = m("attention.head_count")
        self.nkv = m("attention.head_count_kv")
        self.hd = m("attention.key_length")
        self.top_k = m("expert_used_count")
        self.n_shared = m("expert_shared_count", 0)
        self.eps = m("attention.layer_norm_rms_epsilon", 1e-5)
        self.theta = m("rope.freq_base", 1e6)
        self.ctx = m("context_length", 8192)
        self.w = {k: g.tensor(k) for k in g.tensors}
        self.vocab = self.w["token_embd.weight"].shape[0]
        self.k = [[] for _ in range(self.L)]
        self.v = [[] for _ in range(self.L)]

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.eps) * w

    def mv(self, W, x):
        return W @ (actq(x) if self.quant else x)

    def rope(self, v, pos):
        half = self.hd // 2
        i = np.arange(half)
        ang = pos * float(np.float32(self.theta)) ** (-(2.0 * i) / self.hd)
        c, s = np.cos(ang), np.sin(ang)
        z = (v[:half] + 1j * v[half:]) * (c + 1j * s)
        return np.concatenate([z.real, z.imag])

    def block(self, tokens, base):
        """Model::run_block in float64: rows at positions base + r, each attending to the prefix
        rows 0 .. base - 1 already in the cache and to every block row; the cache is unchanged."""
        W = self.w
        b = len(tokens)
        X = np.stack([W["token_embd.weight"][t].copy() for t in tokens])
        qd, kvd, rep = self.nh * self.hd, self.nkv * self.hd, self.nh // self.nkv
        for li in range(self.L):
            p = f"blk.{li}."
            qs, ks, vs = [], [], []
            for r in range(b):
                h = self.rms(X[r], W[p + "attn_norm.weight"])
                qkv = self.mv(W[p + "attn_qkv.weight"], h)
                q = qkv[:qd].reshape(self.nh, self.hd)
                k = qkv[qd:qd + kvd].reshape(self.nkv, self.hd)
                qs.append(np.stack([self.rope(self.rms(qh, W[p + "attn_q_norm.weight"]), base + r) for qh in q]))
                ks.append(np.stack([self.rope(self.rms(kh, W[p + "attn_k_norm.weight"]), base + r) for kh in k]))
                vs.append(qkv[qd + kvd:].reshape(self.nkv, self.hd))
            K = np.stack(self.k[li][:base] + ks)
            V = np.stack(self.v[li][:base] + vs)
            for r in range(b):
                o = np.empty((self.nh, self.hd))
                for hq in range(self.nh):
                    s = K[:, hq // rep, :] @ qs[r][hq] / np.sqrt(self.hd)
                    pr = np.exp(s - s.max())
                    pr /= pr.sum()
                    o[hq] = pr @ V[:, hq // rep, :]
                X[r] = X[r] + self.mv(W[p + "attn_output.weight"], o.reshape(-1))
            for r in range(b):
                X[r] = X[r] + self._ffn(li, self.rms(X[r], W[p + "ffn_norm.weight"]))
        return np.stack([self.mv(W["output.weight"], self.rms(X[r], W["output_norm.weight"])) for r in range(b)])

    def _ffn(self, li, h):
        W, p = self.w, f"blk.{li}."
        if li < self.n_dense:
            gg = self.mv(W[p + "ffn_gate.weight"], h)
            uu = self.mv(W[p + "ffn_up.weight"], h)
            return self.mv(W[p + "ffn_down.weight"], gg / (1 + np.exp(-gg)) * uu)
        logits = W[p + "ffn_gate_inp.weight"] @ h
        sc = 1 / (1 + np.exp(-logits))
        sel = sc + W[p + "exp_probs_b.bias"]
        top = np.argsort(-sel, kind="stable")[: self.top_k]
        out = np.zeros(self.d)
        for e in top:
            gg = self.mv(W[p + "ffn_gate_exps.weight"][e], h)
            uu = self.mv(W[p + "ffn_up_exps.weight"][e], h)
            out += sc[e] * self.mv(W[p + "ffn_down_exps.weight"][e], gg / (1 + np.exp(-gg)) * uu)
        if self.n_shared:
            gg = self.mv(W[p + "ffn_gate_shexp.weight"], h)
            uu = self.mv(W[p + "ffn_up_shexp.weight"], h)
            out += self.mv(W[p + "ffn_down_shexp.weight"], gg / (1 + np.exp(-gg)) * uu)
        return out

    def forward(self, token, pos):
        x = self.w["token_embd.weight"][token].copy()
        W = self.w
        for li in range(self.L):
            p = f"blk.{li}."
            h = self.rms(x, W[p + "attn_norm.weight"])
            qkv = self.mv(W[p + "attn_qkv.weight"], h)
            qd, kvd = self.nh * self.hd, self.nkv * self.hd
            q = qkv[:qd].reshape(self.nh, self.hd)
            k = qkv[qd:qd + kvd].reshape(self.nkv, self.hd)
            v = qkv[qd + kvd:].reshape(self.nkv, self.hd)
            q = np.stack([self.rope(self.rms(qh, W[p + "attn_q_norm.weight"]), pos) for qh in q])
            k = np.stack([self.rope(self.rms(kh, W[p + "attn_k_norm.weight"]), pos) for kh in k])
            self.k[li].append(k)
            self.v[li].append(v)
            K = np.stack(self.k[li])  # [n, nkv, hd]
            V = np.stack(self.v[li])
            rep = self.nh // self.nkv
            o = np.empty((self.nh, self.hd))
            for hq in range(self.nh):
                s = K[:, hq // rep, :] @ q[hq] / np.sqrt(self.hd)
                pr = np.exp(s - s.max())
                pr /= pr.sum()
                o[hq] = pr @ V[:, hq // rep, :]
            x = x + self.mv(W[p + "attn_output.weight"], o.reshape(-1))
            h = self.rms(x, W[p + "ffn_norm.weight"])
            if li < self.n_dense:
                gg = self.mv(W[p + "ffn_gate.weight"], h)
                uu = self.mv(W[p + "ffn_up.weight"], h)
                x = x + self.mv(W[p + "ffn_down.weight"], gg / (1 + np.exp(-gg)) * uu)
            else:
                logits = W[p + "ffn_gate_inp.weight"] @ h
                sc = 1 / (1 + np.exp(-logits))
                sel = sc + W[p + "exp_probs_b.bias"]
                top = np.argsort(-sel, kind="stable")[: self.top_k]
                out = np.zeros(self.d)
                for e in top:
                    gg = self.mv(W[p + "ffn_gate_exps.weight"][e], h)
                    uu = self.mv(W[p + "ffn_up_exps.weight"][e], h)
                    out += sc[e] * self.mv(W[p + "ffn_down_exps.weight"][e], gg / (1 + np.exp(-gg)) * uu)
                if self.n_shared:
                    gg = self.mv(W[p + "ffn_gate_shexp.weight"], h)
                    uu = self.mv(W[p + "ffn_up_shexp.weight"], h)
                    out += self.mv(W[p + "ffn_down_shexp.weight"], gg / (1 + np.exp(-gg)) * uu)
                x = x + out
        h = self.rms(x, W["output_norm.weight"])
        return self.mv(W["output.weight"], h)
