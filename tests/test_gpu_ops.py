"""Operator-level parity of the HIP path against the CPU oracle (run through the C ABI).

Q8 matvec (quant.rs:106-136) and its routed-expert gather, the prompt-path matmul
(quant.rs:144-194), and one decode-attention layer with QK-norm, RoPE and KV append
(model.rs:199-233).  Integer work (requantized weights, activation quantization, cache
rows) and every matvec are bit-exact, because the kernels reproduce qrow_dot_avx2's
lane order and FMAs; fast attention is within 1e-4, exact attention bit-exact.
"""
import numpy as np
import pytest

from hobbylm_amd import gguf_synth as gs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hg():
    import hobbylm_amd
    hobbylm_amd.lib()
    return hobbylm_amd


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _oracle_q8(orc, blocks, n, k):
    deq = orc.dequant_q8_0(blocks.view(np.uint8), n * k).reshape(n, k)
    return orc.q8_quantize(deq)


@pytest.mark.parametrize("n,k", [(1024, 1024), (3072, 1024), (512, 1024), (1024, 512), (50, 192), (7, 96), (1024, 4096)])
def test_q8_matvec_bit_exact(hg, orc, n, k):
    rng = np.random.default_rng(n * 7 + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal(k).astype(np.float32)
    blocks = gs.quantize_q8_0(w)
    t = hg.Q8Tensor.from_q8_0(blocks, n, k)
    y = t.matvec(x)
    sc, qs = _oracle_q8(orc, blocks, n, k)
    want = orc.q8_matvec(sc, qs, x)
    assert _bits_equal(y, want)
    ref = (blocks["qs"].astype(np.float64) * blocks["d"].astype(np.float64)[:, None]).reshape(n, k) @ x.astype(np.float64)
    assert np.max(np.abs(y - ref)) <= 1e-2 * np.max(np.abs(ref))  # activation quantization noise only
    assert t.bytes() == n * k + n * (k // 32) * 4


def test_q8_gather_bit_exact(hg, orc):
    rng = np.random.default_rng(2)
    E, f, d = 36, 512, 1024
    w = (rng.standard_normal((E * f, d)) * 0.02).astype(np.float32)
    x = rng.standard_normal(d).astype(np.float32)
    ids = rng.choice(E, 6, replace=False).astype(np.uint32)
    blocks = gs.quantize_q8_0(w)
    t = hg.Q8Tensor.from_q8_0(blocks, E * f, d)
    y = t.matvec_gather(f, ids, x)
    sc, qs = _oracle_q8(orc, blocks, E * f, d)
    for i, e in enumerate(ids):
        want = orc.q8_matvec(sc[e * f:(e + 1) * f], qs[e * f:(e + 1) * f], x)
        assert _bits_equal(y[i], want), i
    with pytest.raises(hg.HgError):
        t.matvec_gather(f, np.array([E], np.uint32), x)


@pytest.mark.parametrize("n,k,tn", [(256, 1024, 5), (64, 192, 3)])
def test_q8_matmul_prefill_order(hg, orc, n, k, tn):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((tn, k)).astype(np.float32)
    t = hg.Q8Tensor.quantize(w)
    sc, qs = orc.q8_quantize(w)
    assert _bits_equal(t.matmul(x), orc.q8_matmul(sc, qs, x))
    assert _bits_equal(t.matvec(x[0]), orc.q8_matvec(sc, qs, x[0]))


def test_q8_edge_blocks(hg, orc):
    """All-zero blocks (d = 0), exact ties, +-127 extremes and tiny scales."""
    rng = np.random.default_rng(4)
    n, k = 16, 256
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0
    w[1, :32] = np.linspace(-1, 1, 32)
    w[2] *= 1e-30
    x = rng.standard_normal(k).astype(np.float32)
    x[:32] = 0.0
    x[32:64] = np.arange(32) - 15.5
    t = hg.Q8Tensor.quantize(w)
    sc, qs = orc.q8_quantize(w)
    assert _bits_equal(t.matvec(x), orc.q8_matvec(sc, qs, x))


def _attn_case(orc, hg, ctx, exact, seed=0, nh=16, nkv=4, hd=64, theta=10000.0):
    rng = np.random.default_rng(seed + ctx)
    pos = ctx - 1
    kvd = nkv * hd
    kc = np.zeros((ctx, kvd), np.float32)
    vc = np.zeros((ctx, kvd), np.float32)
    kc[:pos] = rng.standard_normal((pos, kvd))
    vc[:pos] = rng.standard_normal((pos, kvd))
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(kvd).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    ones = np.ones(hd, np.float32)
    cos_t, sin_t = orc.rope_table(hd, ctx, theta)
    kc_o, vc_o = kc.copy(), vc.copy()
    want, _, _ = orc.attention_decode(q, k, v, ones, ones, cos_t, sin_t, 1e-5, nh, nkv, hd, pos, kc_o, vc_o)
    kc_g, vc_g = kc.copy(), vc.copy()
    got = hg.attention_decode(q, k, v, ones, ones, 1e-5, theta, ctx, nh, nkv, hd, pos, kc_g, vc_g, fast=not exact)
    assert _bits_equal(kc_g, kc_o) and _bits_equal(vc_g, vc_o)  # the append is bit-exact
    return got, want


@pytest.mark.parametrize("ctx", [1, 2, 65, 512, 2048, 8192])
def test_attention_fast_within_tolerance(hg, orc, ctx):
    got, want = _attn_case(orc, hg, ctx, exact=False)
    assert np.max(np.abs(got - want)) <= 1e-4


# 512 / 2048 / 8192: the attention layer's contexts.  The resident kernel holds windows up to
# 7168 positions, its exact sum as 4 waves x 64 lanes x 8, 12, ..., 28 terms: 2048 / 2049,
# 3072 / 3073, 4096 / 4097, 5120, 6145 and 7168 are the edges of those layouts; 7169 and 8192
# run the LDS product ring.
@pytest.mark.parametrize("ctx", [1, 300, 512, 2048, 2049, 3072, 3073, 4096, 4097, 5120, 6145, 7168, 7169, 8192])
def test_attention_exact_bit_exact(hg, orc, ctx):
    got, want = _attn_case(orc, hg, ctx, exact=True)
    assert _bits_equal(got, want)


@pytest.mark.parametrize("hd,nh,nkv,ctx", [(128, 12, 3, 777), (32, 4, 2, 777), (128, 12, 3, 5000)])
def test_attention_other_head_dims(hg, orc, hd, nh, nkv, ctx):
    for exact in (False, True):
        got, want = _attn_case(orc, hg, ctx, exact=exact, nh=nh, nkv=nkv, hd=hd, theta=1e6)
        if exact:
            assert _bits_equal(got, want)
        else:
            assert np.max(np.abs(got - want)) <= 1e-4
