"""The workgroup-parallel sequential sum against the sequential binary32 sum.

The decode kernels form rmsnorm's `ss += v * v` (ops.rs:101-104) and softmax's `sum += *v`
(ops.rs:119-122) with a parallel method that must reproduce the one-lane sum bit for bit.
The expected value is numpy's float32 cumulative sum (index order, one rounding per add).
Inputs cover the cases the method treats specially: binade crossings (geometric growth, a
late dominant term), ties (terms that are exact half quanta of the running sum), zeros,
subnormals, more than 256 events, overflow, NaN / infinity, and n beyond one workgroup.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hg():
    import hobbylm_amd
    hobbylm_amd.lib()
    return hobbylm_amd


def _seq(x):
    x = np.asarray(x, np.float32)
    return np.cumsum(x, dtype=np.float32)[-1] if x.size else np.float32(0)


def _cases():
    rng = np.random.default_rng(5)
    f = np.float32
    out = [("unif", rng.random(2049, dtype=f)), ("one", np.array([3.5], f)), ("empty", np.zeros(0, f))]
    for sc in (0.5, 2.0, 8.0, 20.0):
        z = rng.standard_normal(2049).astype(f) * f(sc)
        out.append((f"softmax{sc}", np.exp(z - z.max()).astype(f)))
    z = rng.standard_normal(2049).astype(f) * 8
    z[-1] = z.max() + 5
    out.append(("softmax_last_peak", np.exp(z - z.max()).astype(f)))
    out.append(("squares", (rng.standard_normal(1024).astype(f) ** 2).astype(f)))
    out.append(("squares_big", ((rng.standard_normal(1024) * 1e3).astype(f) ** 2).astype(f)))
    t = (rng.random(2049) * 1e-6).astype(f)
    t[::300] = 1.0
    out.append(("tiny_and_big", t))
    out.append(("ties", np.concatenate([[f(2 ** 24)], np.ones(100, f)])))
    out.append(("ties_mixed", np.concatenate([[f(2 ** 24)], np.full(50, 3.0, f), np.ones(50, f)])))
    out.append(("ties_many", np.concatenate([[f(2 ** 24)], np.ones(1000, f)])))
    out.append(("subnormal", (rng.random(2049) * 2.0 ** -140).astype(f)))
    out.append(("subnormal_to_normal", (rng.random(2049) * 2.0 ** -132).astype(f)))
    z = (rng.random(2049) * 2.0).astype(f)
    z[rng.random(2049) < 0.3] = 0
    out.append(("zeros", z))
    out.append(("all_zero", np.zeros(100, f)))
    out.append(("geometric_up", (2.0 ** np.linspace(-60, 10, 2049)).astype(f)))
    out.append(("geometric_down", (2.0 ** np.linspace(10, -60, 2049)).astype(f)))
    out.append(("constant_tenth", np.full(2049, 0.1, f)))
    out.append(("constant_third", np.full(4096, f(1 / 3), f)))
    out.append(("overflow", (rng.random(512) * 1e37).astype(f)))
    nan = rng.random(300).astype(f)
    nan[17] = np.nan
    out.append(("nan", nan))
    inf = rng.random(300).astype(f)
    inf[200] = np.inf
    out.append(("inf", inf))
    neg = rng.random(300).astype(f)
    neg[3] = -0.25
    out.append(("negative", neg))
    out.append(("beyond_one_workgroup", rng.random(5000, dtype=f)))
    for k in range(24):
        n = int(rng.integers(1, 4097))
        kind = k % 4
        if kind == 0:
            v = rng.random(n).astype(f) ** 8
        elif kind == 1:
            v = np.exp(np.minimum(rng.standard_normal(n) * rng.random() * 30, 80)).astype(f)
        elif kind == 2:
            v = (rng.integers(0, 4, n) * 2.0 ** rng.integers(-30, 5, n)).astype(f)
        else:
            v = (rng.random(n) * 2.0 ** int(rng.integers(-149, 20))).astype(f)
        out.append((f"random{k}", v))
    return out


def _long_cases():
    """Up to 16384 terms: the batched attention's softmax sums (8 waves x 32 terms per lane)."""
    rng = np.random.default_rng(11)
    f = np.float32
    out = []
    for n, sc in ((16384, 0.5), (16384, 4.0), (16383, 2.0), (9000, 8.0), (3100, 1.0), (12345, 20.0)):
        z = rng.standard_normal(n).astype(f) * f(sc)
        out.append((f"softmax{n}_{sc}", np.exp(z - z.max()).astype(f)))
    z = rng.standard_normal(16384).astype(f)
    z[-1] = z.max() + 9
    out.append(("softmax_late_peak16384", np.exp(z - z.max()).astype(f)))
    out.append(("ties_long", np.concatenate([[f(2 ** 24)], np.ones(16383, f)])))
    out.append(("constant_third_long", np.full(16384, f(1 / 3), f)))
    out.append(("geometric_long", (2.0 ** np.linspace(-80, 20, 16384)).astype(f)))
    out.append(("unif_long", rng.random(16384, dtype=f)))
    out.append(("beyond_the_layout", rng.random(16385, dtype=f)))
    for k in range(8):
        n = int(rng.integers(4097, 16385))
        v = np.exp(np.minimum(rng.standard_normal(n) * rng.random() * 30, 80)).astype(f) if k % 2 else \
            (rng.integers(0, 4, n) * 2.0 ** rng.integers(-30, 5, n)).astype(f)
        out.append((f"long_random{k}", v))
    return out


@pytest.mark.parametrize("name,x", _long_cases(), ids=lambda v: v if isinstance(v, str) else "")
def test_long_sum_matches_sequential(hg, name, x):
    want = _seq(x)
    got = hg.seq_sum(x, 7)
    assert np.array_equal(np.float32(got).view(np.uint32), np.float32(want).view(np.uint32)), (name, got, want)


@pytest.mark.parametrize("name,x", _cases(), ids=lambda v: v if isinstance(v, str) else "")
def test_workgroup_sum_matches_sequential(hg, name, x):
    want = _seq(x)
    for method in (1, 2, 3, 4, 5, 6, 7, 0):   # every wave layout of the decode kernels, one lane
        got = hg.seq_sum(x, method)
        assert np.array_equal(np.float32(got).view(np.uint32), np.float32(want).view(np.uint32)) or (
            np.isnan(got) and np.isnan(want)), (name, method, got, want)


def test_norm_inputs_of_the_130m_model(hg):
    """Sums of squares of real embeddings (the first RMSNorm of a synthetic 130M model), and
    the same vectors cut to every length the layouts split differently."""
    from hobbylm_amd import gguf_synth as gs
    m = hg.Model(gs.synth_path("130M", 0))
    for t in gs.prompt_ids(7, 4, 50257):
        x = m.token_embedding(int(t))
        sq = (x * x).astype(np.float32)
        for n in (64, 255, 256, 257, 511, 512, len(sq)):
            want = _seq(sq[:n])
            for method in (1, 2, 3, 4, 5, 6, 7):
                got = hg.seq_sum(sq[:n], method)
                assert np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32), (int(t), n, method)
