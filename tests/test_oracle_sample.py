"""The oracle's sampler (sample.rs) pinned by closed forms: the xorshift64* step as a product of
GF(2) matrices, the seed clamp, next_f32's 24-bit grid, and sample::sample on distributions
whose picks follow from the drawn r alone (argmax ties, a one-entry nucleus, index order without
a nucleus against descending order with one, the renormalization of the kept probabilities, the
id order of equal probabilities), plus draw frequencies."""
import numpy as np
import pytest

import oracle

M64 = (1 << 64) - 1
MUL = 0x2545F4914F6CDD1D


def _shift_matrix(k, left):
    """64x64 GF(2) matrix of x -> x << k (left) or x >> k on bit vectors (bit i = row i)."""
    m = np.zeros((64, 64), np.uint8)
    for i in range(64):
        j = i - k if left else i + k   # output bit i takes input bit j
        if 0 <= j < 64:
            m[i, j] = 1
    return m


def _bits(x):
    return np.array([(x >> i) & 1 for i in range(64)], np.uint8)


def _int(b):
    return sum(int(v) << i for i, v in enumerate(b))


def test_rng_state_step_is_the_xorshift_matrix():
    I = np.eye(64, dtype=np.uint8)
    T = (I ^ _shift_matrix(27, False)) @ (I ^ _shift_matrix(25, True)) % 2 @ (I ^ _shift_matrix(12, False)) % 2
    inv = pow(MUL, -1, 1 << 64)
    for seed in (1, 2, 0x9E3779B97F4A7C15, 12345678901234567):
        rng = oracle.Rng(seed)
        state = seed
        for _ in range(50):
            out = rng.next_u64()
            nxt = (out * inv) & M64             # the state, unscrambled
            assert _int(T @ _bits(state) % 2) == nxt
            state = nxt


def test_rng_seed_clamp_and_f32_grid():
    a, b = oracle.Rng(0), oracle.Rng(1)
    assert [a.next_u64() for _ in range(5)] == [b.next_u64() for _ in range(5)]
    r1, r2 = oracle.Rng(77), oracle.Rng(77)
    for _ in range(200):
        u = r1.next_u64()
        f = r2.next_f32()
        assert 0.0 <= f < 1.0 and f * 2**24 == float(u >> 40)


def _draws(seed, k):
    r = oracle.Rng(seed)
    return [r.next_f32() for _ in range(k)]


def test_greedy_and_one_entry_nucleus():
    lg = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    rng = oracle.Rng(5)
    assert oracle.sample(lg, 0.0, 0.9, rng) == 1 and rng.next_u64() == oracle.Rng(5).next_u64()   # no draw
    lg = np.array([0.0, 30.0, 1.0, 2.0], np.float32)   # p[1] > 0.9999
    for seed in range(1, 40):
        rng = oracle.Rng(seed)
        assert oracle.sample(lg, 1.0, 0.5, rng) == 1
        ref = oracle.Rng(seed)
        ref.next_u64()
        assert rng.next_u64() == ref.next_u64()   # exactly one draw per sample


def _two_point(seed, top_p):
    lg = np.array([0.0, np.log(3.0)], np.float32)    # p ~ (0.25, 0.75)
    return oracle.sample(lg, 1.0, top_p, oracle.Rng(seed)), _draws(seed, 1)[0]


def test_index_order_without_nucleus_descending_with_one():
    for seed in range(1, 400):
        pick, r = _two_point(seed, 1.0)
        if abs(r - 0.25) > 1e-4:
            assert pick == (0 if r < 0.25 else 1), (seed, r)    # id order: p0 first
        pick, r = _two_point(seed, 0.99)
        if abs(r - 0.75) > 1e-4:
            assert pick == (1 if r < 0.75 else 0), (seed, r)    # descending: p1 first


def test_nucleus_is_renormalized():
    lg = np.log(np.array([0.5, 0.3, 0.2], np.float32))   # cut after two entries at top_p 0.75
    seen = set()
    for seed in range(1, 600):
        r = _draws(seed, 1)[0]
        pick = oracle.sample(lg, 1.0, 0.75, oracle.Rng(seed))
        assert pick in (0, 1)
        if abs(r - 0.625) > 1e-4:
            assert pick == (0 if r < 0.625 else 1), (seed, r)   # kept (0.5, 0.3) / 0.8
        if 0.5 < r < 0.625:
            seen.add(seed)
    assert seen   # draws that an unnormalized nucleus would send to id 1


def test_equal_probabilities_keep_id_order():
    lg = np.zeros(4, np.float32)   # 0.25 each: the nucleus of top_p 0.5 is ids 0 and 1
    for seed in range(1, 300):
        r = _draws(seed, 1)[0]
        pick = oracle.sample(lg, 1.0, 0.5, oracle.Rng(seed))
        assert pick == (0 if r < 0.5 else 1), (seed, r)


def test_draw_frequencies():
    lg = np.log(np.array([0.1, 0.2, 0.3, 0.4], np.float32))
    rng = oracle.Rng(2024)
    n = 20000
    counts = np.bincount([oracle.sample(lg, 1.0, 1.0, rng) for _ in range(n)], minlength=4)
    expect = np.array([0.1, 0.2, 0.3, 0.4]) * n
    assert np.all(np.abs(counts - expect) < 5 * np.sqrt(expect)), counts
    # temperature 2 flattens: p ~ sqrt(p)
    rng = oracle.Rng(7)
    counts = np.bincount([oracle.sample(lg, 2.0, 1.0, rng) for _ in range(n)], minlength=4)
    q = np.sqrt([0.1, 0.2, 0.3, 0.4])
    expect = q / q.sum() * n
    assert np.all(np.abs(counts - expect) < 5 * np.sqrt(expect)), counts


def test_gumbel_argmax_draws_and_distribution():
    """gumbel_argmax: temp 0 is the argmax with no draw; one draw per finite logit; the picks of
    argmax(l / temp - ln(-ln u)) follow softmax(l / temp) (the Gumbel-max identity)."""
    lg = np.array([0.3, -np.inf, 1.0, np.nan, 0.5, 0.0], np.float32)
    r = oracle.Rng(9)
    assert oracle.gumbel_argmax(lg, 0.0, r) == 2
    assert r.next_u64() == oracle.Rng(9).next_u64()
    r, ref = oracle.Rng(9), oracle.Rng(9)
    oracle.gumbel_argmax(lg, 1.0, r)
    for _ in range(4):   # four finite entries, four draws
        ref.next_u64()
    assert r.next_u64() == ref.next_u64()
    p = np.array([0.1, 0.2, 0.3, 0.4])
    lg = (np.log(p) * 0.7).astype(np.float32)   # at temp 0.7: softmax(l / 0.7) = p
    r = oracle.Rng(31)
    n = 20000
    counts = np.bincount([oracle.gumbel_argmax(lg, 0.7, r) for _ in range(n)], minlength=4)
    assert np.all(np.abs(counts - p * n) < 5 * np.sqrt(p * n)), counts
