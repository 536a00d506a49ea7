"""Batched decode over a paged KV cache (hg_batch_*) against independent oracle forwards.

Every sequence of a batch must equal its own Model::forward (model.rs:152-184) on its own
cache, bit for bit: logits, the per-layer expert picks and weights, and every cache row.  The
oracle has no batched step, so each sequence runs its own oracle cache seeded with the same
rows (KvCache's pub fields, model.rs:60-64).  Contexts are ragged and the block tables are
seeded permutations of the page pool.
"""
import numpy as np
import pytest

from hobbylm_amd import gguf_synth as gs

pytestmark = pytest.mark.gpu
PAGE = 16


@pytest.fixture(scope="module")
def hg():
    import hobbylm_amd
    hobbylm_amd.lib()
    return hobbylm_amd


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _setup(hg, orc, path, lens, steps, seed, max_ctx=0):
    """A batch with len(lens) sequences seeded with random cache rows, and one oracle cache per
    sequence holding the same rows."""
    gm, om = hg.Model(path), orc.Model(path)
    c = gm.cfg
    rng = np.random.default_rng(seed)
    need = [-(-(n + steps) // PAGE) for n in lens]
    n_pages = sum(need) + 7
    b = hg.Batch(gm, len(lens), max_ctx=max_ctx, n_pages=n_pages)
    perm = rng.permutation(n_pages).astype(np.uint32)
    kvd = c.n_kv_heads * c.head_dim
    okvs, at = [], 0
    for s, n in enumerate(lens):
        b.set_pages(s, perm[at:at + need[s]])
        at += need[s]
        k = rng.standard_normal((c.n_layers, n, kvd), dtype=np.float32)
        v = rng.standard_normal((c.n_layers, n, kvd), dtype=np.float32)
        b.load(s, k, v)
        okv = om.new_cache()
        okv.load(k, v)
        okvs.append(okv)
    return gm, om, b, okvs


def _check_steps(om, b, okvs, lens, steps, seed, vocab):
    c = b.model.cfg
    rng = np.random.default_rng(seed + 1)
    valid = min(vocab, 50257)
    for i in range(steps):
        toks = rng.integers(0, valid, len(lens)).astype(np.uint32)
        lg, nxt = b.forward(toks)
        for s, n in enumerate(lens):
            ol = om.forward(int(toks[s]), n + i, okvs[s])
            assert _bits_equal(lg[s], ol), f"logits differ: step {i}, sequence {s} (pos {n + i})"
            assert int(nxt[s]) == int(np.argmax(ol[:valid])), (i, s)
            gi, gw = b.routing(s)
            oi, ow, _ = okvs[s].routing()
            assert np.array_equal(gi[c.n_dense:], oi[c.n_dense:]), (i, s)
            assert _bits_equal(gw[c.n_dense:], ow[c.n_dense:] * np.float32(c.expert_weights_scale)), (i, s)
    for s in range(len(lens)):
        for layer in (0, c.n_layers - 1):
            gk, gv = b.read(s, layer)
            ok, ov = okvs[s].read(layer)
            assert _bits_equal(gk, ok) and _bits_equal(gv, ov), (s, layer)


def test_batch_tiny_bit_exact(hg, orc):
    """hd 64, 12 experts top-4 + shared, renormalized and scaled weights, a dense layer 0."""
    path = gs.synth_path("tiny_wnorm", 41, norm_jitter=0.1)
    lens = [1, 17, 300, 64, 5, 129, 250]
    gm, om, b, okvs = _setup(hg, orc, path, lens, 4, 3)
    _check_steps(om, b, okvs, lens, 4, 3, gm.cfg.vocab_size)


def test_batch_500m_32_sequences(hg, orc):
    """The 500M model, 32 ragged sequences (the batched workload's width) at contexts up to 3000."""
    path = gs.synth_path("500M", 1)
    rng = np.random.default_rng(5)
    lens = [int(x) for x in rng.integers(1, 3000, 32)]
    gm, om, b, okvs = _setup(hg, orc, path, lens, 2, 5)
    _check_steps(om, b, okvs, lens, 2, 5, gm.cfg.vocab_size)


def test_batch_long_contexts(hg, orc):
    """Contexts past the exact parallel sum's 3072 terms, up to 16384 (the workload's longest)."""
    path = gs.synth_path("500M_long", 1)
    lens = [16384, 9000, 3100, 257]
    gm, om, b, okvs = _setup(hg, orc, path, lens, 2, 9, max_ctx=16400)
    _check_steps(om, b, okvs, lens, 2, 9, gm.cfg.vocab_size)


def test_batch_head_dim_128(hg, orc):
    """The joint12 shape: heads of 128, 12 q / 3 kv heads."""
    path = gs.synth_path("joint12", 5)
    lens = [40, 700, 3]
    gm, om, b, okvs = _setup(hg, orc, path, lens, 2, 11)
    _check_steps(om, b, okvs, lens, 2, 11, gm.cfg.vocab_size)


def test_batch_greedy_device_loop(hg, orc):
    """hg_batch_decode_greedy chains each sequence's greedy tokens on the device."""
    path = gs.synth_path("tiny_wnorm", 42, norm_jitter=0.1)
    lens = [3, 90, 33]
    gm, om, b, okvs = _setup(hg, orc, path, lens, 6, 13)
    first = np.array([5, 77, 901], np.uint32)
    ids = b.decode_greedy(first, 6)
    valid = min(gm.cfg.vocab_size, 50257)
    for s, n in enumerate(lens):
        tok = int(first[s])
        for i in range(6):
            ol = om.forward(tok, n + i, okvs[s])
            tok = int(np.argmax(ol[:valid]))
            assert int(ids[i, s]) == tok, (s, i)
        assert b.len(s) == n + 6


def test_batch_errors(hg):
    path = gs.synth_path("tiny_wnorm", 41, norm_jitter=0.1)
    gm = hg.Model(path)
    b = hg.Batch(gm, 2, n_pages=4)
    with pytest.raises(hg.HgError, match="page id"):
        b.set_pages(0, [4])
    b.set_pages(0, [0, 1])
    b.set_pages(1, [2])
    c = gm.cfg
    kvd = c.n_kv_heads * c.head_dim
    with pytest.raises(hg.HgError, match="beyond the sequence's pages"):
        b.load(1, np.zeros((c.n_layers, 17, kvd), np.float32), np.zeros((c.n_layers, 17, kvd), np.float32))
    b.load(1, np.zeros((c.n_layers, 16, kvd), np.float32), np.zeros((c.n_layers, 16, kvd), np.float32))
    with pytest.raises(hg.HgError, match="pages for 16 positions"):
        b.forward([1, 1])                      # sequence 1 is full
    with pytest.raises(hg.HgError, match="out of range"):
        b.forward([c.vocab_size])
    with pytest.raises(hg.HgError, match="sequences"):
        b.forward([1, 1, 1])
