"""The oracle's diffusion block path (model.rs:440-651, lib.rs:214-495) pinned: run_block's K/V
rows equal the prompt path's where the two must agree (every row in layer 0, which sees only
the embeddings; the last row in layer 1, whose residual comes from a layer-0 attention over
every row in both), the float64 model's bidirectional block agrees with
every row's logits (and the causal model does not), and a one-step denoising schedule commits
every position's penalized argmax of one run_block."""
import numpy as np
import pytest

from hobbylm_amd import gguf_synth as gs


@pytest.fixture(scope="module")
def diff_path():
    return gs.synth_path("tiny_diff", 5, norm_jitter=0.1)


def _emb(m, ids):
    return np.stack([m.token_embedding(int(t)) for t in ids])


def test_run_block_last_row_is_the_prompt_paths(orc, diff_path):
    m = orc.Model(diff_path)
    pre, blk = gs.prompt_ids(1, 9, 50257), gs.prompt_ids(2, 7, 50257)
    kv1, kv2 = m.new_cache(), m.new_cache()
    m.prefill(_emb(m, pre), kv1)
    m.prefill(_emb(m, pre), kv2)
    lg, bk, bv = m.run_block(_emb(m, blk), kv1, 9, want_kv=True)
    assert kv1.len == 9                                       # non-destructive
    m.prefill(_emb(m, blk), kv2)                             # causal: its last row sees all 16
    bits = lambda a: np.asarray(a, np.float32).view(np.uint32)
    for layer in (0, 1):
        k, v = kv2.read(layer)
        rows = slice(0, 7) if layer == 0 else slice(6, 7)
        assert np.array_equal(bits(bk[layer][rows]), bits(k[9:][rows])), layer
        assert np.array_equal(bits(bv[layer][rows]), bits(v[9:][rows])), layer
    k1, _ = kv2.read(1)
    assert not np.array_equal(bits(bk[1][0]), bits(k1[9]))   # the first row sees the whole block
    assert np.isfinite(lg).all()


def test_run_block_vs_float64_bidirectional(orc, diff_path):
    from refmodel import RefModel
    m = orc.Model(diff_path)
    ref = RefModel(diff_path)
    pre, blk = gs.prompt_ids(3, 5, 50257), gs.prompt_ids(4, 6, 50257)
    kv = m.new_cache()
    for pos, t in enumerate(pre):
        m.forward(int(t), pos, kv)
        ref.forward(int(t), pos)
    got, _, _ = m.run_block(_emb(m, blk), kv, 5)
    want = ref.block(blk, 5)
    rng_ = want.max() - want.min()
    assert np.max(np.abs(got - want)) <= 2e-3 * rng_
    # the first row's causal logits (attending to the prefix and itself only) are far from it
    causal = ref.forward(int(blk[0]), 5)
    assert np.max(np.abs(causal - want[0])) > 2e-2 * rng_


@pytest.mark.parametrize("cached", [True, False])
def test_one_step_schedule_commits_the_penalized_argmax(orc, diff_path, cached):
    m = orc.Model(diff_path)
    c = m.cfg
    prompt = gs.prompt_ids(6, 8, 50257)
    o = orc.DiffOpts.make(gen_len=12, block=12, steps=1, rep_penalty=1.4, cached=cached)
    out = m.generate_diffusion(prompt, o, eos=10**6)
    if cached:   # the prompt encoded bidirectionally into the cache, then the masked block over it
        kv = m.new_cache()
        _, pk, pv = m.run_block(_emb(m, prompt), kv, 0, want_kv=True)
        kv.load(pk, pv)
        lg, _, _ = m.run_block(_emb(m, [c.mask_token_id] * 12), kv, 8)
    else:        # the whole canvas bidirectionally
        lg = m.forward_bidir(_emb(m, list(prompt) + [c.mask_token_id] * 12))[8:]
    lg[:, 50257:] = -np.inf
    pres = np.zeros(c.vocab_size, bool)
    pres[prompt] = True
    lg[:, pres] = np.where(lg[:, pres] > 0, lg[:, pres] / np.float32(1.4), lg[:, pres] * np.float32(1.4))
    assert np.array_equal(out, np.argmax(lg, axis=1))
    assert np.all(out < 50257)
