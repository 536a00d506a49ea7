"""The diffusion block path on the GPU (model.rs:440-651, lib.rs:214-495) bit for bit against the
oracle: run_block's logits for every block row and its K/V rows over a prefix cache (the tiny
diffusion shape, the 500M model, heads of 128), forward_bidir, appending a finalized block, and
whole cached and uncached denoising runs (the num_transfer schedule, the confidence threshold,
re-masking, the presence penalty, Gumbel draws at temperature > 0, an EOS stop)."""
import numpy as np
import pytest

from hobbylm_amd import gguf_synth as gs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hg():
    import hobbylm_amd
    hobbylm_amd.lib()
    return hobbylm_amd


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _emb(m, ids):
    return np.stack([m.token_embedding(int(t)) for t in ids])


@pytest.mark.parametrize("preset,npre,nblk", [("tiny_diff", 9, 7), ("tiny_diff", 0, 40), ("500M", 20, 32),
                                              ("joint12", 5, 16)])
def test_run_block_bit_exact(hg, orc, preset, npre, nblk):
    path = gs.synth_path(preset, 5, norm_jitter=0.1) if preset.startswith("tiny") else gs.synth_path(preset, 1)
    gm, om = hg.Model(path), orc.Model(path)
    print(f"run_block {preset} prefix {npre} block {nblk}", flush=True)
    pre, blk = gs.prompt_ids(1, npre, 50257), gs.prompt_ids(2, nblk, 50257)
    gkv, okv = gm.new_cache(max_ctx=256), om.new_cache()
    if npre:
        gm.prefill(_emb(om, pre), gkv)
        om.prefill(_emb(om, pre), okv)
    gl, gk, gv = gm.run_block(_emb(om, blk), gkv, npre, want_kv=True)
    ol, ok, ov = om.run_block(_emb(om, blk), okv, npre, want_kv=True)
    assert np.array_equal(_bits(gl), _bits(ol))
    assert np.array_equal(_bits(gk), _bits(ok)) and np.array_equal(_bits(gv), _bits(ov))
    assert gkv.len == npre
    # finalize: append the block on the GPU, load it into the oracle, and continue decoding
    gm.run_block(_emb(om, blk), gkv, npre, append=True)
    assert gkv.len == npre + nblk
    K = np.stack([np.concatenate([okv.read(l)[0], ok[l]]) for l in range(om.cfg.n_layers)])
    V = np.stack([np.concatenate([okv.read(l)[1], ov[l]]) for l in range(om.cfg.n_layers)])
    okv2 = om.new_cache()
    okv2.load(K, V)
    g2, _ = gm.forward(7, npre + nblk, gkv)
    o2 = om.forward(7, npre + nblk, okv2)
    assert np.array_equal(_bits(g2), _bits(o2))


def test_forward_bidir_bit_exact(hg, orc):
    path = gs.synth_path("tiny_diff", 8, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    x = _emb(om, gs.prompt_ids(9, 50, 50257))
    assert np.array_equal(_bits(gm.forward_bidir(x)), _bits(om.forward_bidir(x)))


CASES = [
    dict(gen_len=48, block=16, steps=12, rep_penalty=1.4, cached=True),
    dict(gen_len=40, block=16, steps=40, rep_penalty=1.0, cached=True, remask_steps=2, remask_frac=0.3),
    dict(gen_len=48, block=16, steps=8, rep_penalty=1.4, cached=True, threshold=0.05),
    dict(gen_len=32, block=8, steps=16, rep_penalty=1.4, cached=False),
    dict(gen_len=24, block=12, steps=6, rep_penalty=1.2, cached=False, remask_steps=1, remask_frac=0.5),
    dict(gen_len=40, block=16, steps=20, rep_penalty=1.4, cached=True, temp=0.8, seed=77),
    dict(gen_len=24, block=8, steps=12, rep_penalty=1.0, cached=False, temp=1.2, seed=5, remask_steps=1),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_generate_diffusion_matches_oracle(hg, orc, case):
    path = gs.synth_path("tiny_diff", 5, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    prompt = gs.prompt_ids(11, 10, 50257)
    kw = CASES[case]
    print(f"diffusion {kw}", flush=True)
    g = gm.generate_diffusion(prompt, hg.DiffOpts.make(**kw), eos=10**6)
    o = om.generate_diffusion(prompt, orc.DiffOpts.make(**kw), eos=10**6)
    assert len(o) == kw["gen_len"] and np.array_equal(g, o)
    # an eos inside the generation ends it there on both
    eos = int(o[len(o) // 2])
    g = gm.generate_diffusion(prompt, hg.DiffOpts.make(**kw), eos=eos)
    o = om.generate_diffusion(prompt, orc.DiffOpts.make(**kw), eos=eos)
    assert np.array_equal(g, o) and len(o) < kw["gen_len"]
