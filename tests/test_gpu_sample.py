"""Sampling on the device (sample.rs:66-112, lib.rs:107-162) bit for bit against the oracle: the
pick and the advanced RNG state of sample::sample over seeded logit vectors (the 500M vocabulary
of 50257 ids, which spans four exact-sum segments, and small ones; temperatures, nuclei from
0.3 to 0.999 and none; ties and -inf entries), then seeded generations of 256 steps with the
mask, the repetition penalty, the EOS and context stops."""
import numpy as np
import pytest

from hobbylm_amd import gguf_synth as gs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hg():
    import hobbylm_amd
    hobbylm_amd.lib()
    return hobbylm_amd


def _logits(rng, n, kind):
    if kind == "normal":
        return (rng.standard_normal(n) * 3).astype(np.float32)
    if kind == "flat":      # near-uniform: the nucleus reaches deep into the sorted order
        return (rng.standard_normal(n) * 0.05).astype(np.float32)
    if kind == "ties":      # few distinct values: long runs of equal probabilities
        return rng.integers(-3, 4, n).astype(np.float32)
    if kind == "masked":    # -inf entries (the 50257 mask, banned ids)
        x = (rng.standard_normal(n) * 2).astype(np.float32)
        x[rng.random(n) < 0.3] = -np.inf
        return x
    raise ValueError(kind)


@pytest.mark.parametrize("n", [50257, 1000, 37, 16384])
@pytest.mark.parametrize("kind", ["normal", "flat", "ties", "masked"])
def test_sample_matches_oracle(hg, orc, n, kind):
    print(f"sample n {n} {kind}", flush=True)
    rng = np.random.default_rng(n * 7 + len(kind))
    cases = [(0.0, 0.9), (0.7, 0.9), (1.0, 0.95), (1.5, 0.999), (1.0, 1.0), (0.8, 0.0), (1.0, 0.3)]
    for i, (temp, top_p) in enumerate(cases):
        lg = _logits(rng, n, kind)
        seed = 1000 + i
        gp, gstate = hg.sample(lg, temp, top_p, seed)
        o = orc.Rng(seed)
        op = orc.sample(lg, temp, top_p, o)
        assert gp == op, (n, kind, temp, top_p)
        assert gstate == int(o.state.value), (n, kind, temp, top_p)


@pytest.mark.parametrize("temp,top_p,rep", [(0.9, 0.9, 1.3), (1.0, 1.0, 1.0), (1.2, 0.95, 1.1), (0.0, 0.9, 1.4)])
def test_generate_matches_oracle_tiny(hg, orc, temp, top_p, rep):
    path = gs.synth_path("tiny", 11, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    prompt = gs.prompt_ids(3, 12, gm.cfg.vocab_size)
    print(f"generate tiny temp {temp} top_p {top_p} rep {rep}", flush=True)
    g = gm.generate(prompt, 256, gm.new_cache(), temp=temp, top_p=top_p, seed=42, rep_penalty=rep)
    o = om.generate(prompt, 256, om.new_cache(), temp=temp, top_p=top_p, seed=42, rep_penalty=rep)
    assert len(o) == 256 and np.array_equal(g, o)


def test_generate_eos_and_context_stops(hg, orc):
    path = gs.synth_path("tiny", 4, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    prompt = gs.prompt_ids(9, 20, gm.cfg.vocab_size)
    free = om.generate(prompt, 100, om.new_cache(), temp=1.0, top_p=0.9, seed=3, eos=10**6)
    eos = int(free[57])
    first = int(np.argmax(free == eos))
    gkv, okv = gm.new_cache(), om.new_cache()
    g = gm.generate(prompt, 100, gkv, temp=1.0, top_p=0.9, seed=3, eos=eos)
    o = om.generate(prompt, 100, okv, temp=1.0, top_p=0.9, seed=3, eos=eos)
    assert len(o) == first and np.array_equal(g, o)
    assert gkv.len == 20 + first
    # the cache continues like the oracle's
    gl, _ = gm.forward(int(o[-1]) if len(o) else 1, gkv.len, gkv)
    ol = om.forward(int(o[-1]) if len(o) else 1, 20 + first, okv)
    assert np.array_equal(gl.view(np.uint32), ol.view(np.uint32))
    # context stop: a cache of 64 positions ends the generation at position 63
    g = gm.generate(prompt, 100, gm.new_cache(max_ctx=64), temp=1.0, top_p=0.9, seed=3, eos=10**6)
    assert len(g) == 64 - 20 and np.array_equal(g, free[:44])


def test_generate_matches_oracle_500m(hg, orc):
    path = gs.synth_path("500M", 1)
    gm, om = hg.Model(path), orc.Model(path)
    prompt = gs.prompt_ids(5, 24, 50257)
    print("generate 500M 128 steps", flush=True)
    g = gm.generate(prompt, 128, gm.new_cache(), temp=0.8, top_p=0.95, seed=2026, rep_penalty=1.2)
    o = om.generate(prompt, 128, om.new_cache(), temp=0.8, top_p=0.95, seed=2026, rep_penalty=1.2)
    assert np.array_equal(g, o)
