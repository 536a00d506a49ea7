"""The F32 matrix mode (Engine::load(path, quant = false), lib.rs:85-92) against the oracle's.

Every matrix stays f32 (Mat::Owned, quant.rs:198-222) and is applied with ops::matvec /
ops::matmul, whose per-output arithmetic is ops::dot (ops.rs:7-71).  The prompt runs one step
per row with the routed experts added in expert-id order (ffn_prefill, model.rs:707-731), the
decode steps in rank order (ffn, model.rs:299-311).  Logits, greedy tokens, routing and every
KV row must equal the oracle's F32 model bit for bit.
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


def _pair(hg, orc, path, n_prompt, n_steps, seed):
    gm, om = hg.Model(path, quant=False), orc.Model(path, quant=False)
    assert gm.weight_bytes() == om.weight_bytes()
    V = gm.cfg.vocab_size
    valid = min(V, 50257)
    gkv, okv = gm.new_cache(), om.new_cache()
    emb = np.stack([om.token_embedding(int(t)) for t in gs.prompt_ids(seed, n_prompt, valid)])
    gl, gnext = gm.prefill(emb, gkv)
    ol = om.prefill(emb, okv)
    scale = np.float32(gm.cfg.expert_weights_scale)
    nd = gm.cfg.n_dense

    def check(step, gl, ol, gnext):
        assert _bits_equal(gl, ol), f"logits differ at step {step}"
        assert gnext == int(np.argmax(np.where(np.arange(V) < valid, ol, -np.inf))), step
        gi, gw = gkv.routing()
        oi, ow, _ = okv.routing()
        assert np.array_equal(gi[nd:], oi[nd:]), step
        assert _bits_equal(gw[nd:], ow[nd:] * scale), step

    check(-1, gl, ol, gnext)
    forced = gs.prompt_ids(seed + 1, n_steps, valid)
    for i in range(n_steps):
        pos = n_prompt + i
        gl, gnext = gm.forward(int(forced[i]), pos, gkv)
        ol = om.forward(int(forced[i]), pos, okv)
        check(i, gl, ol, gnext)
    for layer in range(gm.cfg.n_layers):
        gk, gv = gkv.read(layer)
        ok, ov = okv.read(layer)
        assert _bits_equal(gk, ok) and _bits_equal(gv, ov), layer
    return gm, om


@pytest.mark.parametrize("preset", ["tiny", "tiny_noshared", "tiny_softmax", "tiny_wnorm", "tiny_top1"])
def test_f32_prompt_and_steps_bit_exact(hg, orc, preset):
    _pair(hg, orc, gs.synth_path(preset, 21, norm_jitter=0.1), 9, 12, 5)


def test_f32_500m_bit_exact(hg, orc):
    """The 500M shape (a dense layer 0, 36 experts top-6 + 1 shared, vocabulary 50257)."""
    _pair(hg, orc, gs.synth_path("500M", 1), 16, 8, 9)


def test_f32_heads_of_128(hg, orc):
    _pair(hg, orc, gs.synth_path("joint12", 3), 5, 4, 13)


def test_f32_from_kquant_file(hg, orc):
    """Q5_0 / Q4_K / Q6_K / Q8_0 / F16 tensors dequantized at load (gguf.rs:361-468) and kept
    as f32 (Src::Owned -> Mat::Owned, quant.rs:213-222)."""
    _pair(hg, orc, gs.synth_path("tiny", 31, norm_jitter=0.1, qtype="kquant"), 7, 6, 17)


def test_f32_greedy_generation(hg, orc):
    path = gs.synth_path("tiny", 22, norm_jitter=0.1)
    gm, om = hg.Model(path, quant=False), orc.Model(path, quant=False)
    prompt = gs.prompt_ids(23, 7, 1000)
    got = gm.generate_greedy(prompt, 40, gm.new_cache(), eos=2 ** 32 - 1)
    want = om.generate_greedy(prompt, 40, om.new_cache(), eos=2 ** 32 - 1)
    assert list(got) == list(want)


def test_f32_mode_refuses_batched_paths(hg):
    """The batched prompt path and batched decode are Q8 GEMMs; the tree-reduction cache is not
    a parity mode: each is refused with HG_ERR_UNSUPPORTED (-3), not run on other arithmetic."""
    path = gs.synth_path("tiny", 24)
    gm = hg.Model(path, quant=False)
    with pytest.raises(hg.HgError) as e:
        gm.new_cache(fast=True)
    assert e.value.code == -3
    kv = gm.new_cache()
    blk = np.stack([gm.token_embedding(i) for i in (1, 2, 3)])
    with pytest.raises(hg.HgError) as e:
        gm.run_block(blk, kv, 0)
    assert e.value.code == -3
    with pytest.raises(hg.HgError) as e:
        hg.Batch(gm, 2)
    assert e.value.code == -3
