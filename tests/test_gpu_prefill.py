"""The prompt path (Model::prefill, model.rs:340-439) on the GPU: all prompt rows at once as
int8-MFMA GEMMs in Q8Tensor::matmul's order, causal paged attention and the expert-grouped FFN,
bit for bit against the oracle's prefill -- logits, greedy pick, the last row's routing and every
KV row of every layer -- for prompts of 1 to 2048 rows, prompts that continue a cache, prompts
split into chunks of rows, and the decode steps that follow."""
import os

import numpy as np
import pytest

from hobbylm_amd import gguf_synth as gs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hg():
    import hobbylm_amd
    hobbylm_amd.lib()
    return hobbylm_amd


@pytest.fixture(autouse=True)
def _batched_only(monkeypatch):
    """Every prompt here must take the batched path (an unsupported shape is an error)."""
    monkeypatch.setenv("HG_PREFILL", "batched")


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _embed(om, prompt):
    return np.stack([om.token_embedding(int(t)) for t in prompt])


def _check_state(gm, om, gkv, okv, gl, gnext, ol, layers=None):
    V = gm.cfg.vocab_size
    assert _bits_equal(gl, ol), "prefill logits differ"
    assert gnext == int(np.argmax(np.where(np.arange(V) < min(V, 50257), ol, -np.inf)))
    gi, _ = gkv.routing()
    oi, _, _ = okv.routing()
    c = gm.cfg
    moe = [l for l in range(c.n_layers) if l >= c.n_dense]
    assert np.array_equal(gi[moe], oi[moe]), "last row's routing differs"
    assert gkv.len == okv.len
    for layer in (layers if layers is not None else range(c.n_layers)):
        gk, gv = gkv.read(layer)
        ok, ov = okv.read(layer)
        assert _bits_equal(gk, ok) and _bits_equal(gv, ov), f"KV rows differ in layer {layer}"


@pytest.mark.parametrize("preset,n", [("tiny", 1), ("tiny", 16), ("tiny", 133), ("tiny_noshared", 70),
                                      ("tiny_softmax", 48), ("tiny_wnorm", 37)])
def test_prefill_bit_exact(hg, orc, preset, n):
    path = gs.synth_path(preset, 11, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    print(f"prefill {preset} rows {n}", flush=True)
    prompt = gs.prompt_ids(n, n, min(gm.cfg.vocab_size, 50257))
    emb = _embed(om, prompt)
    gkv, okv = gm.new_cache(), om.new_cache()
    gl, gnext = gm.prefill(emb, gkv)
    ol = om.prefill(emb, okv)
    _check_state(gm, om, gkv, okv, gl, gnext, ol)
    # decode continues from the prompt's cache
    tok = gnext
    for i in range(4):
        gl, gnext = gm.forward(tok, n + i, gkv)
        ol = om.forward(tok, n + i, okv)
        assert _bits_equal(gl, ol), f"decode step {i} after the prompt"
        tok = gnext


def test_prefill_continues_cache_in_chunks(hg, orc, monkeypatch):
    """A prompt after decoded positions (base > 0), split into chunks of 64 rows (each chunk's
    attention reads the earlier chunks through the cache)."""
    path = gs.synth_path("tiny", 3, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    V = min(gm.cfg.vocab_size, 50257)
    gkv, okv = gm.new_cache(), om.new_cache()
    p0 = gs.prompt_ids(5, 40, V)
    gm.prefill(_embed(om, p0), gkv)
    om.prefill(_embed(om, p0), okv)
    for i, t in enumerate(gs.prompt_ids(6, 3, V)):
        gm.forward(int(t), 40 + i, gkv)
        om.forward(int(t), 40 + i, okv)
    monkeypatch.setenv("HG_PREFILL_CHUNK", "64")
    p1 = _embed(om, gs.prompt_ids(7, 300, V))
    print("prefill tiny base 43 rows 300 chunks of 64", flush=True)
    gl, gnext = gm.prefill(p1, gkv)
    ol = om.prefill(p1, okv)
    _check_state(gm, om, gkv, okv, gl, gnext, ol)


def test_prefill_2048_rows(hg, orc):
    path = gs.synth_path("tiny_long", 9, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    prompt = gs.prompt_ids(2048, 2048, min(gm.cfg.vocab_size, 50257))
    emb = _embed(om, prompt)
    gkv, okv = gm.new_cache(), om.new_cache()
    print("prefill tiny_long rows 2048", flush=True)
    gl, gnext = gm.prefill(emb, gkv)
    ol = om.prefill(emb, okv)
    _check_state(gm, om, gkv, okv, gl, gnext, ol)


def test_prefill_joint12_hd128(hg, orc):
    """Heads of 128 (the joint12 shape: 12q/3kv, 36 x 320 experts, a 2304-wide dense layer)."""
    path = gs.synth_path("joint12", 5)
    gm, om = hg.Model(path), orc.Model(path)
    prompt = gs.prompt_ids(3, 80, 50257)
    emb = _embed(om, prompt)
    gkv, okv = gm.new_cache(max_ctx=512), om.new_cache()
    print("prefill joint12 rows 80", flush=True)
    gl, gnext = gm.prefill(emb, gkv)
    ol = om.prefill(emb, okv)
    _check_state(gm, om, gkv, okv, gl, gnext, ol, layers=(0, 1, 15))


@pytest.mark.parametrize("n", [16, 512])
def test_prefill_500m(hg, orc, n):
    path = gs.synth_path("500M", 1)
    gm, om = hg.Model(path), orc.Model(path)
    prompt = gs.prompt_ids(n + 1, n, 50257)
    emb = _embed(om, prompt)
    gkv, okv = gm.new_cache(), om.new_cache()
    print(f"prefill 500M rows {n}", flush=True)
    gl, gnext = gm.prefill(emb, gkv)
    ol = om.prefill(emb, okv)
    _check_state(gm, om, gkv, okv, gl, gnext, ol, layers=(0, 1, 12, 23))
