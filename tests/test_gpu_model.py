"""Model-level parity of the HIP decode path against the CPU oracle.

The default cache (reference-order reductions) must reproduce the oracle bit for bit:
logits, greedy tokens, per-layer routing and every KV-cache row.  HG_KV_FAST caches (tree
reductions in RMSNorm and attention) are not a parity mode: near-tied routing decisions can
flip, so they are only checked for a short horizon on a small model.
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


def _run_pair(hg, orc, path, n_prompt, n_steps, fast=False, seed=7, forced=False):
    """Prefill a seeded prompt then decode n_steps on both paths; return per-step records."""
    gm = hg.Model(path)
    om = orc.Model(path)
    V = gm.cfg.vocab_size
    gkv = gm.new_cache(fast=fast)
    okv = om.new_cache()
    prompt = gs.prompt_ids(seed, n_prompt, min(V, 50257))
    emb = np.stack([om.token_embedding(int(t)) for t in prompt])
    assert _bits_equal(emb, np.stack([gm.token_embedding(int(t)) for t in prompt]))
    gl, gnext = gm.prefill(emb, gkv)
    ol = om.prefill(emb, okv)
    recs = [(gl, ol, gnext, gkv.routing(), okv.routing())]
    forced_toks = gs.prompt_ids(seed + 1, n_steps, min(V, 50257))
    valid = min(V, 50257)
    tok = gnext
    for i in range(n_steps):
        otok = int(np.argmax(np.where(np.arange(V) < valid, ol, -np.inf)))
        assert tok == otok, f"greedy token differs at step {i}"
        if forced:
            tok = int(forced_toks[i])
        pos = n_prompt + i
        gl, gnext = gm.forward(tok, pos, gkv)
        ol = om.forward(tok, pos, okv)
        recs.append((gl, ol, gnext, gkv.routing(), okv.routing()))
        tok = gnext
    return gm, om, gkv, okv, recs


@pytest.mark.parametrize("preset", ["tiny", "tiny_noshared", "tiny_softmax", "tiny_wnorm"])
def test_reference_order_bit_exact(hg, orc, preset):
    path = gs.synth_path(preset, 11, norm_jitter=0.1)
    gm, om, gkv, okv, recs = _run_pair(hg, orc, path, 9, 12, forced=True)
    # the device records the weight the expert output is multiplied by, w * expert_weights_scale
    # in f32 (model.rs:307); the oracle records w
    scale = np.float32(gs.PRESETS[preset].expert_weights_scale)
    for i, (gl, ol, gnext, (gi, gw), (oi, ow, _)) in enumerate(recs):
        assert _bits_equal(gl, ol), f"logits differ at step {i}"
        assert np.array_equal(gi[gm.cfg.n_dense:], oi[gm.cfg.n_dense:]), i
        assert _bits_equal(gw[gm.cfg.n_dense:], ow[gm.cfg.n_dense:] * scale), i
    for layer in range(gm.cfg.n_layers):
        gk, gv = gkv.read(layer)
        ok, ov = okv.read(layer)
        assert _bits_equal(gk, ok) and _bits_equal(gv, ov), layer


def test_fast_cache_short_horizon(hg, orc):
    """HG_KV_FAST on the tiny model: the prompt and the first steps stay within 1e-3."""
    path = gs.synth_path("tiny", 12, norm_jitter=0.1)
    gm, om, gkv, okv, recs = _run_pair(hg, orc, path, 9, 3, fast=True, forced=True)
    for i, (gl, ol, gnext, (gi, gw), (oi, ow, gap)) in enumerate(recs):
        assert np.all(np.isfinite(gl))
        assert np.max(np.abs(gl - ol)) <= 1e-3 * (ol.max() - ol.min()), i


def test_130m_exact_bit_exact(hg, orc):
    """The 130M preset: K = 192 expert rows (partial chunk), top-8 of 32, vocab 50304 (masked ids)."""
    path = gs.synth_path("130M", 0)
    gm, om, gkv, okv, recs = _run_pair(hg, orc, path, 16, 6)
    for i, (gl, ol, gnext, (gi, gw), (oi, ow, _)) in enumerate(recs):
        assert _bits_equal(gl, ol), i
        assert np.array_equal(gi[1:], oi[1:]), i


def test_greedy_device_loop_matches_forward(hg, orc):
    path = gs.synth_path("tiny", 13, norm_jitter=0.1)
    gm = hg.Model(path)
    om = orc.Model(path)
    prompt = gs.prompt_ids(3, 6, gm.cfg.vocab_size)
    kv1 = gm.new_cache()
    emb = np.stack([gm.token_embedding(int(t)) for t in prompt])
    _, first = gm.prefill(emb, kv1)
    ids = gm.decode_greedy(first, 20, kv1)
    ref = om.generate_greedy(prompt, 21, om.new_cache(), eos=2 ** 32 - 1)
    assert list(ref) == [first] + list(ids)
    gen = gm.generate_greedy(prompt, 21, gm.new_cache(), eos=2 ** 32 - 1)
    assert list(gen) == list(ref)
    # repetition penalty path (logits on the host) and the EOS stop
    ref_rp = om.generate_greedy(prompt, 15, om.new_cache(), rep_penalty=1.3, eos=2 ** 32 - 1)
    gen_rp = gm.generate_greedy(prompt, 15, gm.new_cache(), rep_penalty=1.3, eos=2 ** 32 - 1)
    assert list(gen_rp) == list(ref_rp)
    eos = int(ref[3])
    assert list(gm.generate_greedy(prompt, 21, gm.new_cache(), eos=eos)) == \
        list(om.generate_greedy(prompt, 21, om.new_cache(), eos=eos))


def test_forward_x_and_errors(hg, orc):
    path = gs.synth_path("tiny", 14)
    gm = hg.Model(path)
    om = orc.Model(path)
    kv, okv = gm.new_cache(), om.new_cache()
    x = np.random.default_rng(0).standard_normal(gm.cfg.d_model).astype(np.float32)
    gl, _ = gm.forward_x(x, 0, kv)
    assert _bits_equal(gl, om.forward_x(x, 0, okv))
    with pytest.raises(hg.HgError):
        gm.forward(gm.cfg.vocab_size, 1, kv)      # token out of range
    with pytest.raises(hg.HgError):
        gm.forward(1, 5, kv)                      # pos does not continue the cache
    small = gm.new_cache(max_ctx=2)
    gm.forward(1, 0, small)
    gm.forward(1, 1, small)
    with pytest.raises(hg.HgError):
        gm.forward(1, 2, small)                   # beyond the cache
    assert gm.weight_bytes() == om.weight_bytes()


def test_kquant_file_bit_exact(hg, orc):
    """A Q4_K / Q6_K / Q5_0 file (dequantized then requantized at load, quant.rs:78-102)."""
    path = gs.synth_path("tiny", 31, norm_jitter=0.1, qtype="kquant")
    gm, om, gkv, okv, recs = _run_pair(hg, orc, path, 9, 8, forced=True)
    for i, (gl, ol, gnext, (gi, gw), (oi, ow, _)) in enumerate(recs):
        assert _bits_equal(gl, ol), f"logits differ at step {i}"
        assert np.array_equal(gi[1:], oi[1:]), i


def test_joint12_shape_bit_exact(hg, orc):
    """The published joint12 shape: d768, 16 layers, 12q/3kv heads of 128, 36 x 320 experts,
    theta 1e6, vocab 50304 (hobby-rs/README.md:9,35)."""
    path = gs.synth_path("joint12", 5)
    gm, om, gkv, okv, recs = _run_pair(hg, orc, path, 16, 6)
    for i, (gl, ol, gnext, (gi, gw), (oi, ow, _)) in enumerate(recs):
        assert _bits_equal(gl, ol), f"logits differ at step {i}"
        assert np.array_equal(gi[1:], oi[1:]), i
    for layer in (0, 7, 15):
        gk, gv = gkv.read(layer)
        ok, ov = okv.read(layer)
        assert _bits_equal(gk, ok) and _bits_equal(gv, ov), layer


@pytest.mark.parametrize("start", [3050, 7150, 8176])
def test_default_capacity_cache_bit_exact(hg, orc, start):
    """The drop-in cache (max_ctx = 0: capacity = context_length = 8192) on the 500M model,
    seeded with the same KV rows on both paths, decoding forced tokens across attention
    windows: across the resident softmax/P.V kernel's sum layouts (start 3050: 12 to 16 terms
    per lane), from that kernel (<= 7168 positions) into the ring kernel (start 7150), and up to
    the last position of the cache (start 8176)."""
    path = gs.synth_path("500M", 1)
    gm, om = hg.Model(path), orc.Model(path)
    c = gm.cfg
    gkv, okv = gm.new_cache(), om.new_cache()
    assert c.context_length == 8192
    rng = np.random.default_rng(start)
    kvd = c.n_kv_heads * c.head_dim
    k = rng.standard_normal((c.n_layers, start, kvd), dtype=np.float32)
    v = rng.standard_normal((c.n_layers, start, kvd), dtype=np.float32)
    gkv.load(k, v)
    okv.load(k, v)
    del k, v
    toks = gs.prompt_ids(start, min(24, c.context_length - start), 50257)
    for i, t in enumerate(toks):
        pos = start + i
        gl, gnext = gm.forward(int(t), pos, gkv)
        ol = om.forward(int(t), pos, okv)
        assert _bits_equal(gl, ol), f"logits differ at pos {pos}"
        assert gnext == int(np.argmax(ol[:50257])), pos
        gi, _ = gkv.routing()
        oi, _, _ = okv.routing()
        assert np.array_equal(gi[1:], oi[1:]), pos
    gk, gv = gkv.read(c.n_layers - 1)
    ok, ov = okv.read(c.n_layers - 1)
    assert _bits_equal(gk, ok) and _bits_equal(gv, ov)


def test_bounded_waits_report_an_error(hg, orc, monkeypatch):
    """The softmax/P.V kernels' LDS waits are bounded (StepParams::spin_cap polls, HG_SPIN_CAP
    overrides the default for tests).  With a cap of one poll the V waves' wait for the exact
    sum (~1 us) gives up: the kernels still run to their normal exit and the call returns
    HG_ERR_DEVICE (-5) instead of results.  With the default cap the same model then decodes
    bit-identically to the oracle on a fresh cache."""
    path = gs.synth_path("tiny", 31, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    toks = gs.prompt_ids(32, 6, 1000)
    emb = np.stack([om.token_embedding(int(t)) for t in toks])
    monkeypatch.setenv("HG_SPIN_CAP", "1")
    kv = gm.new_cache()
    codes = []
    for i, t in enumerate(toks):
        try:
            gm.forward(int(t), kv.len, kv)
            codes.append(0)
        except hg.HgError as e:
            codes.append(e.code)
    assert codes and set(codes) <= {0, -5} and -5 in codes, codes
    monkeypatch.delenv("HG_SPIN_CAP")
    gkv, okv = gm.new_cache(), om.new_cache()
    gl, _ = gm.prefill(emb, gkv)
    ol = om.prefill(emb, okv)
    assert _bits_equal(gl, ol)
    for i in range(4):
        gl, _ = gm.forward(int(toks[i]), len(toks) + i, gkv)
        ol = om.forward(int(toks[i]), len(toks) + i, okv)
        assert _bits_equal(gl, ol), i


@pytest.mark.parametrize("preset,start,rows", [("500M", 2040, False), ("tiny_wnorm", 0, True), ("130M", 0, True)])
def test_scores_in_qkv_launch(hg, orc, monkeypatch, preset, start, rows):
    """Head-64 reference-order steps form the attention scores inside the QKV launch (each score
    workgroup forms its own q head; the softmax + P.V kernel forms the score at pos).  Logits,
    routing and KV rows must equal both the oracle's and those of the separate scores launch
    (HG_QKV_SCORES=0), bit for bit: for the 500M model from seeded KV rows across the windows
    of 2048 and 2304 positions, and for the head-64 presets through a prompt run as one
    replayed step per row (prompt order, HG_PREFILL=rows) followed by decode steps."""
    path = gs.synth_path(preset, 5, norm_jitter=0.1)
    gm, om = hg.Model(path), orc.Model(path)
    c = gm.cfg
    assert c.head_dim == 64
    valid = min(c.vocab_size, 50257)
    rng = np.random.default_rng(start + 1)
    kvd = c.n_kv_heads * c.head_dim
    k = v = None
    if start:
        k = rng.standard_normal((c.n_layers, start, kvd), dtype=np.float32)
        v = rng.standard_normal((c.n_layers, start, kvd), dtype=np.float32)
    prompt = gs.prompt_ids(start + 2, 0 if start else 11, valid)
    toks = gs.prompt_ids(start + 3, 16, valid)
    if rows:
        monkeypatch.setenv("HG_PREFILL", "rows")

    def run(env, dev):
        if env is None:
            monkeypatch.delenv("HG_QKV_SCORES", raising=False)
        else:
            monkeypatch.setenv("HG_QKV_SCORES", env)
        m = gm if dev else om
        kv = m.new_cache()
        if start:
            kv.load(k, v)
        out = []
        if len(prompt):
            emb = np.stack([om.token_embedding(int(t)) for t in prompt])
            r = m.prefill(emb, kv)
            out.append(r[0] if dev else r)
        for i, t in enumerate(toks):
            r = m.forward(int(t), start + len(prompt) + i, kv)
            out.append(r[0] if dev else r)
        return out, kv.routing()[0], kv.read(c.n_layers - 1)

    fused, sep, ref = run(None, True), run("0", True), run(None, False)
    for i, (a, b, o) in enumerate(zip(fused[0], sep[0], ref[0])):
        assert _bits_equal(a, o), f"logits differ from the oracle at step {i}"
        assert _bits_equal(a, b), f"fused and separate scores differ at step {i}"
    nd = c.n_dense
    assert np.array_equal(fused[1][nd:], ref[1][nd:]) and np.array_equal(sep[1][nd:], ref[1][nd:])
    for a, b, o in zip(fused[2], sep[2], ref[2]):
        assert _bits_equal(a, o) and _bits_equal(b, o)
