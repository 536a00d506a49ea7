"""Drives the oracle built with AddressSanitizer / UndefinedBehaviorSanitizer (its path in
ORACLE_LIB) through every entry the tests use, on the tiny shapes: load (valid and malformed
files), forward, prefill, the greedy and sampled generations, the sampler, run_block,
forward_bidir and both diffusion decoders.  Run by tests/test_sanitizers.py with the sanitizer
runtime preloaded; prints OK at the end."""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", ".."))
import oracle  # noqa: E402
from hobbylm_amd import gguf_synth as gs  # noqa: E402



def main():
    bad = sys.argv[1:]
    for p in bad:   # malformed files: errors, never faults
        try:
            oracle.Model(p)
        except oracle.OracleError:
            pass
    for preset in ("tiny", "tiny_noshared", "tiny_softmax", "tiny_wnorm"):
        m = oracle.Model(gs.synth_path(preset, 11, norm_jitter=0.1))
        V = m.cfg.vocab_size
        ids = gs.prompt_ids(1, 9, min(V, 50257))
        kv = m.new_cache()
        m.prefill(np.stack([m.token_embedding(int(t)) for t in ids]), kv)
        for i in range(3):
            m.forward(int(ids[i]), 9 + i, kv)
        m.generate(ids, 8, m.new_cache(), temp=0.9, top_p=0.9, seed=3, rep_penalty=1.3)
        m.generate_greedy(ids, 8, m.new_cache(), rep_penalty=1.2)
    r = oracle.Rng(5)
    for n, tp in ((37, 0.9), (1000, 1.0), (50257, 0.95)):
        oracle.sample(np.random.default_rng(n).standard_normal(n).astype(np.float32), 0.8, tp, r)
    m = oracle.Model(gs.synth_path("tiny_diff", 5, norm_jitter=0.1))
    ids = gs.prompt_ids(2, 6, 50257)
    emb = np.stack([m.token_embedding(int(t)) for t in ids])
    kv = m.new_cache()
    m.prefill(emb, kv)
    m.run_block(emb, kv, 6, want_kv=True)
    m.forward_bidir(emb)
    for cached in (True, False):
        m.generate_diffusion(ids, oracle.DiffOpts.make(gen_len=16, block=8, steps=4, remask_steps=1, cached=cached,
                                                       threshold=0.05 if cached else 0.0))
    print("OK")


if __name__ == "__main__":
    main()
