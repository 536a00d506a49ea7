"""Writes the golden fixtures of the long decode runs with the CPU oracle.

    python tests/golden/make_golden.py [130M|500M ...]

Each fixture holds the synthetic GGUF's sha256 (so a run on another machine proves it
rebuilt the same bytes), the seeded prompt, every greedy token, and at a few positions a
fingerprint of the logits (top-5 ids and values, and 64 logits at fixed indices).
The oracle is the checker: this script only runs it, here, to produce data.
"""
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from hobbylm_amd import gguf_synth as gs  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
RUNS = {
    # config 1: 130M preset, seed 0, 64 greedy tokens after a seeded 16-token prompt
    "130M": dict(preset="130M", seed=0, prompt_seed=0, n_prompt=16, n_new=64, fp_at=(0, 1, 31, 63)),
    # config 4: the 500M-shaped model, seed 1, greedy to position 2047 (the timed window
    # of the decode benchmark is positions 1792..2047)
    "500M": dict(preset="500M", seed=1, prompt_seed=1, n_prompt=16, n_new=2032,
                 fp_at=(0, 1, 1775, 1776, 1777, 1900, 2031)),
    # the same model driven by seeded random tokens (teacher forcing): a non-degenerate input
    # stream, with the argmax and the logit fingerprint of every step
    "500M_forced": dict(preset="500M", seed=1, prompt_seed=1, n_prompt=16, n_new=96,
                        fp_at=tuple(range(96)), forced_seed=2),
}
FP_IDX = np.linspace(0, 50256, 64).astype(np.int64)


def fingerprint(lg):
    top = np.argsort(-lg.astype(np.float64), kind="stable")[:5]
    return {"top5_ids": [int(i) for i in top], "top5_vals": [float(lg[i]) for i in top],
            "probe": [float(lg[i]) for i in FP_IDX if i < lg.size]}


def run(name):
    cfg = RUNS[name]
    path = gs.synth_path(cfg["preset"], cfg["seed"])
    m = oracle.Model(path)
    kv = m.new_cache()
    V = m.cfg.vocab_size
    valid = min(V, 50257)
    prompt = gs.prompt_ids(cfg["prompt_seed"], cfg["n_prompt"], 50257)
    emb = np.stack([m.token_embedding(int(t)) for t in prompt])
    t0 = time.time()
    lg = m.prefill(emb, kv)
    toks, fps, gaps = [], {}, []
    forced = gs.prompt_ids(cfg["forced_seed"], cfg["n_new"], 50257) if "forced_seed" in cfg else None
    for i in range(cfg["n_new"]):
        masked = np.where(np.arange(V) < valid, lg, -np.inf)
        nxt = int(np.argmax(masked))
        s = np.sort(masked[np.isfinite(masked)])
        gaps.append(float(s[-1] - s[-2]))
        if i in cfg["fp_at"]:
            fps[str(i)] = fingerprint(lg)
        toks.append(nxt)
        if i + 1 < cfg["n_new"]:
            feed = int(forced[i]) if forced is not None else nxt
            lg = m.forward(feed, cfg["n_prompt"] + i, kv)
        if i % 200 == 0:
            print(name, i, round(time.time() - t0, 1), "s", flush=True)
    out = {"preset": cfg["preset"], "seed": cfg["seed"], "generator_version": gs.GENERATOR_VERSION,
           "gguf_sha256": gs.file_sha256(path), "prompt": [int(t) for t in prompt],
           "tokens": toks, "logit_fingerprints": fps,
           "forced": [int(t) for t in forced] if forced is not None else None, "min_top1_gap": min(gaps),
           "threads": oracle.threads(), "seconds": round(time.time() - t0, 1)}
    with open(os.path.join(HERE, f"greedy_{name}.json"), "w") as f:
        json.dump(out, f)
    print(name, "done", out["seconds"], "s, min top1 gap", out["min_top1_gap"], flush=True)


if __name__ == "__main__":
    for name in (sys.argv[1:] or list(RUNS)):
        run(name)
