#!/usr/bin/env python3
"""Decode benchmark of the hobbylm sparse-MoE model on one MI355X.

Workload: the 500M-shaped model (d1024, 24 layers, GQA 16q/4kv hd64, layer 0 dense FFN 4096,
36 experts x 512 with top-6 + 1 shared, vocab 50257, tied embeddings), random-init Q8_0 GGUF
from seed 1, batch 1.  A seeded 16-token prompt is prefilled, the model decodes greedily to
position 2047 - steps, `warmup` of those steps run just before the timed window, and the
timed window is the last `steps` greedy decode steps ending at position 2047 (context ~2k).
Weights, the KV cache and the step's control block stay in HBM; the host collects the greedy
tokens once at the end of the window.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16]

Prints one JSON line.  Besides throughput it reports the per-kernel-class split of one step
(HIP events on the cache's stream), the dominant kernel's roofline, the step's algorithmic
HBM bandwidth, greedy-token parity with the committed oracle fixture, and a CPU baseline:
the oracle (a C restatement of hobby-rs's AVX2 path) timed on this host's cores over a
bounded sample of the same window, continuing from the GPU's KV cache.

    python bench.py --window-stats <rocprofv3 dir>   per-kernel stats of the timed window
"""
import argparse
import glob
import json
import os
import sqlite3
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

CTX_END = 2048          # the timed window ends at position CTX_END - 1
N_PROMPT = 16
PEAK_HBM = 8.0e12       # MI355X HBM3E, bytes/s
METRIC = "500M Q8_0 decode tok/s (bs1, ctx2k) + achieved HBM GB/s vs peak"
DOM_KERNEL = "k_attn_softmax_pv_res<64, false, true>"   # softmax + P.V after the QKV + scores launch
SCORES_KERNEL = "k_qkv_head<true, 0, false, 8, 64, true>"   # QKV rows + the attention scores
N_CALIB_STEPS = 2   # --pmc-calib decode steps at context 2049 (24 layers each)


def algorithmic_bytes(cfg, ctx, f32=False):
    """HBM bytes one decode step must read/write at context length ctx (positions 0..ctx-1).

    Matrices at 34 B per 32 Q8_0 weights (4 B per weight in the F32 mode): QKV and attn_output
    every layer, the dense FFN in the leading dense layers, top_k routed + the shared expert's
    gate/up/down in MoE layers, the lm_head; the F32 router and bias, the norm gains, one F32
    embedding row, the K/V row appended per layer and the K/V rows read per layer."""
    d, L, hd = cfg.d_model, cfg.n_layers, cfg.head_dim
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    q8 = (lambda n, k: n * k * 4) if f32 else (lambda n, k: n * k // 32 * 34)
    b = L * (q8(qd + 2 * kvd, d) + q8(d, qd))
    b += cfg.n_dense * (2 * q8(cfg.dense_ffn, d) + q8(d, cfg.dense_ffn))
    n_moe = L - cfg.n_dense
    slots = cfg.top_k + (1 if cfg.n_shared else 0)
    b += n_moe * slots * (2 * q8(cfg.expert_ffn, d) + q8(d, cfg.expert_ffn))
    b += q8(cfg.vocab_size, d)
    b += n_moe * (cfg.n_experts * d + cfg.n_experts) * 4            # router + bias
    b += (2 * L + 1) * d * 4 + L * 2 * hd * 4                        # norm gains, QK-norm gains
    b += d * 4                                                       # embedding row
    b += L * 2 * kvd * 4                                             # KV append
    b += L * 2 * kvd * 4 * ctx                                       # KV read
    return b


def attn_pv_bytes(cfg, ctx):
    """Algorithmic bytes of one softmax+P.V launch (one layer, all heads): the scores and V
    rows of every head's context (V of a kv group is shared by its query heads)."""
    return cfg.n_heads * ctx * 4 + cfg.n_kv_heads * ctx * cfg.head_dim * 4


def window_stats(prof_dir, steps):
    """Per-kernel duration statistics over the dispatches of the last `steps` decode steps
    of a rocprofv3 --kernel-trace run of this benchmark (one decode step ends with exactly one
    k_argmax_final dispatch)."""
    dbs = glob.glob(os.path.join(prof_dir, "**", "*.db"), recursive=True)
    rows = sqlite3.connect(dbs[0]).execute("select name, start, end from kernels order by start").fetchall()
    ends = [i for i, r in enumerate(rows) if "k_argmax_final" in r[0]]
    lo = ends[-steps - 1] + 1 if len(ends) > steps else 0
    agg = {}
    for name, s, e in rows[lo:ends[-1] + 1]:
        a = agg.setdefault(name, [0, 0.0])
        a[0] += 1
        a[1] += (e - s) / 1e3
    tot = sum(v[1] for v in agg.values())
    whole = {}
    for name, s, e in rows:
        a = whole.setdefault(name, [0, 0.0])
        a[0] += 1
        a[1] += (e - s) / 1e3
    print(f"# rocprofv3 kernel stats over the whole run ({len(rows)} dispatches)")
    print(f"{'calls':>7} {'avg_us':>9} {'total_us':>12}  kernel")
    for name, (c, t) in sorted(whole.items(), key=lambda kv: -kv[1][1])[:20]:
        print(f"{c:7d} {t / c:9.2f} {t:12.1f}  {name[:110]}")
    print()
    print(f"# rocprofv3 kernel stats over the last {steps} decode steps ({len(rows) - lo} dispatches)")
    print(f"{'pct':>6} {'calls':>7} {'avg_us':>9} {'total_us':>11}  kernel")
    for name, (c, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"{100 * t / tot:6.2f} {c:7d} {t / c:9.2f} {t:11.1f}  {name[:110]}")


def cpu_baseline(path, gm, gkv, tokens, start, budget_s, max_steps):
    """The oracle, continuing from the GPU's cache at position `start`, over the same tokens."""
    import oracle
    om = oracle.Model(path)
    okv = om.new_cache()
    c = gm.cfg
    kvd = c.n_kv_heads * c.head_dim
    K = np.empty((c.n_layers, start, kvd), np.float32)
    V = np.empty_like(K)
    for l in range(c.n_layers):
        K[l], V[l] = gkv[l]
    okv.load(K, V)
    valid = min(c.vocab_size, 50257)
    n = match = 0
    t0 = time.perf_counter()
    while n < max_steps and time.perf_counter() - t0 < budget_s:
        lg = om.forward(int(tokens[n]), start + n, okv)
        nxt = int(np.argmax(np.where(np.arange(c.vocab_size) < valid, lg, -np.inf)))
        match += nxt == int(tokens[n + 1])
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": oracle.threads(), "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{n} greedy decode steps at positions {start}..{start + n - 1} (context ~2k) of the "
                      f"same model, continuing from the GPU's KV cache; C restatement of hobby-rs's AVX2 "
                      f"decode path, rows in parallel over {oracle.threads()} OpenMP threads",
            "greedy_match": f"{match}/{n}"}


def cpu_model():
    """The host CPU's model name (as lscpu reports it) and logical CPU count."""
    name = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return f"{name} ({os.cpu_count()} logical CPUs visible)"


def op_matvec():
    """Operator-level Q8 matvec (quant.rs:106-136): seeded W ~ N(0, 0.02) quantized by the ggml
    Q8_0 algorithm, x ~ N(0, 1).  Hot: the same weights every call.  Cold: calls rotate through
    replicas totalling >= 320 MB, past the 256 MB last-level cache.  Bytes = N K 34/32 + 4K + 4N."""
    import hobbylm_amd as hg
    from hobbylm_amd import gguf_synth as gs
    rng = np.random.default_rng(2)
    rows = []
    for n, k, gather in [(1024, 1024, None), (3072, 1024, None), (512, 1024, None), (1024, 512, None),
                         (512, 1024, 36)]:
        nm = n * (gather or 1)
        w = (rng.standard_normal((nm, k)) * 0.02).astype(np.float32)
        t = hg.Q8Tensor.from_q8_0(gs.quantize_q8_0(w), nm, k)
        x = rng.standard_normal(k).astype(np.float32)
        if gather:
            ids = np.sort(rng.choice(gather, 6, replace=False)).astype(np.uint32)
            nbytes = 6 * n * k * 34 // 32 + 4 * k + 4 * 6 * n
            mat_bytes = nm * k * 34 // 32
            copies = max(1, -(-320 * 2**20 // mat_bytes))
            hot = t.time_matvec(x, reps=200, rows_per_mat=n, ids=ids)
            cold = t.time_matvec(x, reps=200, copies=copies, rows_per_mat=n, ids=ids)
            shape = f"gather 6 of [{gather}x{n}, {k}]"
        else:
            nbytes = n * k * 34 // 32 + 4 * k + 4 * n
            copies = max(1, -(-320 * 2**20 // (n * k * 34 // 32)))
            hot = t.time_matvec(x, reps=200)
            cold = t.time_matvec(x, reps=200, copies=copies)
            shape = f"{n}x{k}"
        for kind, us in (("hot", hot), ("cold", cold)):
            gbs = nbytes / (us * 1e-6) / 1e9
            rows.append({"shape": shape, "cache": kind, "us": round(us, 3), "bytes": nbytes,
                         "GBps": round(gbs, 1), "frac": round(gbs * 1e9 / PEAK_HBM, 4)})
        t.close()
    print(json.dumps({"metric": "Q8_0 matvec kernel time (bs1)", "unit": "us", "higher_is_better": False,
                      "reps": 200, "data": "synthetic: seeded N(0,0.02) weights, ggml Q8_0", "rows": rows}))


def op_attention():
    """One decode-attention layer (model.rs:199-233): 16 q / 4 kv heads of 64, seeded q, k, v
    and fp32 cache, append at pos = ctx - 1.  Bytes ~ 2 ctx 256 4 + 2 KB + 8 KB."""
    import hobbylm_amd as hg
    rows = []
    for ctx in (512, 2048, 4096, 7168, 8192):
        nbytes = 2 * ctx * 256 * 4 + 2048 + 8192
        for fast in (False, True):
            s_us, p_us = hg.attention_time(16, 4, 64, ctx, reps=50, fast=fast)
            us = s_us + p_us
            gbs = nbytes / (us * 1e-6) / 1e9
            rows.append({"ctx": ctx, "mode": "fast" if fast else "reference-order", "us": round(us, 2),
                         "us_split": [round(s_us, 2), round(p_us, 2)], "bytes": nbytes, "GBps": round(gbs, 1),
                         "frac": round(gbs * 1e9 / PEAK_HBM, 4)})
    print(json.dumps({"metric": "decode attention layer kernel time (16q/4kv, hd64, fp32 cache)", "unit": "us",
                      "higher_is_better": False, "reps": 50, "data": "synthetic seeded", "rows": rows}))


def batched_bytes(cfg, ctxs, experts_read):
    """Algorithmic HBM bytes of one batched decode step: every sequence's K/V rows read and its
    new row appended (49,152 B per position for the 500M shape), the matrices every step reads
    once for the whole batch (QKV, O, dense FFN, shared experts, lm_head, routers, norms), and
    the routed experts' matrices, each distinct (layer, expert) picked in the step read once."""
    d, L, hd = cfg.d_model, cfg.n_layers, cfg.head_dim
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    q8 = lambda n, k: n * k // 32 * 34
    b = L * (q8(qd + 2 * kvd, d) + q8(d, qd))
    b += cfg.n_dense * (2 * q8(cfg.dense_ffn, d) + q8(d, cfg.dense_ffn))
    n_moe = L - cfg.n_dense
    one_expert = 2 * q8(cfg.expert_ffn, d) + q8(d, cfg.expert_ffn)
    b += n_moe * (1 if cfg.n_shared else 0) * one_expert + experts_read * one_expert
    b += q8(cfg.vocab_size, d)
    b += n_moe * (cfg.n_experts * d + cfg.n_experts) * 4 + (2 * L + 1) * d * 4 + L * 2 * hd * 4
    kv_pos = L * 2 * kvd * 4
    b += sum(kv_pos * (c + 1) for c in ctxs) + len(ctxs) * d * 4
    return b


def batched(args):
    """Batched decode of the 500M model: 32 sequences with contexts drawn from U[256, 16384]
    (seed 7), paged KV (16-position pages, a seeded permutation of the pool as block tables),
    seeded cache rows written on the device; `warmup` greedy steps, then `steps` timed greedy
    steps of all sequences (each step one token per sequence, the step loop on the device)."""
    import hobbylm_amd as hg
    from hobbylm_amd import gguf_synth as gs
    rng = np.random.default_rng(7)
    n_seq, steps, warmup = args.batch, args.steps, args.warmup
    ctxs = [int(x) for x in rng.integers(256, 16385, n_seq)]
    path = gs.synth_path("500M_long", 1)
    m = hg.Model(path)
    cfg = m.cfg
    max_ctx = max(ctxs) + warmup + steps + 1
    need = [-(-(c + warmup + steps + 1) // 16) for c in ctxs]
    n_pages = sum(need)
    b = hg.Batch(m, n_seq, max_ctx=max_ctx, n_pages=n_pages)
    perm = rng.permutation(n_pages).astype(np.uint32)
    if args.contiguous_pages:
        perm = np.arange(n_pages, dtype=np.uint32)
    at = 0
    for s_, c in enumerate(ctxs):
        b.set_pages(s_, perm[at:at + need[s_]])
        at += need[s_]
        b.fill(s_, c, 1000 + s_)
    first = rng.integers(0, 50257, n_seq).astype(np.uint32)
    warm = b.decode_greedy(first, warmup) if warmup else first[None, :]
    start = [c + warmup for c in ctxs]
    # parity sample: the caches of two sequences (the longest and the shortest) before the window
    chk = [int(np.argmax(ctxs)), int(np.argmin(ctxs))]
    snaps = {s_: [b.read(s_, l) for l in range(cfg.n_layers)] for s_ in chk} if not args.no_cpu else {}
    # (hg_batch_decode_greedy returns once its stream has drained: the window is bracketed by
    # device synchronizations)
    t0 = time.perf_counter()
    ids = b.decode_greedy(warm[-1], steps)
    dt = time.perf_counter() - t0
    tok_s = n_seq * steps / dt
    # the distinct (layer, expert) pairs of the last step, over all sequences
    picks = set()
    for s_ in range(n_seq):
        idx, _ = b.routing(s_)
        for l in range(cfg.n_dense, cfg.n_layers):
            picks.update((l, int(e)) for e in idx[l])
    mean_ctx = [c + (steps - 1) / 2.0 for c in start]
    by = batched_bytes(cfg, mean_ctx, len(picks))
    ach = by * steps / dt
    parity = None
    if snaps:
        import oracle
        om = oracle.Model(path)
        kvd = cfg.n_kv_heads * cfg.head_dim
        n_chk = min(steps, args.parity_steps)
        ok = 0
        for s_ in chk:
            okv = om.new_cache()
            K = np.stack([kv[0] for kv in snaps[s_]])
            V = np.stack([kv[1] for kv in snaps[s_]])
            okv.load(K, V)
            del K, V
            tok = int(warm[-1][s_])
            for i in range(n_chk):
                lg = om.forward(tok, start[s_] + i, okv)
                tok = int(np.argmax(lg[:50257]))
                ok += tok == int(ids[i][s_])
        parity = {"sequences": [{"seq": s_, "context": start[s_]} for s_ in chk], "steps_each": n_chk,
                  "greedy_tokens_identical": f"{ok}/{len(chk) * n_chk}",
                  "oracle": "C restatement of hobby-rs's decode path, one Model::forward per sequence"}
    out = {
        "metric": "batched decode tok/s (500M Q8_0, 32 ragged sequences, paged KV) + achieved HBM GB/s vs peak",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(dt * 1e3 / steps, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 MFMA (i32 block sums) -> f32, f32 attention",
        "data": "synthetic: random-init 500M-shaped Q8_0 GGUF (seed 1, context_length 16896), seeded cache rows",
        "config": {"workload": f"{n_seq} sequences, contexts U[256,16384] (seed 7, sum {sum(ctxs)}), "
                               f"pages of 16 positions ({'in pool order' if args.contiguous_pages else 'shuffled'}), "
                               f"greedy decode of {steps} steps after {warmup}",
                   "model": "hobbylm-500M-synthetic", "global_batch": n_seq, "parallelism": "none (1 GPU)"},
        "step_bandwidth": {"algorithmic_bytes_per_step": by, "achieved_GBps": round(ach / 1e9, 1),
                           "peak_GBps": PEAK_HBM / 1e9, "frac": round(ach / PEAK_HBM, 4),
                           "experts_read": len(picks)},
        "parity": parity,
    }
    print(json.dumps(out))


def prefill_work(cfg, n):
    """Int8 multiply-accumulates of a prompt of n rows through the Q8 matrices (each row through
    QKV, O, the dense FFN or its top-k routed + shared experts), and the f32 multiply-adds of its
    causal attention (q.k and p.v over positions 0..t for row t, every query head)."""
    d, L, hd = cfg.d_model, cfg.n_layers, cfg.head_dim
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    per_row = L * ((qd + 2 * kvd) * d + d * qd)
    per_row += cfg.n_dense * 3 * cfg.dense_ffn * d
    per_row += (L - cfg.n_dense) * (cfg.top_k + (1 if cfg.n_shared else 0)) * 3 * cfg.expert_ffn * d
    attn = L * cfg.n_heads * hd * 2 * (n * (n + 1) // 2)
    return per_row * n, attn


def prefill_bench(args):
    """Prompt processing of the 500M model into the drop-in cache (capacity = context_length):
    a seeded prompt of --prefill rows, `warmup` untimed prompts, then the median of `repeats`
    timed ones, each into a fresh cache (host input rows to the last row's logits)."""
    import hobbylm_amd as hg
    from hobbylm_amd import gguf_synth as gs
    n = args.prefill
    path = gs.synth_path("500M", 1)
    m = hg.Model(path)
    cfg = m.cfg
    emb = np.stack([m.token_embedding(int(t)) for t in gs.prompt_ids(77, n, 50257)])
    for _ in range(max(min(args.warmup, 2), 1)):
        m.prefill(emb, m.new_cache())
    times = []
    for _ in range(args.repeats):
        kv = m.new_cache()
        t0 = time.perf_counter()
        lg, _ = m.prefill(emb, kv)
        times.append(time.perf_counter() - t0)
        del kv
    dt = float(np.median(times))
    macs, attn = prefill_work(cfg, n)
    out = {
        "metric": "prefill tok/s (500M Q8_0, one prompt into the default cache)",
        "value": round(n / dt, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.repeats, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 MFMA (i32 block sums) -> f32, f32 attention",
        "data": "synthetic: random-init 500M-shaped Q8_0 GGUF (seed 1), seeded prompt rows",
        "config": {"workload": f"prompt of {n} rows from position 0, cache capacity {cfg.context_length}",
                   "model": "hobbylm-500M-synthetic", "parallelism": "none (1 GPU)"},
        "work": {"int8_macs": macs, "attention_fmas": attn,
                 "int8_TOPs": round(2 * macs / dt / 1e12, 2), "int8_peak_TOPs": 5000.0,
                 "int8_frac": round(2 * macs / dt / 5.0e15, 5)},
        "times_ms": [round(t * 1e3, 3) for t in times],
    }
    if not args.no_cpu:
        import oracle
        om = oracle.Model(path)
        k = min(n, args.prefill_cpu_rows)
        okv = om.new_cache()
        t0 = time.perf_counter()
        ol = om.prefill(emb[:k], okv)
        cdt = time.perf_counter() - t0
        gl, _ = m.prefill(emb[:k], m.new_cache())
        out["cpu_baseline"] = {"value": round(k / cdt, 2), "unit": "tok/s", "cores": oracle.threads(),
                               "kind": "port", "sample": f"prefill of the first {k} rows of the prompt",
                               "model": cpu_model()}
        out["parity"] = {"rows": k, "logits_identical": bool(np.array_equal(gl.view(np.uint32), ol.view(np.uint32)))}
    print(json.dumps(out))


def f32_bench(args):
    """The F32 matrix mode (Engine::load(path, quant = false): f32 matrices, ops::dot) on the
    default workload's window: the 500M model, a 16-row prompt, greedy decode to position 1791,
    `warmup` steps, then `steps` timed greedy steps (median of `repeats`).  Parity: the oracle's
    F32 model continues from the GPU's cache at the window's start and must pick the same
    greedy tokens for the first --f32-parity-steps steps."""
    import torch
    import hobbylm_amd as hg
    from hobbylm_amd import gguf_synth as gs
    steps, warmup = args.steps, args.warmup
    start = CTX_END - steps
    path = gs.synth_path("500M", 1)
    m = hg.Model(path, quant=False)
    cfg = m.cfg
    kv = m.new_cache()
    emb = np.stack([m.token_embedding(int(t)) for t in gs.prompt_ids(1, N_PROMPT, 50257)])
    _, first = m.prefill(emb, kv)
    pre = m.decode_greedy(first, start - warmup - N_PROMPT, kv)
    warm = m.decode_greedy(int(pre[-1]), warmup, kv)
    snap = [kv.read(l) for l in range(cfg.n_layers)]
    times = []
    for r in range(max(1, args.repeats)):
        if r:
            kv.truncate(start)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ids_r = m.decode_greedy(int(warm[-1]), steps, kv)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        if r == 0:
            ids = ids_r
        elif list(ids_r) != list(ids):
            sys.exit("repeated window produced different tokens")
    dt = float(np.median(times))
    import oracle
    om = oracle.Model(path, quant=False)
    okv = om.new_cache()
    okv.load(np.stack([s_[0] for s_ in snap]), np.stack([s_[1] for s_ in snap]))
    del snap
    tok, ok, n_chk = int(warm[-1]), 0, min(steps, args.f32_parity_steps)
    for i in range(n_chk):
        lg = om.forward(tok, start + i, okv)
        tok = int(np.argmax(lg[:50257]))
        ok += tok == int(ids[i])
    by = algorithmic_bytes(cfg, CTX_END - steps / 2.0, f32=True)
    out = {
        "metric": "F32-mode decode tok/s (500M, f32 matrices, bs1, ctx 2k) + achieved HBM GB/s vs peak",
        "value": round(steps / dt, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(dt * 1e3 / steps, 4), "higher_is_better": True,
        "repeats_ms_per_step": [round(t * 1e3 / steps, 4) for t in times], "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 (ops::dot order)", "data": "synthetic: random-init 500M-shaped Q8_0 GGUF (seed 1) loaded as f32",
        "config": {"workload": "greedy decode positions 1792..2047 after a 16-token prompt, default cache",
                   "model": "hobbylm-500M-synthetic", "global_batch": 1, "seq_len": 2048, "parallelism": "none (1 GPU)"},
        "step_bandwidth": {"algorithmic_bytes_per_token": by, "achieved_GBps": round(by * steps / dt / 1e9, 1),
                           "peak_GBps": PEAK_HBM / 1e9, "frac": round(by * steps / dt / PEAK_HBM, 4)},
        "parity": {"greedy_tokens_identical": f"{ok}/{n_chk}",
                   "oracle": "C restatement of hobby-rs's F32 decode path, continuing from the GPU's cache"},
    }
    print(json.dumps(out))


COPY_BYTES = 256 * 2**20


def pmc_calib():
    """For rocprofv3 --pmc runs: 4 device copies of COPY_BYTES (the calibration of the byte
    counters); N_CALIB_STEPS decode steps of the bench model at context 2049 on the default
    cache (seeded KV rows; the '@ctx2049' dispatches of the attention kernels); then prefill +
    16 decode steps on a small cache (the other kernels' shapes do not depend on the context)."""
    import torch
    import hobbylm_amd as hg
    from hobbylm_amd import gguf_synth as gs
    a = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    m = hg.Model(gs.synth_path("500M", 1))
    c = m.cfg
    kv = m.new_cache()
    rng = np.random.default_rng(CTX_END)
    rows = rng.standard_normal((c.n_layers, CTX_END, c.n_kv_heads * c.head_dim), dtype=np.float32)
    kv.load(rows, rows[::-1].copy())
    del rows
    for i in range(N_CALIB_STEPS):
        m.forward(int(gs.prompt_ids(2, 1, 50257)[0]), CTX_END + i, kv)
    torch.cuda.synchronize()
    kv = m.new_cache(max_ctx=64)
    prompt = gs.prompt_ids(1, N_PROMPT, 50257)
    emb = np.stack([m.token_embedding(int(t)) for t in prompt])
    _, first = m.prefill(emb, kv)
    m.decode_greedy(first, 16, kv)
    torch.cuda.synchronize()
    print("pmc-calib done", flush=True)


def _counter_rows(d):
    """(kernel name, counter name, value) of every dispatch in a rocprofv3 --pmc output dir,
    in dispatch order."""
    import csv
    out = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            out.append((int(r["Dispatch_Id"]), r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"])))
    return [r[1:] for r in sorted(out)]


def pmc_stats(fetch_dir, write_dir):
    """Per-dispatch FETCH_SIZE and WRITE_SIZE (KiB) of the decode kernels, scaled so that the
    calibration copy (COPY_BYTES read, COPY_BYTES written) reads exactly its size."""
    res = {}
    factors = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = [r for r in _counter_rows(d) if r[1] == counter]
        copy = [v for k, c, v in rows if "copy" in k.lower() or "elementwise" in k.lower()]
        copy = [v for v in copy if v * 1024 > COPY_BYTES / 4]   # the 256 MiB copies only
        if not copy:
            raise SystemExit(f"no calibration copy found in {d}")
        f = COPY_BYTES / (float(np.median(copy)) * 1024)
        factors[counter] = f
        agg = {}
        for k, c, v in rows:
            if k.startswith("void hg::") or k.startswith("hg::"):
                name = k.split("(")[0].replace("void ", "").replace("hg::", "")
                agg.setdefault(name, []).append(v * 1024 * f)
        # the first N_CALIB_STEPS x n_layers dispatches of the attention kernels are --pmc-calib's
        # steps at context 2049
        for name in (SCORES_KERNEL, DOM_KERNEL):
            if name in agg:
                agg[name + " @ctx2049"] = agg[name][:N_CALIB_STEPS * 24]
                agg[name] = agg[name][N_CALIB_STEPS * 24:]
        for name, vals in agg.items():
            if vals:
                res.setdefault(name, {})[counter.lower() + "_bytes"] = float(np.mean(vals))
                res[name]["dispatches"] = len(vals)
    for name, r in res.items():
        r["hbm_bytes_per_dispatch"] = round(r.get("fetch_size_bytes", 0.0) + r.get("write_size_bytes", 0.0))
    return {"calibration": {"copy_bytes": COPY_BYTES, "factor_fetch": factors.get("FETCH_SIZE"),
                            "factor_write": factors.get("WRITE_SIZE")}, "kernels": res}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--repeats", type=int, default=3, help="timed windows; the median is reported")
    ap.add_argument("--window-stats", metavar="ROCPROF_DIR")
    ap.add_argument("--op", choices=["matvec", "attention"], help="operator-level measurement instead")
    ap.add_argument("--batched", action="store_true",
                    help="the batched workload: 32 ragged sequences over a paged cache (its own JSON line)")
    ap.add_argument("--batch", type=int, default=32, help="sequences of --batched")
    ap.add_argument("--prefill", type=int, metavar="ROWS", help="prompt-processing measurement of ROWS rows instead")
    ap.add_argument("--f32", action="store_true", help="the F32 matrix mode (quant = false) on the decode window instead")
    ap.add_argument("--f32-parity-steps", type=int, default=8, help="oracle-checked steps of --f32")
    ap.add_argument("--prefill-cpu-rows", type=int, default=128, help="oracle-timed rows of --prefill")
    ap.add_argument("--parity-steps", type=int, default=3, help="oracle-checked steps per sequence (--batched)")
    ap.add_argument("--contiguous-pages", action="store_true",
                    help="--batched: each sequence's pages in pool order instead of a seeded shuffle")
    ap.add_argument("--pmc-calib", action="store_true",
                    help="a copy of known size, then a short decode window (for rocprofv3 --pmc runs)")
    ap.add_argument("--pmc-stats", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="HBM traffic per dispatch from two rocprofv3 --pmc runs of --pmc-calib")
    args = ap.parse_args()
    if args.window_stats:
        window_stats(args.window_stats, args.steps)
        return
    if args.pmc_stats:
        print(json.dumps(pmc_stats(*args.pmc_stats)))
        return
    if args.op == "matvec":
        op_matvec()
        return
    if args.op == "attention":
        op_attention()
        return
    if args.pmc_calib:
        pmc_calib()
        return
    if args.prefill:
        if args.gpus != 1:
            sys.exit("bench.py measures one GPU")
        prefill_bench(args)
        return
    if args.batched:
        if args.gpus != 1:
            sys.exit("bench.py measures one GPU")
        batched(args)
        return
    if args.f32:
        if args.gpus != 1:
            sys.exit("bench.py measures one GPU")
        f32_bench(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this decode path does not shard (--gpus {args.gpus} requested)",
              file=sys.stderr)
        sys.exit(2)
    steps, warmup = args.steps, args.warmup
    start = CTX_END - steps
    if start - warmup < N_PROMPT + 1:
        sys.exit("--steps + --warmup leave no room for the prompt")

    import torch
    import hobbylm_amd as hg
    from hobbylm_amd import gguf_synth as gs

    path = gs.synth_path("500M", 1)
    m = hg.Model(path)
    cfg = m.cfg
    kv = m.new_cache()   # the drop-in default: capacity = context_length (8192)
    prompt = gs.prompt_ids(1, N_PROMPT, 50257)
    emb = np.stack([m.token_embedding(int(t)) for t in prompt])
    _, first = m.prefill(emb, kv)
    pre = m.decode_greedy(first, start - warmup - N_PROMPT, kv)
    warm = m.decode_greedy(int(pre[-1]), warmup, kv)
    assert kv.len == start
    snap = [kv.read(l) for l in range(cfg.n_layers)] if not args.no_cpu else None

    times = []
    for r in range(max(1, args.repeats)):
        if r:
            kv.truncate(start)   # the same window again: identical tokens, rows rewritten
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ids_r = m.decode_greedy(int(warm[-1]), steps, kv)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        if r == 0:
            ids = ids_r
        elif list(ids_r) != list(ids):
            sys.exit("repeated window produced different tokens")
    dt = float(np.median(times))
    tok_s = steps / dt

    # parity of the whole greedy stream with the oracle's fixture
    stream = [first] + [int(t) for t in pre] + [int(t) for t in warm] + [int(t) for t in ids]
    fx = os.path.join(ROOT, "tests", "golden", "greedy_500M.json")
    golden = None
    if os.path.exists(fx):
        g = json.load(open(fx))
        n = min(len(g["tokens"]), len(stream))
        golden = {"tokens_compared": n, "identical": g["tokens"][:n] == stream[:n]}

    # per-kernel-class split of one step at the window's end (pos 2048, a free row of the cache)
    prof = m.profile_step(int(ids[-1]), kv, reps=10)
    step_us = sum(v[0] for v in prof.values())
    dom = max(prof, key=lambda k: prof[k][0])
    mean_ctx = CTX_END - steps / 2.0
    bytes_step = algorithmic_bytes(cfg, mean_ctx)
    ach = bytes_step * tok_s
    dom_us = prof[dom][0] / prof[dom][1]
    if dom == "attn_softmax_pv":
        dom_bytes = attn_pv_bytes(cfg, CTX_END + 1)
        dom_note = "scores + V rows of all heads at context 2049 per launch (one layer)"
    else:
        dom_bytes = None
        dom_note = "no algorithmic byte count for this kernel class"
    roof = None
    if dom_bytes:
        a = dom_bytes / (dom_us * 1e-6)
        traffic, tnote = None, None
        tf = os.path.join(ROOT, "profiles", "traffic_decode_500M_ctx2k.json")
        if os.path.exists(tf):
            tj = json.load(open(tf))
            k = tj.get("kernels", {}).get(DOM_KERNEL + " @ctx2049")
            if k:
                traffic = k["hbm_bytes_per_dispatch"]
                tnote = f"rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch, copy-calibrated ({os.path.relpath(tf, ROOT)})"
        roof = {"bound": "hbm", "achieved": round(a / 1e9, 2), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": round(a / PEAK_HBM, 5), "traffic": traffic, "kernel": DOM_KERNEL,
                "avg_launch_us": round(dom_us, 2), "bytes_per_launch": dom_bytes, "bytes_note": dom_note}
        if tnote:
            roof["traffic_note"] = tnote

    cpu = None
    if not args.no_cpu:
        all_tokens = [int(warm[-1])] + [int(t) for t in ids]
        cpu = cpu_baseline(path, m, snap, all_tokens, start, args.cpu_seconds, steps)

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(dt * 1e3 / steps, 4), "higher_is_better": True,
        "repeats_ms_per_step": [round(t * 1e3 / steps, 4) for t in times],
        "scaling": "weak", "vs_baseline": None, "dtype": "int8xint8->f32 (Q8_0), f32 attention",
        "data": "synthetic: random-init 500M-shaped Q8_0 GGUF (seed 1), seeded 16-token prompt",
        "config": {"workload": f"hobbylm 500M-shaped sparse MoE, Q8_0, batch 1, greedy decode positions "
                               f"{start}..{CTX_END - 1} after a 16-token prompt",
                   "model": "hobbylm-500M-synthetic", "global_batch": 1, "seq_len": CTX_END,
                   "parallelism": "none (1 GPU)",
                   "kv_cache": f"f32, layer-major, capacity {cfg.context_length} (the default), "
                               f"reference-order reductions"},
        "step_bandwidth": {"algorithmic_bytes_per_token": bytes_step, "achieved_GBps": round(ach / 1e9, 2),
                           "peak_GBps": PEAK_HBM / 1e9, "frac": round(ach / PEAK_HBM, 5)},
        "roofline": roof,
        "kernel_split_us": {k: round(v[0], 2) for k, v in sorted(prof.items(), key=lambda kv: -kv[1][0])},
        "profiled_step_us": round(step_us, 1),
        "parity": golden,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
