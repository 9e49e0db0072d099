#!/usr/bin/env python3
"""Benchmark of the north-star path: speculative decoding on one MI355X with a
Llama-3-8B-shape Q4_K target and a Llama-3.2-1B-shape Q4_K draft (BASELINE.json
configs[2]), k = 7, f16 KV prefilled to 4096 positions, batch 1, greedy.

A "step" is one speculative step (sh_spec_step): 7 greedy draft tokens on the
device, one verify forward of k+1 = 8 tokens with all-position logits, greedy
acceptance and KV rollback. value = accepted tok/s over the timed steps, the
reference's own definition (generated tokens / decode seconds,
apps/seeker-cli/src/commands/run.rs:702-710). Weights and KV are resident in
HBM before timing; synthetic random-init weights (N(0, 0.02) quantized to Q4_K).

Also reported: verify-step latency and HBM roofline (hipEvents inside the
library), the dominant kernel's roofline, and the CPU oracle's speculative step
timed on this host's cores from the same state (with a token-for-token check).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       python bench.py --profile-only   (target verify steps only, for rocprofv3: the
           KV position is set to the context length without a prefill, which leaves
           the bytes read and the work done unchanged)

roofline.traffic (HBM bytes per launch of the dominant kernel) comes from
profiles/verify_8b_q4k_traffic.json, written from rocprofv3 FETCH_SIZE /
WRITE_SIZE runs of `bench.py --profile-only`, when it names the same kernel.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16 MFMA, MI355X


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def verify_bytes(d, P, L):
    """Algorithmic bytes of one verify step: every Q4_K weight matrix (144 B per
    256 elements, lm_head included, norms and the L gathered embedding rows
    excluded) + f16 K/V read for [0, P+L) + K/V write of L rows."""
    dkv = d.head_dim * d.n_head_kv
    per_layer = (2 * d.n_embd * d.n_embd + 2 * dkv * d.n_embd + 3 * d.n_ff * d.n_embd)
    elems = d.n_layer * per_layer + d.n_vocab * d.n_embd
    w = elems * 144 // 256
    kv_read = 2 * d.n_layer * (P + L) * dkv * 2
    kv_write = 2 * d.n_layer * L * dkv * 2
    return w, kv_read, kv_write


def measured_traffic(kernel_tag):
    """HBM bytes per launch (FETCH + WRITE, calibrated) of kernel_tag from the
    committed rocprofv3 counter summary, or None."""
    path = os.path.join(ROOT, "profiles", "verify_8b_q4k_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    k = t.get("kernels", {}).get(kernel_tag)
    return None if k is None else k["fetch_bytes"] + k["write_bytes"]


def measure_draft(eng, P=4096, reps=30):
    """The draft forward alone (1B shape, 1 column, context P): eager
    sh_forward_full calls with greedy logits at KV position P (set without a
    prefill; the bytes read and the work are the same), then a pass with
    per-kernel profiling events. Bytes per forward: every weight matrix once +
    f16 K/V read for [0, P + 1) + one K/V row written."""
    import numpy as np
    from seeker_amd import synth as S
    img = S.GgufImage(S.L1B_DRAFT, seed=1)
    dm = eng.upload_weights(img)
    img.close()
    d = dm.dims
    kv = eng.allocate_kv_cache(dm, P + 64)
    tok = [int(S.tokens(5, 1, d.n_vocab)[0])]
    for _ in range(3):
        kv.set_position(P)
        eng.forward_full_readback(dm, kv, tok, P, full_logits=False, want_residual=False)
    lat = []
    for _ in range(reps):
        kv.set_position(P)
        t = time.perf_counter()
        eng.forward_full_readback(dm, kv, tok, P, full_logits=False, want_residual=False)
        lat.append((time.perf_counter() - t) * 1e3)
    eng.set_profiling(True)
    eng.profile(reset=True)
    for _ in range(reps):
        kv.set_position(P)
        eng.forward_full_readback(dm, kv, tok, P, full_logits=False, want_residual=False)
    prof = eng.profile(reset=True)
    eng.set_profiling(False)
    kv.close()
    dm.close()
    w, kr, kw = verify_bytes(d, P, 1)
    kern_ms = sum(s["ms"] for s in prof.values()) / reps
    per = {n: round(s["ms"] / reps * 1e3, 2) for n, s in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])}
    log(f"draft forward (P={P}): median {statistics.median(lat):.3f} ms eager wall, {kern_ms:.3f} ms in kernels; "
        f"us/forward by kernel {per}")
    return {"config": f"1B draft shape, 1 column, ctx {P}, eager", "wall_ms": round(statistics.median(lat), 4),
            "kernel_ms": round(kern_ms, 4), "alg_bytes": w + kr + kw, "kernel_us": per}


def measure_rejection(eng, tm, dm, tkv, dkv, last, k, steps, warmup=2, T=0.8, seed=5):
    """REJECTION spec steps at temperature T (graph-replayed like the greedy
    steps): draft i drawn from softmax(q / T), accepted iff u q(d) < p(d),
    first rejection resampled from max(0, p - q)."""
    from seeker_amd._native import sh_sampling
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = 2, T, seed, 0
    for _ in range(warmup):
        last = eng.decode_speculative(tm, dm, tkv, dkv, last, k, s).last_token
    eng.sync()
    t = time.perf_counter()
    emitted = accepted = 0
    for _ in range(steps):
        r = eng.decode_speculative(tm, dm, tkv, dkv, last, k, s)
        emitted += len(r.emitted)
        accepted += r.accepted
        last = r.last_token
    eng.sync()
    dt = time.perf_counter() - t
    log(f"REJECTION T={T}: {dt * 1e3 / steps:.3f} ms/step, {emitted} tokens, acceptance {accepted / (steps * k):.3f}")
    return {"temperature": T, "ms_per_step": round(dt * 1e3 / steps, 4), "tok_s": round(emitted / dt, 2),
            "acceptance_rate": round(accepted / (steps * k), 4), "steps": steps}, last


def measure_forced(eng, tm, dm, tkv, dkv, last, k, steps, warmup=2):
    """The forced-acceptance diagnostic: every step's drafts are the target's
    greedy continuation (single-token target forwards from the same state,
    computed outside the timed steps), fed through the draft model by
    sh_spec_step_forced, so a step does a real step's work and accepts all k
    drafts. tok/s = emitted tokens / summed step wall times. A near-tie where
    the 8-column verify's argmax differs from the single-token forward's ends
    the continuation early: it is recomputed from there (untimed)."""
    cont, j = [], 0

    def extend():
        P = tkv.position
        c = [last]
        for i in range((steps + warmup - done) * (k + 1) + k):
            c.append(int(eng.verify_greedy(tm, tkv, [c[-1]], P + i)[0]))
        tkv.truncate(P)
        return c
    times, emitted, accepted, resyncs = [], 0, 0, 0
    done = 0
    while done < steps + warmup:
        if j + k + 1 >= len(cont):
            cont, j = extend(), 0
        t = time.perf_counter()
        r = eng.decode_speculative_forced(tm, dm, tkv, dkv, cont[j], cont[j + 1:j + 1 + k])
        dt = time.perf_counter() - t
        if done >= warmup:
            times.append(dt)
            emitted += len(r.emitted)
            accepted += r.accepted
        done += 1
        last = r.last_token
        if r.emitted != cont[j + 1:j + 2 + k]:
            resyncs += 1
            cont, j = [], 0
        else:
            j += len(r.emitted)
    total = sum(times)
    log(f"forced acceptance: {total * 1e3 / steps:.3f} ms/step, {emitted} tokens in {steps} steps, "
        f"{emitted / total:.1f} tok/s ({resyncs} continuation resyncs)")
    return {"tok_s": round(emitted / total, 2), "ms_per_step": round(total * 1e3 / steps, 4),
            "acceptance_rate": round(accepted / (steps * k), 4), "steps": steps, "resyncs": resyncs,
            "definition": "measured: each step's drafts are the target's greedy continuation (single-token target "
                          "forwards), fed through the draft model (sh_spec_step_forced: the draft forwards run over "
                          "them), so every draft is accepted; tokens emitted / summed step wall times "
                          "(apps/seeker-cli/src/commands/run.rs:702-710 counts emitted tokens)"}, last


def measure_acceptance(eng, reps=20, cpu=True):
    """the acceptance kernel alone (REJECTION, T = 0.8), B = 32, k = 8,
    V = 128256; target logits N(0, 3), draft = target + N(0, 1), drafts sampled
    from the draft distribution (numpy), uniforms Philox (seed 7) in the kernel.
    Bytes per call = 4 V B (2k + 1) (one read of every target and draft logit)."""
    import numpy as np
    from seeker_amd import synth as S
    from seeker_amd._native import SH_SAMPLE_REJECTION, sh_sampling
    B, k, V, T = 32, 8, 128256, 0.8
    p = S.normal_f32(7, 10, B * (k + 1) * V, 0.0, 3.0).reshape(B, k + 1, V)
    q = (p[:, :k] + S.normal_f32(7, 11, B * k * V, 0.0, 1.0).reshape(B, k, V)).astype(np.float32)
    rng = np.random.default_rng(7)
    z = q.reshape(B * k, V).astype(np.float64) / T
    z = np.exp(z - z.max(axis=1, keepdims=True))
    cdf = np.cumsum(z, axis=1)
    u = rng.random(B * k) * cdf[:, -1]
    drafts = np.array([int(np.searchsorted(cdf[i], u[i], side="right")) for i in range(B * k)],
                      dtype=np.uint32).reshape(B, k)
    pd, qd, dd = eng.to_device(p), eng.to_device(q), eng.to_device(drafts)
    acc, nxt = eng.dev_alloc(4 * B), eng.dev_alloc(4 * B)
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = SH_SAMPLE_REJECTION, T, 7, 0
    for _ in range(3):
        eng.accept_sample(pd, qd, dd, B, k, V, s, acc, nxt)
    eng.sync()
    # the call as a caller sees it: back-to-back calls on the engine stream,
    # one synchronization at the end (no per-launch events)
    t = time.perf_counter()
    for _ in range(reps):
        eng.accept_sample(pd, qd, dd, B, k, V, s, acc, nxt)
    eng.sync()
    wall_ms = (time.perf_counter() - t) * 1e3 / reps
    # kernel time: the same calls with per-launch events
    eng.set_profiling(True)
    eng.profile(reset=True)
    for _ in range(reps):
        eng.accept_sample(pd, qd, dd, B, k, V, s, acc, nxt)
    prof = eng.profile(reset=True)
    eng.set_profiling(False)
    kern_ms = sum(prof[n]["ms"] for n in ("accept_stats", "accept_decide") if n in prof) / reps
    al, nt = acc.read(np.uint32, B), nxt.read(np.uint32, B)
    for x in (pd, qd, dd, acc, nxt):
        x.free()
    nbytes = 4 * V * B * (2 * k + 1)
    log(f"acceptance kernel B={B} k={k} V={V}: {kern_ms * 1e3:.1f} us in kernels, {wall_ms * 1e3:.1f} us per call")
    out = {"config": "B=32, k=8, V=128256, REJECTION T=0.8, Philox seed 7", "kernel_us": round(kern_ms * 1e3, 2),
           "call_us": round(wall_ms * 1e3, 2), "alg_bytes": nbytes,
           "GBps": round(nbytes / kern_ms / 1e6, 1), "frac": round(nbytes / kern_ms / 1e6 / HBM_PEAK_GBS, 4),
           "mean_accepted": round(float(al.mean()), 3)}
    if cpu:
        # the C oracle's rejection rule (f64, one thread) over the same logits,
        # drafts and Philox words: the CPU time of the same call, and the check
        # that every sequence's (accepted length, next token) is the GPU's
        import oracle as O
        U = O.philox_uniforms(7, 0x5EC, 0, 2 * B * (k + 1)).reshape(B, k + 1, 2)
        t = time.perf_counter()
        ref = [O.rejection(p[b], q[b], drafts[b], T, U[b, :k, 0].copy(), U[b, :, 1].copy()) for b in range(B)]
        cpu_ms = (time.perf_counter() - t) * 1e3
        same = sum(int(al[b]) == ref[b][0] and int(nt[b]) == ref[b][1] for b in range(B))
        log(f"acceptance on the CPU (C oracle, 1 thread): {cpu_ms:.1f} ms per call; {same}/{B} sequences equal")
        out["cpu_baseline"] = {"value": round(cpu_ms * 1e3, 1), "unit": "us per call", "cores": 1, "kind": "port",
                               "sample": f"the whole call: {B} sequences, f64 C restatement (oracle/oracle.c)"}
        out["parity"] = {"sequences_equal": same, "sequences": B}
    return out


def measure_tree(eng, tm, d, P=8192, reps=3):
    """one tree verification step (sh_tree_verify_step) on the 8B
    target, B = 4 sequences at context 8192, trees of depth 3 with branching
    4, 3, 2 (41 nodes with the root), REJECTION at T = 1.0 (Philox seed 11)
    against synthetic draft logits N(0, 3), then compaction of the accepted
    paths. The KV position is set to 8192 without a prefill (the bytes read and
    the work are the same). Bytes per step: every weight matrix once + K/V read
    for [0, P + 41) of each sequence + 41 K/V rows written per sequence."""
    import numpy as np
    from seeker_amd import synth as S
    from seeker_amd._native import SH_SAMPLE_REJECTION, sh_sampling
    B, branching = 4, (4, 3, 2)
    parents, level = [-1], [0]
    for b in branching:
        nxt_level = []
        for v in level:
            for _ in range(b):
                parents.append(v)
                nxt_level.append(len(parents) - 1)
        level = nxt_level
    n = len(parents)
    V = d.n_vocab
    caches = [eng.allocate_kv_cache(tm, P + 64) for _ in range(B)]
    tokens = np.stack([S.tokens(900 + b, n, V) for b in range(B)]).astype(np.uint32)
    par = np.tile(np.array(parents, np.int32), (B, 1))
    qd = eng.to_device(S.normal_f32(11, 12, B * n * V, 0.0, 3.0))
    s = sh_sampling()
    s.mode, s.temperature, s.seed, s.counter = SH_SAMPLE_REJECTION, 1.0, 11, 0
    times, plens = [], []
    for i in range(reps + 1):
        for c in caches:
            c.set_position(P)
        t = time.perf_counter()
        paths, _ = eng.tree_verify_step(tm, caches, tokens, par, qd, s)
        if i:
            times.append((time.perf_counter() - t) * 1e3)
            plens += [len(x) for x in paths]
    for c in caches:
        c.set_position(P)
    eng.set_profiling(True)
    eng.profile(reset=True)
    eng.tree_verify_step(tm, caches, tokens, par, qd, s)
    prof = eng.profile(reset=True)
    eng.set_profiling(False)
    kern = {k: round(v["ms"], 4) for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])}
    qd.free()
    for c in caches:
        c.close()
    w, _, _ = verify_bytes(d, 0, 0)
    dkv = d.head_dim * d.n_head_kv
    kv = B * 2 * d.n_layer * ((P + n) * dkv * 2 + n * dkv * 2)
    ms = statistics.median(times)
    log(f"tree verify step B={B} n={n} ctx {P}: {ms:.2f} ms, mean path {np.mean(plens):.2f} nodes")
    for k, v in list(kern.items())[:10]:
        log(f"  {k:16s} {v:8.3f} ms")
    # the dense matmuls' rate: 2 x (every weight element) x the B n columns
    # against the summed event time of their GEMM kernels (split partials
    # written; their finishing kernels are counted under the preps)
    gemm_ms = sum(v for k, v in kern.items() if k.startswith("gemv_"))
    elems = w * 256 // 144
    gemm_tflops = 2.0 * elems * B * n / (gemm_ms * 1e-3) / 1e12 if gemm_ms else 0.0
    log(f"  dense GEMMs: {gemm_ms:.3f} ms, {gemm_tflops:.0f} TFLOP/s ({gemm_tflops / MFMA_F16_PEAK_TFLOPS:.3f} of "
        f"the dense f16 MFMA peak)")
    return {"config": f"B={B}, tree 4x3x2 ({n} nodes), ctx {P}, REJECTION T=1.0 seed 11, synthetic draft logits",
            "arithmetic": ("reference wide-GEMM (f16 weights and activations, f32 accumulation; "
                           "ops/matmul.rs:433-446)" if tm.wide_f16 else "f32-level (hi/lo f16 activations)"),
            "ms": round(ms, 3), "alg_bytes": w + kv, "GBps": round((w + kv) / ms / 1e6, 1),
            "frac": round((w + kv) / ms / 1e6 / HBM_PEAK_GBS, 4), "mean_path_nodes": round(float(np.mean(plens)), 3),
            "gemm": {"ms": round(gemm_ms, 4), "flop": 2 * elems * B * n, "TFLOPs": round(gemm_tflops, 1),
                     "mfma_frac": round(gemm_tflops / MFMA_F16_PEAK_TFLOPS, 4), "peak_TFLOPs": MFMA_F16_PEAK_TFLOPS},
            "kernel_ms": kern}


def measure_q4km(eng, P=4096, L=8, reps=30):
    """The configs[2] verify (L = 8 at context 4096) on a Q4_K_M-style 8B: the
    attn_v and ffn_down of every other layer and output.weight in Q6_K, the rest
    Q4_K (llama.cpp's Q4_K_M mix). Such a model runs on the multi-group path
    (graph-replayed), not on the tuned uniform-Q4_K GEMVs. KV positions set
    without a prefill. Algorithmic bytes: the model's weight bytes (Q6_K at
    210 B per 256 elements) + K/V read and written."""
    import dataclasses
    import numpy as np
    from seeker_amd import synth as S
    from seeker_amd._native import GGML_Q6_K
    sh = dataclasses.replace(S.L8B_TARGET, out_type=GGML_Q6_K, mix=1)
    t0 = time.time()
    img = S.GgufImage(sh, seed=3)
    m = eng.upload_weights(img)
    img.close()
    log(f"Q4_K_M-style 8B synthesized and uploaded in {time.time() - t0:.1f}s")
    d = m.dims
    kv = eng.allocate_kv_cache(m, P + 64)
    toks = S.tokens(778, L, d.n_vocab)
    times = []
    for i in range(reps + 3):
        kv.set_position(P)
        eng.sync()
        t = time.perf_counter()
        eng.verify_greedy(m, kv, toks, P)
        if i >= 3:
            times.append((time.perf_counter() - t) * 1e3)
    kv.set_position(P)
    eng.set_profiling(True)
    eng.profile(reset=True)
    eng.verify_greedy(m, kv, toks, P)
    prof = eng.profile(reset=True)
    eng.set_profiling(False)
    for n, st in sorted(prof.items(), key=lambda kv_: -kv_[1]["ms"]):
        log(f"  {n:16s} {st['launches']:4d}/step {st['ms']:8.3f} ms/step")
    _, kvr, kvw = verify_bytes(d, P, L)
    wb = int(d.weight_bytes)
    ms = statistics.median(times)
    kv.close()
    m.close()
    log(f"Q4_K_M-style 8B verify (L={L}, P={P}): {ms:.3f} ms, {(wb + kvr + kvw) / ms / 1e6:.0f} GB/s")
    return {"config": "Llama-3-8B shape, Q4_K_M-style mix (Q6_K attn_v / ffn_down of even layers and output), "
                      f"L={L}, ctx {P}, multi-group path, graph-replayed",
            "ms": round(ms, 4), "alg_bytes": wb + kvr + kvw,
            "GBps": round((wb + kvr + kvw) / ms / 1e6, 1),
            "frac": round((wb + kvr + kvw) / ms / 1e6 / HBM_PEAK_GBS, 4)}


def measure_moe(eng, P=16384, B=8, L=7, reps=5):
    """batched verify (sh_verify_unified) of B = 8 sequences x L = k+1 = 7
    columns on the Qwen3-30B-A3B-shape Q4_K MoE target (48 layers, d 2048, 32 / 4
    heads, head_dim 128, 128 experts top-8, expert FFN 768, vocab 151936) at
    context 16384 (KV positions set without a prefill: the same bytes read and
    work done). Algorithmic bytes: attention / router / lm_head matrices once,
    the expected number of distinct routed experts per layer, 128 (1 -
    (120/128)^56) = 124.6, times one expert's gate + up + down bytes, plus K/V
    read for [0, P + L) of each sequence and the L new rows written."""
    import numpy as np
    from seeker_amd import synth as S
    sh = S.Q30B_A3B_TARGET
    t0 = time.time()
    img = S.GgufImage(sh, seed=2)
    log(f"moe target GGUF {img.size / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    t0 = time.time()
    m = eng.upload_weights(img)
    img.close()
    log(f"moe upload + repack {time.time() - t0:.1f}s")
    d = m.dims
    V = d.n_vocab
    caches = [eng.allocate_kv_cache(m, P + 64) for _ in range(B)]
    toks = np.concatenate([S.tokens(700 + b, L, V) for b in range(B)])
    times = []
    for i in range(reps + 2):
        for c in caches:
            c.set_position(P)
        eng.sync()
        t = time.perf_counter()
        eng.verify_unified(m, caches, toks, [L] * B)
        if i >= 2:
            times.append((time.perf_counter() - t) * 1e3)
    for c in caches:
        c.set_position(P)
    eng.set_profiling(True)
    eng.profile(reset=True)
    eng.verify_unified(m, caches, toks, [L] * B)
    prof = eng.profile(reset=True)
    eng.set_profiling(False)
    q4 = 144 / 256
    qd, kvd = d.n_head * d.head_dim, d.n_head_kv * d.head_dim
    dense = d.n_layer * (d.n_embd * (qd + 2 * kvd) + qd * d.n_embd) * q4 + V * d.n_embd * q4
    router = d.n_layer * sh.n_expert * d.n_embd * 4
    N = B * L
    distinct = sh.n_expert * (1 - (1 - sh.n_expert_used / sh.n_expert) ** N)
    experts = d.n_layer * distinct * 3 * sh.expert_ff * d.n_embd * q4
    kv = B * d.n_layer * 2 * ((P + L) * kvd * 2 + L * kvd * 2)
    nbytes = dense + router + experts + kv
    ms = statistics.median(times)
    for c in caches:
        c.close()
    m.close()
    kern = {n: round(v["ms"], 4) for n, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])}
    log(f"moe verify B={B} L={L} ctx {P}: {ms:.2f} ms, {nbytes / 1e9:.2f} GB -> {nbytes / ms / 1e6:.0f} GB/s")
    for n, v in list(kern.items())[:8]:
        log(f"  {n:16s} {v:8.3f} ms")
    return {"config": f"Qwen3-30B-A3B-shape Q4_K MoE target, B={B} x L={L} (k=6), ctx {P}, greedy ids",
            "ms": round(ms, 3), "alg_bytes": int(nbytes), "expected_distinct_experts_per_layer": round(distinct, 2),
            "GBps": round(nbytes / ms / 1e6, 1), "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
            "kernel_ms": kern}


def measure_moe_spec(eng, P=16384, B=8, k=6, steps=6, warmup=1):
    """configs[4] as a batch-8 spec decode (sh_spec_step_batch, the server's step,
    server/inference.rs:2777-2924): the Qwen3-30B-A3B-shape Q4_K MoE target (48
    layers) and the Qwen3-0.6B-shape Q4_K draft (28 layers), 8 sequences at
    context 16384 (both caches' positions set without a prefill: the same bytes
    read and work done), k = 6 greedy drafts per sequence, one batched verify
    of 8 x 7 columns, per-sequence acceptance and rollback. Accepted tok/s =
    emitted tokens / wall time over the timed steps (run.rs:702-710's count);
    draft ms per position = (step - verify) / k, verify ms from the batched
    verify of the same columns timed alone."""
    import numpy as np
    from seeker_amd import synth as S
    t0 = time.time()
    timg = S.GgufImage(S.Q30B_A3B_TARGET, seed=2)
    dimg = S.GgufImage(S.Q06B_DRAFT, seed=3)
    tm, dm = eng.upload_weights(timg), eng.upload_weights(dimg)
    timg.close()
    dimg.close()
    log(f"moe spec: target + draft synthesized and uploaded in {time.time() - t0:.1f}s")
    V = tm.dims.n_vocab
    tk = [eng.allocate_kv_cache(tm, P + 64) for _ in range(B)]
    dk = [eng.allocate_kv_cache(dm, P + 64) for _ in range(B)]
    for c in tk + dk:
        c.set_position(P)
    last = [int(t) for t in S.tokens(710, B, V)]
    emitted = accepted = 0
    for _ in range(warmup):
        em, _ = eng.spec_step_batch(tm, dm, tk, dk, last, k)
        last = [e[-1] for e in em]
    eng.sync()
    t = time.perf_counter()
    for _ in range(steps):
        em, _ = eng.spec_step_batch(tm, dm, tk, dk, last, k)
        emitted += sum(len(e) for e in em)
        accepted += sum(len(e) - 1 for e in em)
        last = [e[-1] for e in em]
    eng.sync()
    dt = time.perf_counter() - t
    # the verify of the same shape alone (the step's verify share)
    toks = np.concatenate([S.tokens(720 + b, k + 1, V) for b in range(B)])
    vt = []
    for i in range(4):
        for c in tk:
            c.set_position(P)
        eng.sync()
        t1 = time.perf_counter()
        eng.verify_unified(tm, tk, toks, [k + 1] * B)
        if i >= 1:
            vt.append((time.perf_counter() - t1) * 1e3)
    v_ms = statistics.median(vt)
    step_ms = dt * 1e3 / steps
    for c in tk + dk:
        c.close()
    tm.close()
    dm.close()
    out = {"config": f"configs[4]: Qwen3-30B-A3B-shape Q4_K MoE target + Qwen3-0.6B-shape Q4_K draft, B={B}, k={k}, "
                     f"ctx {P}, greedy, batched spec step (sh_spec_step_batch)",
           "tok_s": round(emitted / dt, 2), "ms_per_step": round(step_ms, 3),
           "acceptance_rate": round(accepted / (steps * B * k), 4), "verify_ms": round(v_ms, 3),
           "verify_share": round(v_ms / step_ms, 4), "draft_ms_per_position": round((step_ms - v_ms) / k, 3),
           "steps": steps}
    log(f"moe spec decode B={B} k={k} ctx {P}: {step_ms:.2f} ms/step, {emitted / dt:.1f} tok/s, verify {v_ms:.2f} ms")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--k", type=int, default=7)
    ap.add_argument("--verify-reps", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the acceptance-kernel, tree and MoE lines")
    ap.add_argument("--moe-only", action="store_true", help="only the configs[4] MoE verify measurement")
    ap.add_argument("--q4km-only", action="store_true", help="only the Q4_K_M-style 8B verify measurement")
    ap.add_argument("--moe-spec-only", action="store_true", help="only the configs[4] batched spec-decode measurement")
    ap.add_argument("--tree-only", action="store_true", help="only the configs[3] tree verify measurement")
    ap.add_argument("--acceptance-only", action="store_true", help="only the configs[1] acceptance measurement")
    ap.add_argument("--draft-only", action="store_true", help="only the draft forward (eager, per-kernel events)")
    ap.add_argument("--profile-only", action="store_true")
    ap.add_argument("--spec-eager", action="store_true",
                    help="only greedy spec steps, launched kernel by kernel (no graph replay): the step's kernel mix "
                         "for a kernel tracer")
    ap.add_argument("--spec-mode", type=int, default=0, help="sampling mode of --spec-eager (0 greedy, 2 REJECTION)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build targets one MI355X; the verify path has no multi-GPU mode "
              "(a batch-1 verify does not shard profitably: tensor parallelism would add two all-reduces "
              "per layer)", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    from seeker_amd import Engine
    from seeker_amd import synth as S

    if args.moe_only:
        with Engine(0) as eng:
            print(json.dumps({"metric": "moe verify step", "moe_verify": measure_moe(eng)}), flush=True)
        return
    if args.moe_spec_only:
        with Engine(0) as eng:
            print(json.dumps({"metric": "moe spec decode", "moe_spec": measure_moe_spec(eng)}), flush=True)
        return
    if args.spec_eager:
        os.environ["SH_GRAPH"] = "0"  # read once, at the first step
    if args.draft_only:
        with Engine(0) as eng:
            print(json.dumps({"metric": "draft forward", "draft": measure_draft(eng, args.ctx)}), flush=True)
        return
    if args.q4km_only:
        with Engine(0) as eng:
            print(json.dumps({"metric": "Q4_K_M-style 8B verify", "q4km_verify": measure_q4km(eng)}), flush=True)
        return
    if args.acceptance_only:
        with Engine(0) as eng:
            print(json.dumps({"metric": "acceptance kernel", "acceptance": measure_acceptance(eng)}), flush=True)
        return
    if args.tree_only:
        img = S.GgufImage(S.L8B_TARGET, seed=0)
        with Engine(0) as eng:
            tm = eng.upload_weights(img)
            img.close()
            print(json.dumps({"metric": "tree verify step", "tree_verify": measure_tree(eng, tm, tm.dims)}), flush=True)
            tm.close()
        return

    t0 = time.time()
    timg = S.GgufImage(S.L8B_TARGET, seed=0)
    dimg = None if args.profile_only else S.GgufImage(S.L1B_DRAFT, seed=1)
    log(f"synthetic GGUF: target {timg.size / 1e9:.2f} GB" + ("" if dimg is None else f", draft {dimg.size / 1e9:.2f} GB")
        + f" in {time.time() - t0:.1f}s")
    eng = Engine(0)
    t0 = time.time()
    tm = eng.upload_weights(timg)
    dm = None if dimg is None else eng.upload_weights(dimg)
    log(f"upload + repack {time.time() - t0:.1f}s")
    d = tm.dims
    V = d.n_vocab
    P0 = args.ctx
    max_seq = P0 + 16 + (args.steps + args.warmup + 2) * (args.k + 1) + 64
    tkv = eng.allocate_kv_cache(tm, max_seq)
    dkv = None if dm is None else eng.allocate_kv_cache(dm, max_seq)
    prompt = S.tokens(1234, P0, V)
    t0 = time.time()
    if args.profile_only:
        tkv.set_position(P0)
        last = int(prompt[-1])
    else:
        eng.prefill(tm, tkv, prompt[:-1], 0)
        lg, _ = eng.forward_full_readback(tm, tkv, prompt[-1:], P0 - 1, full_logits=False, want_residual=False)
        if dm is not None:
            eng.prefill(dm, dkv, prompt, 0)
        last = int(np.argmax(lg[0]))
    last0 = last  # the token after the prefill: each stepped leg below starts from (P0, last0)
    log(f"prefill {P0} tokens in {time.time() - t0:.1f}s")
    if args.spec_eager:
        s = None
        if args.spec_mode:
            from seeker_amd._native import sh_sampling
            s = sh_sampling()
            s.mode, s.temperature, s.seed, s.counter = args.spec_mode, 0.8, 5, 0
        for i in range(args.warmup + args.steps):
            if i == args.warmup:
                eng.sync()
                t = time.perf_counter()
            last = eng.decode_speculative(tm, dm, tkv, dkv, last, args.k, s).last_token
        eng.sync()
        ms = (time.perf_counter() - t) * 1e3 / args.steps
        print(json.dumps({"metric": "eager spec steps", "ms_per_step": round(ms, 4), "steps": args.steps,
                          "graph_stats": eng.graph_stats()}), flush=True)
        return

    # ---- verify step: latency + roofline (target only) -------------------
    vt = S.tokens(777, args.k + 1, V)
    vt[0] = last
    P = tkv.position
    for _ in range(3):
        eng.verify_greedy(tm, tkv, vt, P)
        tkv.truncate(P)
    lat = []
    for _ in range(args.verify_reps):
        t = time.perf_counter()
        eng.verify_greedy(tm, tkv, vt, P)
        lat.append((time.perf_counter() - t) * 1e3)
        tkv.truncate(P)
    eng.set_profiling(True)
    eng.profile(reset=True)
    for _ in range(args.verify_reps):
        eng.verify_greedy(tm, tkv, vt, P)
        tkv.truncate(P)
    prof = eng.profile(reset=True)
    eng.set_profiling(False)
    wb, kvr, kvw = verify_bytes(d, P, args.k + 1)
    vbytes = wb + kvr + kvw
    vms = statistics.median(lat)
    gemv = {n: s for n, s in prof.items() if n.startswith("gemv")}
    dom_name = max(gemv, key=lambda n: gemv[n]["ms"])
    dom = gemv[dom_name]
    dom_avg_ms = dom["ms"] / dom["launches"]
    dom_bytes = dom["bytes"] / dom["launches"]
    kern_ms = sum(s["ms"] for s in prof.values()) / args.verify_reps
    log(f"verify step (L={args.k + 1}, P={P}): median {vms:.3f} ms wall, {kern_ms:.3f} ms in kernels; "
        f"{vbytes / 1e9:.3f} GB -> {vbytes / vms / 1e6:.0f} GB/s")
    for n, s in sorted(prof.items(), key=lambda kv: -kv[1]["ms"]):
        per = s["ms"] / args.verify_reps
        gbs = s["bytes"] / s["ms"] / 1e6 if s["ms"] > 0 and s["bytes"] else 0
        log(f"  {n:16s} {s['launches'] // args.verify_reps:4d}/step {per:8.3f} ms/step  {gbs:7.0f} GB/s")

    if args.profile_only:
        print(json.dumps({"metric": "verify-only profile run", "verify_ms": vms, "dominant": dom_name}))
        return

    # ---- CPU baseline + full-size greedy parity from the same state --------
    cpu = None
    parity = None
    gpu_first = eng.decode_speculative(tm, dm, tkv, dkv, last, args.k) if args.no_cpu_baseline else None
    if not args.no_cpu_baseline:
        import oracle as O

        cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        cpu_model = "unknown"
        try:
            with open("/proc/cpuinfo") as f:
                cpu_model = next(ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name"))
        except (OSError, StopIteration):
            pass
        ot, od = O.Model(timg), O.Model(dimg)
        ot.set_mm16(2 if tm.wide_f16 else 0)  # wide calls as the GPU computes them
        od.set_mm16(2 if dm.wide_f16 else 0)
        ot.set_attn_cm1(tm.cm1_attention)  # the verify's cm1 attention as the GPU computes it
        od.set_attn_cm1(dm.cm1_attention)
        okt, okd = O.KvCache(ot, max_seq), O.KvCache(od, max_seq)
        for (gkv, okv, m) in ((tkv, okt, tm), (dkv, okd, dm)):
            n = gkv.position
            for layer in range(m.dims.n_layer):
                for isv in (False, True):
                    okv.layer(layer, isv, n)[:] = gkv.read_layer(layer, isv, n)
            okv.set_position(n)
        # parity: the f64 check build takes one step from the GPU's state
        o_em, o_dr = O.spec_step_greedy(ot, od, okt, okd, last, args.k)
        g = eng.decode_speculative(tm, dm, tkv, dkv, last, args.k)
        gpu_first = g
        parity = {"oracle_emitted": o_em, "gpu_emitted": g.emitted, "drafts_equal": o_dr == g.drafts,
                  "emitted_equal": o_em == g.emitted}
        # baseline: the f32 timing build continues from there, 1 warm-up + 3 timed steps
        lastc, rates, step_s = o_em[-1], [], []
        for i in range(4):
            t = time.perf_counter()
            em, _ = O.spec_step_greedy(ot, od, okt, okd, lastc, args.k, fast=True)
            dt_s = time.perf_counter() - t
            if i:
                rates.append(len(em) / dt_s)
                step_s.append(round(dt_s, 3))
            lastc = em[-1]
        log(f"cpu oracle (f32, {cores} threads, {cpu_model}): steps {step_s} s; parity emitted {o_em} vs {g.emitted}")
        cpu = {"value": round(statistics.mean(rates), 4), "sd": round(statistics.stdev(rates), 4),
               "unit": "accepted tok/s", "cores": cores, "cpu_model": cpu_model, "kind": "port",
               "sample": f"3 timed speculative steps (k={args.k}, greedy; 1 warm-up) continuing from the GPU's "
                         f"post-prefill state (ctx {P0}, same weights and KV): the C restatement built -O3 AVX2/FMA "
                         f"with f32 accumulation (the reference's FLOAT_TYPE=float), OpenMP over rows and heads",
               "step_s": step_s}
        for x in (okt, okd):
            x.close()
        ot.close(); od.close()
    last = gpu_first.last_token

    # ---- timed speculative steps ------------------------------------------
    for _ in range(args.warmup):
        r = eng.decode_speculative(tm, dm, tkv, dkv, last, args.k)
        last = r.last_token
    eng.sync()
    t = time.perf_counter()
    emitted = 0
    accepted = 0
    for _ in range(args.steps):
        r = eng.decode_speculative(tm, dm, tkv, dkv, last, args.k)
        emitted += len(r.emitted)
        accepted += r.accepted
        last = r.last_token
    eng.sync()
    dt = time.perf_counter() - t
    value = emitted / dt
    log(f"{args.steps} spec steps: {dt * 1e3 / args.steps:.3f} ms/step, {emitted} tokens, "
        f"acceptance {accepted / (args.steps * args.k):.3f}")

    # draft forward per token: the step minus its verify, over k drafts, against the
    # draft's weight bytes + its f16 K/V read per token
    dd = dm.dims
    dw, dkr, dkw = verify_bytes(dd, P0, 1)
    d_ms = (dt * 1e3 / args.steps - vms) / args.k
    draft_stats = {"ms_per_token": round(d_ms, 4), "alg_bytes_per_token": dw + dkr + dkw,
                   "GBps": round((dw + dkr + dkw) / d_ms / 1e6, 1),
                   "frac": round((dw + dkr + dkw) / d_ms / 1e6 / HBM_PEAK_GBS, 4),
                   "method": "(spec step ms - verify ms) / k, graph-replayed steps"}
    for kv in (tkv, dkv):
        kv.truncate(P0)
    rej, _ = measure_rejection(eng, tm, dm, tkv, dkv, last0, args.k, args.steps)
    for kv in (tkv, dkv):
        kv.truncate(P0)
    forced, _ = measure_forced(eng, tm, dm, tkv, dkv, last0, args.k, args.steps)
    extra_acc = extra_tree = extra_moe = None
    if not args.no_extra:
        extra_acc = measure_acceptance(eng)
        extra_tree = measure_tree(eng, tm, d)

    out = {
        "metric": "spec-decode accepted tok/s (8B Q4_K, k=7, 1 GPU); verify HBM GB/s vs peak",
        "value": round(value, 3),
        "unit": "accepted tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, f32 activations (f16 hi/lo MFMA), f16 KV",
        "data": "synthetic: random-init N(0,0.02) Q4_K weights, uniform random prompt ids",
        "config": {"workload": "spec decode: Llama-3-8B-shape Q4_K target + Llama-3.2-1B-shape Q4_K draft, "
                               "k=7 (verify L=8), f16 KV ctx 4096, batch 1, greedy",
                   "k": args.k, "ctx": P0, "batch": 1, "acceptance_rate": round(accepted / (args.steps * args.k), 4)},
        "verify_step": {"ms": round(vms, 4), "kernel_ms": round(kern_ms, 4), "alg_bytes": vbytes,
                        "GBps": round(vbytes / vms / 1e6, 1), "frac": round(vbytes / vms / 1e6 / HBM_PEAK_GBS, 4)},
        "roofline": {"kernel": dom_name, "bound": "hbm", "achieved": round(dom_bytes / dom_avg_ms / 1e6, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_bytes / dom_avg_ms / 1e6 / HBM_PEAK_GBS, 4),
                     "bytes_per_launch": dom_bytes, "avg_launch_ms": round(dom_avg_ms, 5),
                     "traffic": measured_traffic(dom_name)},
        "forced_acceptance": forced,
        "rejection_step": rej,
        "draft_forward": draft_stats,
        "cpu_baseline": cpu,
        "parity": parity,
        "acceptance_kernel": extra_acc,
        "tree_verify": extra_tree,
        "q4km_verify": None,
        "moe_verify": None,
        "moe_spec": None,
    }
    for x in (tkv, dkv, tm, dm):
        x.close()
    timg.close()
    dimg.close()
    if not args.no_extra:  # the 8B models are freed first: the MoE target is 17 GB
        out["q4km_verify"] = measure_q4km(eng)
        out["moe_verify"] = measure_moe(eng)
        out["moe_spec"] = measure_moe_spec(eng)
    print(json.dumps(out), flush=True)
    eng.close()


if __name__ == "__main__":
    main()
