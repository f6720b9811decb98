"""Headline benchmark: paged GQA decode attention at the Llama-3-8B layer shape
(benchmark config 2) on one MI355X, plus the CPU oracle timed on the same host.

A "step" is one paged decode-attention pass over the whole batch: 64 query
rows (one per sequence, contexts U[128, 4096]), 32 query / 8 KV heads,
head_dim 128, bf16 KV cache in the reference arena layout, block size 16,
block tables scattered over a pool of 1.25x the blocks needed.  Inputs are
resident in HBM before the timed region.

value = algorithmic HBM bytes per step / step time, where the bytes are the
compulsory traffic: every attended K and V vector once (sum(ctx) * 2 * Hkv *
d * 2 B), the f32 queries and outputs, and the block-table entries.

Prints ONE JSON line (the driver's contract).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "orionserve-rs_amd"), os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "paged_decode_cfg2_pmc.txt")


def copy_ceiling(be, achieved_gbs, nbytes=1 << 30, reps=10):
    """This box's HBM copy rate: a 1 GiB device-to-device copy (read + write
    bytes), median of `reps` event-timed copies after two warm-ups.  A copy
    moves read and write traffic at once, so it is a practical ceiling for
    mixed traffic; the read-only decode kernel can pass it."""
    src, dst = be.alloc(nbytes), be.alloc(nbytes)
    for _ in range(2):
        be.memcpy_d2d(dst.ptr, src.ptr, nbytes)
    be.synchronize()
    samples = []
    for _ in range(reps):
        be.timer_start()
        be.memcpy_d2d(dst.ptr, src.ptr, nbytes)
        samples.append(be.timer_stop())
    src.free()
    dst.free()
    gbs = 2 * nbytes / (float(np.median(samples)) * 1e-3) / 1e9
    return {"copy_GBps": round(gbs, 1), "achieved_over_copy": round(achieved_gbs / gbs, 4),
            "copy_note": "1 GiB device copy on this box, (read + write bytes) / median time"}


def measured_traffic():
    """HBM bytes per launch of the decode split-K kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (None when absent)."""
    import re
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch\s*=\s*(\d+)", text)
    return int(m.group(1)) if m else None


def prefill_cfg3(be, steps=20, warmup=3, head_major=False):
    """benchmark config 3: chunked-prefill causal attention over the paged
    cache as an MFMA contraction (8 seqs x 512-token chunks on prefixes
    U[0,7680], 32q/8kv, d 128, bf16).  Timed per kernel with HIP events."""
    import orion_hip as oh
    from paged_cases import cfg3

    case = cfg3(head_major=head_major)
    n = len(case.positions)
    kv = case.kv_layout()
    bufs = [be.to_device(case.arena_device_bytes()), be.to_device(case.q),
            be.to_device(case.row_start), be.to_device(case.row_count),
            be.to_device(case.first_pos), be.to_device(case.bt_offsets),
            be.to_device(case.bt_ids), be.alloc(n * case.hq * case.d * 4)]
    arena, dq, drs, drc, dfp, dbo, dbi, dout = bufs
    flops = case.flops()
    res = {"workload": "chunked-prefill attention, config 3: 8 seqs x 512-token chunks, prefix "
                       "U[0,7680], 32q/8kv, head_dim 128, bf16, block 16",
           "flops_per_call": flops}
    rng = np.random.default_rng(3)
    rows = np.array(sorted({r for c in range(case.S)
                            for r in [512 * c, 512 * c + 511] + list(512 * c + rng.integers(
                                0, 512, size=30))}))
    want = case.oracle_rows(rows)
    for hilo, key in ((0, "bf16"), (1, "hilo"), (2, "q_hilo"), (3, "p_hilo")):
        def call():
            oh.paged_attention_prefill(be, kv, arena.ptr, 0, dq.ptr, case.hq, case.S, drs.ptr,
                                       drc.ptr, dfp.ptr, dbo.ptr, dbi.ptr, 512,
                                       int(case.positions.max()), dout.ptr, hilo=hilo)
        for _ in range(warmup):
            call()
        be.kernel_timing(True)
        for _ in range(steps):
            call()
        samples = be.kernel_timing_samples(be.K_PREFILL)
        be.kernel_timing(False)
        ms = float(np.median(samples))
        tf = flops / (ms * 1e-3) / 1e12
        res[key] = {"ms": round(ms, 4), "ms_mean": round(float(samples.mean()), 4),
                    "launches": int(len(samples)), "tflops": round(tf, 1),
                    "frac_of_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
        # check of the timed output: the first, the last and 30 random rows
        # of every chunk (all 32 heads) against the oracle
        got = dout.download(np.float32, (n, case.hq * case.d))
        res[key]["max_abs_err_vs_oracle"] = float(np.abs(got[rows] - want).max())
        res[key]["rows_checked"] = f"{len(rows)} of {n}"
    res["operands"] = ("bf16: Q and softmax weights P rounded to bf16 (MFMA rate); hilo: each as "
                       "a hi+lo bf16 pair (2x MFMA work); q_hilo: Q as a pair, P rounded; "
                       "p_hilo: Q rounded, P as a pair")
    for b in bufs:
        b.free()
    return res


def algorithmic_bytes(case):
    kv = case.kv_bytes_read()
    q = case.S * case.hq * case.d * 4
    out = case.S * case.hq * case.d * 4
    tables = int(sum(len(t) for t in case.tables)) * 4
    return kv + q + out + tables


def host_threads():
    """(threads used, nproc): nproc = CPUs this process may run on; the oracle
    uses at most 16 (the GPU box's CPU share for one GPU)."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    return min(16, nproc), nproc


def timed_median(fn, reps, budget_s):
    """Median wall time of `fn` over `reps` calls (fewer if `budget_s` runs out)."""
    times = []
    t_end = time.perf_counter() + budget_s
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end:
            break
    return float(np.median(times)), len(times)


def cpu_baseline(case):
    """The oracle (C++ restatement of the reference CPU attention) on the same
    workload: all allowed host threads (OpenMP over independent (row, head)
    pairs), and one thread (the reference's own execution model)."""
    import oracle as orc

    threads, nproc = host_threads()
    orc.set_num_threads(threads)
    case.oracle()  # warm caches / page in
    dt, reps = timed_median(case.oracle, 20, 10.0)
    orc.set_num_threads(1)
    dt1, reps1 = timed_median(case.oracle, 20, 12.0)
    orc.set_num_threads(threads)
    return {
        "value": algorithmic_bytes(case) / dt / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "nproc": nproc,
        "kind": "port",
        "sample": f"full config-2 step ({case.S} rows, sum ctx {int(case.ctxs.sum())}), median "
                  f"of {reps} steps, {dt * 1e3:.1f} ms/step, f32 arena holding the same bf16 "
                  f"values",
        "single_thread": {"value": algorithmic_bytes(case) / dt1 / 1e9, "unit": "GB/s",
                          "cores": 1, "sample": f"median of {reps1} full steps, {dt1:.3f} s"},
    }


def decode_e2e(steps=64, seqs=32, seed=20261204, cpu=True):
    """benchmark config 4: full decode step of a random-init TinyLlama-1.1B-shape
    model (bf16 weights N(0, 0.02), bf16 KV cache), 32 sequences with prompt
    lengths U[16, 1024] (random token ids), prefilled in one forward, then
    `steps` greedy decode steps (device argmax).  The greedy tokens are
    compared with the CPU oracle's greedy decode of the same batch
    (tests/golden/cfg4_greedy_bf16kv.npz), and an untimed f32-KV run with the
    reference-exact oracle (cfg4_greedy_f32kv.npz).  Returns a dict of results."""
    import orion_hip as oh
    from cfg4_case import TINYLLAMA, cfg4_case

    cfg = TINYLLAMA
    case = cfg4_case(seed, seqs, steps)
    lens, tables, num_blocks, bs = case.lens, case.tables, case.num_blocks, 16
    meta = oh.ModelMetadata(hidden_size=cfg["H"], num_layers=cfg["L"],
                            num_attention_heads=cfg["hq"], num_kv_heads=cfg["hkv"],
                            head_dim=cfg["d"], vocab_size=cfg["V"], intermediate_size=cfg["F"],
                            max_position_embeddings=cfg["max_pos"], rope_theta=cfg["theta"],
                            rms_norm_eps=cfg["eps"])
    be = oh.HipBackend(0)
    model = oh.HipTransformerModel(meta, num_blocks, bs, be, oh.BF16)
    model.init_synthetic(seed, 0.02)
    toks = [t for p in case.prompts for t in p]
    pos = [i for n in lens for i in range(int(n))]
    pf_batch = oh.ForwardBatch(toks, pos, list(range(seqs)), [int(n) for n in lens],
                               [int(n) for n in lens], tables, True)
    # The first forward also writes the packed weight copies (once per weight
    # write) and frees the row-major ones; the prefill is then timed again (it
    # rewrites the same K/V).
    t0 = time.perf_counter()
    out = model.forward(pf_batch, want_logits=False, want_argmax=True)
    be.synchronize()
    prefill_first_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    out = model.forward(pf_batch, want_logits=False, want_argmax=True)
    be.synchronize()
    prefill_s = time.perf_counter() - t0
    last = out.argmax.tolist()
    ctx = [int(n) for n in lens]
    generated = [last]
    # The decode batch is flattened once; each step then replaces its tokens
    # and advances positions and context lengths in place (advance_decode).
    # The library still validates and plans every step.
    dec = None

    def step():
        nonlocal last, dec
        if dec is None:
            dec = oh.ForwardBatch(last, list(ctx), list(range(seqs)), [1] * seqs,
                                  [c + 1 for c in ctx], tables, False).prepare()
        else:
            dec.advance_decode(last)
        o = model.forward(dec, want_logits=False, want_argmax=True)
        last = o.argmax.tolist()
        generated.append(last)
        for i in range(seqs):
            ctx[i] += 1

    for _ in range(2):  # warm-up steps (they also extend the sequences)
        step()
    be.synchronize()
    n_steps = steps - 2
    # KV bytes the timed steps read (every attended position, all layers, K
    # and V) and write (one new position per sequence and step)
    kv_pos_bytes = cfg["L"] * 2 * cfg["hkv"] * cfg["d"] * 2
    kv_read = sum(sum(c + k + 1 for c in ctx) for k in range(n_steps)) * kv_pos_bytes
    kv_write = n_steps * seqs * kv_pos_bytes
    # every step ends in a device-to-host copy of its tokens (a full sync), so
    # each step is timed on its own; tokens/s uses the median step
    per_step = []
    t0 = time.perf_counter()
    for _ in range(n_steps):
        t1 = time.perf_counter()
        step()
        per_step.append(time.perf_counter() - t1)
    be.synchronize()
    dt = time.perf_counter() - t0
    med = float(np.median(per_step))
    res = {
        "decode_tokens_per_s": round(seqs / med, 1),
        "decode_ms_per_step": round(med * 1e3, 4),
        "step_ms_mean": round(dt / n_steps * 1e3, 4),
        "step_ms_min_max": [round(min(per_step) * 1e3, 4), round(max(per_step) * 1e3, 4)],
        "timed_steps": n_steps,
        "prefill_tokens": int(sum(lens)),
        "prefill_s": round(prefill_s, 4),
        "prefill_tokens_per_s": round(int(sum(lens)) / prefill_s, 1),
        "prefill_first_s": round(prefill_first_s, 4),
        "workload": "TinyLlama-1.1B shape (22L, hidden 2048, 32q/4kv, d 64, ffn 5632, vocab "
                    "32000), bf16 weights N(0,0.02) synthetic, bf16 KV, 32 seqs, prompts "
                    "U[16,1024], greedy decode",
        "weight_bytes_per_step": int((22 * (2048 * (2048 + 512) + 2048 * 2048 + 3 * 2048 * 5632)
                                      + 32000 * 2048) * 2),
    }
    # HBM roofline of the step: weights + KV read + KV write per step at 8 TB/s
    res["hbm_bytes_per_step"] = int(res["weight_bytes_per_step"] + (kv_read + kv_write) / n_steps)
    res["frac_of_hbm_roofline"] = round(
        res["hbm_bytes_per_step"] / (res["decode_ms_per_step"] * 1e-3) / HBM_PEAK_GBS / 1e9, 4)
    res["greedy_vs_oracle"] = greedy_vs_golden(generated, steps, seqs, "bf16")
    model.close()
    # The same free-running greedy decode (untimed) on an f32 arena, the
    # reference's KV dtype, against the reference-exact oracle's decode.
    model = oh.HipTransformerModel(meta, num_blocks, bs, be, oh.F32)
    model.init_synthetic(seed, 0.02)
    out = model.forward(pf_batch, want_logits=False, want_argmax=True)
    last = out.argmax.tolist()
    ctx = [int(n) for n in lens]
    generated = [last]
    dec = None
    for _ in range(steps):
        step()
    res["greedy_vs_oracle_f32kv"] = greedy_vs_golden(generated, steps, seqs, "f32")
    model.close()
    be.close()
    if cpu:
        res["cpu_baseline"] = cpu_decode_step(cfg, lens, tables, num_blocks, seqs, seed)
        res["speedup_vs_cpu"] = round(res["decode_tokens_per_s"] / res["cpu_baseline"]["value"], 1)
    return res


def greedy_vs_golden(generated, steps, seqs, kv):
    """The bench's free-running greedy tokens against the CPU oracle's greedy
    decode of the same batch with the same KV dtype
    (tests/golden/cfg4_greedy_{kv}kv.npz; for bf16 the oracle rounds each K/V
    element to bf16 when written): per sequence, the tokens that agree up to
    the first difference (after one, the two sequences continue from
    different inputs), and at each first difference the oracle's margin
    between its own token and the device's (from the golden's 8 largest
    logits; None when the device's token is not among them)."""
    path = os.path.join(ROOT, "tests", "golden", f"cfg4_greedy_{kv}kv.npz")
    if not os.path.exists(path):
        return None
    g = np.load(path)
    gold = g["tokens"]
    got = np.asarray(generated, np.int64)
    if got.shape != gold.shape:
        return {"error": f"shape {got.shape} against golden {gold.shape}"}
    agree = got == gold
    prefix = [int(np.argmin(agree[:, s])) if not agree[:, s].all() else steps + 1
              for s in range(seqs)]
    margins = []
    for s, p in enumerate(prefix):
        if p > steps:
            continue
        idx = list(g["top_idx"][p, s])
        tok = int(got[p, s])
        margins.append(float(g["top_val"][p, s, 0] - g["top_val"][p, s, idx.index(tok)])
                       if tok in idx else None)
    known = [m for m in margins if m is not None]
    return {"tokens_compared": int(gold.size), "tokens_matched": int(sum(prefix)),
            "sequences_identical": int(sum(p == steps + 1 for p in prefix)),
            "first_difference_steps": [p for p in prefix if p <= steps],
            "oracle_margin_at_first_differences": [None if m is None else round(m, 6)
                                                   for m in margins],
            "smallest_margin": round(min(known), 6) if known else None,
            "note": f"{kv} KV on both sides; matched = tokens up to each sequence's first "
                    "difference; margin = oracle top-1 logit minus the oracle's logit of "
                    "the device's token"}


def gemm_shapes(reps=10):
    """The projection GEMMs of the config-4 model at prefill M (the 17,526-token
    prefill of decode_e2e) and decode M (32 rows), through orion_hip_gemm on
    zero-filled operands (timing only).  Prefill shapes report algorithmic
    TFLOP/s (2*M*N*K; the MFMA work issued is twice that, hi/lo activations);
    decode shapes report weight-streaming GB/s (N*K*2 bytes of bf16 weights).
    W is row-major here (the op-level entry point); the forward's decode GEMMs
    read packed copies and are timed in decode_e2e's kernel trace.  Each
    figure is the median over `reps` calls of HIP events around the call's
    launches (GEMM plus split-K reduce)."""
    import orion_hip as oh

    be = oh.HipBackend(0)
    out = []
    shapes = [("qkv", 2560, 2048, oh.GEMM_STORE), ("o", 2048, 2048, oh.GEMM_ACCUMULATE),
              ("gate_up", 11264, 2048, oh.GEMM_SWIGLU), ("down", 2048, 5632, oh.GEMM_ACCUMULATE),
              ("lm_head", 32000, 2048, oh.GEMM_STORE)]
    for M in (17526, 32):
        for name, N, K, ep in shapes:
            if M > 64 and name == "lm_head":
                continue  # the forward runs the head on the last rows only
            x, w, o = be.alloc(M * K * 4), be.alloc(N * K * 2), be.alloc(M * N * 4)
            for buf, n in ((x, M * K * 4), (w, N * K * 2), (o, M * N * 4)):
                oh._check(be.lib.orion_hip_memset(be.handle, buf.ptr, 0, n))
            for _ in range(2):
                oh.gemm(be, x.ptr, w.ptr, None, M, N, K, ep, o.ptr)
            be.synchronize()
            # HIP events around each call's launches (GEMM + split-K reduce):
            # the decode shapes take less GPU time than a host call costs
            be.kernel_timing(True)
            for _ in range(reps):
                oh.gemm(be, x.ptr, w.ptr, None, M, N, K, ep, o.ptr)
            ms = float(np.median(be.kernel_timing_samples(be.K_GEMM)))
            be.kernel_timing(False)
            rec = {"gemm": name, "M": M, "N": N, "K": K, "us": round(ms * 1e3, 1)}
            if M > 64:
                rec["tflops"] = round(2 * M * N * K / (ms * 1e-3) / 1e12, 1)
            else:
                rec["weight_GBps"] = round(N * K * 2 / (ms * 1e-3) / 1e9, 1)
            out.append(rec)
            for buf in (x, w, o):
                buf.free()
    be.close()
    return out


def sampling_bench(rows=32, vocab=32000, reps=10, seed=20261206):
    """The device sampler (runtime/src/sampling.rs DefaultSampler) on the
    config-4 decode batch's logits shape, per call including the token copy
    back, against the oracle's restatement on the host for the same rows."""
    import oracle as orc
    import orion_hip as oh

    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((rows, vocab)) * 2.0).astype(np.float32)
    prev = [rng.integers(0, vocab, 64).tolist() for _ in range(rows)]
    uni = rng.random(rows, dtype=np.float32).tolist()
    cases = {"greedy": oh.SamplingParams(temperature=0.0),
             "top_k50_top_p0.9": oh.SamplingParams(temperature=0.8, top_k=50, top_p=0.9,
                                                   repetition_penalty=1.1),
             "top_p0.95_full_vocab": oh.SamplingParams(temperature=1.0, top_p=0.95)}
    be = oh.HipBackend(0)
    d = be.alloc(rows * vocab * 4)
    out = {"rows": rows, "vocab": vocab}
    for name, p in cases.items():
        times = []
        for _ in range(reps + 2):
            d.upload(logits)
            be.synchronize()
            t0 = time.perf_counter()
            oh.sample(be, d.ptr, rows, vocab, [p] * rows, prev, uni)
            times.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        for r in range(rows):
            orc.sample(logits[r], prev[r], p.temperature, p.top_k, p.top_p,
                       p.repetition_penalty, uni[r])
        cpu = time.perf_counter() - t0
        out[name] = {"device_ms": round(float(np.median(times[2:])) * 1e3, 3),
                     "oracle_1thread_ms": round(cpu * 1e3, 2)}
    d.free()
    be.close()
    return out


QWEN2_7B_LAYER = dict(H=3584, hq=28, hkv=4, d=128, F=18944, V=1024, eps=1e-6, theta=1000000.0,
                      max_pos=16640)


def mixed_cfg5(steps=10, warmup=2, seed=20261205):
    """benchmark config 5: one Qwen2-7B-shape layer (hidden 3584, 28q/4kv heads,
    d 128, ffn 18944, QKV bias; bf16 weights synthetic N(0,0.02), RoPE theta
    1e6) over a mixed continuous batch: 8 prefill chunks of 256 tokens + 192
    decode rows, half the sequences sharing a 2048-token prefix through
    identical leading block ids, other context lognormal (median 1024) capped
    at 16384, block 16.  The KV cache (bf16) is filled with N(0,1) values.
    The LM head is cut to a 1024-token vocabulary so the figure is the layer's
    (the real 152k-row head would dominate).  Also times the two attention
    kernels alone on the same cache: decode rows against unique and logical
    K/V bytes, prefill chunks in TFLOP/s."""
    import orion_hip as oh
    from paged_cases import cfg5_batch

    cfg = QWEN2_7B_LAYER
    b = cfg5_batch(cfg["V"], seed)
    be = oh.HipBackend(0)
    meta = oh.ModelMetadata(hidden_size=cfg["H"], num_layers=1, num_attention_heads=cfg["hq"],
                            num_kv_heads=cfg["hkv"], head_dim=cfg["d"], vocab_size=cfg["V"],
                            intermediate_size=cfg["F"], max_position_embeddings=cfg["max_pos"],
                            rope_theta=cfg["theta"], rms_norm_eps=cfg["eps"],
                            architecture="qwen2")
    model = oh.HipTransformerModel(meta, b.num_blocks, b.bs, be, oh.BF16)
    model.init_synthetic(seed, 0.02)
    arena_ptr, arena_bytes = model.kv_arena()
    rng = np.random.default_rng(seed + 1)
    chunk = 1 << 26  # bf16 elements per upload
    for off in range(0, arena_bytes // 2, chunk):
        n = min(chunk, arena_bytes // 2 - off)
        bits = oh.f32_to_bf16_bits(rng.standard_normal(n, dtype=np.float32))
        oh._check(be.lib.orion_hip_memcpy_h2d(be.handle, arena_ptr + off * 2, bits.ctypes.data,
                                              bits.nbytes))
    batch = oh.ForwardBatch(b.tokens.tolist(), b.positions.tolist(), list(range(b.S)),
                            b.counts.tolist(), b.ctx.tolist(), [t.tolist() for t in b.tables],
                            True).prepare()  # Python list flattening once, outside the loop
    for _ in range(warmup):
        model.forward(batch, want_logits=False, want_argmax=True)
    be.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.forward(batch, want_logits=False, want_argmax=True)
    be.synchronize()
    layer_ms = (time.perf_counter() - t0) / steps * 1e3
    n_rows = len(b.positions)

    # attention kernels alone, same cache and tables
    kv = model.kv_layout()
    hq, hkv, d = cfg["hq"], cfg["hkv"], cfg["d"]
    offs = np.zeros(b.S + 1, np.int64)
    offs[1:] = np.cumsum([len(t) for t in b.tables])
    ids = np.concatenate(b.tables)
    dec = np.nonzero(~b.is_prefill)[0]
    pos_d = (b.ctx[dec] - 1).astype(np.uint32)
    rs_d = dec.astype(np.int32)
    q_d = rng.standard_normal((len(dec), hq * d), dtype=np.float32)
    pf = np.nonzero(b.is_prefill)[0]
    q_p = rng.standard_normal((len(pf) * 256, hq * d), dtype=np.float32)
    bufs = dict(bo=be.to_device(offs), bi=be.to_device(ids), qd=be.to_device(q_d),
                pos=be.to_device(pos_d), rs=be.to_device(rs_d), od=be.alloc(q_d.nbytes),
                qp=be.to_device(q_p), op=be.alloc(q_p.nbytes),
                pst=be.to_device((np.arange(len(pf)) * 256).astype(np.int32)),
                pcnt=be.to_device(np.full(len(pf), 256, np.int32)),
                pfp=be.to_device(b.cached[pf].astype(np.uint32)),
                pbo=be.to_device(offs[pf].astype(np.int64)))
    plan = oh.DecodePlan(be, pos_d, rs_d, offs, ids, hq, hkv, d, b.bs)

    def attn():
        oh.paged_attention_decode(be, kv, arena_ptr, 0, bufs["qd"].ptr, len(dec), hq,
                                  bufs["pos"].ptr, bufs["rs"].ptr, bufs["bo"].ptr, bufs["bi"].ptr,
                                  plan, bufs["od"].ptr)
        oh.paged_attention_prefill(be, kv, arena_ptr, 0, bufs["qp"].ptr, hq, len(pf),
                                   bufs["pst"].ptr, bufs["pcnt"].ptr, bufs["pfp"].ptr,
                                   bufs["pbo"].ptr, bufs["bi"].ptr, 256, int(b.ctx.max()),
                                   bufs["op"].ptr, hilo=False)
    for _ in range(warmup):
        attn()
    be.kernel_timing(True)
    for _ in range(steps):
        attn()
    split_ms = be.kernel_timing_read(be.K_DECODE_SPLIT)[0] / steps
    merge_ms = be.kernel_timing_read(be.K_DECODE_MERGE)[0] / steps
    pre_ms = be.kernel_timing_read(be.K_PREFILL)[0] / steps
    be.kernel_timing(False)
    uniq, logical = b.kv_bytes(hkv, d)
    pf_flops = 4 * hq * d * int(sum(256 * int(b.cached[s]) + 256 * 257 // 2 for s in pf))
    dec_ms = split_ms + merge_ms
    res = {
        "workload": "Qwen2-7B-shape layer (hidden 3584, 28q/4kv, d 128, ffn 18944, QKV bias; "
                    "vocab cut to 1024), bf16 weights N(0,0.02) + bf16 KV N(0,1); 8 prefill "
                    "chunks x 256 + 192 decodes, 50% share a 2048-token prefix, rest lognormal "
                    "(median 1024, sigma 1.0) capped 16384, block 16",
        "rows": n_rows,
        "layer_ms": round(layer_ms, 4),
        "layer_timing": "forward calls on one prepared batch (ForwardBatch.prepare: the Python "
                        "list flattening runs once); each call still validates, plans and "
                        "stages the batch in the library",
        "layer_rows_per_s": round(n_rows / (layer_ms * 1e-3), 1),
        "decode_attention": {
            "rows": int(len(dec)), "ms": round(dec_ms, 5), "split_ms": round(split_ms, 5),
            "unique_kv_bytes": uniq, "logical_kv_bytes": logical,
            "unique_GBps": round(uniq / (dec_ms * 1e-3) / 1e9, 1),
            "logical_GBps": round(logical / (dec_ms * 1e-3) / 1e9, 1),
            "unique_frac_of_hbm_peak": round(uniq / (dec_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "prefill_attention": {
            "chunks": int(len(pf)), "ms": round(pre_ms, 5), "flops": pf_flops,
            "tflops": round(pf_flops / (pre_ms * 1e-3) / 1e12, 1)},
    }
    plan.close()
    for v in bufs.values():
        v.free()
    model.close()
    be.close()
    return res


def cpu_decode_step(cfg, lens, tables, num_blocks, seqs, seed=20261204):
    """The oracle (C++ restatement of the reference CPU TransformerModel) on
    greedy decode steps of the benchmarked model and batch: the same synthetic
    bf16 weights (the oracle's restatement of the library's generator), the
    same 32 sequences and block tables, positions advancing from the prompt
    lengths, each step fed its own argmax, bf16-rounded KV as on the GPU.  The
    prompts are not prefilled on the CPU (about 10 minutes of work): the KV
    entries the steps attend hold zeros, which changes no timing."""
    import oracle as orc
    from cfg4_case import oracle_tinyllama

    threads, nproc = host_threads()
    orc.set_num_threads(threads)
    t0 = time.perf_counter()
    m = oracle_tinyllama(orc, num_blocks, seed=seed, cfg=cfg, kv_bf16=True)
    t_weights = time.perf_counter() - t0
    pos = [int(n) for n in lens]
    toks = [1] * seqs

    def step():
        nonlocal toks
        lg = m.forward(toks, pos, [1] * seqs, [p + 1 for p in pos], tables)
        toks = [orc.argmax(r) for r in lg]
        for i in range(seqs):
            pos[i] += 1

    step()  # warm-up (pages in the weights)
    dt, reps = timed_median(step, 20, 12.0)
    # The reference's own execution model (single-threaded): a bounded sample.
    orc.set_num_threads(1)
    dt1, reps1 = timed_median(step, 5, 12.0)
    orc.set_num_threads(threads)
    m.close()
    return {"value": round(seqs / dt, 3), "unit": "tokens/s", "cores": threads, "nproc": nproc,
            "kind": "port",
            "sample": f"greedy decode steps of the benchmarked model (synthetic weights, "
                      f"{seqs} sequences, positions advancing from the prompt lengths, prompts "
                      f"not prefilled on the CPU), median of {reps}, {dt:.3f} s/step, OpenMP "
                      f"over independent outputs; weight set-up {t_weights:.1f} s untimed",
            "single_thread": {"value": round(seqs / dt1, 3), "unit": "tokens/s", "cores": 1,
                              "sample": f"median of {reps1} further decode steps, {dt1:.2f} s"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-4 decode step")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-3 prefill kernel")
    ap.add_argument("--no-mixed", action="store_true", help="skip the config-5 mixed batch")
    ap.add_argument("--no-gemm", action="store_true", help="skip the GEMM shape timings")
    ap.add_argument("--no-sampling", action="store_true", help="skip the device sampler timing")
    ap.add_argument("--e2e-steps", type=int, default=64,
                    help="greedy decode steps of the config-4 run (64 as benchmarked; fewer for "
                         "profiling its prefill forward; the golden comparison needs 64)")
    ap.add_argument("--kv-layout", choices=["head-major", "reference"], default="reference",
                    help="block-internal order of the KV arena (reference = attention.rs order)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 3 plain 1 GiB device copies (PMC byte-counter scale)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (this build is single-GPU); --gpus {a.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)

    import orion_hip as oh
    from paged_cases import cfg2

    head_major = a.kv_layout == "head-major"
    case = cfg2(head_major=head_major)
    be = oh.HipBackend(0)
    kv = case.kv_layout()
    arena = be.to_device(case.arena_device_bytes())
    dq = be.to_device(case.q)
    dpos = be.to_device(case.positions)
    drs = be.to_device(case.row_seq)
    dbo = be.to_device(case.bt_offsets)
    dbi = be.to_device(case.bt_ids)
    dout = be.alloc(case.S * case.hq * case.d * 4)
    # The plan depends only on the batch's positions; a forward pass builds it
    # once and reuses it for every layer, so it is built outside the timed loop.
    plan = oh.DecodePlan(be, case.positions, case.row_seq, case.bt_offsets, case.bt_ids, case.hq,
                         case.hkv, case.d, case.bs)

    def step():
        oh.paged_attention_decode(be, kv, arena.ptr, 0, dq.ptr, case.S, case.hq, dpos.ptr,
                                  drs.ptr, dbo.ptr, dbi.ptr, plan, dout.ptr)

    for _ in range(a.warmup):
        step()
    be.synchronize()
    be.timer_start()
    for _ in range(a.steps):
        step()
    ms = be.timer_stop()
    be.synchronize()
    ms_per_step = ms / a.steps
    # The dominant kernel alone (split-K pass; the merge kernel is separate),
    # HIP events on the library's stream around each launch.
    be.kernel_timing(True)
    for _ in range(max(a.steps, 20)):
        step()
    split_ms, split_n = be.kernel_timing_read(be.K_DECODE_SPLIT)
    merge_ms, merge_n = be.kernel_timing_read(be.K_DECODE_MERGE)
    split_samples = be.kernel_timing_samples(be.K_DECODE_SPLIT)
    merge_samples = be.kernel_timing_samples(be.K_DECODE_MERGE)
    be.kernel_timing(False)
    split_avg = split_ms / max(split_n, 1)
    merge_avg = merge_ms / max(merge_n, 1)
    # Whole steps one at a time (events around each), for the median.
    step_samples = []
    for _ in range(max(a.steps, 20)):
        be.timer_start()
        step()
        step_samples.append(be.timer_stop())
    be.synchronize()
    step_med = float(np.median(step_samples))
    split_med = float(np.median(split_samples)) if len(split_samples) else split_avg

    # correctness spot-check of the measured output (cheap: 4 rows)
    got = dout.download(np.float32, (case.S, case.hq * case.d))
    rows = np.arange(4)
    want = case.oracle(case.positions[rows], case.row_seq[rows], case.q[rows])
    max_err = float(np.abs(got[rows] - want).max())

    nbytes = algorithmic_bytes(case)
    gbs = nbytes / (ms_per_step * 1e-3) / 1e9
    kern_gbs = nbytes / (split_avg * 1e-3) / 1e9
    result = {
        "metric": "paged-attn decode HBM GB/s (% peak) at Llama-3-8B shape; decode tokens/sec",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "paged GQA decode attention, Llama-3-8B layer shape (config 2): 64 seqs, "
                        "ctx U[128,4096], 32q/8kv heads, head_dim 128, bf16 KV, block 16, "
                        "pool 1.25x",
            "num_seqs": case.S,
            "sum_context": int(case.ctxs.sum()),
            "algorithmic_bytes_per_step": nbytes,
            "kv_dtype": "bf16",
            "kv_layout": a.kv_layout,
            "accumulate": "f32",
            "decode_plan": plan.info(),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_decode_mfma2_kernel (split-K pass)",
            "achieved": round(kern_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "kernel_ms": round(split_avg, 5),
            "kernel_ms_median": round(split_med, 5),
            "kernel_launches_timed": int(split_n),
            "merge_kernel_ms": round(merge_avg, 5),
            "merge_kernel_ms_median": round(float(np.median(merge_samples)), 5)
            if len(merge_samples) else None,
            **copy_ceiling(be, kern_gbs),
        },
        "step_ms_median": round(step_med, 5),
        "value_at_step_median": round(nbytes / (step_med * 1e-3) / 1e9, 1),
        "max_abs_err_vs_oracle": max_err,
    }
    if not a.no_cpu:
        result["cpu_baseline"] = cpu_baseline(case)
    for b in (arena, dq, dpos, drs, dbo, dbi, dout):
        b.free()
    plan.close()
    if not a.no_prefill:
        result["prefill_cfg3"] = prefill_cfg3(be, head_major=head_major)
    if a.copy_calibration:
        # Plain device-to-device copies of known size, for scaling the PMC
        # byte counters (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE).
        src, dst = be.alloc(1 << 30), be.alloc(1 << 30)
        for _ in range(3):
            be.memcpy_d2d(dst.ptr, src.ptr, 1 << 30)
        be.synchronize()
        src.free()
        dst.free()
        result["copy_calibration_bytes"] = 1 << 30
    be.close()
    if not a.no_e2e:
        result["decode_e2e"] = decode_e2e(steps=a.e2e_steps, cpu=not a.no_cpu)
    if not a.no_mixed:
        result["mixed_cfg5"] = mixed_cfg5()
    if not a.no_gemm:
        result["gemm"] = gemm_shapes()
    if not a.no_sampling:
        result["sampling"] = sampling_bench()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
