"""Greedy-token parity at benchmark config 4 exactly as the bench decodes it.

The HIP model (TinyLlama-1.1B shape, the bench's synthetic bf16 weights)
runs the bench's batch: 32 sequences, prompts U[16, 1024], scattered block
tables, one prefill forward, then 64 decode steps.  The steps are
teacher-forced with the oracle's tokens, so both sides see the same inputs at
every step.  Two arenas, each against the oracle's greedy decode of the same
batch with the same KV dtype (tests/golden/make_golden_cfg4.py):
  * bf16 KV (the bench's configuration) against the oracle with every K/V
    element rounded to bf16 when written (cfg4_greedy_bf16kv.npz);
  * f32 KV (the reference's dtype) against the reference-exact oracle
    (cfg4_greedy_f32kv.npz).

Checked per step and sequence (reference: transformer.rs:359-442 forward,
runtime/src/sampling.rs:196-207 argmax, lowest index on ties):
  * the logit error, measured on the oracle's 8 largest logits of every
    sequence, stays within the stated bound of max |logit| (f32 arithmetic
    in a different summation order; for bf16 KV also a K/V element that
    rounds the other way when the two sides' f32 values straddle a bf16
    rounding boundary);
  * the device argmax equals the oracle's token, except at near-ties: the
    device's token is then among the oracle's 8 best, and the oracle's margin
    between the two tokens is within twice that sequence's measured logit
    error.  Measured on the MI355X: 2 or 3 such tokens of 2,080 with f32 KV
    (two runs; logit error 6.7e-5 and 7.6e-5 of max |logit|), 6 with bf16 KV
    (two runs; 1.0e-3: a K/V element whose f32 value differs in its last bits
    between the two sides can round to the neighbouring bf16 value).  The
    caps are the largest measured count + 1: 4 (f32) and 7 (bf16).
"""
import os

import numpy as np
import pytest

import orion_hip as oh
from cfg4_case import SEED, STD, TINYLLAMA, cfg4_case

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("kv,bound,cap", [("bf16", 2e-3, 7), ("f32", 1e-4, 4)])
def test_cfg4_bench_batch_greedy_tokens_match_oracle(backend, kv, bound, cap):
    g = np.load(os.path.join(GOLDEN, f"cfg4_greedy_{kv}kv.npz"))
    case = cfg4_case()
    assert list(g["lens"]) == case.lens
    cfg = TINYLLAMA
    meta = oh.ModelMetadata(hidden_size=cfg["H"], num_layers=cfg["L"],
                            num_attention_heads=cfg["hq"], num_kv_heads=cfg["hkv"],
                            head_dim=cfg["d"], vocab_size=cfg["V"], intermediate_size=cfg["F"],
                            max_position_embeddings=cfg["max_pos"], rope_theta=cfg["theta"],
                            rms_norm_eps=cfg["eps"])
    m = oh.HipTransformerModel(meta, case.num_blocks, 16, backend,
                               oh.BF16 if kv == "bf16" else oh.F32)
    m.init_synthetic(SEED, STD)
    S, steps = case.seqs, case.steps
    toks = [t for p in case.prompts for t in p]
    pos = [i for n in case.lens for i in range(n)]
    print(f"[cfg4 greedy] prefill {len(toks)} tokens, {S} sequences, {kv} KV", flush=True)
    out = m.forward(oh.ForwardBatch(toks, pos, list(range(S)), case.lens, case.lens,
                                    case.tables, True), want_argmax=True)
    ctx = list(case.lens)
    compared = mismatches = 0
    worst = 0.0
    margins = []
    for step in range(steps + 1):
        lg, am = out.logits, out.argmax
        top_idx, top_val = g["top_idx"][step], g["top_val"][step]
        err_s = np.abs(np.take_along_axis(lg, top_idx, axis=1) - top_val).max(axis=1)
        err = float(err_s.max())
        scale = max(float(np.abs(top_val).max()), 1.0)
        worst = max(worst, err / scale)
        assert err <= bound * scale, (step, err, scale)
        for s in range(S):
            compared += 1
            if int(am[s]) != int(g["tokens"][step, s]):
                k = list(top_idx[s]).index(int(am[s])) if int(am[s]) in top_idx[s] else -1
                assert k > 0, (step, s, int(am[s]))
                gap = float(top_val[s, 0] - top_val[s, k])
                assert gap <= 2 * float(err_s[s]), (step, s, gap, float(err_s[s]))
                margins.append(gap)
                mismatches += 1
        if step == steps:
            break
        feed = g["tokens"][step].tolist()
        out = m.forward(oh.ForwardBatch(feed, ctx, list(range(S)), [1] * S,
                                        [c + 1 for c in ctx], case.tables, False),
                        want_argmax=True)
        ctx = [c + 1 for c in ctx]
    print(f"[cfg4 greedy] {compared} tokens compared, {mismatches} near-tie mismatches, "
          f"worst logit error {worst:.2e} of max |logit|, oracle margins at the mismatches "
          f"{sorted(round(x, 6) for x in margins)}", flush=True)
    assert mismatches <= cap
    m.close()
