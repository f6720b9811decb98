"""The HIP model under the positions the reference engine really sends
(decode at total_len, leaving slot P unwritten; scheduler.rs:262-305,
engine.rs:311-330,456-482), against the CPU oracle step by step: a fresh
arena (the hole reads as zeros on both sides) and reused blocks (the hole
reads the previous tenant's K/V on both sides)."""
import numpy as np
import pytest

import oracle as orc
import orion_hip as oh
from engine_sim import SimSeq, build_batch, record_tokens
from model_fixtures import oracle_model, random_weights
from test_gpu_model import batch, gpu_model, rel_err, small_spec

pytestmark = pytest.mark.gpu


def drive(gm, om, seqs, steps, chunk, tol):
    """Runs the engine loop until every sequence has `steps` tokens; both
    models consume the oracle's greedy tokens."""
    worst = 0.0
    while min(len(s.output) for s in seqs) < steps:
        toks, pos, cnt, ctx, tables, fin = build_batch(seqs, chunk, quirk=True)
        g = gm.forward(batch(toks, pos, cnt, tables, ctx)).logits
        o = om.forward(toks, pos, cnt, ctx, tables)
        e = rel_err(g, o)
        worst = max(worst, e)
        assert e <= tol, (pos.tolist(), e)
        record_tokens(seqs, fin, [orc.argmax(r) for r in o])
    return worst


@pytest.mark.parametrize("kv", [oh.F32, oh.BF16])
def test_engine_positions_fresh_and_reused_blocks(backend, kv):
    rng = np.random.default_rng(41)
    spec = small_spec(L=2)
    W = random_weights(spec, rng, std=0.05)
    gm = gpu_model(backend, spec, W, kv)
    om = oracle_model(spec, W)
    tol = 1e-4 if kv == oh.F32 else 2e-2
    try:
        perm = [int(b) for b in rng.permutation(spec.num_blocks)]
        prompt = lambda n: [int(t) for t in rng.integers(0, spec.V, n)]
        # fresh arena: prompts of 21, 32 (the unwritten slot opens a new block)
        # and 7 tokens, chunked by 16
        seqs = [SimSeq(prompt(21), perm[0:6]), SimSeq(prompt(32), perm[6:12]),
                SimSeq(prompt(7), perm[12:18])]
        print(f"[engine] kv={kv} fresh", flush=True)
        drive(gm, om, seqs, steps=6, chunk=16, tol=tol)
        # reuse: new sequences take the freed tables with shorter prompts, so
        # their unwritten slot P holds what the old tenant wrote there
        seqs = [SimSeq(prompt(11), perm[0:6]), SimSeq(prompt(19), perm[6:12])]
        print(f"[engine] kv={kv} reused", flush=True)
        drive(gm, om, seqs, steps=6, chunk=16, tol=tol)
        for layer in range(spec.L):
            blk, slot = orc.locate(perm[0:6], 11, spec.block_size)
            assert gm.kv_read(layer, blk, slot, 0, False).any()  # the old tenant's key
    finally:
        gm.close()

