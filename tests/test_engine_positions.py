"""The reference engine's decode positions, characterised on the CPU oracle
(crates/orion-scheduler/src/scheduler.rs:262-305, crates/orion-runtime/src/
engine.rs:311-330,456-482): after a prompt of length P the first decode is
sent at position P+1, so slot P is never written and every later step
attends over it as the arena left it."""
import numpy as np

import oracle as orc
from engine_sim import SimSeq, build_batch, record_tokens
from model_fixtures import Spec, oracle_model, random_weights


def spec():
    return Spec(2, 64, 4, 2, 16, 128, 97, max_pos=256, num_blocks=24, block_size=4)


def slot_of(om, s, table, p, layer, head, is_v):
    blk, slot = orc.locate(table, p, s.block_size)
    off = orc.lib().oracle_kv_offset(s.L, s.num_blocks, s.block_size, s.hkv, s.d, layer, blk,
                                     int(is_v), slot, head)
    return om.kv()[off:off + s.d]


def run(quirk, steps=4, P=21, chunk=8):
    s = spec()
    W = random_weights(s, np.random.default_rng(7), std=0.1)
    om = oracle_model(s, W)
    seq = SimSeq(prompt=list(np.random.default_rng(8).integers(0, s.V, P)), table=list(range(12)))
    positions, logits = [], []
    while len(seq.output) < steps:
        toks, pos, cnt, ctx, tables, fin = build_batch([seq], chunk, quirk)
        positions.append(pos.tolist())
        out = om.forward(toks, pos, cnt, ctx, tables)
        logits.append(out[0])
        record_tokens([seq], fin, [orc.argmax(out[0])])
    return s, om, seq, positions, logits


def test_decode_positions_skip_the_prompt_length():
    _, _, _, positions, _ = run(quirk=True)
    assert positions == [list(range(0, 8)), list(range(8, 16)), list(range(16, 21)), [22], [23],
                         [24]]
    _, _, _, fixed, _ = run(quirk=False)
    assert fixed[3:] == [[21], [22], [23]]


def test_the_skipped_slot_stays_as_the_arena_held_it():
    s, om, seq, _, _ = run(quirk=True)
    for layer in range(s.L):
        for h in range(s.hkv):
            for is_v in (False, True):
                assert not slot_of(om, s, seq.table, 21, layer, h, is_v).any()  # never written
                assert slot_of(om, s, seq.table, 22, layer, h, is_v).any()


def test_the_quirk_changes_what_decode_computes():
    # Prefill logits agree; from the first decode on, the zero slot enters
    # every softmax (score 0, value 0) and the positions are shifted by one.
    _, _, _, _, lq = run(quirk=True)
    _, _, _, _, lf = run(quirk=False)
    np.testing.assert_array_equal(lq[2], lf[2])
    assert np.abs(lq[3] - lf[3]).max() > 1e-3
