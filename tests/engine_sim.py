"""How the reference engine builds a ForwardBatch, restated for tests: chunked
prefill, then one token per step per sequence, with the positions the engine
really sends.

The engine schedules a decode at ``start_position = total_len`` (prompt +
outputs so far, crates/orion-scheduler/src/scheduler.rs:262-305) and feeds the
LAST generated token there (crates/orion-runtime/src/engine.rs:456-482); the
first token is sampled from the final prefill chunk's logits
(engine.rs:311-330).  That token belongs at position ``total_len - 1``, so
with prompt length P the first decode writes position P+1 and position P is
never written: every decode attends over a slot that still holds what the
arena held before (zeros in a fresh arena, crates/orion-models/src/
attention.rs:45-56; a previous tenant's K/V in a reused block).  ``quirk=False``
gives the contiguous positions a corrected scheduler would send.
"""
from dataclasses import dataclass, field
from typing import List

import numpy as np


@dataclass
class SimSeq:
    prompt: List[int]
    table: List[int]
    computed: int = 0  # prompt tokens already prefilled
    output: List[int] = field(default_factory=list)

    @property
    def prefill_done(self):
        return self.computed >= len(self.prompt)

    @property
    def total_len(self):
        return len(self.prompt) + len(self.output)


def build_batch(seqs, chunk, quirk=True):
    """One engine step's batch: (tokens, positions, counts, context_lens,
    tables, prefill-finished flags).  Prefilling sequences get their next
    chunk of at most `chunk` prompt tokens; decoding ones one token."""
    toks, pos, counts, ctx, tables, finishing = [], [], [], [], [], []
    for s in seqs:
        if not s.prefill_done:
            start = s.computed
            t = s.prompt[start:min(start + chunk, len(s.prompt))]
            s.computed += len(t)
            finishing.append(s.prefill_done)
        else:
            start = s.total_len if quirk else s.total_len - 1
            t = [s.output[-1] if s.output else s.prompt[-1]]
            finishing.append(True)
        toks += t
        pos += range(start, start + len(t))
        counts.append(len(t))
        ctx.append(start + len(t))
        tables.append(s.table)
    return (np.array(toks, np.uint32), np.array(pos, np.uint32), counts, ctx, tables, finishing)


def record_tokens(seqs, finishing, tokens):
    """A token for every sequence whose logits row is final this step."""
    for s, fin, t in zip(seqs, finishing, tokens):
        if fin:
            s.output.append(int(t))
