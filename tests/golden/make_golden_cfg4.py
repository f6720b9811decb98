"""Writes tests/golden/cfg4_greedy_{f32,bf16}kv.npz: the CPU oracle's greedy
decode of benchmark config 4 exactly as bench.py runs it.

The TinyLlama-1.1B-shape model with the library's synthetic bf16 weights
(seed 20261204, N(0, 0.02)), the bench's 32 sequences (prompts U[16, 1024],
scattered block tables), one prefill forward of all prompts, then 64 greedy
decode steps, each feeding the previous step's argmax at position
prompt_len + step.  The oracle's KV arena is f32 (the reference's dtype,
--kv f32) or holds every K/V element rounded to bf16 when written (--kv
bf16: the bench's KV dtype).

Stored per step (step 0 = the prefill's last rows, steps 1..64 = decode
steps) and sequence: the greedy token (reference argmax, lowest index wins
ties), the 8 largest logits and their ids (descending), and the top-2 margin.
Also stored: the prompt lengths and a checksum of the prompts and tables, so
a test can tell that the case generator still draws the same batch.

Run: python tests/golden/make_golden_cfg4.py --kv {f32,bf16} [--threads N]
(about 10 min on 8 cores)
"""
import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as orc  # noqa: E402
from cfg4_case import cfg4_case, oracle_tinyllama  # noqa: E402

TOPN = 8


def case_checksum(case):
    acc = []
    for p, t in zip(case.prompts, case.tables):
        acc.append(int(np.sum(np.asarray(p, np.int64) * np.arange(1, len(p) + 1))))
        acc.append(int(np.sum(np.asarray(t, np.int64) * np.arange(1, len(t) + 1))))
    return np.asarray(acc, np.int64)


def top_of(logits):
    idx = np.argsort(-logits, axis=1, kind="stable")[:, :TOPN]
    val = np.take_along_axis(logits, idx, axis=1)
    return idx.astype(np.int32), val.astype(np.float32)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--kv", choices=["f32", "bf16"], required=True)
    a = ap.parse_args()
    orc.set_num_threads(a.threads)
    case = cfg4_case()
    S, steps = case.seqs, case.steps
    t0 = time.time()
    m = oracle_tinyllama(orc, case.num_blocks, kv_bf16=a.kv == "bf16")
    print(f"weights {time.time() - t0:.0f} s", flush=True)
    toks = [t for p in case.prompts for t in p]
    pos = [i for n in case.lens for i in range(n)]
    t0 = time.time()
    lg = m.forward(toks, pos, case.lens, case.lens, case.tables)
    print(f"prefill {len(toks)} tokens {time.time() - t0:.0f} s", flush=True)
    tokens = np.zeros((steps + 1, S), np.int32)
    top_idx = np.zeros((steps + 1, S, TOPN), np.int32)
    top_val = np.zeros((steps + 1, S, TOPN), np.float32)
    ctx = list(case.lens)
    for step in range(steps + 1):
        tokens[step] = [orc.argmax(r) for r in lg]
        top_idx[step], top_val[step] = top_of(lg)
        if step == steps:
            break
        t0 = time.time()
        lg = m.forward(tokens[step].tolist(), ctx, [1] * S, [c + 1 for c in ctx], case.tables)
        ctx = [c + 1 for c in ctx]
        if step % 8 == 0:
            print(f"step {step} {time.time() - t0:.1f} s", flush=True)
    m.close()
    name = f"cfg4_greedy_{a.kv}kv.npz"
    np.savez_compressed(os.path.join(HERE, name), lens=np.asarray(case.lens),
                        checksum=case_checksum(case), tokens=tokens, top_idx=top_idx,
                        top_val=top_val, margin=top_val[:, :, 0] - top_val[:, :, 1])
    print("wrote", name)


if __name__ == "__main__":
    main()
