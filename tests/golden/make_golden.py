"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

cfg1_decode.npz: benchmark config 1 (4 seqs, ctx U[1,512], bs 16, 8q/2kv,
d 64, f32) — context lengths, block tables, a checksum of the generated
inputs and the oracle's attention output [4, 8*64].
tiny_model.npz: the reference's fixture model (transformer.rs:459-523) —
logits of the scenarios in its tests.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from paged_cases import cfg1  # noqa: E402
from model_fixtures import oracle_model, tiny_spec, tiny_weights  # noqa: E402


def input_checksum(case):
    return np.array([float(np.float64(case.arena_f32).sum()), float(np.float64(case.q).sum())])


def main():
    case = cfg1()
    out = case.oracle()
    np.savez_compressed(os.path.join(HERE, "cfg1_decode.npz"), ctxs=case.ctxs,
                        bt_ids=case.bt_ids, bt_offsets=case.bt_offsets,
                        checksum=input_checksum(case), out=out)
    spec = tiny_spec(2)
    m = oracle_model(spec, tiny_weights(spec))
    full = m.forward([1, 2, 3, 4, 5], [0, 1, 2, 3, 4], [5], [5], [[0, 1]])
    m2 = oracle_model(spec, tiny_weights(spec))
    two = m2.forward([1, 2, 5, 6, 7], [0, 1, 0, 1, 2], [2, 3], [2, 3], [[0], [4]])
    np.savez_compressed(os.path.join(HERE, "tiny_model.npz"), full=full, two=two)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
