"""The config-4 greedy golden fixture and the inputs it is made from (CPU).

* The synthetic weight generator: the numpy restatement, the oracle's C
  restatement and the HIP library's host entry point agree bit for bit.
* The case generator still draws the batch the fixture was made from.
* The fixture is self-consistent (token = the largest of the stored logits,
  lowest index on ties; margins non-negative).
* The oracle reproduces the fixture for the shortest sequence run alone:
  the reference's batching-independence invariant (transformer.rs:601-640)
  makes its logits bit-identical to those of the 32-sequence batch.
"""
import os

import numpy as np
import pytest

import oracle as orc
from cfg4_case import (SEED, STD, TINYLLAMA, W_DOWN, W_EMBED, W_GATE, W_INPUT_NORM, W_LM_HEAD,
                       W_Q, W_UP, cfg4_case, oracle_tinyllama, synthetic_weight_np)

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDENS = {"f32": os.path.join(HERE, "golden", "cfg4_greedy_f32kv.npz"),
           "bf16": os.path.join(HERE, "golden", "cfg4_greedy_bf16kv.npz")}


@pytest.mark.parametrize("which,layer", [(W_EMBED, -1), (W_LM_HEAD, -1), (W_Q, 0), (W_GATE, 7),
                                         (W_UP, 7), (W_DOWN, 21), (W_INPUT_NORM, 3)])
def test_synthetic_weights_agree_with_the_library(which, layer):
    import orion_hip as oh

    n = 4096
    a = synthetic_weight_np(SEED, which, layer, n)
    b = orc.synthetic_weight(SEED, which, layer, n, STD)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    rng = np.random.default_rng(which * 100 + layer + 1)
    for i in rng.integers(0, n, 64).tolist() + [0, n - 1]:
        v = np.float32(oh.synthetic_value(SEED, which, layer, i, STD))
        assert v.view(np.uint32) == a[i].view(np.uint32), (which, layer, i)
    if which not in (W_INPUT_NORM,):
        assert 0.018 < float(a.std()) < 0.022
        # bf16-exact values
        assert np.all((a.view(np.uint32) & 0xFFFF) == 0)


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_golden_matches_the_case_generator(kv):
    from golden.make_golden_cfg4 import case_checksum

    g = np.load(GOLDENS[kv])
    case = cfg4_case()
    assert list(g["lens"]) == case.lens
    assert np.array_equal(g["checksum"], case_checksum(case))
    assert g["tokens"].shape == (case.steps + 1, case.seqs)


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_golden_is_self_consistent(kv):
    g = np.load(GOLDENS[kv])
    assert np.array_equal(g["tokens"], g["top_idx"][:, :, 0])
    assert np.all(g["margin"] >= 0)
    assert np.all(np.diff(g["top_val"], axis=2) <= 0)
    assert np.all((g["tokens"] >= 0) & (g["tokens"] < TINYLLAMA["V"]))


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_oracle_reproduces_golden_for_one_sequence_alone(kv):
    g = np.load(GOLDENS[kv])
    case = cfg4_case()
    s = int(np.argmin(case.lens))
    steps = 3
    m = oracle_tinyllama(orc, case.num_blocks, kv_bf16=kv == "bf16")
    try:
        n = case.lens[s]
        lg = m.forward(case.prompts[s], list(range(n)), [n], [n], [case.tables[s]])
        for step in range(steps + 1):
            row = lg[0]
            top = np.argsort(-row, kind="stable")[:8]
            assert np.array_equal(top, g["top_idx"][step, s]), step
            assert np.array_equal(row[top].view(np.uint32), g["top_val"][step, s].view(np.uint32))
            assert orc.argmax(row) == g["tokens"][step, s]
            if step == steps:
                break
            p = n + step
            lg = m.forward([int(g["tokens"][step, s])], [p], [1], [p + 1], [case.tables[s]])
    finally:
        m.close()
