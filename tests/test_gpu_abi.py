"""The C-ABI called from C++ (tests/abi/abi_check.cpp) the way the Rust FFI
would call it, against the same model driven through the ctypes binding:
identical structs marshalled two ways must give bit-identical logits."""
import os
import subprocess

import numpy as np
import pytest

import orion_hip as oh
from conftest import ROOT

pytestmark = pytest.mark.gpu

ABI_CHECK = os.path.join(ROOT, "tests", "abi", "abi_check")


def test_cpp_caller_forward_matches_ctypes_caller(backend, tmp_path):
    out = str(tmp_path / "abi_forward.bin")
    print("[abi_check] forward from C++", flush=True)
    p = subprocess.run([ABI_CHECK, "forward", out], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stdout + p.stderr
    V = 1000
    raw = open(out, "rb").read()
    lg = np.frombuffer(raw[:2 * V * 4], np.float32).reshape(2, V)
    lg2 = np.frombuffer(raw[2 * V * 4:4 * V * 4], np.float32).reshape(2, V)
    am = np.frombuffer(raw[4 * V * 4:4 * V * 4 + 16], np.int64)
    am2 = np.frombuffer(raw[4 * V * 4 + 16:], np.int64)
    meta = oh.ModelMetadata(hidden_size=256, num_layers=2, num_attention_heads=4, num_kv_heads=2,
                            head_dim=64, vocab_size=V, intermediate_size=512,
                            max_position_embeddings=512, rope_theta=10000.0, rms_norm_eps=1e-5,
                            architecture="qwen2", tied_lm_head=False)
    m = oh.HipTransformerModel(meta, 32, 16, backend, oh.F32)
    m.init_synthetic(77, 0.05)
    toks = [1, 17, 300, 5, 999, 42, 42, 7, 8, 650, 11, 12, 13, 14]
    pos = [0, 1, 2, 3, 4, 0, 1, 2, 3, 4, 5, 6, 7, 8]
    o = m.forward(oh.ForwardBatch(toks, pos, [0, 1], [5, 9], [5, 9], [[3, 4], [10, 11]], True),
                  want_argmax=True)
    assert np.array_equal(o.logits.view(np.uint32), lg.view(np.uint32))
    assert list(o.argmax) == list(am)
    o2 = m.forward(oh.ForwardBatch([int(a) for a in am], [5, 9], [0, 1], [1, 1], [6, 10],
                                   [[3, 4], [10, 11]], False), want_argmax=True)
    assert np.array_equal(o2.logits.view(np.uint32), lg2.view(np.uint32))
    assert list(o2.argmax) == list(am2)
    m.close()
