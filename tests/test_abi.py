"""The C-ABI library loads and exports every symbol include/orion_hip.h
declares (no GPU needed: no compute call is made)."""
import os
import re
import subprocess
import ctypes as C

import numpy as np
import pytest

from conftest import ROOT

import orion_hip

HEADER = os.path.join(ROOT, "include", "orion_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(orion_hip_\w+)\s*\(", text)))


def test_header_and_binding_list_agree():
    assert declared_symbols() == sorted(orion_hip.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = orion_hip.load_library()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", orion_hip.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\b(orion_hip_\w+)\b", out))
    assert set(declared_symbols()) <= exported


def test_library_is_built_for_gfx950_only():
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o",
                          f"--input={orion_hip.LIB_PATH}"], capture_output=True, text=True)
    if out.returncode == 0 and out.stdout.strip():
        targets = [t for t in out.stdout.split() if "gfx" in t]
        assert targets and all("gfx950" in t for t in targets), targets


def test_synthetic_generator_statistics_and_determinism():
    # Host-side generator (no GPU call): zero mean, requested sd, bf16 values,
    # different tensors/layers give different streams.
    v = np.array([orion_hip.synthetic_value(3, orion_hip.W_Q, 0, i, 0.02) for i in range(20000)])
    assert abs(v.mean()) < 1e-3 and abs(v.std() - 0.02) < 1e-3
    assert np.array_equal(orion_hip.f32_to_bf16_bits(v.astype(np.float32)).astype(np.uint32) << 16,
                          v.astype(np.float32).view(np.uint32))
    w = np.array([orion_hip.synthetic_value(3, orion_hip.W_Q, 1, i, 0.02) for i in range(64)])
    assert not np.array_equal(v[:64], w)
    assert orion_hip.synthetic_value(3, orion_hip.W_INPUT_NORM, 0, 5, 0.02) == 1.0


def test_bf16_helpers_round_to_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.4e38, np.inf], np.float32)
    b = orion_hip.f32_to_bf16_bits(x)
    back = orion_hip.bf16_bits_to_f32(b)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 3*2^-8 is a tie -> 1 + 2^-6
    assert back[0] == 1.0 and back[1] == 1.0 and back[2] == np.float32(1.015625)
    assert back[3] == -2.5 and np.isinf(back[5])


ABI_CHECK = os.path.join(ROOT, "tests", "abi", "abi_check")


def test_c_struct_layouts_match_the_ctypes_binding():
    # tests/abi/abi_check.cpp static_asserts the header's layouts against the
    # #[repr(C)] structs of the Rust bindings; here the same layouts are
    # compared with the ctypes binding's structures.
    import json

    out = subprocess.run([ABI_CHECK, "layout"], capture_output=True, text=True, check=True)
    lay = json.loads(out.stdout)
    for cname, py in [("orion_hip_model_desc", orion_hip.ModelDesc),
                      ("orion_hip_batch", orion_hip.BatchDesc),
                      ("orion_hip_sampling_params", orion_hip.SamplingParams),
                      ("orion_hip_kv_layout", orion_hip.KvLayout)]:
        assert lay[cname]["size"] == C.sizeof(py), cname
        fields = [f[0] for f in py._fields_]
        assert list(lay[cname]["offsets"]) == fields, cname
        for f in fields:
            assert lay[cname]["offsets"][f] == getattr(py, f).offset, (cname, f)


def test_prepared_batch_reuses_the_flattened_arrays():
    """ForwardBatch.prepare validates once and keeps the CSR arrays that
    forward() would otherwise rebuild on every call (traits.rs:193-261)."""
    oh = orion_hip
    b = oh.ForwardBatch([5, 6, 7], [0, 1, 9], [0, 1], [2, 1], [2, 10], [[3], [4]], True)
    want = b.to_csr()
    assert b.prepare() is b
    for got, w in zip(b._prepared, want):
        assert np.array_equal(got, w)
    assert list(want[4]) == [0, 1, 2] and list(want[5]) == [3, 4]
    bad = oh.ForwardBatch([5], [0, 1], [0], [1], [1], [[3]], True)
    with pytest.raises(oh.InternalError):
        bad.prepare()


def test_advance_decode_updates_lists_and_prepared_arrays():
    """ForwardBatch.advance_decode: the next decode step of a prepared batch
    equals the batch built from scratch for that step (the reference's
    scheduler gives each decoding sequence its next token at position + 1,
    context + 1, the same table)."""
    oh = orion_hip
    b = oh.ForwardBatch([5, 6], [3, 9], [0, 1], [1, 1], [4, 10], [[3], [4]], False).prepare()
    assert b.advance_decode([7, 8]) is b
    want = oh.ForwardBatch([7, 8], [4, 10], [0, 1], [1, 1], [5, 11], [[3], [4]], False)
    assert (b.tokens, b.positions, b.context_lens) == ([7, 8], [4, 10], [5, 11])
    for got, w in zip(b._prepared, want.to_csr()):
        assert np.array_equal(got, w)
    with pytest.raises(oh.InternalError):  # not prepared
        oh.ForwardBatch([5], [0], [0], [1], [1], [[3]], False).advance_decode([1])
    with pytest.raises(oh.InternalError):  # a prefill chunk
        oh.ForwardBatch([5, 6], [0, 1], [0], [2], [2], [[3]], True).prepare().advance_decode([1, 2])
    with pytest.raises(oh.InternalError):  # wrong number of tokens
        b.advance_decode([1])
    with pytest.raises(OverflowError):  # a token id that is no u32
        b.advance_decode([-1, 2])


def test_bench_measures_one_gpu_only():
    """bench.py --gpus N with N > 1 exits with a message (this build measures
    one GPU); the check runs before the library is loaded."""
    import sys
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr


def test_serve_backend_patch_applies_to_the_reference():
    # crates/orion-hip/serve-backend.patch (the `orion serve --backend hip`
    # selection) must apply cleanly to the reference sources it targets; run
    # only where the reference tree is present (a dry run, nothing written).
    import shutil
    import subprocess
    ref = "/root/reference"
    patch = os.path.join(ROOT, "crates", "orion-hip", "serve-backend.patch")
    if not os.path.isdir(ref) or not shutil.which("patch"):
        pytest.skip("reference tree or patch(1) not present")
    p = subprocess.run(["patch", "-p1", "--dry-run", "-d", ref, "-i", patch],
                       capture_output=True, text=True)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "FAILED" not in p.stdout
