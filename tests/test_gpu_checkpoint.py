"""TransformerModel::from_directory on the MI355X: a Hugging Face directory
(config.json + sharded safetensors) loaded straight to the device, against the
same weights uploaded one by one and against the CPU oracle
(crates/orion-models/src/transformer.rs:62-120,180-204)."""
import os

import numpy as np
import pytest

import hf_config as hc
import orion_hip as oh
from ckpt_fixtures import write_model_dir
from model_fixtures import Spec, oracle_model, random_weights
from test_gpu_model import KEYS, batch, gpu_model, rel_err

pytestmark = pytest.mark.gpu


def spec_of(bias, tied):
    return Spec(2, 256, 4, 2, 64, 512, 1000, max_pos=1024, bias=bias, tied=tied,
                num_blocks=64, block_size=16)


def prompts(spec, rng):
    lens = [21, 40]
    perm = rng.permutation(spec.num_blocks)
    tables = [perm[0:4], perm[4:8]]
    toks = rng.integers(0, spec.V, sum(lens))
    pos = np.concatenate([np.arange(n) for n in lens])
    return toks, pos, lens, tables


@pytest.mark.parametrize("bias,tied,dtype,shards", [(False, False, "BF16", 2),
                                                    (True, False, "F32", 3),
                                                    (False, True, "F16", 1)])
def test_from_directory_matches_uploaded_weights_and_oracle(backend, tmp_path, bias, tied,
                                                            dtype, shards):
    rng = np.random.default_rng(11)
    spec = spec_of(bias, tied)
    W = random_weights(spec, rng, std=0.05)  # bf16-representable values
    if dtype == "F16":  # keep values both bf16 and f16 hold exactly (others -> 0)
        def both(v):
            v16 = v.astype(np.float16).astype(np.float32)
            return np.where(v16 == v, v, np.float32(0)).astype(np.float32)
        for l in W["layers"]:
            for k, v in l.items():
                if v is not None:
                    l[k] = both(v)
        for k in ("embed", "final_norm", "lm_head"):
            if W[k] is not None:
                W[k] = both(W[k])
    write_model_dir(str(tmp_path), spec, W, dtype=dtype, shards=shards)
    print(f"[ckpt] bias={bias} tied={tied} dtype={dtype} shards={shards}", flush=True)
    m = oh.HipTransformerModel.from_directory(str(tmp_path), spec.num_blocks, spec.block_size,
                                              backend, oh.F32)
    ref = gpu_model(backend, spec, W, oh.F32)
    try:
        assert m.meta.architecture == ("qwen2" if bias else "llama")
        assert m.meta.tied_lm_head == tied
        # every weight the device holds equals the same array uploaded directly
        for key, wid in KEYS:
            src = W["layers"][1][key]
            if src is None:
                continue
            got = m.download_weight(wid, 1, src.size)
            want = ref.download_weight(wid, 1, src.size)
            assert np.array_equal(got, want), key
        toks, pos, lens, tables = prompts(spec, rng)
        g = m.forward(batch(toks, pos, lens, tables))
        r = ref.forward(batch(toks, pos, lens, tables))
        assert np.array_equal(g.logits, r.logits)
        o = oracle_model(spec, W).forward(toks, pos, lens, lens, tables)
        assert rel_err(g.logits, o) <= 1e-4, rel_err(g.logits, o)
    finally:
        m.close()
        ref.close()


def test_untied_model_without_lm_head_uses_the_embedding(backend, tmp_path):
    # transformer.rs:108-112: an absent lm_head.weight means the tied head.
    rng = np.random.default_rng(12)
    spec = spec_of(False, False)
    W = random_weights(spec, rng, std=0.05)
    W["lm_head"] = None
    write_model_dir(str(tmp_path), spec, W, dtype="BF16", shards=2)
    m = oh.HipTransformerModel.from_directory(str(tmp_path), spec.num_blocks, spec.block_size,
                                              backend, oh.F32)
    try:
        head = m.download_weight(oh.W_LM_HEAD, -1, spec.V * spec.H)
        assert np.array_equal(head, W["embed"].reshape(-1))
        tied = spec_of(False, True)
        toks, pos, lens, tables = prompts(spec, rng)
        o = oracle_model(tied, W).forward(toks, pos, lens, lens, tables)
        g = m.forward(batch(toks, pos, lens, tables))
        assert rel_err(g.logits, o) <= 1e-4
    finally:
        m.close()


def test_shape_mismatch_and_missing_tensor_are_model_errors(backend, tmp_path):
    rng = np.random.default_rng(13)
    spec = spec_of(False, True)
    W = random_weights(spec, rng)
    W["layers"][0]["q"] = W["layers"][0]["q"][:, :128]  # wrong in-features
    write_model_dir(str(tmp_path / "bad_shape"), spec, W)
    with pytest.raises(hc.ShapeMismatch, match="q_proj"):
        oh.HipTransformerModel.from_directory(str(tmp_path / "bad_shape"), spec.num_blocks,
                                              spec.block_size, backend)
    W = random_weights(spec, rng)
    W["layers"][1]["down"] = None
    write_model_dir(str(tmp_path / "missing"), spec, W)
    with pytest.raises(hc.TensorNotFound, match="model.layers.1.mlp.down_proj.weight"):
        oh.HipTransformerModel.from_directory(str(tmp_path / "missing"), spec.num_blocks,
                                              spec.block_size, backend)
    os.makedirs(tmp_path / "arch", exist_ok=True)
    write_model_dir(str(tmp_path / "arch"), spec, random_weights(spec, rng),
                    config_extra={"architectures": ["GPT2LMHeadModel"], "model_type": "gpt2"})
    with pytest.raises(hc.UnsupportedArchitecture):
        oh.HipTransformerModel.from_directory(str(tmp_path / "arch"), spec.num_blocks,
                                              spec.block_size, backend)
