"""Checkpoint loading on the host (no GPU): the library's safetensors reader
against the reference loader's tests (crates/orion-models/src/loader.rs:
238-386), files written by the `safetensors` package itself, the dtype
widening closed forms, malformed files, and config.json parsing against the
reference's config tests (crates/orion-models/src/config.rs:245-445)."""
import json
import os

import numpy as np
import pytest

import hf_config as hc
import orion_hip as oh
from ckpt_fixtures import bf16_bits, tensor_entry, write_safetensors


def write_f32(directory, tensors, name="model.safetensors"):
    """The reference tests' write_checkpoint (loader.rs:243-262), via the
    safetensors package."""
    from safetensors.numpy import save_file

    os.makedirs(directory, exist_ok=True)
    save_file({k: np.asarray(v, np.float32).reshape(s) for k, (s, v) in tensors.items()},
              os.path.join(directory, name))


def test_loads_tensors_by_name_with_their_shapes(tmp_path):  # loader.rs:272-291
    write_f32(tmp_path, {"weight": ([2, 3], [1, 2, 3, 4, 5, 6]), "norm": ([3], [0.5] * 3)})
    with oh.Checkpoint(str(tmp_path)) as ck:
        assert len(ck) == 2
        assert ck.contains("weight") and not ck.contains("absent")
        assert ck.names() == ["norm", "weight"]
        data, shape = ck.tensor("weight")
        assert shape == [2, 3]
        assert data.tolist() == [1, 2, 3, 4, 5, 6]


def test_a_missing_tensor_names_itself(tmp_path):  # loader.rs:317-325
    write_f32(tmp_path, {"present": ([2], [1, 2])})
    with oh.Checkpoint(str(tmp_path)) as ck:
        with pytest.raises(hc.TensorNotFound, match="absent"):
            ck.tensor("absent")


def test_a_directory_with_no_checkpoint_is_refused(tmp_path):  # loader.rs:345-353
    with pytest.raises(hc.MissingFile):
        oh.Checkpoint(str(tmp_path))


def test_a_nonexistent_directory_is_refused():  # loader.rs:355-361
    with pytest.raises(hc.PathNotFound):
        oh.Checkpoint("/definitely/not/here")


def test_tensors_are_indexed_across_multiple_shards(tmp_path):  # loader.rs:363-385
    write_f32(tmp_path, {"first": ([2], [1, 2])}, "a.safetensors")
    write_f32(tmp_path, {"second": ([2], [1, 2])}, "b.safetensors")
    with oh.Checkpoint(str(tmp_path)) as ck:
        assert len(ck) == 2
        assert ck.contains("first") and ck.contains("second")
        assert ck.tensor("second")[0].tolist() == [1, 2]


def test_a_duplicated_name_resolves_to_the_first_file(tmp_path):  # loader.rs:127-131,149-152
    write_f32(tmp_path, {"w": ([2], [7, 7])}, "b.safetensors")
    write_f32(tmp_path, {"w": ([2], [3, 3])}, "a.safetensors")
    with oh.Checkpoint(str(tmp_path)) as ck:
        assert len(ck) == 1
        assert ck.tensor("w")[0].tolist() == [3, 3]


def test_dtype_widening_closed_forms(tmp_path):
    # loader.rs:74-98 with half 2.7.1: bf16 -> f32 is the bit pattern shifted
    # left by 16; f16 -> f32 is exact (IEEE binary16 widening); f32 is copied.
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 16, 4096, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7F80) != 0x7F80]  # finite values only
    f16 = rng.standard_normal(1000).astype(np.float16)
    f16[:4] = [0.0, -0.0, 65504.0, np.float16(6e-8)]  # zero, max, subnormal
    f32 = rng.standard_normal(1000).astype(np.float32)
    write_safetensors(str(tmp_path / "m.safetensors"), {
        "b": ("BF16", [len(bits)], bits.tobytes()),
        "h": ("F16", [len(f16)], f16.tobytes()),
        "s": ("F32", [len(f32)], f32.tobytes()),
    })
    with oh.Checkpoint(str(tmp_path)) as ck:
        got_b = ck.tensor("b")[0]
        assert np.array_equal(got_b.view(np.uint32), bits.astype(np.uint32) << 16)
        assert np.array_equal(ck.tensor("h")[0], f16.astype(np.float32))
        assert np.array_equal(ck.tensor("s")[0].view(np.uint32), f32.view(np.uint32))
        assert [ck.info(i)[1] for i in range(3)] == [oh.BF16, oh.F16, oh.F32]


def test_metadata_and_header_padding_are_accepted(tmp_path):
    write_safetensors(str(tmp_path / "m.safetensors"),
                      {"x": tensor_entry(np.arange(6, dtype=np.float32).reshape(2, 3), "F32")},
                      metadata={"format": "pt", "note": "a \"quoted\" \\ value é"})
    with oh.Checkpoint(str(tmp_path)) as ck:
        data, shape = ck.tensor("x")
        assert shape == [2, 3] and data.tolist() == [0, 1, 2, 3, 4, 5]


def test_unsupported_dtypes_are_listed_but_not_read(tmp_path):  # loader.rs:91-96
    write_safetensors(str(tmp_path / "m.safetensors"),
                      {"i": ("I32", [2], np.array([1, 2], np.int32).tobytes())})
    with oh.Checkpoint(str(tmp_path)) as ck:
        assert ck.info(0)[:2] == ("i", -1)
        with pytest.raises(hc.UnsupportedDtype, match="I32"):
            ck.tensor("i")


def _raw_file(path, header_obj, data=b"", header_bytes=None):
    h = header_bytes if header_bytes is not None else json.dumps(header_obj).encode()
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        f.write(data)


@pytest.mark.parametrize("case", ["truncated", "bad_json", "outside", "size", "overlap",
                                  "short_len", "no_offsets", "trailing", "wrap"])
def test_malformed_files_are_refused(tmp_path, case):
    p = str(tmp_path / "m.safetensors")
    z = b"\0" * 16
    if case == "truncated":
        open(p, "wb").write(b"\x05\0\0")
    elif case == "bad_json":
        _raw_file(p, None, z, header_bytes=b'{"a": {"dtype": "F32",')
    elif case == "outside":
        _raw_file(p, {"a": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]}}, z)
    elif case == "size":
        _raw_file(p, {"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, z)
    elif case == "overlap":
        _raw_file(p, {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
                      "b": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}, z)
    elif case == "short_len":
        with open(p, "wb") as f:
            f.write((1 << 40).to_bytes(8, "little"))
            f.write(b"{}")
    elif case == "no_offsets":
        _raw_file(p, {"a": {"dtype": "F32", "shape": [2]}}, z)
    elif case == "trailing":
        _raw_file(p, None, z, header_bytes=b'{} {}')
    elif case == "wrap":
        # 2^62 f32 elements: count * 4 wraps to 0 in 64 bits, matching the
        # empty data_offsets unless the size check refuses it first
        _raw_file(p, {"a": {"dtype": "F32", "shape": [1 << 62], "data_offsets": [0, 0]}}, z)
    with pytest.raises(hc.Malformed):
        oh.Checkpoint(str(tmp_path))


# ---- config.json (config.rs tests) ----

LLAMA = {
    "architectures": ["LlamaForCausalLM"], "model_type": "llama", "hidden_size": 4096,
    "num_hidden_layers": 32, "num_attention_heads": 32, "num_key_value_heads": 8,
    "vocab_size": 128256, "intermediate_size": 14336, "max_position_embeddings": 8192,
    "rope_theta": 500000.0, "rms_norm_eps": 1e-05, "torch_dtype": "bfloat16",
    "eos_token_id": [128001, 128009], "bos_token_id": 128000,
}
SMALL = {"architectures": ["LlamaForCausalLM"], "hidden_size": 64, "num_hidden_layers": 2,
         "num_attention_heads": 4, "vocab_size": 100}


def cfg(**kw):
    return hc.HfConfig.from_json(json.dumps(kw))


def test_parses_a_realistic_llama_config():  # config.rs:270-286
    c = cfg(**LLAMA)
    m = c.to_metadata("llama-3-8b")
    assert (m.architecture, m.num_layers, m.num_kv_heads, m.head_dim) == ("llama", 32, 8, 128)
    assert c.dtype() == "bf16"
    assert c.eos_token_ids() == [128001, 128009] and c.bos_token_id == 128000
    assert m.num_attention_heads // m.num_kv_heads == 4
    assert (m.intermediate_size, m.rope_theta, m.max_position_embeddings) == (14336, 500000.0, 8192)


def test_a_single_eos_id_is_accepted_as_well_as_a_list():  # config.rs:288-298
    assert cfg(**SMALL, eos_token_id=2).eos_token_ids() == [2]


def test_absent_kv_heads_means_multi_head_attention():  # config.rs:300-310
    assert cfg(**SMALL).to_metadata("t").num_kv_heads == 4


def test_unknown_fields_are_ignored():  # config.rs:312-324
    cfg(**SMALL, transformers_version="4.40.0", use_cache=True,
        some_future_field={"nested": [1, 2, 3]})


def test_alternate_field_names_are_accepted():  # config.rs:326-339
    c = cfg(model_type="llama", hidden_size=64, n_layer=2, n_head=4, vocab_size=100,
            n_positions=1024)
    m = c.to_metadata("t")
    assert (m.num_layers, m.num_attention_heads, m.max_position_embeddings) == (2, 4, 1024)
    assert cfg(**SMALL, layer_norm_eps=1e-6).to_metadata("t").rms_norm_eps == 1e-6


def test_an_unsupported_architecture_is_refused():  # config.rs:341-351
    c = cfg(**{**SMALL, "architectures": ["BertForMaskedLM"]})
    with pytest.raises(hc.UnsupportedArchitecture, match="BertForMaskedLM"):
        c.to_metadata("t")


def test_qwen2_is_detected_and_declares_qkv_bias():  # config.rs:353-366
    m = cfg(**{**SMALL, "architectures": ["Qwen2ForCausalLM"]}).to_metadata("t")
    assert m.architecture == "qwen2" and m.has_qkv_bias()
    assert not cfg(**SMALL).to_metadata("t").has_qkv_bias()
    assert cfg(**{k: v for k, v in SMALL.items() if k != "architectures"},
               model_type="qwen2").architecture() == "qwen2"


def test_inconsistent_head_counts_are_rejected():  # config.rs:368-381
    with pytest.raises(hc.Malformed):
        cfg(**{**SMALL, "num_attention_heads": 7, "num_key_value_heads": 2}).to_metadata("t")


@pytest.mark.parametrize("field", ["num_hidden_layers", "vocab_size"])
def test_zero_valued_dimensions_are_rejected(field):  # config.rs:383-398
    with pytest.raises(hc.Malformed):
        cfg(**{**SMALL, field: 0}).to_metadata("t")


def test_an_unsupported_dtype_is_refused():  # config.rs:400-412
    with pytest.raises(hc.UnsupportedDtype):
        cfg(**SMALL, torch_dtype="float8_e4m3fn").to_metadata("t")


def test_explicit_head_dim_overrides_the_derived_value():  # config.rs:414-425
    assert cfg(**SMALL, head_dim=32).to_metadata("t").head_dim == 32


def test_ffn_dim_falls_back_to_the_llama_convention():  # config.rs:427-437
    c = cfg(**SMALL)
    assert c.ffn_dim() == 256 and not c.ties_embeddings()
    m = c.to_metadata("t")
    assert (m.rope_theta, m.rms_norm_eps, m.max_position_embeddings) == (10000.0, 1e-5, 2048)


def test_a_missing_config_file_names_the_path():  # config.rs:439-443
    with pytest.raises(hc.MissingFile, match="/nonexistent/model"):
        hc.HfConfig.load("/nonexistent/model")


def test_bf16_bit_helper_rounds_to_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5], np.float32)  # ties at the half-ulp
    assert bf16_bits(x).tolist() == [0x3F80, 0x3F80, 0x3F82, 0xC020]
