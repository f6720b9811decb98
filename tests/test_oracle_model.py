"""Oracle forward pinned by the reference's model tests
(crates/orion-models/src/transformer.rs:525-809) on its own fixture model and
by an independent float64 dense-attention restatement."""
import numpy as np
import pytest

import oracle as orc
from model_fixtures import (Spec, dense_forward_f64, oracle_model, random_weights, tiny_spec,
                            tiny_weights)


def tiny(num_layers):
    spec = tiny_spec(num_layers)
    return oracle_model(spec, tiny_weights(spec))


def fwd(m, tokens, positions, blocks, counts=None, ctx=None):
    counts = counts or [len(tokens)]
    ctx = ctx or counts
    tables = blocks if isinstance(blocks[0], list) else [blocks]
    return m.forward(tokens, positions, counts, ctx, tables)


def test_forward_gives_finite_logits_of_the_right_shape():  # :525-540
    out = fwd(tiny(2), [1, 2, 3], [0, 1, 2], [0])
    assert out.shape == (1, 8) and np.all(np.isfinite(out))


def test_only_the_last_position_yields_logits():  # :542-549
    assert fwd(tiny(1), [1, 2, 3, 4, 5], [0, 1, 2, 3, 4], [0, 1]).shape == (1, 8)


def test_an_empty_batch_returns_empty_output():  # :551-566
    assert tiny(1).forward([], [], [], [], []).shape == (0, 8)


def test_a_batch_of_several_sequences_yields_one_row_each():  # :568-588
    out = fwd(tiny(1), [1, 2, 3, 4], [0, 1, 0, 1], [[0], [1]], [2, 2], [2, 2])
    assert out.shape == (2, 8)


def test_batched_sequences_do_not_influence_each_other():  # :590-638
    m = tiny(2)
    alone = fwd(m, [1, 2], [0, 1], [0])
    together = fwd(m, [1, 2, 5, 6, 7], [0, 1, 0, 1, 2], [[0], [4]], [2, 3], [2, 3])
    assert np.allclose(alone[0], together[0], atol=1e-4)


def test_incremental_decode_matches_a_full_prefill():  # :640-677
    full = fwd(tiny(2), [1, 2, 3], [0, 1, 2], [0])[0]
    m = tiny(2)
    fwd(m, [1, 2], [0, 1], [0])
    inc = m.forward([3], [2], [1], [3], [[0]])[0]
    assert np.allclose(full, inc, atol=1e-4)


def test_chunked_prefill_matches_a_single_pass():  # :679-713
    whole = fwd(tiny(2), [1, 2, 3, 4], [0, 1, 2, 3], [0])[0]
    m = tiny(2)
    fwd(m, [1, 2], [0, 1], [0])
    chunked = m.forward([3, 4], [2, 3], [2], [4], [[0]])[0]
    assert np.allclose(whole, chunked, atol=1e-4)


def test_a_scattered_block_table_gives_identical_logits():  # :715-746
    a = fwd(tiny(2), [1, 2, 3, 4, 5], [0, 1, 2, 3, 4], [0, 1])[0]
    b = fwd(tiny(2), [1, 2, 3, 4, 5], [0, 1, 2, 3, 4], [11, 3])[0]
    assert np.allclose(a, b, atol=1e-5)


def test_different_prompts_give_different_logits():  # :748-767
    m = tiny(2)
    a = fwd(m, [1, 1, 1], [0, 1, 2], [0])[0]
    b = fwd(m, [5, 6, 4], [0, 1, 2], [2])[0]
    assert np.any(np.abs(a - b) > 1e-4)


def test_an_out_of_vocabulary_token_is_an_error():  # :769-776
    with pytest.raises(orc.OracleError):
        fwd(tiny(1), [999], [0], [0])


def test_a_position_beyond_the_rope_table_is_an_error():  # :778-793
    with pytest.raises(orc.OracleError):
        fwd(tiny(1), [1], [100], list(range(26)))


def test_an_inconsistent_batch_is_rejected():  # :795-801
    with pytest.raises(orc.OracleError):
        tiny(1).forward([1, 2], [0, 1], [5], [5], [[0]])


@pytest.mark.parametrize("bias,tied", [(False, True), (True, False)])
def test_forward_matches_dense_float64(bias, tied):
    # Llama-style (tied) and Qwen2-style (QKV bias, untied) small models.
    rng = np.random.default_rng(7)
    spec = Spec(2, 64, 4, 2, 16, 96, 50, max_pos=128, bias=bias, tied=tied, num_blocks=32,
                block_size=4)
    W = random_weights(spec, rng, std=0.2, bf16=False)
    tokens = rng.integers(0, spec.V, size=23).tolist()
    m = oracle_model(spec, W)
    table = rng.permutation(spec.num_blocks)[:6].tolist()
    got = m.forward(tokens, list(range(23)), [23], [23], [table])[0]
    want = dense_forward_f64(spec, W, tokens)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)


def test_tiny_model_golden_logits():
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "tiny_model.npz"))
    assert np.array_equal(fwd(tiny(2), [1, 2, 3, 4, 5], [0, 1, 2, 3, 4], [0, 1]), g["full"])
    two = fwd(tiny(2), [1, 2, 5, 6, 7], [0, 1, 0, 1, 2], [[0], [4]], [2, 3], [2, 3])
    assert np.array_equal(two, g["two"])


def test_bf16_kv_arena_holds_the_rounded_f32_values():
    # kv_bf16 rounds each K/V element to bf16 (nearest even) when it is
    # written: layer 0 (same inputs in both models) must hold exactly the
    # rounded values of the f32 arena; every stored value is bf16-exact, and
    # the logits move only by the rounding.
    from model_fixtures import bf16_round

    rng = np.random.default_rng(11)
    spec = Spec(2, 64, 4, 2, 16, 96, 50, max_pos=128, bias=True, tied=False, num_blocks=16,
                block_size=4)
    W = random_weights(spec, rng, std=0.2)
    tokens = rng.integers(0, spec.V, size=13).tolist()
    m32 = oracle_model(spec, W)
    m16 = orc.OracleTransformer(spec.L, spec.H, spec.hq, spec.hkv, spec.d, spec.F, spec.V,
                                spec.max_pos, spec.eps, spec.theta, spec.bias, spec.tied,
                                spec.num_blocks, spec.block_size, kv_bf16=True)
    for key, wid in [("input_norm", orc.W_INPUT_NORM), ("q", orc.W_Q), ("k", orc.W_K),
                     ("v", orc.W_V), ("o", orc.W_O), ("post_norm", orc.W_POST_NORM),
                     ("gate", orc.W_GATE), ("up", orc.W_UP), ("down", orc.W_DOWN),
                     ("q_bias", orc.W_Q_BIAS), ("k_bias", orc.W_K_BIAS), ("v_bias", orc.W_V_BIAS)]:
        for l in range(spec.L):
            m16.set_weight(wid, l, W["layers"][l][key])
    m16.set_weight(orc.W_EMBED, -1, W["embed"])
    m16.set_weight(orc.W_FINAL_NORM, -1, W["final_norm"])
    m16.set_weight(orc.W_LM_HEAD, -1, W["lm_head"])
    table = [3, 7, 1, 12]
    a = m32.forward(tokens, list(range(13)), [13], [13], [table])
    b = m16.forward(tokens, list(range(13)), [13], [13], [table])
    kv32, kv16 = m32.kv().copy(), m16.kv().copy()
    half = kv32.size // spec.L
    assert np.array_equal(kv16[:half].view(np.uint32), bf16_round(kv32[:half]).view(np.uint32))
    assert np.all((kv16.view(np.uint32) & 0xFFFF) == 0)
    assert not np.array_equal(a, b)
    assert float(np.abs(a - b).max()) <= 2e-2 * float(np.abs(a).max())
