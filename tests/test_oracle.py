"""The CPU oracle pinned against the reference's own known-answer tests
(crates/orion-models/src/{tensor,attention,transformer}.rs test modules,
crates/orion-cuda/src/lib.rs, crates/orion-runtime/src/sampling.rs), closed
forms, brute force and independent float64 / torch restatements."""
import math

import numpy as np
import pytest

import oracle as orc


def approx(a, b, tol):
    return abs(a - b) < tol


# ---------------------------------------------------------------- tensor.rs
def test_linear_computes_x_times_w_transposed():  # tensor.rs:315-325
    out = orc.linear(np.array([[1.0, 2.0]]), np.array([[1.0, 0.0], [0.0, 1.0], [1.0, 1.0]]))
    assert out.shape == (1, 3)
    assert out.tolist() == [[1.0, 2.0, 3.0]]


def test_linear_applies_bias():  # tensor.rs:327-333
    out = orc.linear(np.array([[1.0, 1.0]]), np.array([[1.0, 1.0]]), np.array([10.0]))
    assert out.tolist() == [[12.0]]


def test_linear_handles_multiple_tokens():  # tensor.rs:335-341
    out = orc.linear(np.array([[1.0, 0.0], [0.0, 1.0]]), np.array([[2.0, 3.0]]))
    assert out.tolist() == [[2.0], [3.0]]


def test_linear_rejects_mismatched_shapes():  # tensor.rs:343-355
    with pytest.raises(orc.OracleError):
        orc.linear(np.ones((1, 3)), np.ones((2, 2)))
    with pytest.raises(orc.OracleError):
        orc.linear(np.ones((1, 3)), np.ones((1, 3)), np.array([1.0, 2.0]))


def test_linear_is_the_sequential_f32_dot():
    # The reference accumulates left to right in f32 from 0.0 (tensor.rs:96-130).
    # The restatement runs 16-row blocks x column pairs in vector registers;
    # check it bit for bit against an explicit f32 loop (each product rounded,
    # then each sum) at row counts inside one block, exactly one, and several
    # with ragged ends (n = 17, 33, 48), odd and even out_features (a column
    # pair cut short) and K not a multiple of 4, and against float64 within
    # f32 rounding.
    rng = np.random.default_rng(1)
    for n in (1, 3, 4, 7, 16, 17, 33, 48):
        for out_f, k in ((5, 37), (6, 38), (1, 3)):
            x = rng.standard_normal((n, k)).astype(np.float32)
            w = rng.standard_normal((out_f, k)).astype(np.float32)
            b = rng.standard_normal(out_f).astype(np.float32)
            out = orc.linear(x, w, b)
            acc = np.zeros((n, out_f), np.float32)
            for t in range(k):  # vectorised over (i, j); sequential over t
                acc = (acc + (x[:, t, None] * w[None, :, t]).astype(np.float32)).astype(np.float32)
            ref = (acc + b[None, :]).astype(np.float32)
            assert np.array_equal(out, ref), (n, out_f, k)
            np.testing.assert_allclose(out, x.astype(np.float64) @ w.T.astype(np.float64) + b,
                                       rtol=1e-5, atol=1e-5)
    # a slip in the block index (rows of block 2 taken from block 1) shows
    # as a swapped row: rows must depend on their own inputs only
    x = rng.standard_normal((48, 8)).astype(np.float32)
    w = rng.standard_normal((3, 8)).astype(np.float32)
    full = orc.linear(x, w)
    for i in (0, 15, 16, 31, 32, 47):
        assert np.array_equal(full[i], orc.linear(x[i:i + 1], w)[0])


def test_rms_norm_normalizes_to_unit_rms():  # tensor.rs:357-373
    x = orc.rms_norm(np.array([[3.0, 4.0]]), np.array([1.0, 1.0]), 0.0)
    r = math.sqrt(12.5)
    assert approx(x[0, 0], 3.0 / r, 1e-5) and approx(x[0, 1], 4.0 / r, 1e-5)
    assert approx(float(np.sqrt((x.astype(np.float64) ** 2).mean())), 1.0, 1e-5)


def test_rms_norm_applies_the_gain_vector():  # tensor.rs:375-382
    x = orc.rms_norm(np.array([[1.0, 1.0]]), np.array([2.0, 3.0]), 0.0)
    assert approx(x[0, 0], 2.0, 1e-6) and approx(x[0, 1], 3.0, 1e-6)


def test_rms_norm_rows_are_independent():  # tensor.rs:384-390
    x = orc.rms_norm(np.array([[1.0, 1.0], [100.0, 100.0]]), np.array([1.0, 1.0]), 0.0)
    assert approx(x[0, 0], x[1, 0], 1e-4)


def test_rms_norm_survives_an_all_zero_row():  # tensor.rs:392-399
    x = orc.rms_norm(np.zeros((1, 2)), np.ones(2), 1e-5)
    assert np.all(np.isfinite(x))


def test_rms_norm_rejects_a_mismatched_weight():  # tensor.rs:401-405
    with pytest.raises(orc.OracleError):
        orc.rms_norm(np.ones((1, 4)), np.ones(2), 1e-5)


def test_rms_norm_matches_float64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((6, 513)).astype(np.float32) * 3
    w = rng.standard_normal(513).astype(np.float32)
    out = orc.rms_norm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * w
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=1e-6)


def test_silu_matches_known_values():  # tensor.rs:407-415
    assert approx(orc.silu(0.0), 0.0, 1e-6)
    assert approx(orc.silu(1.0), 0.7310586, 1e-5)
    assert orc.silu(-1.0) < 0.0 and orc.silu(-1.0) > -0.3
    assert approx(orc.silu(20.0), 20.0, 1e-3)


def test_swiglu_multiplies_activated_gate_by_up():  # tensor.rs:417-425
    g = orc.swiglu(np.array([[1.0, 0.0]]), np.array([[2.0, 5.0]]))
    assert approx(g[0, 0], orc.silu(1.0) * 2.0, 1e-6) and approx(g[0, 1], 0.0, 1e-6)


def test_swiglu_rejects_mismatched_shapes():  # tensor.rs:427-432
    with pytest.raises(orc.OracleError):
        orc.swiglu(np.zeros((1, 2)), np.zeros((1, 3)))


def test_softmax_sums_to_one_and_is_stable():  # tensor.rs:434-445
    x = orc.softmax_inplace(np.array([1.0, 2.0, 3.0]))
    assert approx(float(x.sum()), 1.0, 1e-5) and x[2] > x[1] > x[0]
    big = orc.softmax_inplace(np.array([1000.0, 1001.0]))
    assert np.all(np.isfinite(big)) and approx(float(big.sum()), 1.0, 1e-5)


def test_softmax_matches_float64_and_nonfinite_rule():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(300) * 5).astype(np.float32)
    out = orc.softmax_inplace(x)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(out, e / e.sum(), rtol=1e-5, atol=1e-7)
    # tensor.rs:194-198: a non-finite max gives the uniform distribution.
    u = orc.softmax_inplace(np.array([np.inf, 1.0, 2.0, 3.0], np.float32))
    assert np.all(u == np.float32(0.25))


def test_rope_tables_have_the_expected_shape():  # tensor.rs:447-459
    t = orc.RopeTable(4, 8, 10000.0)
    cos, sin = t.at(0)
    assert cos.size == 2 and sin.size == 2
    assert np.allclose(cos, 1.0, atol=1e-6) and np.allclose(sin, 0.0, atol=1e-6)
    assert t.at(8) is None


def test_rope_requires_an_even_head_dim():  # tensor.rs:461-464
    with pytest.raises(orc.OracleError):
        orc.RopeTable(3, 8, 10000.0)


def test_rope_at_position_zero_is_the_identity():  # tensor.rs:466-475
    t = orc.RopeTable(4, 4, 10000.0)
    v = orc.apply_rope(np.array([1.0, 2.0, 3.0, 4.0]), *t.at(0))
    assert np.allclose(v, [1.0, 2.0, 3.0, 4.0], atol=1e-6)


def test_rope_pairs_i_with_i_plus_half_not_i_plus_one():  # tensor.rs:477-493
    v = orc.apply_rope(np.array([1.0, 2.0, 3.0, 4.0]), np.array([0.0, 0.0]), np.array([1.0, 1.0]))
    assert np.allclose(v, [-3.0, -4.0, 1.0, 2.0], atol=1e-6)


def test_rope_preserves_vector_norm():  # tensor.rs:495-506
    t = orc.RopeTable(8, 16, 10000.0)
    v0 = np.arange(1, 9, dtype=np.float32)
    v = orc.apply_rope(v0, *t.at(7))
    assert approx(float(np.linalg.norm(v0)), float(np.linalg.norm(v)), 1e-4)


def test_rope_encodes_relative_position():  # tensor.rs:508-530
    t = orc.RopeTable(8, 64, 10000.0)
    base = np.arange(1, 9, dtype=np.float32) * 0.1
    rot = lambda p: orc.apply_rope(base, *t.at(p))
    assert approx(float(rot(5) @ rot(8)), float(rot(20) @ rot(23)), 1e-3)


def test_rope_rejects_a_mismatched_table_width():  # tensor.rs:532-536
    with pytest.raises(orc.OracleError):
        orc.apply_rope(np.ones(4), np.array([1.0]), np.array([0.0]))


def test_rope_table_matches_float64_formula():
    # inv_freq = theta^(-2i/d), angle = pos * inv_freq; f32 rounding of the
    # angle dominates at large positions, so compare with a relative bound on
    # the angle error (|d angle| <= pos * |inv| * 2^-22).
    d, P, theta = 128, 4096, 500000.0
    t = orc.RopeTable(d, P, theta)
    i = np.arange(d // 2)
    inv = (1.0 / np.power(np.float32(theta), (2.0 * i / d).astype(np.float32))).astype(np.float32)
    ang = np.arange(P)[:, None].astype(np.float64) * inv.astype(np.float64)[None, :]
    tol = np.arange(P)[:, None] * inv[None, :].astype(np.float64) * 2.0 ** -22 + 2e-7
    assert np.all(np.abs(t.cos - np.cos(ang)) <= tol)
    assert np.all(np.abs(t.sin - np.sin(ang)) <= tol)


# ------------------------------------------------------------- attention.rs
def store():
    return orc.KvStore(2, 4, 2, 2, 4)


def test_the_arena_is_sized_from_its_dimensions():  # attention.rs:307-313
    s = store()
    assert len(s) == 2 * 4 * 2 * 2 * 2 * 4 and s.block_size() == 2 and s.num_blocks() == 4


def test_a_written_vector_reads_back_unchanged():  # attention.rs:315-320
    s = store()
    s.write(1, 2, 1, 0, False, [1.0, 2.0, 3.0, 4.0])
    assert s.read(1, 2, 1, 0, False).tolist() == [1.0, 2.0, 3.0, 4.0]


def test_keys_and_values_occupy_distinct_storage():  # attention.rs:322-329
    s = store()
    s.write(0, 0, 0, 0, False, [1.0] * 4)
    s.write(0, 0, 0, 0, True, [2.0] * 4)
    assert s.read(0, 0, 0, 0, False)[0] == 1.0 and s.read(0, 0, 0, 0, True)[0] == 2.0


def test_every_index_dimension_is_independent():  # attention.rs:331-346
    s = store()
    for i, idx in enumerate([(0, 0, 0, 0), (1, 0, 0, 0), (0, 1, 0, 0), (0, 0, 1, 0), (0, 0, 0, 1)]):
        s.write(*idx, False, [float(i + 1)] * 4)
    for i, idx in enumerate([(0, 0, 0, 0), (1, 0, 0, 0), (0, 1, 0, 0), (0, 0, 1, 0), (0, 0, 0, 1)]):
        assert s.read(*idx, False)[0] == float(i + 1)


def test_out_of_range_indices_are_errors_not_panics():  # attention.rs:348-356
    s = store()
    for args in [(9, 0, 0, 0), (0, 9, 0, 0), (0, 0, 9, 0), (0, 0, 0, 9)]:
        with pytest.raises(orc.OracleError):
            s.write(*args, False, [0.0] * 4)
    with pytest.raises(orc.OracleError):
        s.write(0, 0, 0, 0, False, [0.0] * 3)


def test_locate_maps_logical_positions_through_the_block_table():  # attention.rs:358-366
    t = [7, 3, 9]
    assert orc.locate(t, 0, 4) == (7, 0)
    assert orc.locate(t, 3, 4) == (7, 3)
    assert orc.locate(t, 4, 4) == (3, 0)
    assert orc.locate(t, 11, 4) == (9, 3)
    assert orc.locate(t, 12, 4) is None


def test_locate_handles_non_contiguous_physical_blocks():  # attention.rs:368-373
    assert orc.locate([100, 2, 57], 5, 4) == (2, 1)


def test_locate_and_offsets_brute_force():
    # Every position of random tables against pos // bs, pos % bs, and every
    # arena offset against the row-major index of [L][nb][2][bs][hkv][d].
    rng = np.random.default_rng(4)
    for bs in (4, 16, 64):
        table = rng.permutation(50)[:9].tolist()
        for pos in range(len(table) * bs + bs):
            got = orc.locate(table, pos, bs)
            want = (table[pos // bs], pos % bs) if pos // bs < len(table) else None
            assert got == want
    L, nb, bs, hkv, d = 2, 5, 4, 3, 8
    s = orc.KvStore(L, nb, bs, hkv, d)
    idx = np.arange(L * nb * 2 * bs * hkv * d).reshape(L, nb, 2, bs, hkv, d)
    for l in range(L):
        for b in range(nb):
            for kv in (0, 1):
                for sl in range(bs):
                    for h in range(hkv):
                        assert s.offset(l, b, kv, sl, h) == idx[l, b, kv, sl, h, 0]


def attn(s, q, table, ctx, qpos, hq, hkv, d, bs, layer=0):
    return orc.paged_attention(s, q, table, ctx, qpos, layer, hq, hkv, d, bs)


def test_attention_over_one_position_returns_that_value():  # attention.rs:375-403
    s = orc.KvStore(1, 2, 4, 1, 4)
    s.write(0, 0, 0, 0, False, [1.0, 0, 0, 0])
    s.write(0, 0, 0, 0, True, [9.0, 8.0, 7.0, 6.0])
    assert attn(s, [1.0, 0, 0, 0], [0], 1, 0, 1, 1, 4, 4).tolist() == [9.0, 8.0, 7.0, 6.0]


def test_attention_output_is_a_convex_combination_of_values():  # attention.rs:405-440
    s = orc.KvStore(1, 2, 4, 1, 2)
    for p in range(4):
        s.write(0, 0, p, 0, False, [float(p), 0.0])
        s.write(0, 0, p, 0, True, [p * 10.0, 1.0])
    out = attn(s, [1.0, 0.0], [0], 4, 3, 1, 1, 2, 4)
    assert 0.0 <= out[0] <= 30.0 and abs(out[1] - 1.0) < 1e-5


def test_causal_masking_ignores_future_positions():  # attention.rs:442-477
    s = orc.KvStore(1, 4, 4, 1, 2)
    s.write(0, 0, 0, 0, False, [1.0, 0.0])
    s.write(0, 0, 0, 0, True, [5.0, 5.0])
    for p in range(1, 4):
        s.write(0, 0, p, 0, False, [1.0, 0.0])
        s.write(0, 0, p, 0, True, [1000.0, 1000.0])
    assert attn(s, [1.0, 0.0], [0], 4, 0, 1, 1, 2, 4).tolist() == [5.0, 5.0]


def test_attention_spans_multiple_blocks():  # attention.rs:479-510
    s = orc.KvStore(1, 4, 2, 1, 2)
    for p in range(4):
        b, sl = orc.locate([0, 1], p, 2)
        s.write(0, b, sl, 0, False, [1.0, 0.0])
        s.write(0, b, sl, 0, True, [float(p), 1.0])
    assert abs(attn(s, [1.0, 0.0], [0, 1], 4, 3, 1, 1, 2, 2)[0] - 1.5) < 1e-5


def test_a_scattered_block_table_gives_the_same_answer():  # attention.rs:512-548
    def run(blocks):
        s = orc.KvStore(1, 8, 2, 1, 2)
        for p in range(4):
            b, sl = orc.locate(blocks, p, 2)
            s.write(0, b, sl, 0, False, [p * 0.5, 1.0])
            s.write(0, b, sl, 0, True, [float(p), 2.0])
        return attn(s, [0.7, 0.3], blocks, 4, 3, 1, 1, 2, 2)
    assert np.allclose(run([0, 1]), run([6, 2]), atol=1e-6)


def test_grouped_query_heads_share_kv_heads():  # attention.rs:550-582
    s = orc.KvStore(1, 1, 2, 2, 2)
    s.write(0, 0, 0, 0, False, [1.0, 0.0])
    s.write(0, 0, 0, 0, True, [10.0, 10.0])
    s.write(0, 0, 0, 1, False, [1.0, 0.0])
    s.write(0, 0, 0, 1, True, [20.0, 20.0])
    out = attn(s, [1.0, 0.0] * 4, [0], 1, 0, 4, 2, 2, 2)
    assert out.tolist() == [10.0, 10.0, 10.0, 10.0, 20.0, 20.0, 20.0, 20.0]


def test_attention_favours_the_most_similar_key():  # attention.rs:584-614
    s = orc.KvStore(1, 1, 4, 1, 2)
    s.write(0, 0, 0, 0, False, [0.0, 1.0])
    s.write(0, 0, 0, 0, True, [1.0, 0.0])
    s.write(0, 0, 1, 0, False, [10.0, 0.0])
    s.write(0, 0, 1, 0, True, [0.0, 1.0])
    out = attn(s, [10.0, 0.0], [0], 2, 1, 1, 1, 2, 4)
    assert out[1] > 0.9 and out[0] < 0.1


def test_mismatched_head_grouping_is_rejected():  # attention.rs:616-637
    s = orc.KvStore(1, 1, 2, 2, 2)
    with pytest.raises(orc.OracleError):
        attn(s, [0.0] * 6, [0], 1, 0, 3, 2, 2, 2)


def test_a_position_outside_the_block_table_is_an_error():  # attention.rs:639-658
    s = orc.KvStore(1, 1, 2, 1, 2)
    with pytest.raises(orc.OracleError):
        attn(s, [1.0, 0.0], [0], 6, 5, 1, 1, 2, 2)


def test_paged_attention_matches_torch_sdpa_on_depaged_kv():
    # cfg1 shape: 4 sequences, ctx U[1,512], bs 16, 8 q / 2 kv heads, d 64.
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(20261201)
    L, nb, bs, hkv, hq, d = 1, 256, 16, 2, 8, 64
    s = orc.KvStore(L, nb, bs, hkv, d)
    perm = rng.permutation(nb)
    ctxs = rng.integers(1, 513, size=4)
    cursor = 0
    for ctx in ctxs:
        nblk = -(-int(ctx) // bs)
        table = perm[cursor:cursor + nblk].tolist()
        cursor += nblk
        K = rng.standard_normal((ctx, hkv, d)).astype(np.float32)
        Vv = rng.standard_normal((ctx, hkv, d)).astype(np.float32)
        for p in range(ctx):
            b, sl = orc.locate(table, p, bs)
            for h in range(hkv):
                s.write(0, b, sl, h, False, K[p, h])
                s.write(0, b, sl, h, True, Vv[p, h])
        q = rng.standard_normal(hq * d).astype(np.float32)
        out = attn(s, q, table, int(ctx), int(ctx) - 1, hq, hkv, d, bs)
        qt = torch.from_numpy(q.reshape(1, hq, 1, d)).double()
        kt = torch.from_numpy(K).double().permute(1, 0, 2).repeat_interleave(hq // hkv, 0)[None]
        vt = torch.from_numpy(Vv).double().permute(1, 0, 2).repeat_interleave(hq // hkv, 0)[None]
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt).reshape(-1).numpy()
        np.testing.assert_allclose(out, ref, rtol=1e-4, atol=2e-5)


# -------------------------------------------------------- sampling / validate
def test_argmax_lowest_index_wins_ties():  # sampling.rs:196-207
    assert orc.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert orc.argmax([float("nan"), 0.5]) == 1
    assert orc.argmax([-np.inf, -np.inf]) is None
    assert orc.argmax([]) is None


def test_tolerance_and_validate_semantics():  # orion-cuda/src/lib.rs:319-453
    mm, ma, mr, wi = orc.validate([1.0, 2.0, 3.0], [1.0, 2.0, 3.0], orc.Tolerance.F32)
    assert mm == 0 and ma == 0.0
    mm, ma, mr, wi = orc.validate([1.0, 2.0, 3.0], [1.0, 2.5, 3.0], orc.Tolerance.F32)
    assert mm == 1 and wi == 1 and abs(ma - 0.5) < 1e-7
    # relative tolerance admits large magnitudes
    assert orc.validate([1e6], [1e6 + 5.0], orc.Tolerance.F32)[0] == 0
    # NaN matches only NaN, inf only the same inf
    assert orc.validate([float("nan")], [float("nan")], orc.Tolerance.F32)[0] == 0
    assert orc.validate([float("nan")], [0.0], orc.Tolerance.F32)[0] == 1
    assert orc.validate([float("inf")], [float("-inf")], orc.Tolerance.F32)[0] == 1
    with pytest.raises(orc.OracleError):
        orc.validate([1.0], [1.0, 2.0], orc.Tolerance.F32)


def test_oracle_reproduces_the_committed_cfg1_golden():
    import os
    from paged_cases import cfg1
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1_decode.npz"))
    case = cfg1()
    assert np.array_equal(case.ctxs, g["ctxs"]) and np.array_equal(case.bt_ids, g["bt_ids"])
    np.testing.assert_allclose(
        [float(np.float64(case.arena_f32).sum()), float(np.float64(case.q).sum())],
        g["checksum"], rtol=0, atol=1e-9)
    assert np.array_equal(case.oracle(), g["out"])


def test_cfg1_oracle_matches_torch_sdpa():
    # The whole config-1 workload against torch SDPA on the de-paged K/V.
    torch = pytest.importorskip("torch")
    from paged_cases import cfg1
    case = cfg1()
    out = case.oracle()
    a = case.arena_f32.reshape(case.num_blocks, 2, case.bs, case.hkv, case.d)
    for s in range(case.S):
        ctx = int(case.ctxs[s])
        tab = case.tables[s]
        K = np.stack([a[tab[p // case.bs], 0, p % case.bs] for p in range(ctx)])
        V = np.stack([a[tab[p // case.bs], 1, p % case.bs] for p in range(ctx)])
        g = case.hq // case.hkv
        qt = torch.from_numpy(case.q[s].reshape(1, case.hq, 1, case.d)).double()
        kt = torch.from_numpy(K).double().permute(1, 0, 2).repeat_interleave(g, 0)[None]
        vt = torch.from_numpy(V).double().permute(1, 0, 2).repeat_interleave(g, 0)[None]
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt).reshape(-1).numpy()
        np.testing.assert_allclose(out[s], ref, rtol=1e-4, atol=2e-5)
