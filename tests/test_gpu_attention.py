"""Paged decode attention on the MI355X against the CPU oracle
(crates/orion-models/src/attention.rs:219-295 restated in oracle/)."""
import numpy as np
import pytest

import oracle as orc
import orion_hip as oh
from paged_cases import PagedCase, cfg1, cfg2

pytestmark = pytest.mark.gpu


def run_decode(be, case, positions=None, row_seq=None, q=None):
    positions = case.positions if positions is None else np.asarray(positions, np.uint32)
    row_seq = case.row_seq if row_seq is None else np.asarray(row_seq, np.int32)
    q = case.q if q is None else q
    rows = len(positions)
    kv = case.kv_layout()
    bufs = [be.to_device(case.arena_device_bytes()), be.to_device(q), be.to_device(positions),
            be.to_device(row_seq), be.to_device(case.bt_offsets), be.to_device(case.bt_ids),
            be.alloc(rows * case.hq * case.d * 4)]
    arena, dq, dpos, drs, dbo, dbi, dout = bufs
    print(f"[decode] rows={rows} hq={case.hq} hkv={case.hkv} d={case.d} bs={case.bs} "
          f"dtype={case.dtype} maxpos={int(positions.max())}", flush=True)
    plan = oh.DecodePlan(be, positions, row_seq, case.bt_offsets, case.bt_ids, case.hq, case.hkv,
                         case.d, case.bs)
    oh.paged_attention_decode(be, kv, arena.ptr, 0, dq.ptr, rows, case.hq, dpos.ptr, drs.ptr,
                              dbo.ptr, dbi.ptr, plan, dout.ptr)
    out = dout.download(np.float32, (rows, case.hq * case.d))
    plan.close()
    for b in bufs:
        b.free()
    return out


def test_cfg1_matches_oracle_f32_tolerance(backend):
    case = cfg1()
    got = run_decode(backend, case)
    want = case.oracle()
    mm, ma, mr, wi = orc.validate(want, got, orc.Tolerance.F32)
    assert mm == 0, (ma, mr, wi)


@pytest.mark.parametrize("head_major", [False, True])
def test_cfg2_full_size_bf16_kv(backend, head_major):
    case = cfg2(head_major=head_major)
    got = run_decode(backend, case)
    want = case.oracle()
    err = np.abs(got - want).max()
    assert err <= 1e-2, err          # north-star tolerance on attention outputs
    assert err <= 1e-4, err          # what f32 accumulation over exact bf16 values gives


@pytest.mark.parametrize("which", ["cfg2", "few_long_rows"])
def test_balanced_and_fixed_plans_agree(backend, monkeypatch, which):
    # The planner cuts each row into equal pieces that fit one round of wave
    # slots (the default) or into fixed power-of-two chunks
    # (ORION_DECODE_BALANCE=0).  Both must match the oracle; their split
    # boundaries differ, so they agree to f32 rounding, not bit for bit.
    # few_long_rows: rows of 16,384 and 12,000 tokens over 8 KV heads are cut
    # into more than 64 pieces per row (the merge's general path).
    case = cfg2() if which == "cfg2" else PagedCase(77, [16384, 12000], 32, 8, 128, 16,
                                                    dtype="bf16")
    want = case.oracle()
    outs, infos = {}, {}
    for bal in ("1", "0"):
        monkeypatch.setenv("ORION_DECODE_BALANCE", bal)
        plan = oh.DecodePlan(backend, case.positions, case.row_seq, case.bt_offsets,
                             case.bt_ids, case.hq, case.hkv, case.d, case.bs)
        infos[bal] = plan.info()
        plan.close()
        outs[bal] = run_decode(backend, case)
        err = float(np.abs(outs[bal] - want).max())
        print(f"[plans] {which} balance={bal} {infos[bal]} err {err:.2e}", flush=True)
        assert err <= 1e-4, (bal, err)
    assert np.abs(outs["1"] - outs["0"]).max() <= 2e-5
    if which == "cfg2":
        assert infos["1"]["num_work"] <= 2048 < infos["0"]["num_work"]
    else:
        assert infos["1"]["max_splits"] > 64


@pytest.mark.parametrize("hq,hkv,d,bs,dtype", [
    (8, 8, 64, 16, "f32"), (16, 8, 128, 16, "bf16"), (12, 4, 128, 8, "bf16"),
    (28, 4, 128, 16, "bf16"), (32, 4, 64, 16, "bf16"), (20, 4, 64, 32, "f32"),
    (10, 2, 128, 4, "f32"), (6, 1, 64, 256, "bf16"), (64, 8, 128, 64, "bf16"),
])
@pytest.mark.parametrize("head_major", [False, True])
def test_shapes_groups_and_block_sizes(backend, hq, hkv, d, bs, dtype, head_major):
    ctxs = [1, 2, 15, 16, 17, 63, 64, 65, 255, 256, 257, 511, 512, 513, 1000, 2049]
    case = PagedCase(hq * 1000 + d + bs, ctxs, hq, hkv, d, bs, dtype=dtype, head_major=head_major)
    got = run_decode(backend, case)
    want = case.oracle()
    tol = orc.Tolerance.F32 if dtype == "f32" else orc.Tolerance(1e-4, 1e-4)
    mm, ma, mr, wi = orc.validate(want, got, tol)
    assert mm == 0, (ma, mr, wi)


@pytest.mark.parametrize("hq,hkv,d,bs,dtype", [
    # head_dim other than 64/128 (the reference accepts any even head_dim,
    # attention.rs:244-249) and groups above 8 (any divisible grouping):
    # the general decode wave and merge
    (8, 1, 80, 16, "bf16"), (16, 1, 96, 16, "f32"), (32, 2, 256, 16, "bf16"),
    (32, 1, 64, 16, "bf16"), (24, 2, 128, 8, "f32"), (4, 2, 2, 16, "f32"),
    (6, 3, 160, 32, "bf16"), (12, 1, 48, 4, "bf16"),
    # head_dim above 256, up to the kernels' 2048: 2, 4, 8 and 16
    # 128-dimension chunks per lane (and a partial last chunk)
    (4, 2, 258, 16, "f32"), (8, 2, 512, 16, "bf16"), (4, 1, 1000, 16, "bf16"),
    (2, 1, 2048, 16, "f32"), (6, 2, 1538, 8, "bf16"),
    # groups of 9 to 16 on bf16 arenas at head_dim 64/128: the MFMA wave
    (16, 1, 128, 16, "bf16"), (24, 2, 128, 16, "bf16"), (18, 2, 64, 16, "bf16"),
    (64, 4, 64, 16, "bf16"), (20, 2, 128, 8, "bf16"),
])
def test_any_head_dim_and_group(backend, hq, hkv, d, bs, dtype):
    ctxs = [1, 2, 17, 64, 65, 300, 513, 1000, 2049]
    case = PagedCase(hq * 100 + d + bs, ctxs, hq, hkv, d, bs, dtype=dtype)
    got = run_decode(backend, case)
    want = case.oracle()
    tol = orc.Tolerance.F32 if dtype == "f32" else orc.Tolerance(1e-4, 1e-4)
    mm, ma, mr, wi = orc.validate(want, got, tol)
    assert mm == 0, (ma, mr, wi)


def shared_prefix_case(seed, hq, hkv, d, bs, head_major=False):
    # 40 rows: rows 0-19 share 1,024 tokens; rows 20-26 share 320; rows
    # 30-35 share 640 with row 30 except row 33, which shares 288 (a pack's
    # prefix is what all its rows share); rows 36-39 share 2 blocks (too
    # short to pack); the rest are private.
    rng = np.random.default_rng(seed)
    ctxs = rng.integers(1100, 3000, 40)
    case = PagedCase(seed, ctxs, hq, hkv, d, bs, dtype="bf16", head_major=head_major)
    tok = lambda n: -(-n // bs)
    return case.share_prefixes([(list(range(20)), tok(1024)), (list(range(20, 27)), tok(320)),
                                ([30, 31, 32, 34, 35], tok(640)), ([30, 33], tok(288)),
                                ([36, 37, 38, 39], 2)])


@pytest.mark.parametrize("hq,hkv,d,bs,hm", [(28, 4, 128, 16, False), (32, 8, 128, 16, False),
                                            (8, 8, 64, 16, False), (16, 4, 64, 16, False),
                                            (16, 2, 128, 32, False), (12, 4, 64, 8, False),
                                            (28, 4, 128, 16, True)])
def test_packed_shared_prefixes(backend, monkeypatch, hq, hkv, d, bs, hm):
    # Rows whose tables start with the same block ids attend that prefix
    # together: up to 16 / G rows' query heads fill one MFMA wave's query
    # columns, and the prefix pieces are splits of every row of the pack.
    # Against the oracle, and against the same plan without packing
    # (ORION_DECODE_PACK=0), which plans no packed item.
    case = shared_prefix_case(hq + d + bs, hq, hkv, d, bs, head_major=hm)
    args = (case.positions, case.row_seq, case.bt_offsets, case.bt_ids, hq, hkv, d, bs)
    items = oh.DecodePlan(backend, *args)
    info = items.info()
    items.close()
    got = run_decode(backend, case)
    monkeypatch.setenv("ORION_DECODE_PACK", "0")
    items = oh.DecodePlan(backend, *args)
    info_plain = items.info()
    items.close()
    plain = run_decode(backend, case)
    monkeypatch.delenv("ORION_DECODE_PACK")
    want = case.oracle()
    err, diff = float(np.abs(got - want).max()), float(np.abs(got - plain).max())
    print(f"[packed prefixes] G={hq // hkv} {info['packed_items']} packed items of "
          f"{info['num_work']} ({info['rows_per_pack']} rows each), unpacked plan "
          f"{info_plain['num_work']} items; err {err:.2e}, vs unpacked {diff:.2e}", flush=True)
    assert info["packed_items"] > 0 and info["rows_per_pack"] == 16 // (hq // hkv)
    assert info_plain["packed_items"] == 0
    assert err <= 1e-4 and float(np.abs(plain - want).max()) <= 1e-4
    assert diff <= 2e-5


def test_packed_plan_on_an_f32_arena_takes_the_unpacked_copy(backend):
    # The plan is built before the arena's dtype is known; an f32 arena (VALU
    # waves, no packed items) runs the unpacked copy of the same plan.
    case = shared_prefix_case(3, 28, 4, 128, 16)
    case.dtype = "f32"
    got = run_decode(backend, case)
    assert float(np.abs(got - case.oracle()).max()) <= 1e-4


def test_ragged_positions_and_shared_sequences(backend):
    # Several query rows per sequence at arbitrary positions (what a chunked
    # prefill batch looks like to the decode kernel) and sequences sharing
    # leading blocks (prefix sharing, non-disjoint tables).
    case = PagedCase(11, [300, 1200, 40], 16, 4, 128, 16, dtype="bf16", disjoint=False,
                     num_blocks=40)
    rng = np.random.default_rng(5)
    row_seq = np.array([0, 0, 0, 1, 1, 2, 1, 0], np.int32)
    positions = np.array([0, 299, 150, 1199, 17, 39, 640, 31], np.uint32)
    q = rng.standard_normal((len(row_seq), case.hq * case.d), dtype=np.float32)
    got = run_decode(backend, case, positions, row_seq, q)
    want = case.oracle(positions, row_seq, q)
    assert np.abs(got - want).max() <= 1e-4


def test_consecutive_calls_of_different_sizes(backend):
    # Split-K partials live in per-device scratch reused by every call: calls
    # with many rows, then few, then many again (and one plan replayed) must
    # each match the oracle, and replays must repeat the same bits.
    ctxs = [3000, 70, 1500, 900, 2048, 5, 700, 1300] * 4
    big = PagedCase(41, ctxs, 32, 8, 128, 16, dtype="bf16")
    small = PagedCase(42, [4000, 33], 32, 8, 128, 16, dtype="bf16")
    outs = []
    for case in (big, small, big, big):
        got = run_decode(backend, case)
        assert np.abs(got - case.oracle()).max() <= 1e-4
        outs.append(got)
    assert np.array_equal(outs[0], outs[2]) and np.array_equal(outs[2], outs[3])


def test_single_position_returns_value_exactly(backend):
    # attention.rs:375-403 at a supported head_dim: one position -> softmax 1.0 -> V.
    case = PagedCase(3, [1, 1, 1], 8, 2, 64, 16, dtype="f32")
    got = run_decode(backend, case)
    for s in range(3):
        b = int(case.tables[s][0])
        for h in range(8):
            off = (b * 2 + 1) * 16 * 2 * 64 + (h // 4) * 64
            v = case.arena_f32[off:off + 64]
            assert np.array_equal(got[s, h * 64:(h + 1) * 64], v)


def test_uniform_keys_give_the_mean_of_values(backend):
    # attention.rs:479-510: identical keys -> uniform weights -> mean of V.
    case = PagedCase(9, [777], 4, 1, 128, 16, dtype="f32")
    a = case.arena_f32.reshape(case.num_blocks, 2, 16, 1, 128)
    a[:, 0] = 0.25
    got = run_decode(backend, case)
    vals = np.stack([a[case.tables[0][p // 16], 1, p % 16, 0] for p in range(777)])
    np.testing.assert_allclose(got.reshape(4, 128), np.broadcast_to(vals.mean(0), (4, 128)),
                               rtol=1e-5, atol=1e-6)


def test_golden_cfg1_fixture(backend):
    # Committed golden output of the oracle on config 1 (tests/golden/).
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1_decode.npz"))
    case = cfg1()
    assert np.array_equal(case.ctxs, g["ctxs"])
    got = run_decode(backend, case)
    mm, ma, mr, wi = orc.validate(g["out"], got, orc.Tolerance.F32)
    assert mm == 0, (ma, mr, wi)


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_packed_random_sharing_patterns(backend, seed):
    # Random batches of rows sharing prefixes of random depths (several
    # groups, nested depths, rows whose context barely passes the prefix),
    # random grouping and head_dim 64/128 on bf16 arenas, against the oracle.
    rng = np.random.default_rng(1000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 3, 4, 5, 7, 8]))
    d = int(rng.choice([64, 128]))
    bs = int(rng.choice([8, 16, 32]))
    rows = int(rng.integers(8, 48))
    ctxs = rng.integers(300, 2600, rows)
    case = PagedCase(2000 + seed, ctxs, G * hkv, hkv, d, bs, dtype="bf16")
    groups, r = [], 0
    while r < rows - 1:
        n = int(rng.integers(2, 9))
        members = list(range(r, min(rows, r + n)))
        depth = int(min(ctxs[m] for m in members) // bs)
        nb = int(rng.integers(1, depth + 1))
        groups.append((members, nb))
        r += n + int(rng.integers(0, 3))
    case.share_prefixes(groups)
    plan = oh.DecodePlan(backend, case.positions, case.row_seq, case.bt_offsets, case.bt_ids,
                         case.hq, hkv, d, bs)
    info = plan.info()
    plan.close()
    got = run_decode(backend, case)
    err = float(np.abs(got - case.oracle()).max())
    print(f"[packed random] seed={seed} G={G} hkv={hkv} d={d} bs={bs} rows={rows} "
          f"packed items {info['packed_items']} of {info['num_work']}, err {err:.2e}", flush=True)
    assert err <= 1e-4
