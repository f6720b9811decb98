"""Chunked-prefill attention (MFMA) on the MI355X against the CPU oracle's
paged_attention (crates/orion-models/src/attention.rs:219-295), and against
the decode kernel on the same rows."""
import numpy as np
import pytest

import oracle as orc
import orion_hip as oh
from paged_cases import PrefillCase, cfg3
from test_gpu_attention import run_decode

pytestmark = pytest.mark.gpu


def run_prefill(be, case, hilo):
    n = len(case.positions)
    kv = case.kv_layout()
    bufs = [be.to_device(case.arena_device_bytes()), be.to_device(case.q),
            be.to_device(case.row_start), be.to_device(case.row_count),
            be.to_device(case.first_pos), be.to_device(case.bt_offsets),
            be.to_device(case.bt_ids), be.alloc(max(n, 1) * case.hq * case.d * 4)]
    arena, dq, drs, drc, dfp, dbo, dbi, dout = bufs
    max_rows = int(case.row_count.max()) if case.S else 0
    max_pos = int(case.positions.max()) if n else 0
    print(f"[prefill] seqs={case.S} rows={n} hq={case.hq} hkv={case.hkv} d={case.d} "
          f"bs={case.bs} hilo={hilo} max_rows={max_rows} max_pos={max_pos}", flush=True)
    try:
        oh.paged_attention_prefill(be, kv, arena.ptr, 0, dq.ptr, case.hq, case.S, drs.ptr,
                                   drc.ptr, dfp.ptr, dbo.ptr, dbi.ptr, max_rows, max_pos,
                                   dout.ptr, hilo=hilo)
        return dout.download(np.float32, (n, case.hq * case.d))
    finally:
        for b in bufs:
            b.free()


def sample_rows(case, per_seq, seed=0):
    """First, last and `per_seq` random rows of every sequence's chunk."""
    rng = np.random.default_rng(seed)
    rows = []
    for s in range(case.S):
        a, c = int(case.row_start[s]), int(case.row_count[s])
        if c == 0:
            continue
        pick = {a, a + c - 1} | set((a + rng.integers(0, c, size=min(per_seq, c))).tolist())
        rows += sorted(pick)
    return np.array(rows, np.int64)


@pytest.mark.parametrize("hilo,head_major", [(False, False), (True, False), (False, True)])
def test_cfg3_full_size_sampled_rows(backend, hilo, head_major):
    case = cfg3(head_major=head_major)
    got = run_prefill(backend, case, hilo)
    rows = sample_rows(case, 24)
    want = case.oracle_rows(rows)
    err = float(np.abs(got[rows] - want).max())
    print(f"cfg3 hilo={hilo} sampled rows={len(rows)} max_abs_err={err:.3g}", flush=True)
    assert err <= 1e-2, err                    # north-star tolerance on attention outputs
    if hilo:
        assert err <= 1e-4, err                # hi/lo operands: f32-class products
    assert np.isfinite(got).all()


@pytest.mark.parametrize("hq,hkv,d,bs", [
    (32, 8, 128, 16), (28, 4, 128, 16), (32, 4, 64, 16), (8, 2, 64, 16), (8, 8, 64, 8),
    (12, 4, 128, 32), (6, 1, 64, 1), (16, 16, 128, 64),
    # groups above 8 (Llama-3.1-405B has 16 query heads per KV head; MQA)
    (32, 2, 128, 16), (12, 1, 128, 16), (32, 1, 64, 16),
    # head_dim 256 (one 16-row tile per wave, a 2-stage ring)
    (8, 2, 256, 16), (16, 1, 256, 16), (4, 4, 256, 32),
])
@pytest.mark.parametrize("hilo", [False, True])
@pytest.mark.parametrize("head_major", [False, True])
def test_shapes_against_oracle(backend, hq, hkv, d, bs, hilo, head_major):
    # Prefixes 0 / inside a block / block- and tile-aligned; chunks of 1, 2,
    # a ragged tile and several tiles.
    prefixes = [0, 0, 5, 16, 63, 64, 200, 1000]
    chunks = [1, 2, 33, 64, 129, 17, 300, 70]
    case = PrefillCase(hq * 100 + d + bs, prefixes, chunks, hq, hkv, d, bs,
                       head_major=head_major)
    got = run_prefill(backend, case, hilo)
    want = case.oracle()
    tol = orc.Tolerance(1e-4, 1e-4) if hilo else orc.Tolerance(1e-2, 1e-2)
    mm, ma, mr, wi = orc.validate(want, got, tol)
    assert mm == 0, (ma, mr, wi)
    assert float(np.abs(got - want).max()) <= (1e-4 if hilo else 1e-2)


# (prefixes, chunks, hq, hkv, d): the first is config 5's imbalance (one chunk
# on a 9,000-token prefix beside short ones: parts, but no empty part and no
# part boundary inside a row tile); the second is cut by the planner (256 CUs)
# into 27 parts with 3 empty parts and a part whose first key lies inside the
# positions of one 16-row MFMA tile of queries (some attend no key of the
# part, others do).  tests/test_prefill_plan.py asserts those plan shapes on
# the CPU, so this test cannot silently stop covering them.
KEY_PART_CASES = [
    ([9000, 400, 60, 0], [256, 256, 100, 1500], 28, 4, 128),
    ([0, 0, 0, 26474], [2575, 414, 1096, 343], 2, 1, 128),
    ([0, 12000, 300], [700, 200, 500], 8, 2, 256),  # head_dim 256 with parts
]


@pytest.mark.parametrize("which", [0, 1, 2])
@pytest.mark.parametrize("hilo", [False, True])
def test_key_parts_for_long_prefixes(backend, monkeypatch, hilo, which):
    # Sequences whose tiles read far more keys than an even share of the CUs
    # are cut into key parts (partial results merged afterwards).  Against the
    # oracle on sampled rows (every row of the split sequences' chunks in the
    # second case) and against ORION_PREFILL_SPLIT=0 (whole sequences); every
    # output finite.
    prefixes, chunks, hq, hkv, d = KEY_PART_CASES[which]
    case = PrefillCase(31 + which, prefixes, chunks, hq, hkv, d, 16)
    rows = sample_rows(case, 24, seed=3)
    if which == 1:
        a = int(case.row_start[3])
        rows = np.union1d(rows, np.arange(a, a + int(case.row_count[3])))
    want = case.oracle_rows(rows)
    got = run_prefill(backend, case, hilo)
    monkeypatch.setenv("ORION_PREFILL_SPLIT", "0")
    whole = run_prefill(backend, case, hilo)
    monkeypatch.delenv("ORION_PREFILL_SPLIT")
    tol = 1e-4 if hilo else 1e-2
    err = float(np.abs(got[rows] - want).max())
    print(f"[prefill parts] hilo={hilo} err {err:.2e} "
          f"vs whole {float(np.abs(got - whole).max()):.2e}", flush=True)
    assert err <= tol
    assert float(np.abs(whole[rows] - want).max()) <= tol
    assert float(np.abs(got - whole).max()) <= (2e-5 if hilo else 2e-3)
    assert np.isfinite(got).all()


def test_matches_decode_kernel_on_same_rows(backend):
    # The two kernels restate the same per-row computation; with hi/lo
    # operands they agree to f32-class rounding.
    case = PrefillCase(77, [0, 900, 3000], [150, 64, 257], 32, 8, 128, 16)
    got = run_prefill(backend, case, True)
    dec = run_decode(backend, case)
    assert float(np.abs(got - dec).max()) <= 5e-5


def test_single_row_and_uniform_keys(backend):
    # Closed forms: a row at position 0 returns V[0] exactly (one weight of 1);
    # identical keys give the mean of the attended V rows.
    case = PrefillCase(5, [0], [40], 8, 2, 64, 16)
    kvd = case.hkv * case.d
    a = case.arena_f32.reshape(case.num_blocks, 2, case.bs, kvd)
    tbl = case.tables[0]
    a[tbl, 0] = a[tbl[0], 0, 0]                      # every key identical
    got = run_prefill(backend, case, False)
    v = a[:, 1][tbl].reshape(-1, case.hkv, case.d)   # V rows in position order
    for r in range(40):
        for h in range(case.hq):
            want = v[:r + 1, h // (case.hq // case.hkv)].mean(axis=0)
            np.testing.assert_allclose(got[r, h * case.d:(h + 1) * case.d], want,
                                       rtol=0, atol=2e-6 * (r + 1))


def test_empty_and_zero_row_sequences(backend):
    case = PrefillCase(9, [10, 0, 50], [0, 3, 0], 8, 2, 64, 16)
    got = run_prefill(backend, case, False)
    want = case.oracle()
    assert float(np.abs(got - want).max()) <= 1e-2


def test_f32_arena_is_a_backend_error(backend):
    case = PrefillCase(3, [4], [8], 8, 2, 64, 16, dtype="f32")
    with pytest.raises(oh.BackendError):
        run_prefill(backend, case, False)


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 80), (4, 2, 192), (8, 1, 96)])
def test_uncovered_prefill_shapes_are_backend_errors(backend, hq, hkv, d):
    # The MFMA prefill kernel covers head_dim 64/128/256 with any grouping; the
    # model forward sends other shapes' rows to the decode kernel (which
    # covers every even head_dim up to 2048 and any group), and the op-level
    # entry point refuses them with a Backend error before any launch.
    case = PrefillCase(4, [20], [8], hq, hkv, d, 16)
    with pytest.raises(oh.BackendError):
        run_prefill(backend, case, False)


@pytest.mark.parametrize("mode", [2, 3])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (32, 4, 64), (28, 4, 128)])
def test_single_operand_hilo_modes(backend, mode, hq, hkv, d):
    # Mode 2 carries Q as a hi/lo pair and rounds the softmax weights P to
    # bf16; mode 3 the reverse.  Each sits between the bf16 and the hi/lo
    # modes: within the north-star 1e-2 of the oracle, and its error is
    # printed beside the two full modes' for the record.
    case = PrefillCase(500 + mode + d, [0, 37, 700, 3000], [64, 200, 129, 300], hq, hkv, d, 16)
    want = case.oracle()
    errs = {m: float(np.abs(run_prefill(backend, case, m) - want).max()) for m in (0, mode, 1)}
    print(f"[prefill operands] hq={hq} hkv={hkv} d={d} max abs err bf16 {errs[0]:.2e} "
          f"mode{mode} {errs[mode]:.2e} hilo {errs[1]:.2e}", flush=True)
    assert errs[mode] <= 1e-2
    assert errs[1] <= 1e-4


def test_split_output_layout_is_the_split_of_the_f32_output(backend):
    # Operand mode + 16 writes each finished row as the O GEMM's pre-split
    # operand: per 8 dims, 8 hi bf16 (the f32 value's top 16 bits) then 8 lo
    # bf16 (the top 16 bits of value - hi).  It must be exactly the split of
    # the f32 output the same launch writes without it.
    case = PrefillCase(61, [0, 37, 300], [100, 64, 129], 32, 8, 128, 16)
    f32 = run_prefill(backend, case, 1)
    raw = run_prefill(backend, case, 1 | 16).view(np.uint32).reshape(f32.shape[0], -1, 8)
    u16 = raw.view(np.uint16).reshape(f32.shape[0], -1, 16)
    bits = f32.view(np.uint32).reshape(f32.shape[0], -1, 8)
    hi = (bits >> 16).astype(np.uint16)
    rem = f32.reshape(bits.shape) - (bits & np.uint32(0xFFFF0000)).view(np.float32)
    lo = (rem.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(u16[..., :8], hi)
    assert np.array_equal(u16[..., 8:], lo)


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5, 6])
def test_random_prefill_batches(backend, seed):
    # Random batches: 1-6 sequences with prefixes 0-6000 and chunks 1-700,
    # random grouping, head_dim 64/128/256 and block size, both operand
    # precisions; every output row against the oracle on sampled rows, and
    # everything finite.
    rng = np.random.default_rng(3000 + seed)
    S = int(rng.integers(1, 7))
    hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 4, 7, 8, 12, 16]))
    d = int(rng.choice([64, 128, 256]))
    bs = int(rng.choice([8, 16, 32]))
    prefixes = [int(rng.integers(0, 6000)) if rng.random() < 0.7 else 0 for _ in range(S)]
    chunks = [int(rng.integers(1, 700)) for _ in range(S)]
    case = PrefillCase(4000 + seed, prefixes, chunks, G * hkv, hkv, d, bs)
    rows = sample_rows(case, 12, seed=seed)
    want = case.oracle_rows(rows)
    for hilo, tol in ((True, 1e-4), (False, 1e-2)):
        got = run_prefill(backend, case, hilo)
        err = float(np.abs(got[rows] - want).max())
        print(f"[prefill random] seed={seed} S={S} G={G} hkv={hkv} d={d} bs={bs} hilo={hilo} "
              f"rows={len(rows)} err {err:.2e}", flush=True)
        assert np.isfinite(got).all()
        assert err <= tol
