"""Per-op parity on the MI355X against the CPU oracle: GEMM (linear), RMSNorm,
RoPE + slot-mapped KV write, SwiGLU, argmax (the validation gate of
docs/cuda.md:80-116 in the reference)."""
import numpy as np
import pytest

import oracle as orc
import orion_hip as oh
from model_fixtures import bf16_round

pytestmark = pytest.mark.gpu


def gemm_case(be, M, N, K, bias=False, accumulate=False, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = bf16_round(rng.standard_normal((N, K), dtype=np.float32) * 0.05)
    b = rng.standard_normal(N, dtype=np.float32) if bias else None
    init = rng.standard_normal((M, N), dtype=np.float32) if accumulate else np.zeros((M, N), np.float32)
    dx, dw = be.to_device(x), be.to_device(oh.f32_to_bf16_bits(w))
    db = be.to_device(b) if bias else None
    dout = be.to_device(init)
    print(f"[gemm] M={M} N={N} K={K} bias={bias} acc={accumulate}", flush=True)
    oh.gemm(be, dx.ptr, dw.ptr, db.ptr if db else None, M, N, K, accumulate, dout.ptr)
    got = dout.download(np.float32, (M, N))
    want = orc.linear(x, w, b) + (init if accumulate else 0)
    ref64 = x.astype(np.float64) @ w.T.astype(np.float64) + (0 if b is None else b) + (
        init if accumulate else 0)
    for buf in (dx, dw, db, dout):
        if buf:
            buf.free()
    return got, want, ref64


@pytest.mark.parametrize("M,N,K", [(1, 16, 32), (7, 40, 64), (32, 2560, 2048), (64, 512, 5632),
                                   (65, 96, 256), (130, 2048, 512), (32, 32000, 2048),
                                   # LDS-tiled (prefill) kernel: M >= 256, ragged M/N edges
                                   (256, 128, 32), (300, 96, 256), (1000, 2560, 2048),
                                   (777, 2048, 5632), (513, 32000, 2048),
                                   # wide (128 x 256) tiles with a ragged last column tile
                                   (300, 8200, 512)])
def test_gemm_matches_linear(backend, M, N, K):
    got, want, ref64 = gemm_case(backend, M, N, K, seed=M + N + K)
    scale = np.abs(ref64).max()
    # hi/lo split keeps x to ~2^-17 relative; the rest is summation order.
    assert np.abs(got - ref64).max() <= 2e-5 * scale + 1e-6
    assert np.abs(got - want).max() <= 2e-5 * scale + 1e-6


@pytest.mark.parametrize("M", [33, 400])
def test_gemm_bias_and_accumulate_epilogues(backend, M):
    got, want, ref64 = gemm_case(backend, M, 272, 384, bias=True, seed=1)
    assert np.abs(got - ref64).max() <= 1e-4
    got, want, ref64 = gemm_case(backend, M, 272, 384, accumulate=True, seed=2)
    assert np.abs(got - ref64).max() <= 1e-4


@pytest.mark.parametrize("M,N,K", [(400, 272, 2048), (1100, 1024, 3584), (200, 1024, 3584),
                                   (2048, 2048, 8192), (300, 8192, 4096)])
def test_tiled_gemm_k_splits(backend, monkeypatch, M, N, K):
    # LDS-tiled shapes with few output tiles split K (sums reduced in split
    # order by a second kernel): store with bias, and accumulate, against
    # float64 and against the unsplit kernel (ORION_GEMM_TILED_SPLIT=1).
    # 200 x 1024 x 3584 is config 5's LM head on the last rows; 2048 x 2048 x
    # 8192 (256 tiles, 256 k-steps) takes the long-K rule's 4 splits; 300 x
    # 8192 x 4096 splits K with the wide 128 x 256 tiles.
    for kw in (dict(bias=True), dict(accumulate=True)):
        got, want, ref64 = gemm_case(backend, M, N, K, seed=M + K, **kw)
        monkeypatch.setenv("ORION_GEMM_TILED_SPLIT", "1")
        one, _, _ = gemm_case(backend, M, N, K, seed=M + K, **kw)
        monkeypatch.delenv("ORION_GEMM_TILED_SPLIT")
        scale = np.abs(ref64).max()
        assert np.abs(got - ref64).max() <= 2e-5 * scale + 1e-6, kw
        assert np.abs(got - one).max() <= 2e-5 * scale + 1e-6, kw


@pytest.mark.parametrize("M,F,K", [(5, 48, 64), (32, 5632, 2048), (300, 176, 256), (600, 5632, 2048),
                                   (300, 4104, 256)])  # wide tiles, ragged last tile
def test_gemm_swiglu_epilogue(backend, M, F, K):
    # Gate and up rows interleaved in groups of 8 (the model's fused W_gu
    # layout); the epilogue returns swiglu(x.Wg^T, x.Wu^T) (tensor.rs:175-189).
    rng = np.random.default_rng(M + F)
    x = rng.standard_normal((M, K), dtype=np.float32)
    wg = bf16_round(rng.standard_normal((F, K), dtype=np.float32) * 0.05)
    wu = bf16_round(rng.standard_normal((F, K), dtype=np.float32) * 0.05)
    w = np.empty((2 * F, K), np.float32)
    for g in range(F // 8):
        w[16 * g:16 * g + 8] = wg[8 * g:8 * g + 8]
        w[16 * g + 8:16 * g + 16] = wu[8 * g:8 * g + 8]
    dx, dw = backend.to_device(x), backend.to_device(oh.f32_to_bf16_bits(w))
    dout = backend.alloc(M * F * 4)
    print(f"[gemm-swiglu] M={M} F={F} K={K}", flush=True)
    oh.gemm(backend, dx.ptr, dw.ptr, None, M, 2 * F, K, oh.GEMM_SWIGLU, dout.ptr)
    got = dout.download(np.float32, (M, F))
    g64 = x.astype(np.float64) @ wg.T.astype(np.float64)
    u64 = x.astype(np.float64) @ wu.T.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u64
    assert np.abs(got - want).max() <= 3e-5 * max(np.abs(want).max(), 1.0)
    for b in (dx, dw, dout):
        b.free()


@pytest.mark.parametrize("rows,cols", [(1, 64), (5, 2048), (33, 3584), (3, 100),
                                       # the scalar path: odd width, wider than 8192
                                       (3, 99), (2, 10000)])
def test_rmsnorm_matches_oracle(backend, rows, cols):
    rng = np.random.default_rng(rows * cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    w = rng.standard_normal(cols).astype(np.float32)
    dx, dw, do = backend.to_device(x), backend.to_device(w), backend.alloc(x.nbytes)
    oh.rmsnorm(backend, dx.ptr, dw.ptr, rows, cols, 1e-5, do.ptr)
    got = do.download(np.float32, x.shape)
    want = orc.rms_norm(x, w, 1e-5)
    # f64 sum of squares in a different order: the f32 scale may differ by 1 ulp.
    np.testing.assert_allclose(got, want, rtol=3e-7, atol=0)
    # all-zero row stays finite (tensor.rs:392-399)
    dz = backend.to_device(np.zeros((1, cols), np.float32))
    oh.rmsnorm(backend, dz.ptr, dw.ptr, 1, cols, 1e-5, do.ptr)
    assert np.all(do.download(np.float32, (1, cols)) == 0)


@pytest.mark.parametrize("dtype,head_major,shift,d", [
    ("f32", False, 0, 128), ("bf16", False, 0, 128), ("bf16", True, 0, 128),
    ("f32", False, 1, 128), ("bf16", False, 1, 128),
    # head_dim above 256: several elements per thread in the scalar kernel
    ("f32", False, 1, 1000), ("bf16", False, 1, 2048), ("bf16", False, 0, 512)])
def test_rope_and_cache_is_bit_exact(backend, dtype, head_major, shift, d):
    # RoPE + slot mapping + KV write against the oracle's apply_rope and
    # KvStore.write: the rotated Q, and every arena element, bit for bit.
    # shift 1 moves the q/k/v inputs off 16-byte alignment, which takes the
    # one-element-per-thread kernel instead of the vectorised one.
    rng = np.random.default_rng(17)
    L, nb, bs, hkv, hq = 2, 40, 16, 4, 16
    layer = 1
    n = 37
    S = 3
    counts = [20, 1, 16]
    row_seq = np.repeat(np.arange(S), counts).astype(np.int32)
    perm = rng.permutation(nb).astype(np.uint32)
    tables = [perm[8 * i:8 * i + 8] for i in range(S)]  # disjoint: no two rows share a slot
    offs = np.array([0, 8, 16, 24], np.int64)
    ids = np.concatenate(tables)
    positions = np.concatenate([np.arange(20) + 5, [100], np.arange(16) + 64]).astype(np.uint32)
    qkvd = (hq + 2 * hkv) * d
    qkv = rng.standard_normal((n, qkvd), dtype=np.float32)
    rope = orc.RopeTable(d, 256, 500000.0)
    kvl = oh.kv_layout(L, nb, bs, hkv, d, oh.BF16 if dtype == "bf16" else oh.F32, head_major)
    esz = 2 if dtype == "bf16" else 4
    arena_el = L * nb * 2 * bs * hkv * d
    darena = backend.alloc(arena_el * esz)
    oh._check(backend.lib.orion_hip_memset(backend.handle, darena.ptr, 0, arena_el * esz))
    dqkv_buf = backend.to_device(np.concatenate([np.zeros(shift, np.float32), qkv.ravel()]))
    dqo = backend.alloc(n * hq * d * 4)
    qkv_ptr = dqkv_buf.ptr + 4 * shift  # the q/k/v base, `shift` floats into the buffer
    bufs = [backend.to_device(a) for a in (positions, row_seq, offs, ids, rope.cos, rope.sin)]
    dpos, drs, dbo, dbi, dcos, dsin = bufs
    oh.rope_and_cache(backend, kvl, darena.ptr, layer, n, hq, qkv_ptr, qkvd, dqo.ptr,
                      qkv_ptr + hq * d * 4, qkvd, qkv_ptr + (hq + hkv) * d * 4, qkvd, dpos.ptr,
                      drs.ptr, dbo.ptr, dbi.ptr, dcos.ptr, dsin.ptr)
    q_got = dqo.download(np.float32, (n, hq * d))
    raw = darena.download(np.uint16 if dtype == "bf16" else np.float32, (arena_el,))
    arena_got = oh.bf16_bits_to_f32(raw) if dtype == "bf16" else raw
    if head_major:  # back to the reference block order [k|v][slot][kv_head][dim]
        arena_got = arena_got.reshape(L, nb, hkv, 2, bs, d).transpose(0, 1, 3, 4, 2, 5).reshape(-1)
    store = orc.KvStore(L, nb, bs, hkv, d)
    for r in range(n):
        c, s = rope.at(int(positions[r]))
        for h in range(hq):
            want = orc.apply_rope(qkv[r, h * d:(h + 1) * d], c, s)
            assert np.array_equal(q_got[r, h * d:(h + 1) * d], want)
        blk, slot = orc.locate(tables[row_seq[r]], int(positions[r]), bs)
        for h in range(hkv):
            k = orc.apply_rope(qkv[r, (hq + h) * d:(hq + h + 1) * d], c, s)
            v = qkv[r, (hq + hkv + h) * d:(hq + hkv + h + 1) * d]
            if dtype == "bf16":
                k, v = bf16_round(k), bf16_round(v)
            store.write(layer, blk, slot, h, False, k)
            store.write(layer, blk, slot, h, True, v)
    assert np.array_equal(arena_got, store.data)


def test_silu_mul_matches_swiglu(backend):
    rng = np.random.default_rng(3)
    g = (rng.standard_normal(10001) * 4).astype(np.float32)
    u = rng.standard_normal(10001).astype(np.float32)
    dg, du = backend.to_device(g), backend.to_device(u)
    oh.silu_mul(backend, dg.ptr, du.ptr, g.size)
    np.testing.assert_allclose(dg.download(np.float32, g.shape), orc.swiglu(g, u), rtol=2e-6,
                               atol=1e-7)


def test_argmax_semantics(backend):
    rows = np.array([
        [1.0, 3.0, 3.0, 2.0] + [0.0] * 1000,
        [np.nan, 0.5] + [0.1] * 1002,
        [-np.inf] * 1004,
        [0.0] * 1003 + [7.0],
    ], np.float32)
    rng = np.random.default_rng(0)
    big = rng.standard_normal((5, 32000)).astype(np.float32)
    big[2, 31999] = big[2, 17] = 100.0  # tie: lowest index wins
    big[3, 4 * 4096 + 1] = big[3, 4 * 1024 + 3] = 50.0    # tie across threads / unroll steps
    big[4, 8] = big[4, 9] = big[4, 10] = 60.0             # tie inside one float4
    odd = rng.standard_normal((3, 32003)).astype(np.float32)  # unaligned rows: scalar scan
    odd[1, 32002] = odd[1, 1025] = 9.0
    odd[2, :] = -np.inf
    odd[2, 31000] = np.nan
    for arr in (rows, big, odd):
        dl, do = backend.to_device(arr), backend.alloc(arr.shape[0] * 8)
        oh.argmax(backend, dl.ptr, arr.shape[0], arr.shape[1], do.ptr)
        got = do.download(np.int64, (arr.shape[0],))
        want = [orc.argmax(r) for r in arr]
        assert got.tolist() == [(-1 if w is None else w) for w in want]
