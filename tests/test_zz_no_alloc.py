"""orion_hip_gemm_noalloc (the GEMM entry point that allocates nothing)
against orion_hip_gemm, through the C-ABI: identical kernels, so the outputs
must be bit-identical.  Calls run back to back on one device, each later one
smaller than the one before, so a call that read partial tiles left by the
previous (larger) call would show.  A shape whose split-K partials exceed the
fixed device array is refused with a Backend error before any launch; a
long-K shape whose optional extra K splits do not fit runs with fewer splits
(the same kernels, f32 sums in another order)."""
import ctypes as C

import numpy as np
import pytest

import orion_hip as oh
from model_fixtures import bf16_round

pytestmark = pytest.mark.gpu


def run_both(be, M, N, K, ep, bias, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = bf16_round(rng.standard_normal((N, K), dtype=np.float32) * 0.05)
    b = rng.standard_normal(N, dtype=np.float32) if bias else None
    n_out = N // 2 if ep == oh.GEMM_SWIGLU else N
    init = rng.standard_normal((M, n_out), dtype=np.float32)
    dx, dw = be.to_device(x), be.to_device(oh.f32_to_bf16_bits(w))
    db = be.to_device(b) if bias else None
    d1, d2 = be.to_device(init), be.to_device(init)
    print(f"[gemm_noalloc] M={M} N={N} K={K} ep={ep} bias={bias}", flush=True)
    bp = db.ptr if db else None
    oh._check(be.lib.orion_hip_gemm(be.handle, dx.ptr, dw.ptr, bp, M, N, K, ep, d1.ptr))
    oh._check(be.lib.orion_hip_gemm_noalloc(be.handle, dx.ptr, dw.ptr, bp, M, N, K, ep, d2.ptr))
    a = d1.download(np.float32, (M, n_out))
    c = d2.download(np.float32, (M, n_out))
    for buf in (dx, dw, db, d1, d2):
        if buf:
            buf.free()
    return a, c


# Larger first, then smaller: LM-head-sized partials (32 MB), a tiled shape
# with few output tiles (its K split 8 ways, sums in the array), then QKV with
# bias, a down projection (22 K slices), SwiGLU, a residual accumulate, a
# single-slice shape and one row; a skinny (M = 100) and a tiled (M = 300)
# shape, which use no partials.
SEQUENCE = [(32, 32000, 2048, oh.GEMM_STORE, False), (400, 256, 4096, oh.GEMM_STORE, True),
            (8, 2560, 2048, oh.GEMM_STORE, True),
            (64, 2048, 5632, oh.GEMM_ACCUMULATE, False), (32, 11264, 2048, oh.GEMM_SWIGLU, False),
            (17, 2048, 2048, oh.GEMM_ACCUMULATE, False), (5, 96, 256, oh.GEMM_STORE, True),
            (1, 512, 1024, oh.GEMM_STORE, False), (100, 1024, 512, oh.GEMM_STORE, False),
            (300, 384, 256, oh.GEMM_ACCUMULATE, False)]


def test_noalloc_gemm_matches_gemm_on_consecutive_calls(backend):
    for i, (M, N, K, ep, bias) in enumerate(SEQUENCE):
        a, c = run_both(backend, M, N, K, ep, bias, seed=100 + i)
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32)), (M, N, K, ep)


def test_noalloc_gemm_twice_in_a_row_smaller_second(backend):
    for (M, N, K) in [(48, 16384, 4096), (3, 640, 2048)]:
        a, c = run_both(backend, M, N, K, oh.GEMM_STORE, False, seed=M)
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32)), (M, N, K)


def test_noalloc_gemm_runs_long_k_without_its_optional_splits(backend):
    # config 5's down projection: 3 preferred K splits need 96 MB of sums, more
    # than the 64 MiB array, so the no-allocation call runs it unsplit.
    M, N, K = 2240, 3584, 18944
    a, c = run_both(backend, M, N, K, oh.GEMM_ACCUMULATE, False, seed=5)
    scale = float(np.abs(a).max())
    assert np.isfinite(c).all()
    assert float(np.abs(a - c).max()) <= 2e-5 * scale + 1e-6


def test_noalloc_gemm_refuses_shapes_beyond_its_scratch(backend):
    # 64 rows x 200,000 columns over K = 4096 needs ~800 MB of partials
    with pytest.raises(oh.BackendError, match="no-allocation entry point holds"):
        oh._check(backend.lib.orion_hip_gemm_noalloc(backend.handle, C.c_void_p(16),
                                                     C.c_void_p(16), None, 64, 200000, 4096,
                                                     oh.GEMM_STORE, C.c_void_p(16)))


def test_noalloc_gemm_ordered_across_device_handles(backend):
    # Two handles on GPU 0 each have their own stream, and both use the GPU's
    # one scratch array.  Calls alternate between the handles with no host
    # synchronisation between them; each must still be bit-identical to
    # orion_hip_gemm (the library orders them with a per-GPU event).
    be2 = oh.HipBackend(backend.ordinal)
    cases = []
    try:
        shapes = [(32, 32000, 2048, oh.GEMM_STORE), (48, 11264, 2048, oh.GEMM_SWIGLU),
                  (64, 2048, 5632, oh.GEMM_STORE), (8, 2560, 2048, oh.GEMM_STORE)]
        rng = np.random.default_rng(77)
        for (M, N, K, ep) in shapes:
            x = rng.standard_normal((M, K), dtype=np.float32)
            w = bf16_round(rng.standard_normal((N, K), dtype=np.float32) * 0.05)
            n_out = N // 2 if ep == oh.GEMM_SWIGLU else N
            dx, dw = backend.to_device(x), backend.to_device(oh.f32_to_bf16_bits(w))
            ref = backend.alloc(M * n_out * 4)
            oh._check(backend.lib.orion_hip_gemm(backend.handle, dx.ptr, dw.ptr, None, M, N, K,
                                                 ep, ref.ptr))
            outs = [backend.alloc(M * n_out * 4) for _ in range(2)]
            cases.append((M, N, K, ep, n_out, dx, dw, ref, outs))
        backend.synchronize()
        print("[gemm_noalloc] two handles, alternating calls", flush=True)
        for rnd in range(2):
            for i, (M, N, K, ep, n_out, dx, dw, ref, outs) in enumerate(cases):
                be = backend if (i + rnd) % 2 == 0 else be2
                oh._check(be.lib.orion_hip_gemm_noalloc(be.handle, dx.ptr, dw.ptr, None, M, N, K,
                                                        ep, outs[rnd].ptr))
        backend.synchronize()
        be2.synchronize()
        for (M, N, K, ep, n_out, dx, dw, ref, outs) in cases:
            want = ref.download(np.float32, (M, n_out))
            for o in outs:
                got = o.download(np.float32, (M, n_out))
                assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), (M, N, K, ep)
    finally:
        be2.close()
        for (M, N, K, ep, n_out, dx, dw, ref, outs) in cases:
            for b in (dx, dw, ref, *outs):
                b.free()
