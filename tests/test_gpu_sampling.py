"""Device-side DefaultSampler (runtime/src/sampling.rs:266-293) on the MI355X:
the reference's own sampling tests (sampling.rs:296-552) run through the
device, and rows at vocabulary scale against the CPU oracle's restatement
with the same uniform draws."""
import numpy as np
import pytest

import oracle as orc
import orion_hip as oh

pytestmark = pytest.mark.gpu
MASKED = -1.0e30


def run(be, rows, params, previous=None, uniforms=None):
    """Samples every row of `rows` (a list of equal-length logit lists) on the
    device; returns (tokens, filtered logits)."""
    x = np.ascontiguousarray(rows, dtype=np.float32)
    n, V = x.shape
    previous = previous or [[] for _ in range(n)]
    uniforms = uniforms if uniforms is not None else [0.5] * n
    if isinstance(params, oh.SamplingParams):
        params = [params] * n
    d = be.to_device(x)
    try:
        t = oh.sample(be, d.ptr, n, V, params, previous, uniforms)
        return t, d.download(np.float32, x.shape)
    finally:
        d.free()


def kept(x):
    return [i for i, v in enumerate(x) if v > MASKED]


def nucleus_probs(row, p, previous):
    """Float64 probabilities the top-p filter ranks (sampling.rs:108-144), and
    how many candidates it ranks."""
    x = np.asarray(row, np.float64).copy()
    for t in set(previous):
        if t < len(x):
            x[t] = x[t] / p.repetition_penalty if x[t] > 0 else x[t] * p.repetition_penalty
    x /= p.temperature
    live = np.ones(len(x), bool)
    if 0 < p.top_k < len(x):
        live = x >= np.sort(x)[::-1][p.top_k - 1]
    e = np.where(live, np.exp(x - x[live].max()), 0.0)
    return e / e.sum(), int(live.sum())


def test_reference_sampler_cases(backend):
    be = backend
    # greedy is deterministic, ties go low (sampling.rs:300-318)
    t, _ = run(be, [[0.1, 0.9, 0.3, 0.2]] * 4, oh.SamplingParams(temperature=0.0),
               uniforms=[0.0, 0.3, 0.6, 0.99])
    assert t == [1, 1, 1, 1]
    assert run(be, [[5.0, 5.0, 1.0]], oh.SamplingParams(temperature=0.0))[0] == [0]
    # top-k keeps exactly k (sampling.rs:371-382), disabled at 0 or >= len (:384-392)
    _, x = run(be, [[1.0, 5.0, 3.0, 2.0, 4.0]], oh.SamplingParams(top_k=2))
    assert kept(x[0]) == [1, 4]
    for k in (0, 3, 100):
        _, x = run(be, [[1.0, 5.0, 3.0]], oh.SamplingParams(top_k=k))
        assert x[0].tolist() == [1.0, 5.0, 3.0]
    # top-k never masks everything (:394-402)
    _, x = run(be, [[2.0] * 4], oh.SamplingParams(top_k=1))
    assert kept(x[0])
    # top-p nucleus (:404-413), no-op at 1 (:415-421), never empty (:423-433)
    _, x = run(be, [[5.0, 3.0, 0.0, -1.0]], oh.SamplingParams(top_p=0.9))
    assert x[0][0] > MASKED and x[0][2] <= MASKED and x[0][3] <= MASKED
    _, x = run(be, [[1.0, 2.0, 3.0]], oh.SamplingParams(top_p=1.0))
    assert x[0].tolist() == [1.0, 2.0, 3.0]
    _, x = run(be, [[1.0] * 4], oh.SamplingParams(top_p=0.01))
    assert len(kept(x[0])) == 1
    # repetition penalty: sign-aware (:435-444), once per distinct token (:446-451),
    # a no-op at 1, out-of-range ignored (:453-465)
    _, x = run(be, [[2.0, -2.0, 1.0]], oh.SamplingParams(temperature=0.0, repetition_penalty=2.0),
               previous=[[0, 1]])
    assert x[0].tolist() == [1.0, -4.0, 1.0]
    _, x = run(be, [[4.0, 1.0]], oh.SamplingParams(temperature=0.0, repetition_penalty=2.0),
               previous=[[0, 0, 0, 0]])
    assert x[0][0] == 2.0
    _, x = run(be, [[1.0, 2.0]], oh.SamplingParams(temperature=0.0, repetition_penalty=2.0),
               previous=[[99]])
    assert x[0].tolist() == [1.0, 2.0]
    # top-k of one collapses to greedy (:510-523)
    t, _ = run(be, [[1.0, 9.0, 2.0]] * 50, oh.SamplingParams(top_k=1),
               uniforms=list(np.linspace(0, 0.999, 50)))
    assert set(t) == {1}


def test_sampling_reflects_the_distribution(backend):  # sampling.rs:525-551
    rng = np.random.default_rng(11)
    t, _ = run(backend, [[0.0, 4.0, 0.0]] * 3000, oh.SamplingParams(),
               uniforms=rng.random(3000, dtype=np.float32).tolist())
    counts = np.bincount(t, minlength=3)
    assert counts[1] > 2500 and counts[0] > 0 and counts[2] > 0


@pytest.mark.parametrize("V", [8, 1000, 32000, 151936])
def test_rows_match_the_oracle(backend, V):
    rng = np.random.default_rng(V)
    n = 24
    rows = (rng.standard_normal((n, V)) * rng.uniform(0.5, 3.0, (n, 1))).astype(np.float32)
    rows[0, :3] = rows[0].max() + 1.0  # ties at the top
    params, previous, uniforms = [], [], []
    for i in range(n):
        params.append(oh.SamplingParams(
            temperature=float(rng.choice([0.0, 0.7, 1.0, 1.5])),
            top_k=int(rng.choice([0, 1, 40, V // 2, V + 3])),
            top_p=float(rng.choice([1.0, 0.95, 0.6])),
            repetition_penalty=float(rng.choice([1.0, 1.2]))))
        previous.append(rng.integers(0, V + 10, int(rng.integers(0, 64))).tolist())
        uniforms.append(float(rng.random(dtype=np.float32)))
    print(f"[sample] V={V} rows={n}", flush=True)
    tokens, filtered = run(backend, rows, params, previous, uniforms)
    for i in range(n):
        p = params[i]
        want, wx, margin = orc.sample(rows[i], previous[i], p.temperature, p.top_k, p.top_p,
                                      p.repetition_penalty, uniforms[i])
        # the filters are value-based: identical masked sets and values, except
        # a top-p crossing that lies within f32 summation rounding of p
        got_k, want_k = kept(filtered[i]), kept(wx)
        if got_k != want_k:
            # Both are prefixes of the same descending order that differ only
            # by where a cumulative f32 sum crosses p: the tokens between the
            # two cutoffs must carry no more mass than the rounding of a
            # sum over n candidates (n * 2^-23).
            assert p.temperature != 0.0 and p.top_p < 1.0, i
            probs, n_live = nucleus_probs(rows[i], p, previous[i])
            diff = sorted(set(got_k) ^ set(want_k))
            mass = float(probs[diff].sum())
            print(f"row {i}: nucleus differs by {len(diff)} tokens, mass {mass:.2e} "
                  f"over {n_live} candidates", flush=True)
            assert mass <= n_live * 2.0 ** -23, (i, mass, n_live)
            smallest_kept = min(probs[list(set(got_k) & set(want_k))])
            assert probs[diff].max() <= smallest_kept, i
            continue
        np.testing.assert_array_equal(filtered[i][np.array(want_k, int)],
                                      wx[np.array(want_k, int)])
        # the draw: identical unless r lies within f32 rounding of a boundary
        if p.temperature == 0.0 or margin > 1e-5:
            assert tokens[i] == want, (i, tokens[i], want, margin)


def test_model_sample_uses_the_last_forward_logits(backend):
    from model_fixtures import random_weights
    from test_gpu_model import batch, gpu_model, small_spec

    rng = np.random.default_rng(5)
    spec = small_spec(False, True)
    m = gpu_model(backend, spec, random_weights(spec, rng, std=0.05), oh.BF16)
    try:
        lens = [9, 30, 17]
        tables = [[0], [1, 2], [3, 4]]
        toks = rng.integers(0, spec.V, sum(lens))
        pos = np.concatenate([np.arange(k) for k in lens])
        out = m.forward(batch(toks, pos, lens, tables))
        params = [oh.SamplingParams(temperature=0.0), oh.SamplingParams(top_k=20, top_p=0.9),
                  oh.SamplingParams(temperature=0.8, repetition_penalty=1.3)]
        previous = [toks[:9].tolist(), toks[9:39].tolist(), toks[39:].tolist()]
        uniforms = [0.25, 0.5, 0.75]
        got = m.sample(params, previous, uniforms)
        for i, p in enumerate(params):
            want, _, margin = orc.sample(out.logits[i], previous[i], p.temperature, p.top_k,
                                         p.top_p, p.repetition_penalty, uniforms[i])
            if p.temperature == 0.0 or margin > 1e-5:
                assert got[i] == want
    finally:
        m.close()


def test_invalid_parameters_are_internal_errors(backend):
    for bad in (oh.SamplingParams(temperature=-1.0), oh.SamplingParams(top_p=0.0),
                oh.SamplingParams(top_p=1.5), oh.SamplingParams(repetition_penalty=0.0),
                oh.SamplingParams(temperature=float("nan"))):
        with pytest.raises(oh.InternalError):
            run(backend, [[1.0, 2.0]], bad)
    with pytest.raises(oh.InternalError):
        run(backend, [[1.0, 2.0]], oh.SamplingParams(), uniforms=[1.0])
