"""The oracle's DefaultSampler restatement (runtime/src/sampling.rs) against
the reference's own sampling tests (sampling.rs:296-552) and an independent
float64 numpy restatement of the filters and the draw."""
import numpy as np
import pytest

import oracle as orc

MASKED = -1.0e30


def kept(x):
    return [i for i, v in enumerate(x) if v > MASKED]


def test_argmax_picks_the_largest_and_breaks_ties_low():  # sampling.rs:300-305
    assert orc.argmax([1.0, 5.0, 3.0]) == 1
    assert orc.argmax([5.0, 5.0, 1.0]) == 0
    assert orc.argmax([]) is None


def test_greedy_decoding_is_deterministic():  # sampling.rs:307-318
    for r in np.linspace(0, 0.999, 20):
        assert orc.sample([0.1, 0.9, 0.3, 0.2], temperature=0.0, r=float(r))[0] == 1


def test_top_k_keeps_exactly_k_candidates():  # sampling.rs:371-382
    _, x, _ = orc.sample([1.0, 5.0, 3.0, 2.0, 4.0], top_k=2)
    assert kept(x) == [1, 4]


@pytest.mark.parametrize("k", [0, 3, 100])
def test_top_k_is_disabled_at_zero_or_beyond_the_vocabulary(k):  # sampling.rs:384-392
    _, x, _ = orc.sample([1.0, 5.0, 3.0], top_k=k)
    assert x.tolist() == [1.0, 5.0, 3.0]


def test_top_k_never_masks_everything():  # sampling.rs:394-402
    _, x, _ = orc.sample([2.0, 2.0, 2.0, 2.0], top_k=1)
    assert kept(x)


def test_top_p_keeps_the_nucleus_and_masks_the_tail():  # sampling.rs:404-413
    _, x, _ = orc.sample([5.0, 3.0, 0.0, -1.0], top_p=0.9)
    assert x[0] > MASKED and x[2] <= MASKED and x[3] <= MASKED


def test_top_p_of_one_is_a_no_op():  # sampling.rs:415-421
    _, x, _ = orc.sample([1.0, 2.0, 3.0], top_p=1.0)
    assert x.tolist() == [1.0, 2.0, 3.0]


def test_top_p_always_keeps_at_least_one_token():  # sampling.rs:423-433
    _, x, _ = orc.sample([1.0, 1.0, 1.0, 1.0], top_p=0.01)
    assert len(kept(x)) == 1


def test_repetition_penalty_lowers_logits_in_both_directions():  # sampling.rs:435-444
    _, x, _ = orc.sample([2.0, -2.0, 1.0], previous=[0, 1], repetition_penalty=2.0,
                         temperature=0.0)
    assert x.tolist() == [1.0, -4.0, 1.0]


def test_repetition_penalty_applies_once_per_distinct_token():  # sampling.rs:446-451
    _, x, _ = orc.sample([4.0, 1.0], previous=[0, 0, 0, 0], repetition_penalty=2.0,
                         temperature=0.0)
    assert x[0] == 2.0


def test_repetition_penalty_of_one_is_a_no_op_and_out_of_range_is_ignored():  # :453-465
    _, x, _ = orc.sample([2.0, -2.0], previous=[0, 1], repetition_penalty=1.0, temperature=0.0)
    assert x.tolist() == [2.0, -2.0]
    _, x, _ = orc.sample([1.0, 2.0], previous=[99], repetition_penalty=2.0, temperature=0.0)
    assert x.tolist() == [1.0, 2.0]


def test_sampling_always_returns_a_valid_token_id():  # sampling.rs:485-501
    rng = np.random.default_rng(7)
    for _ in range(200):
        t, _, _ = orc.sample([1.0, 2.0, 3.0, 0.5, -1.0, 4.0, 0.0, 2.5], previous=[1, 2],
                             temperature=0.8, top_k=3, top_p=0.9, repetition_penalty=1.1,
                             r=float(rng.random(dtype=np.float32)))
        assert 0 <= t < 8


def test_an_empty_logits_row_has_no_token():  # sampling.rs:503-508 (Internal error there)
    assert orc.sample([])[0] is None


def test_stochastic_sampling_respects_a_top_k_of_one():  # sampling.rs:510-523
    for r in np.linspace(0, 0.999, 50):
        assert orc.sample([1.0, 9.0, 2.0], top_k=1, r=float(r))[0] == 1


def test_sampling_reflects_the_distribution():  # sampling.rs:525-551
    rng = np.random.default_rng(11)
    counts = [0, 0, 0]
    for _ in range(3000):
        counts[orc.sample([0.0, 4.0, 0.0], r=float(rng.random(dtype=np.float32)))[0]] += 1
    assert counts[1] > 2500 and counts[0] > 0 and counts[2] > 0


def ref64(logits, prev, temperature, top_k, top_p, penalty, r):
    """Independent float64 restatement: filters as sets, draw by inverse CDF."""
    x = np.asarray(logits, np.float64).copy()
    if penalty != 1.0:
        for t in set(int(p) for p in prev):
            if t < len(x):
                x[t] = x[t] / penalty if x[t] > 0 else x[t] * penalty
    if temperature == 0.0:
        return int(np.argmax(x)), None
    x = x / temperature
    live = np.ones(len(x), bool)
    if 0 < top_k < len(x):
        thr = np.sort(x)[::-1][top_k - 1]
        live &= x >= thr
    def probs(mask):
        e = np.where(mask, np.exp(x - x[mask].max()), 0.0)
        return e / e.sum()
    if top_p < 1.0:
        p = probs(live)
        order = sorted(np.flatnonzero(live), key=lambda i: (-p[i], i))
        cum, keep = 0.0, []
        for i in order:
            keep.append(i)
            cum += p[i]
            if cum >= top_p:
                break
        live = np.zeros(len(x), bool)
        live[keep] = True
    p = probs(live)
    c = np.cumsum(p)
    return int(np.searchsorted(c, r, side="right")), live


@pytest.mark.parametrize("seed", range(40))
def test_matches_an_independent_float64_restatement(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(2, 300))
    logits = (rng.standard_normal(V) * rng.uniform(0.5, 4)).astype(np.float32)
    prev = rng.integers(0, V + 5, int(rng.integers(0, 20)))
    temperature = float(rng.choice([0.0, 0.7, 1.0, 1.3]))
    top_k = int(rng.choice([0, 1, 5, 50, V + 1]))
    top_p = float(rng.choice([1.0, 0.9, 0.5, 0.05]))
    penalty = float(rng.choice([1.0, 1.3]))
    r = float(rng.random(dtype=np.float32))
    t, x, margin = orc.sample(logits, prev, temperature, top_k, top_p, penalty, r)
    want, live = ref64(logits, prev, temperature, top_k, top_p, penalty, r)
    if live is not None:
        assert kept(x) == list(np.flatnonzero(live))
    if margin > 1e-5 or temperature == 0.0:
        assert t == want, (t, want, margin)
