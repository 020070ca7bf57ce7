"""Sampling (sampler.rs:1-92): the oracle's restatement pinned by closed
forms, and the library's host sampler (pi_sample) equal to it (CPU only).

* SplitMix64: the constants and steps of sampler.rs:1-19, restated here in
  integer Python (a wrong constant or shift changes every draw).
* CDF inversion: weights 1/4, 1/2, 3/4, 1 (logits log 1..4 at temp 1) have
  cumulative sums 0.25, 0.75, 1.5, 2.5; the draw u * 2.5 falls in one of
  those intervals, which fixes the id from u alone.
* Top-p: weights 1, 1/2, 1/4, 1/8, 1/8 (sum 2) with top_p 0.7 keep exactly
  the first two (running shares 0.5, 0.75); top_p 0.5 keeps only the first.
* Equal weights at the cut are kept by index.
* Non-finite logits (all -inf, or a NaN sum) give id 0; temp <= 0 is greedy.
"""
import ctypes as C
import math

import numpy as np
import pytest

M64 = 0xFFFFFFFFFFFFFFFF


def splitmix_next(state):
    z = (state + 0x9E3779B97F4A7C15) & M64
    state = z
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return state, z ^ (z >> 31)


def u_of(seed):
    """next_f32 of Rng::new(seed), exactly (a 24-bit fraction)."""
    _, z = splitmix_next((seed + 0x9E3779B97F4A7C15) & M64)
    return (z >> 40) / float(1 << 24)


def oracle_sample(oracle, logits, temp, top_p, seed):
    """(id, weights left in the logits) of the oracle's po_sample."""
    v = np.array(logits, np.float32)
    r = oracle.PoRng()
    oracle.lib().po_rng_init(C.byref(r), seed)
    tok = oracle.lib().po_sample(v.ctypes.data, v.size, temp, top_p, C.byref(r))
    return tok, v


def lib_sample(pih, logits, temp, top_p, seed):
    v = np.array(logits, np.float32)
    tok = pih.sample(v, temp, top_p, pih.Rng(seed))
    return tok, v


@pytest.fixture(params=["oracle", "library"])
def sampler(request, oracle, pih):
    if request.param == "oracle":
        return lambda lg, t, p, s: oracle_sample(oracle, lg, t, p, s)[0]
    return lambda lg, t, p, s: lib_sample(pih, lg, t, p, s)[0]


def test_splitmix64_streams(oracle, pih):
    for seed in (0, 1, 0xC0FFEE, 2 ** 63 + 5):
        st = (seed + 0x9E3779B97F4A7C15) & M64
        r = oracle.PoRng()
        oracle.lib().po_rng_init(C.byref(r), seed)
        rl = pih.Rng(seed)
        for _ in range(5):
            st, want = splitmix_next(st)
            assert oracle.lib().po_rng_next_u64(C.byref(r)) == want
            assert rl.next_u64() == want


def _cdf_case(u):
    cum = [0.25, 0.75, 1.5, 2.5]
    r = u * 2.5
    if min(abs(r - c) for c in cum) < 1e-4:
        return None      # too close to a boundary for float rounding to be irrelevant
    return next(i for i, c in enumerate(cum) if r <= c)


def test_cdf_inversion_closed_form(sampler):
    logits = [math.log(1), math.log(2), math.log(3), math.log(4)]
    seen = set()
    for seed in range(200):
        want = _cdf_case(u_of(seed))
        if want is None:
            continue
        assert sampler(logits, 1.0, 1.0, seed) == want, seed
        seen.add(want)
    assert seen == {0, 1, 2, 3}


def test_top_p_keeps_the_hand_computed_set(sampler):
    # weights 1, 1/2, 1/4, 1/8, 1/8 at temp 1 (sum 2)
    logits = [0.0, -math.log(2), -math.log(4), -math.log(8), -math.log(8)]
    for seed in range(200):
        u = u_of(seed)
        # top_p 0.7: keeps ids 0, 1 (new sum 1.5); the draw picks 0 when u * 1.5 <= 1
        r = u * 1.5
        if abs(r - 1.0) > 1e-4:
            assert sampler(logits, 1.0, 0.7, seed) == (0 if r <= 1.0 else 1), seed
        # top_p 0.5: the first share already reaches it, only id 0 survives
        assert sampler(logits, 1.0, 0.5, seed) == 0


def test_top_p_ties_kept_by_index(sampler):
    # weights 1/2, 1, 1/2, 1 (sum 3): order 1, 3, 0, 2; top_p 0.6 -> shares
    # 1/3, 2/3: keeps ids 1 and 3; top_p 0.8 -> 5/6: keeps 1, 3 and then the
    # lower index of the tie (0), never 2
    logits = [-math.log(2), 0.0, -math.log(2), 0.0]
    got6 = {sampler(logits, 1.0, 0.6, s) for s in range(300)}
    assert got6 == {1, 3}
    got8 = {sampler(logits, 1.0, 0.8, s) for s in range(300)}
    assert got8 == {0, 1, 3}


def test_degenerate_inputs(sampler):
    assert sampler([-np.inf] * 5, 0.7, 0.95, 1) == 0            # (v - max) is NaN: sum is not > 0
    assert sampler([1.0, np.nan, 2.0], 0.7, 0.95, 1) == 0       # NaN weight: the sum is NaN
    assert sampler([0.5, 3.0, 3.0, 1.0], 0.0, 0.95, 1) == 1     # temp 0: first maximum
    assert sampler([0.5, 3.0, 3.0, 1.0], -1.0, 0.95, 9) == 1


@pytest.mark.parametrize("temp,top_p", [(0.7, 0.95), (1.0, 1.0), (0.3, 0.5), (1.5, 0.99), (0.7, 0.0)])
def test_library_sampler_equals_oracle(oracle, pih, temp, top_p):
    """Same ids and the same weights left in the logits, bit for bit, over
    near-flat and peaked logit vectors."""
    rng = np.random.default_rng(5)
    for trial in range(40):
        n = int(rng.integers(2, 3000))
        scale = 0.05 if trial % 2 else 4.0
        logits = (rng.standard_normal(n) * scale).astype(np.float32)
        if trial % 5 == 0:
            logits[rng.integers(0, n, size=3)] = logits.max()          # ties at the top
        seed = int(rng.integers(0, 2 ** 63))
        a, wa = oracle_sample(oracle, logits, temp, top_p, seed)
        b, wb = lib_sample(pih, logits, temp, top_p, seed)
        assert a == b, (trial, n, temp, top_p)
        assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32)), trial
