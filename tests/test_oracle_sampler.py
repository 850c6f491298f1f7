"""Pins the sampler oracle: Philox KATs, exp accuracy, scan exactness, special cases, float64 restatement."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import sampler as S

# Random123 known-answer vectors for philox4x32 with 10 rounds: (counter, key, output).
PHILOX_KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter,key,expected", PHILOX_KAT)
def test_philox_known_answers(counter, key, expected):
    assert S.philox4x32(counter, key) == expected


def test_uniforms_are_in_unit_interval_and_counter_local():
    us = [S.uniform_from_counter(7, off) for off in range(0, 512 * 40, 32)]
    assert all(0.0 <= u < 1.0 for u in us)
    assert len(set(us)) == len(us)
    assert S.uniform_from_counter(3, 544) == S.uniform_from_counter(3, 544)


def test_exp_within_two_ulp_of_float64():
    x = np.linspace(-86.9, 0.0, 400001, dtype=np.float32)
    got = S.nq_exp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) <= 2.0
    assert S.nq_exp(np.float32(0.0)) == 1.0
    assert S.nq_exp(np.float32(-np.inf)) == 0.0 and S.nq_exp(np.float32(-87.0)) == 0.0


@pytest.mark.parametrize("k", [1, 5, 64, 65, 200, 3072])
def test_scan_is_exact_on_integers(k):
    w = np.random.default_rng(k).integers(0, 50, size=k).astype(np.float32)
    np.testing.assert_array_equal(S.wave_scan(w), np.cumsum(w.astype(np.int64)).astype(np.float32))


def test_greedy_is_argmax_with_lowest_id():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal(3072).astype(np.float32)
    assert S.sample_row(logits, 0.0, 50, 0.9, 0.7) == int(np.argmax(logits))
    logits[10] = logits[20] = logits.max() + 1
    assert S.sample_row(logits, 0.0, 50, 0.9, 0.7) == 10


def test_special_cases():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal(2048).astype(np.float32)
    top = int(np.argmax(logits))
    assert S.sample_row(logits, 0.9, 1, 1.0, 0.999) == top  # k = 1
    assert S.sample_row(logits, 0.9, 50, 0.95, 0.0) == top  # u = 0 -> rank 0
    assert S.sample_row(logits, 0.9, 50, 1e-7, 0.999) == top  # tiny p keeps only rank 0
    onehot = np.full(2048, -1e4, dtype=np.float32)
    onehot[777] = 10.0
    assert all(S.sample_row(onehot, 1.0, 50, 1.0, u) == 777 for u in (0.0, 0.5, 0.999999))


def test_penalty_and_masks():
    logits = np.array([2.0, -1.0, 1.9, 0.5], dtype=np.float32)
    seen = np.array([True, True, False, False])
    x = S.prepare(logits, 2.0, seen, 4, -1, False)
    np.testing.assert_array_equal(x, np.array([1.0, -2.0, 1.9, 0.5], dtype=np.float32))
    assert S.sample_row(logits, 0.0, 0, 1.0, 0.0, 2.0, seen) == 2  # greedy + penalty flips the winner
    x = S.prepare(np.zeros(3000, np.float32), 1.0, None, 2048, 2150, True)
    assert np.isneginf(x[2048:]).all() and np.isneginf(x[2150])
    x = S.prepare(np.zeros(3000, np.float32), 1.0, None, 2048, 2150, False)
    assert np.isneginf(x[2049:2150]).all() and x[2150] == 0.0


def _float64_reference(logits, t, k, p, u):
    """The reference fused sampler (executor/sampling.py:265-301) in float64, u given."""

    s = logits.astype(np.float64) / t
    order = np.lexsort((np.arange(len(s)), -s))[:k]
    w = np.exp(s[order] - s[order[0]])
    cum = np.cumsum(w)
    keep = (cum - w) < p * cum[-1]
    mass = w[keep].sum()
    hit = np.nonzero(keep & (cum >= u * mass))[0]
    return int(order[hit[0]]), cum, mass


def test_agrees_with_float64_restatement_away_from_boundaries():
    rng = np.random.default_rng(2)
    agree = skipped = 0
    for _ in range(400):
        logits = rng.standard_normal(3072).astype(np.float32) * 2
        u = float(rng.random())
        ref, cum, mass = _float64_reference(logits, 0.9, 50, 0.95, u)
        if np.min(np.abs(cum - u * mass)) < 1e-5 * mass:
            skipped += 1
            continue
        assert S.sample_row(logits, 0.9, 50, 0.95, u) == ref
        agree += 1
    assert agree > 350


def test_brute_force_distribution_small_vocab():
    """V = 6: sweeping u over [0,1) hits each kept token in proportion to its probability."""

    logits = np.array([0.3, -1.0, 2.0, 0.9, 0.9, -3.0], dtype=np.float32)
    us = (np.arange(20000) + 0.5) / 20000
    counts = np.bincount([S.sample_row(logits, 1.0, 4, 1.0, u) for u in us], minlength=6) / len(us)
    s = logits.astype(np.float64)
    top = np.lexsort((np.arange(6), -s))[:4]
    probs = np.zeros(6)
    probs[top] = np.exp(s[top]) / np.exp(s[top]).sum()
    np.testing.assert_allclose(counts, probs, atol=2e-4)
