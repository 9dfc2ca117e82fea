"""Oracle relocation against a brute-force linear scan and hand cases.

Rule (build definition): the last interval i with lo_i <= w moves w to
w - lo_i + new_lo_i if w < hi_i (w <= hi_i under the inclusive policy)."""
import random

import numpy as np
import pytest

import oracle


def brute(w, ivs, policy):
    hit = None
    for lo, hi, nlo in ivs:
        if lo <= w:
            hit = (lo, hi, nlo)
    if hit is None:
        return w
    lo, hi, nlo = hit
    inside = w <= hi if policy else w < hi
    return (w - lo + nlo) & ((1 << 64) - 1) if inside else w


def cols(ivs):
    a = np.array(ivs, dtype=np.uint64).reshape(-1, 3)
    return a[:, 0].copy(), a[:, 1].copy(), a[:, 2].copy()


def table(rng, n, gaps=True):
    ivs, at = [], rng.randrange(0, 1 << 20)
    for _ in range(n):
        if gaps and rng.random() < 0.5:
            at += rng.randrange(1, 1 << 12)
        size = rng.randrange(1, 1 << 14)
        ivs.append((at, at + size, rng.randrange(0, 1 << 48)))
        at += size
    return ivs


@pytest.mark.parametrize("policy", [0, 1])
def test_brute_force(policy):
    rng = random.Random(11 + policy)
    for _ in range(60):
        ivs = table(rng, rng.randrange(1, 40), gaps=rng.random() < 0.7)
        words = []
        for lo, hi, _ in ivs:
            words += [lo - 1, lo, lo + 1, hi - 1, hi, hi + 1, rng.randrange(lo, hi)]
        words += [rng.randrange(0, 1 << 64) for _ in range(20)] + [0, (1 << 64) - 1]
        words = [w & ((1 << 64) - 1) for w in words]
        lo, hi, nlo = cols(ivs)
        got = oracle.relocate_words(words, lo, hi, nlo, policy=policy, threads=2)
        assert got.tolist() == [brute(w, ivs, policy) for w in words]
        for w in words[:10]:
            assert oracle.relocate_word(w, lo, hi, nlo, policy) == brute(w, ivs, policy)


def test_hand_cases_adjacent_intervals():
    lo, hi, nlo = cols([(100, 200, 1000), (200, 300, 5000), (400, 500, 9000)])
    cases = {  # w: (exclusive, inclusive)
        99: (99, 99), 100: (1000, 1000), 199: (1099, 1099),
        200: (5000, 5000),          # one past interval 0 is interval 1's first byte
        299: (5099, 5099), 300: (300, 5100),  # one past the end: only the inclusive policy moves it
        350: (350, 350), 400: (9000, 9000), 500: (500, 9100), 501: (501, 501),
    }
    for w, (ex, inc) in cases.items():
        assert oracle.relocate_word(w, lo, hi, nlo, 0) == ex, w
        assert oracle.relocate_word(w, lo, hi, nlo, 1) == inc, w


def test_identity_at_zero_shift_and_empty_table():
    rng = random.Random(3)
    ivs = [(lo, hi, lo) for lo, hi, _ in table(rng, 30)]
    lo, hi, nlo = cols(ivs)
    words = [rng.randrange(0, 1 << 22) for _ in range(500)]
    assert oracle.relocate_words(words, lo, hi, nlo).tolist() == words
    e = np.zeros(0, dtype=np.uint64)
    assert oracle.relocate_words(words, e, e, e).tolist() == words


def test_shift_wraps_modulo_2_64():
    lo, hi, nlo = cols([(1 << 63, (1 << 63) + 100, 5)])
    assert oracle.relocate_word((1 << 63) + 7, lo, hi, nlo, 0) == 12
