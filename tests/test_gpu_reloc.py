"""Standalone relocation kernel vs the oracle (relocation-heavy workload)."""
import numpy as np
import pytest

import oracle
from foundry_amd import synth
from foundry_amd._lib import FoundryError
from foundry_amd.restore import RelocPlan

pytestmark = pytest.mark.gpu


def _gpu_relocate(torch, words, lo, hi, nlo, policy=0, offset_words=0):
    plan = RelocPlan(lo, hi, nlo, policy)
    n = len(words)
    d_in = torch.from_numpy(words.view(np.int64)).to("cuda")
    d_out = torch.empty(n + offset_words, dtype=torch.int64, device="cuda")
    plan.relocate(d_in.data_ptr(), d_out.data_ptr() + 8 * offset_words, n)
    torch.cuda.synchronize()
    out = d_out.cpu().numpy().view(np.uint64)[offset_words:]
    plan.close()
    return out


@pytest.mark.parametrize("intervals", [1, 100, 4096, 4097, 70000, 2_000_000])
def test_relocate_words_matches_oracle(cuda, intervals):
    p = synth.preset(4, num_words=1 << 20, num_intervals=intervals, seed=0xC4 + intervals)
    print(f"[case] relocate intervals={intervals} words={p.num_words}", flush=True)
    s = synth.SynthArchive(p)
    words = np.array(s.words(), copy=True)
    lo, hi, nlo = s.intervals()
    for policy in (0, 1):
        got = _gpu_relocate(cuda, words, lo, hi, nlo, policy)
        want = oracle.relocate_words(words, lo, hi, nlo, policy, threads=8)
        np.testing.assert_array_equal(got, want)


def test_relocate_unaligned_and_odd_length(cuda):
    p = synth.preset(4, num_words=100_001, num_intervals=5000, seed=7)
    s = synth.SynthArchive(p)
    words = np.array(s.words(), copy=True)
    lo, hi, nlo = s.intervals()
    got = _gpu_relocate(cuda, words, lo, hi, nlo, 0, offset_words=1)  # 8-B aligned, not 16-B
    np.testing.assert_array_equal(got, oracle.relocate_words(words, lo, hi, nlo, 0))


@pytest.mark.parametrize("n,offset", [(1 << 20, 0), (100_001, 1)])
def test_relocate_in_place(cuda, n, offset):
    """in == out (the header allows it), on a 16-byte-aligned even array and
    on an 8-byte-aligned odd one."""
    p = synth.preset(4, num_words=n, num_intervals=5000, seed=11 + n)
    print(f"[case] relocate in place words={n} offset={offset}", flush=True)
    s = synth.SynthArchive(p)
    words = np.array(s.words(), copy=True)
    lo, hi, nlo = s.intervals()
    plan = RelocPlan(lo, hi, nlo, 0)
    d = cuda.zeros(n + offset, dtype=cuda.int64, device="cuda")
    d[offset:] = cuda.from_numpy(words.view(np.int64)).to("cuda")
    ptr = d.data_ptr() + 8 * offset
    plan.relocate(ptr, ptr, n)
    cuda.cuda.synchronize()
    got = d.cpu().numpy().view(np.uint64)[offset:]
    plan.close()
    np.testing.assert_array_equal(got, oracle.relocate_words(words, lo, hi, nlo, 0, threads=8))


def test_relocate_full_size_round_trip(cuda):
    # 1 GiB of words against 2M intervals: relocating with the inverse table
    # restores every word that was relocated (size-independent check).
    p = synth.preset(4)
    print(f"[case] relocate full words={p.num_words} intervals={p.num_intervals}", flush=True)
    s = synth.SynthArchive(p)
    words = s.words()
    lo, hi, nlo = s.intervals()
    torch = cuda
    plan = RelocPlan(lo, hi, nlo, 0)
    order = np.argsort(nlo)
    inv = RelocPlan(nlo[order], (nlo + (hi - lo))[order], lo[order], 0)
    d_in = torch.from_numpy(np.asarray(words).view(np.int64)).to("cuda")
    d_mid = torch.empty_like(d_in)
    d_back = torch.empty_like(d_in)
    plan.relocate(d_in.data_ptr(), d_mid.data_ptr(), len(words))
    inv.relocate(d_mid.data_ptr(), d_back.data_ptr(), len(words))
    torch.cuda.synchronize()
    moved = (d_mid != d_in)
    # Every word that moved came back; words that did not move (outside the
    # old region, hence outside the new one too) stay put under the inverse.
    assert torch.equal(d_back, d_in)
    frac = moved.double().mean().item()
    assert 0.35 < frac < 0.45, frac  # ~40% pointers
    # A sampled slice checked exactly against the oracle.
    idx = slice(12_345_678, 12_345_678 + 200_000)
    want = oracle.relocate_words(np.asarray(words)[idx], lo, hi, nlo, 0, threads=8)
    np.testing.assert_array_equal(d_mid[idx].cpu().numpy().view(np.uint64), want)


def test_empty_table_zero_words_and_refused_tables(cuda):
    """A plan of no intervals leaves every word as it is (the reference's
    relocation of a pointer outside every interval), a call for zero words
    writes nothing, and tables that break the interval rules are refused
    when the plan is made."""
    print("[case] relocation: empty table, zero words, refused tables", flush=True)
    rng = np.random.default_rng(5)
    words = rng.integers(0, 1 << 63, 10_001, dtype=np.uint64) * np.uint64(2) + np.uint64(1)
    words[:3] = [0, 1, np.uint64((1 << 64) - 1)]
    empty = np.zeros(0, np.uint64)
    for policy in (0, 1):
        plan = RelocPlan(empty, empty, empty, policy)
        assert plan.lines().shape == (0, 8)
        d_in = cuda.from_numpy(words.view(np.int64)).to("cuda")
        d_out = cuda.full_like(d_in, 7)
        plan.relocate(d_in.data_ptr(), d_out.data_ptr(), 0)
        cuda.cuda.synchronize()
        assert (d_out.cpu().numpy() == 7).all()
        plan.relocate(d_in.data_ptr(), d_out.data_ptr(), len(words))
        cuda.cuda.synchronize()
        got = d_out.cpu().numpy().view(np.uint64)
        np.testing.assert_array_equal(got, words)
        np.testing.assert_array_equal(got, oracle.relocate_words(words, empty, empty, empty, policy))
        plan.close()
    bad = {
        "overlapping": ([100, 150], [200, 300]),
        "unsorted": ([300, 100], [400, 200]),
        "empty interval": ([100, 300], [100, 400]),
        "ending at 2^64-1": ([100], [(1 << 64) - 1]),
    }
    for name, (lo, hi) in bad.items():
        lo, hi = np.array(lo, np.uint64), np.array(hi, np.uint64)
        with pytest.raises(FoundryError, match="interval"):
            RelocPlan(lo, hi, lo)
    with pytest.raises(FoundryError, match="policy"):
        RelocPlan(np.array([100], np.uint64), np.array([200], np.uint64), np.array([0], np.uint64), 2)
