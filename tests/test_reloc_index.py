"""The interval index (foundry_amd/csrc/reloc_index.h) and its search
(reloc_batch in foundry_amd/csrc/restore_dev.h, the code the kernels run),
executed on the CPU by tests/native/reloc_index_check and compared with the
oracle's binary search (oracle.cpp relocate_word, which follows the
reference's relocation rule) on tables shaped to reach every kind of line:
leaves, fence lines one and several levels deep, lines wider than any
interval, abutting intervals under both policies, a table at the top of the
address space, and the relocation-heavy workload's interval mix.  Every
fence line must name children inside the index and after itself."""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle
from foundry_amd import synth

CHECK = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "_build", "reloc_index_check")


def _run(tmp_path, lo, hi, nlo, words, policy, per=None):
    assert os.path.exists(CHECK), "build first: make -C tests/native"
    t, w, o = (str(tmp_path / f) for f in ("t.bin", "w.bin", "o.bin"))
    np.concatenate([np.array([len(lo), policy], np.uint64), lo, hi, nlo]).astype(np.uint64).tofile(t)
    np.asarray(words, np.uint64).tofile(w)
    extra = [] if per is None else [str(per)]
    p = subprocess.run([CHECK, t, w, o] + extra, capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    stats = json.loads(p.stdout)
    return stats, (None if "error" in stats else np.fromfile(o, np.uint64))


def _probe_words(lo, hi, rng, extra=20000):
    """Every interval's edges (lo - 1, lo, lo + 1, hi - 1, hi, hi + 1) and
    random words inside and around the table."""
    edges = np.concatenate([lo - 1, lo, lo + 1, hi - 1, hi, hi + 1])
    span_lo, span_hi = int(lo[0]), int(hi[-1])
    r = rng.integers(0, 1 << 63, extra, dtype=np.int64).view(np.uint64)
    inside = np.uint64(span_lo) + r % np.uint64(span_hi - span_lo + 1)
    outside = np.array([0, 1, span_lo - 2, min(span_hi + 2, (1 << 64) - 1), (1 << 64) - 1], dtype=np.uint64)
    return np.concatenate([edges, inside, outside])


def _check(tmp_path, lo, hi, nlo, rng, max_reads=None, words=None, per=None):
    lo, hi, nlo = (np.asarray(a, np.uint64) for a in (lo, hi, nlo))
    w = _probe_words(lo, hi, rng) if words is None else words
    for policy in (0, 1):
        stats, got = _run(tmp_path, lo, hi, nlo, w, policy, per)
        assert stats["bad_refs"] == 0, stats
        want = oracle.relocate_words(w, lo, hi, nlo, policy, threads=8)
        np.testing.assert_array_equal(got, want)
        if max_reads is not None:
            assert stats["max_reads"] <= max_reads, stats
    return stats


def test_dense_tiny_intervals_build_fence_lines_several_levels_deep(tmp_path):
    """20,000 adjacent 16-byte intervals beside one 1 GiB interval: every
    root line over the tiny ones holds thousands of them, so the search
    descends three or more fence levels."""
    rng = np.random.default_rng(1)
    n = 20000
    base = 1 << 40
    lo = base + 16 * np.arange(n, dtype=np.uint64)
    hi = lo + 16
    lo = np.append(lo, hi[-1] + 4096)
    hi = np.append(hi, lo[-1] + (1 << 30))
    nlo = (1 << 44) + rng.permutation(len(lo)).astype(np.uint64) * (1 << 31)
    stats = _check(tmp_path, lo, hi, nlo, rng)
    assert stats["fence_lines"] > 0 and stats["max_reads"] >= 4, stats


def test_gaps_and_abutting_intervals(tmp_path):
    """Random sizes with random gaps, a third of them abutting (hi == next
    lo): the point hi belongs to the next interval under both policies, and
    to the interval itself under the inclusive one when a gap follows."""
    rng = np.random.default_rng(2)
    n = 30000
    sizes = rng.integers(1, 1 << 14, n).astype(np.uint64)
    gaps = np.where(rng.random(n) < 0.33, 0, rng.integers(1, 1 << 16, n)).astype(np.uint64)
    lo = (1 << 36) + np.cumsum(sizes + gaps) - sizes
    hi = lo + sizes
    nlo = lo + rng.integers(-(1 << 30), 1 << 30, n).astype(np.int64).view(np.uint64)
    _check(tmp_path, lo, hi, nlo, rng)


def test_wide_sparse_span_and_single_interval(tmp_path):
    """A few intervals over 2^44 bytes (lines of the widest width, 2^31), and
    a table of one interval."""
    rng = np.random.default_rng(3)
    lo = np.sort(rng.choice(1 << 20, 64, replace=False).astype(np.uint64)) << np.uint64(24)
    hi = lo + rng.integers(1, 1 << 24, 64).astype(np.uint64)
    stats = _check(tmp_path, lo, hi, lo + (1 << 50), rng)
    assert stats["shift"] == 31, stats
    _check(tmp_path, [4096], [8192], [1 << 30], rng, max_reads=1)


def test_table_at_the_top_of_the_address_space(tmp_path):
    """Intervals ending just below 2^64 - 1 (line starts past the last root
    line saturate instead of wrapping)."""
    rng = np.random.default_rng(4)
    top = (1 << 64) - (1 << 34)
    lo = np.uint64(top) + np.arange(0, 1 << 33, 1 << 20, dtype=np.uint64)
    hi = lo + np.uint64(1 << 19)
    hi[-1] = np.uint64((1 << 64) - 2)
    nlo = lo - np.uint64(1 << 40)
    _check(tmp_path, lo, hi, nlo, rng)


def test_relocation_heavy_interval_mix(tmp_path):
    """The relocation-heavy workload's table (2M log-uniform intervals tiling
    200 GB) and its packed words: at most two line reads per search."""
    p = synth.preset(4, num_words=1 << 20)
    s = synth.SynthArchive(p)
    lo, hi, nlo = s.intervals()
    stats = _check(tmp_path, lo, hi, nlo, np.random.default_rng(5), max_reads=2,
                   words=np.array(s.words(), copy=True))
    print(stats)
    assert stats["line_reads"] <= 1.7 * stats["searched"], stats


@pytest.mark.parametrize("per", [1, 16])
def test_plan_sized_index(tmp_path, per):
    """The same lookups with 1 and with 16 root lines per interval (the
    relocation plan's index): the relocation-heavy mix, where 16 per interval
    takes fewer line reads, and the dense fence-line and top-of-address-space
    tables."""
    p = synth.preset(4, num_words=1 << 19)
    s = synth.SynthArchive(p)
    lo, hi, nlo = s.intervals()
    words = np.array(s.words(), copy=True)
    stats = _check(tmp_path, lo, hi, nlo, np.random.default_rng(6), words=words, per=per)
    base, _ = _run(tmp_path, np.asarray(lo, np.uint64), np.asarray(hi, np.uint64), np.asarray(nlo, np.uint64),
                   words, 0)
    if per == 16:
        assert stats["line_reads"] < base["line_reads"], (stats, base)
        assert stats["root_lines"] >= 4 * base["root_lines"], (stats, base)
    rng = np.random.default_rng(7)
    n = 20000
    tlo = (1 << 40) + 16 * np.arange(n, dtype=np.uint64)
    _check(tmp_path, tlo, tlo + 16, (1 << 44) + rng.permutation(n).astype(np.uint64) * (1 << 31), rng, per=per)
    top = np.uint64((1 << 64) - (1 << 34)) + np.arange(0, 1 << 33, 1 << 20, dtype=np.uint64)
    thi = top + np.uint64(1 << 19)
    thi[-1] = np.uint64((1 << 64) - 2)
    _check(tmp_path, top, thi, top - np.uint64(1 << 40), rng, per=per)


def test_refused_tables(tmp_path):
    """Unsorted or overlapping intervals are refused before any line is built."""
    stats, _ = _run(tmp_path, np.array([100, 50], np.uint64), np.array([200, 60], np.uint64),
                    np.array([0, 0], np.uint64), np.array([1], np.uint64), 0)
    assert stats == {"error": -1}  # FDY_E_INVALID


def test_tables_of_unequal_length_are_refused_before_the_library():
    """The Python binding checks that lo, hi and new_lo have one entry per
    interval: the library reads n entries of each."""
    from foundry_amd.restore import Archive, RelocPlan, relocate_words_static
    lo, hi = np.array([100, 300], np.uint64), np.array([200, 400], np.uint64)
    with pytest.raises(ValueError):
        RelocPlan(lo, hi, np.array([0], np.uint64))
    with pytest.raises(ValueError):
        relocate_words_static(lo, hi[:1], lo, 0, 0, 0)
    with pytest.raises(ValueError):
        Archive.set_relocation(None, lo, np.zeros((2, 1), np.uint64), lo)
