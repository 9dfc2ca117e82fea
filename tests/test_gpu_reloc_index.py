"""The interval index built on the device (fdy_reloc_plan_create: the
builder of foundry_amd/csrc/reloc_index.h run as kernels, one thread per
root line) against the host build of the same table
(tests/native/reloc_index_check, the same builder on the CPU, which the CPU
tests pin against the oracle's search): equal line for line, 16 root lines
per interval as in every plan, on tables shaped to reach every kind of line:
fence lines several levels deep (dense tiny intervals beside a huge one),
random gaps with abutting intervals, the widest root lines over a sparse
span, one interval, a table at the top of the address space, and the
relocation-heavy workload's interval mix.  Each plan then relocates its
table's edge words as the oracle does."""
import os
import subprocess

import numpy as np
import pytest
import torch

import oracle
from foundry_amd import synth
from foundry_amd._lib import RELOC_HALF_OPEN, RELOC_INCLUSIVE
from foundry_amd.restore import RelocPlan

pytestmark = pytest.mark.gpu

CHECK = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "_build", "reloc_index_check")
PLAN_ROOT_LINES_PER_INTERVAL = 16


def _host_lines(tmp_path, lo, hi, nlo, policy):
    assert os.path.exists(CHECK), "build first: make -C tests/native"
    t, w, o, x = (str(tmp_path / f) for f in ("t.bin", "w.bin", "o.bin", "x.bin"))
    np.concatenate([np.array([len(lo), policy], np.uint64), lo, hi, nlo]).astype(np.uint64).tofile(t)
    np.zeros(0, np.uint64).tofile(w)
    p = subprocess.run([CHECK, t, w, o, str(PLAN_ROOT_LINES_PER_INTERVAL), x], capture_output=True, text=True,
                       timeout=300)
    assert p.returncode == 0, p.stderr
    return np.fromfile(x, np.uint64).reshape(-1, 8)


def _check(tmp_path, name, lo, hi, nlo):
    lo, hi, nlo = (np.asarray(a, np.uint64) for a in (lo, hi, nlo))
    print(f"[case] device interval index: {name}, {len(lo)} intervals", flush=True)
    edges = np.concatenate([lo - np.uint64(1), lo, hi - np.uint64(1), hi])
    for policy in (RELOC_HALF_OPEN, RELOC_INCLUSIVE):
        plan = RelocPlan(lo, hi, nlo, policy)
        try:
            got = plan.lines()
            want = _host_lines(tmp_path, lo, hi, nlo, policy)
            assert got.shape == want.shape, (got.shape, want.shape)
            bad = np.nonzero((got != want).any(axis=1))[0]
            assert bad.size == 0, f"{name}: {bad.size} lines differ, first {bad[:8].tolist()}"
            d_in = torch.from_numpy(edges.view(np.int64)).cuda()
            d_out = torch.empty_like(d_in)
            plan.relocate(d_in.data_ptr(), d_out.data_ptr(), edges.size)
            torch.cuda.synchronize()
            out = d_out.cpu().numpy().view(np.uint64)
            np.testing.assert_array_equal(out, oracle.relocate_words(edges, lo, hi, nlo, policy, threads=8))
        finally:
            plan.close()


def test_dense_tiny_intervals_beside_a_huge_one(tmp_path):
    rng = np.random.default_rng(1)
    n = 20000
    lo = (1 << 40) + 16 * np.arange(n, dtype=np.uint64)
    hi = lo + np.uint64(16)
    lo = np.append(lo, hi[-1] + np.uint64(4096))
    hi = np.append(hi, lo[-1] + np.uint64(1 << 30))
    nlo = (1 << 44) + rng.permutation(len(lo)).astype(np.uint64) * np.uint64(1 << 31)
    _check(tmp_path, "dense tiny intervals", lo, hi, nlo)


def test_gaps_and_abutting_intervals(tmp_path):
    rng = np.random.default_rng(2)
    n = 30000
    sizes = rng.integers(1, 1 << 14, n).astype(np.uint64)
    gaps = np.where(rng.random(n) < 0.33, 0, rng.integers(1, 1 << 16, n)).astype(np.uint64)
    lo = np.uint64(1 << 36) + np.cumsum(sizes + gaps) - sizes
    hi = lo + sizes
    nlo = lo + rng.integers(-(1 << 30), 1 << 30, n).astype(np.int64).view(np.uint64)
    _check(tmp_path, "gaps and abutting intervals", lo, hi, nlo)


def test_sparse_span_single_interval_and_top_of_address_space(tmp_path):
    rng = np.random.default_rng(3)
    lo = np.sort(rng.choice(1 << 20, 64, replace=False).astype(np.uint64)) << np.uint64(24)
    hi = lo + rng.integers(1, 1 << 24, 64).astype(np.uint64)
    _check(tmp_path, "sparse span", lo, hi, lo + np.uint64(1 << 50))
    _check(tmp_path, "one interval", [4096], [8192], [1 << 30])
    top = np.uint64((1 << 64) - (1 << 34)) + np.arange(0, 1 << 33, 1 << 20, dtype=np.uint64)
    thi = top + np.uint64(1 << 19)
    thi[-1] = np.uint64((1 << 64) - 2)
    _check(tmp_path, "top of the address space", top, thi, top - np.uint64(1 << 40))


def test_relocation_heavy_interval_mix(tmp_path):
    s = synth.SynthArchive(synth.preset(4, num_words=1 << 10))
    lo, hi, nlo = s.intervals()
    _check(tmp_path, "relocation-heavy mix (2M intervals)", lo, hi, nlo)
