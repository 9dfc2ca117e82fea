"""HIP restore vs the oracle over a seeded sweep of archive shapes.

Each case draws the generator's knobs at random (within their documented
ranges): graph and group counts, node counts, blob sizes and param splits,
ragged params, arg-buffer params, memset / memcpy / event nodes,
batch-size-dependent grids and layouts, clustered or scattered differences,
pointer fraction, interval count, and the relocation policy -- so that the
combinations no hand-written case names are compared output for output too.
"""
import random

import pytest

from foundry_amd import synth
from tests.parity import assert_live_matches, assert_restore_parity, gpu_and_oracle

pytestmark = pytest.mark.gpu

CASES = 40
WIDE = 12  # more cases whose kernel nodes take 17-48 params (past the 16 kept field-major)


def _params(seed: int):
    rng = random.Random(seed)
    base = rng.choice([1, 2, 3])
    groups = rng.choice([1, 2, 3, 5])
    p = synth.preset(
        base,
        num_graphs=rng.randrange(groups, groups * 6 + 1),
        num_groups=groups,
        nodes_per_graph=rng.choice([1, 7, 64, 255, 256, 257, 600]),
        min_blob_bytes=8 * rng.randrange(1, 4),
        max_blob_bytes=8 * rng.randrange(4, 160),
        max_params=rng.randrange(1, 17),
        ragged=rng.randrange(2),
        extra_style_pct=rng.choice([0, 0, 10, 40]),
        memset_pct=rng.choice([0, 5, 15]),
        memcpy_pct=rng.choice([0, 5, 10]),
        event_pct=rng.choice([0, 4]),
        grid_bs_pct=rng.choice([0, 20]),
        layout_var_pct=rng.choice([0, 0, 5]),
        pointer_frac=rng.choice([0.0, 0.25, 0.6]),
        diff_lo=0.0,
        diff_hi=rng.choice([0.0, 0.03, 0.2]),
        seed=0x5EED5000 + seed,
        num_intervals=rng.choice([1, 64, 4096]),
    )
    if rng.random() < 0.3:
        p.run_min_bytes, p.run_max_bytes = 64, 256
    policy = rng.randrange(2)
    if seed >= CASES:
        p.max_params = 17 + (7 * seed) % 32
        p.max_blob_bytes = max(p.max_blob_bytes, 16 * p.max_params)
    return p, policy


@pytest.mark.parametrize("seed", range(CASES + WIDE))
def test_random_shape(cuda, seed):
    p, policy = _params(seed)
    print(f"[case] sweep seed={seed}: base preset {p.preset}, graphs={p.num_graphs} groups={p.num_groups} "
          f"nodes={p.nodes_per_graph} blob={p.min_blob_bytes}-{p.max_blob_bytes} params<={p.max_params} "
          f"ragged={p.ragged} extra={p.extra_style_pct}% memset={p.memset_pct}% memcpy={p.memcpy_pct}% "
          f"events={p.event_pct}% layout_var={p.layout_var_pct}% intervals={p.num_intervals} policy={policy}",
          flush=True)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s, policy=policy)
    assert_restore_parity(arch, ref)
    groups = arch.groups()
    for t in sorted(set(groups.tolist()))[:2]:
        members = [g for g in range(s.num_graphs) if groups[g] == t]
        for g in members[1:3] + members[:1]:
            arch.switch(g)
            ref.switch(g)
        assert_live_matches(arch, ref, t)
    arch.close()
