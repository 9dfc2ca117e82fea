"""Members whose words equal the template's only after relocation: the
search pass places records by per-slot bounds that such words leave unused,
and the finishing pass closes the gaps.  Everything bit for bit against the
oracle, including a switch through the gapped override set."""
import numpy as np
import pytest

import gap_cases
import oracle
from foundry_amd import synth
from foundry_amd.restore import Archive
from parity import assert_live_matches, assert_restore_parity

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tiles", [(0, 1, -1), (1,), (-1,)])
def test_gaps_are_closed(cuda, tiles):
    s = synth.SynthArchive(synth.preset(2, num_graphs=6, nodes_per_graph=240, num_groups=2, num_intervals=500))
    iv = s.intervals()
    images = list(s.images())
    groups = oracle.Restore(images, iv).groups()
    members = [g for g in range(len(images)) if groups[g] != g]
    imgs = images
    planted = 0
    for g in members[:2]:
        imgs, words = gap_cases.plant_equal_after_relocation(imgs, iv, g, int(groups[g]), tiles=tiles, per_tile=3)
        planted += len(words)
    assert planted >= 2
    print(f"gaps: tiles={tiles} planted={planted}", flush=True)
    arch = Archive.from_images(imgs)
    arch.set_relocation(*iv)
    arch.restore()
    ref = oracle.Restore(imgs, iv)
    assert_restore_parity(arch, ref)
    g = members[0]
    t = int(groups[g])
    arch.switch(g)
    ref.switch(g)
    assert_live_matches(arch, ref, t)
    arch.close()
