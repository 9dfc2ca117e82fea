"""The planted equal-after-relocation words (tests/gap_cases.py) are what
they claim to be, checked on the CPU against the oracle: each differs from
the template's raw word, makes no override record, and the member's
relocated image holds the template's relocated word there."""
import numpy as np
import pytest

import gap_cases
import oracle
from foundry_amd import synth


@pytest.fixture(scope="module")
def planted():
    s = synth.SynthArchive(synth.preset(2, num_graphs=6, nodes_per_graph=240, num_groups=2, num_intervals=500))
    iv = s.intervals()
    images = list(s.images())
    ref0 = oracle.Restore(images, iv)
    groups = ref0.groups()
    members = [g for g in range(len(images)) if groups[g] != g]
    g = members[0]
    imgs, words = gap_cases.plant_equal_after_relocation(images, iv, g, int(groups[g]), tiles=(0, 1, -1))
    return images, imgs, iv, g, int(groups[g]), words, ref0


def test_planted_words_make_no_records(planted):
    images, imgs, iv, g, t, words, ref0 = planted
    assert len(words) >= 4, "the generator offers pointers to plant in at least two tiles"
    assert len({w // 4096 for w in words}) >= 2
    ref = oracle.Restore(imgs, iv)
    np.testing.assert_array_equal(ref.groups(), ref0.groups())
    ri, rt = ref.param_image(g), ref.param_image(t)
    nw = ref.node_words(g)
    for w in words:
        assert ri[w] == rt[w], "relocated member word equals the template's"
    # The planted words changed raw bytes but no record, and the other
    # records are unchanged.
    np.testing.assert_array_equal(ref.overrides(g), ref0.overrides(g))
    assert nw[-1] > 4096, "the member spans more than one tile"
