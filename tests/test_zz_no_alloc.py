"""fdy_relocate_words_static (relocation whose interval index lives in the
library's static per-GPU array, with no device allocation) against
fdy_relocate_words with a plan of the same table: two calls in a row, the
second on a smaller table and fewer words (the array keeps the first call's
index, which must not leak into the second), plus in place."""
import ctypes as C

import numpy as np
import pytest

from foundry_amd import _lib, synth
from foundry_amd.restore import RelocPlan, relocate_words_static


def _case(n_words, n_iv, seed):
    p = synth.preset(4, num_words=n_words, num_intervals=n_iv, seed=seed)
    s = synth.SynthArchive(p)
    return np.array(s.words(), copy=True), s.intervals()


def test_static_index_too_large_is_refused():
    """Refused on the host, before anything is enqueued (no device needed)."""
    n = 400_000
    lo = np.arange(n, dtype=np.uint64) * 4096 + (1 << 40)
    hi = lo + 1024
    with pytest.raises(_lib.FoundryError, match="FDY_E_CAPACITY"):
        relocate_words_static(lo, hi, lo + (1 << 30), 0, 0, 0)


@pytest.mark.gpu
def test_static_relocation_matches_the_plan(cuda):
    torch = cuda
    cases = [(1 << 20, 60_000, 0x51A7), (100_001, 300, 0x51A8)]  # second: smaller table and odd length
    for n_words, n_iv, seed in cases:
        print(f"[case] static relocation words={n_words} intervals={n_iv}", flush=True)
        words, (lo, hi, nlo) = _case(n_words, n_iv, seed)
        for policy in (0, 1):
            d_in = torch.from_numpy(words.view(np.int64)).to("cuda")
            d_plan = torch.empty_like(d_in)
            d_static = torch.full_like(d_in, -1)
            plan = RelocPlan(lo, hi, nlo, policy)
            plan.relocate(d_in.data_ptr(), d_plan.data_ptr(), n_words)
            relocate_words_static(lo, hi, nlo, d_in.data_ptr(), d_static.data_ptr(), n_words, policy)
            torch.cuda.synchronize()
            plan.close()
            want = d_plan.cpu().numpy()
            np.testing.assert_array_equal(d_static.cpu().numpy(), want)
            # in place, on the current stream
            relocate_words_static(lo, hi, nlo, d_in.data_ptr(), d_in.data_ptr(), n_words, policy,
                                  torch.cuda.current_stream())
            torch.cuda.synchronize()
            np.testing.assert_array_equal(d_in.cpu().numpy(), want)
            assert (want != words.view(np.int64)).any()  # the table moved some words
