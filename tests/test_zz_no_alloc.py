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


@pytest.mark.gpu
def test_static_relocation_allocates_no_device_memory(cuda):
    """After a first call on the device, further calls (the same table, a
    smaller one, then the first again) leave the device's free memory and
    torch's allocation counts exactly as they were, and each call's words
    equal the plan's."""
    torch = cuda
    big_words, big_iv = _case(1 << 18, 20_000, 0x51A9)
    small_words, small_iv = _case(50_001, 700, 0x51AA)
    d_big = torch.from_numpy(big_words.view(np.int64)).to("cuda")
    d_small = torch.from_numpy(small_words.view(np.int64)).to("cuda")
    want = {}
    for name, d, (lo, hi, nlo), n in (("big", d_big, big_iv, len(big_words)),
                                      ("small", d_small, small_iv, len(small_words))):
        out = torch.empty_like(d)
        plan = RelocPlan(lo, hi, nlo, 0)
        plan.relocate(d.data_ptr(), out.data_ptr(), n)
        torch.cuda.synchronize()
        plan.close()
        want[name] = out.cpu().numpy()
    out_big = torch.full_like(d_big, -1)
    out_small = torch.full_like(d_small, -1)
    relocate_words_static(*big_iv, d_big.data_ptr(), out_big.data_ptr(), len(big_words), 0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out_big.cpu().numpy(), want["big"])
    free0 = torch.cuda.mem_get_info()[0]

    def requests():  # torch's cumulative counts of device allocation requests and segments
        return {k: v for k, v in torch.cuda.memory_stats().items()
                if k.startswith(("allocation.", "segment.")) and k.endswith(".allocated")}

    stats0 = requests()
    for name, d, dst, iv, n in (("big", d_big, out_big, big_iv, len(big_words)),
                                ("small", d_small, out_small, small_iv, len(small_words)),
                                ("big", d_big, out_big, big_iv, len(big_words))):
        print(f"[case] static relocation, {name} table again: words={n} intervals={len(iv[0])}", flush=True)
        dst.fill_(-1)
        relocate_words_static(*iv, d.data_ptr(), dst.data_ptr(), n, 0)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, "device free memory changed"
        assert requests() == stats0, "torch allocated device memory"
        np.testing.assert_array_equal(dst.cpu().numpy(), want[name])
