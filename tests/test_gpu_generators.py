"""Generator state on LOAD (row A11): graphs saved with a GENERATORS section
register their states in finish_one_graph_load before the allocator replay
(csrc/CUDAGraphParallel.cpp:2048-2059), so the state's seed and offset words
land where the saved kernel params point, and every replay runs the
replay prologue first (csrc/CUDAGraph.cpp:469-472, 79-86): seed and offset
written, offset advanced by the increment rounded up to 4.

SAVE is simulated with a planning region at the reference's default base
(which MI355X cannot map, so LOAD relocates).  The captured kernel,
probe_rng, writes *seed and *offset + its intragraph offset into the
output buffer."""
import json
import os

import numpy as np
import pytest
import torch

import cugraph_writer as W
import graph_cases as GC
from cugraph_writer import le
from foundry_amd import api, ops
from foundry_amd.region import MiB, Region

pytestmark = pytest.mark.gpu

SAVED_BASE = 0x500000000000
SIZE = 1 << 30
WEIGHTS = 3 * MiB
STATE_ID = 0x6E7E0001  # an id no other test registers (the registry is process-wide)
SEED = 0xF00DF00DCAFEBABE  # above 2^63: the words hold int64_t(seed)
INCREMENTS = [10, 20, 0, 7]  # graph 2 captured no random numbers of this state


def _save(dirpath, bhash):
    plan = Region.plan(SAVED_BASE, SAVED_BASE, SIZE)
    plan.alloc(WEIGHTS)
    # The state registers before the first capture: its segment is not an
    # allocator event of any graph.
    gen = plan.alloc(2 * MiB)
    paths, out = [], None
    for g, inc in enumerate(INCREMENTS):
        plan.clear_events()
        plan.record(True)
        if g == 0:
            out = plan.alloc(GC.BUF_BYTES)
        events = plan.events_json().encode()
        plan.record(False)
        outputs = json.dumps({"type": 1, "tensors": [{
            "data_ptr": out, "sizes": [16], "strides": [1], "dtype": 4, "device_type": 1, "device_index": 0,
            "requires_grad": False, "numel": 16, "element_size": 8}]}).encode()
        nodes = [W.Kernel("probe_rng", bhash, params=[le(out), le(0, 4), le(GC.CAP, 4), le(gen), le(gen + 512),
                                                      le(16 * g, 4)])]
        stem = os.path.join(dirpath, f"graph_{g}_bs{g + 1}")
        with open(stem + ".cugraph", "wb") as f:
            f.write(W.write(nodes, alloc_events=events, output_tensors=outputs,
                            generators=[(STATE_ID, SEED, inc)]))
        paths.append(stem + ".json")
    return paths, gen - SAVED_BASE


def _expected(order):
    """(seed word, offset word + intragraph) per replay, from the prologue's
    rules: no write when the increment is 0, else write then advance by the
    increment rounded up to a multiple of 4."""
    words, offset, out = None, 0, []
    for g in order:
        inc = INCREMENTS[g]
        if inc:
            words = (SEED, offset)
            offset += (inc + 3) // 4 * 4
        out.append((words[0], words[1] + 16 * g))
    return out


def test_generator_state_registered_and_advanced(tmp_path):
    torch.cuda.set_device(0)
    bhash = ops.registry().add_file(GC.PROBE_CO)
    paths, gen_offset = _save(str(tmp_path), bhash)
    api.set_allocation_region(SAVED_BASE, SIZE)
    try:
        info = ops._region().info()
        assert info["base"] != SAVED_BASE
        ops.region_alloc(WEIGHTS)
        pending = api.CUDAGraph.start_graph_builds(paths)
        try:
            print("[case] 4 graphs with one generator state, 7 replays", flush=True)
            results = api.CUDAGraph.finish_graph_loads(pending)
            state = ops.global_generator_state_registry.get_state_from_id(STATE_ID, 0)
            assert state.seed == SEED
            # registered before the allocator replay: at SAVE's region offset,
            # where the relocated kernel params point (words 3 and 4: the
            # params out, idx, cap, seed, offset, intragraph, each padded to 8 B)
            assert state.seed_ptr == info["base"] + gen_offset and state.offset_ptr == state.seed_ptr + 512
            img = [int(x) for x in pending.archive.param_image(0)]
            assert img[3] == state.seed_ptr and img[4] == state.offset_ptr
            out = results[0][1]
            order = [0, 1, 0, 2, 3, 3, 1]
            got = []
            for g in order:
                out.zero_()
                results[g][0].replay()
                torch.cuda.synchronize()
                v = out.cpu().numpy().view(np.uint64)
                got.append((int(v[0]), int(v[1])))
            assert got == _expected(order)
            assert state.philox_offset_per_thread == 80
        finally:
            pending.close()
    finally:
        ops.release_allocation_region()
