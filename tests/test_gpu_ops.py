"""The reference's LOAD API end to end on the GPU (foundry_amd.ops /
foundry_amd.api): archives saved against an allocation region at the
reference's default base, loaded in a process where the MI355X cannot map
that base -- so the region moves, the restore relocates every saved pointer,
the allocator events map the graphs' buffer at its new address, and the
output tensors are views there.

SAVE is simulated with a planning region (placement arithmetic only).  Every
pointer a replay dereferences is compared with the relocated buffer before
the first replay."""
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

SAVED_BASE = 0x500000000000  # the reference's default base; unmappable on MI355X
SIZE = 1 << 30
WEIGHTS = 5 * MiB            # allocated before capture, on SAVE and on LOAD alike
SPECS = [dict(a=100 + g, b=7, v=0x01010101 * (g + 1)) for g in range(4)]


def _save(dirpath, bhash):
    plan = Region.plan(SAVED_BASE, SAVED_BASE, SIZE)
    plan.alloc(WEIGHTS)
    paths, out = [], None
    for g, sp in enumerate(SPECS):
        plan.clear_events()
        plan.record(True)
        if g == 0:
            out = plan.alloc(GC.BUF_BYTES)  # the first capture allocates the output buffer
        events = plan.events_json().encode()
        plan.record(False)
        outputs = json.dumps({"type": 1, "tensors": [{
            "data_ptr": out, "sizes": [16], "strides": [1], "dtype": 4, "device_type": 1, "device_index": 0,
            "requires_grad": False, "numel": 16, "element_size": 8}]}).encode()
        nodes = [
            W.Kernel("probe_mix", bhash, grid=(2, 1, 1), block=(64, 1, 1),
                     params=[le(out), le(0, 4), le(GC.CAP, 4), le(sp["a"]), le(sp["b"])]),
            W.Memset(dst=out + GC.FILL_OFF, value=sp["v"], width=32, element_size=4),
            W.Kernel("probe_chain", bhash, params=[le(out), le(1, 4), le(GC.CAP, 4), le(0, 4)]),
        ]
        stem = os.path.join(dirpath, f"graph_{g}_bs{g + 1}")
        with open(stem + ".cugraph", "wb") as f:
            f.write(W.write(nodes, [(0, 2)], alloc_events=events, output_tensors=outputs))
        paths.append(stem + ".json")
    api.save_graph_manifest(dirpath)
    return paths, out


@pytest.fixture()
def loaded(tmp_path):
    torch.cuda.set_device(0)
    assert api.load_cuda_modules_and_libraries(os.path.dirname(GC.PROBE_CO)) >= 1
    bhash = ops.registry().add_file(GC.PROBE_CO)
    paths, saved_out = _save(str(tmp_path), bhash)
    api.set_allocation_region(SAVED_BASE, SIZE)
    region = ops._region()
    info = region.info()
    assert info["base"] != SAVED_BASE and info["saved_base"] == SAVED_BASE
    weights = ops.region_alloc(WEIGHTS)  # the model's allocations come first, as on SAVE
    assert weights == info["base"]
    pending = api.CUDAGraph.start_graph_builds(paths)
    yield pending, saved_out - SAVED_BASE + info["base"]
    pending.close()
    ops.release_allocation_region()


def test_load_relocates_replays_and_outputs(loaded):
    pending, out = loaded
    assert pending.used_manifest
    assert list(pending.template_of) == [0, 0, 0, 0]
    for g in range(4):  # pointer check before anything runs
        img = [int(x) for x in pending.archive.param_image(g)]
        ptrs = [int(x) for x in pending.archive.node_pointers(g)]
        assert img[0] == out and img[5] == out and ptrs[2] == out + GC.FILL_OFF
    results = api.CUDAGraph.finish_graph_loads(pending)
    assert ops._region().info()["live_allocations"] == 2  # weights + the replayed buffer
    outs = [o for _, o in results]
    assert outs[0].data_ptr() == out and outs[0].shape == (16,) and outs[0].dtype == torch.int64
    whole = ops.tensor_at(out, [GC.BUF_BYTES // 8], [1], torch.int64)
    for g in [0, 1, 2, 3, 0, 2, 3]:
        whole.zero_()
        results[g][0].replay()
        torch.cuda.synchronize()
        sp = SPECS[g]
        r0 = GC.mix_expect(sp["a"], sp["b"], 2, 64)
        got = outs[g].cpu().numpy().view(np.uint64)
        assert int(got[0]) == r0 and int(got[1]) == GC.mix(r0, 1), g
        fill = whole.cpu().numpy().view(np.uint64).tobytes()[GC.FILL_OFF:GC.FILL_OFF + 128]
        assert fill == le(sp["v"], 4) * 32, g
    del whole, outs, results


def test_pack_and_reload_through_ops(loaded, tmp_path):
    """pack_fatbins_to_folder writes the process registry's code objects as
    the packed pair; load_cuda_modules_and_libraries reads the pair back."""
    ops.pack_fatbins_to_folder(str(tmp_path))
    assert (tmp_path / "fatbin_image_packed.img").stat().st_size > 16
    records = (tmp_path / "fatbin_entrypoint_packed.txt").read_text().count("---\n")
    assert records >= 1
    assert api.load_cuda_modules_and_libraries(str(tmp_path)) == records


def test_finish_one_out_of_range(loaded):
    pending, _ = loaded
    with pytest.raises(IndexError):
        api.CUDAGraph.finish_one_graph_load(pending, 4)


def test_debug_dump_and_raw_handles(loaded, tmp_path):
    pending, _ = loaded
    results = api.CUDAGraph.finish_graph_loads(pending)
    g1 = results[1][0]
    with pytest.warns(UserWarning, match="debug not enabled"):
        g1.debug_dump(str(tmp_path / "no.dot"))
    assert not (tmp_path / "no.dot").exists()
    g1.enable_debug_mode()
    g1.debug_dump(str(tmp_path / "g1.dot"))
    dot = (tmp_path / "g1.dot").read_text()
    assert "digraph" in dot
    exec_handle = g1.raw_cuda_graph_exec()
    assert exec_handle != 0 and exec_handle == results[2][0].raw_cuda_graph_exec()  # one exec per group
    with pytest.raises(RuntimeError, match="keep_graph"):
        g1.raw_cuda_graph()
    assert g1.pool() == (0, 0)
    assert ops.get_graph_ptr(g1) == ops.get_graph_ptr(g1) != ops.get_graph_ptr(results[2][0])
