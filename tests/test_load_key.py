"""The key a graph read from its JSON document is grouped by
(csrc/CUDAGraphParallel.cpp:1791-1841): the product (fdy_load_topology_key,
no device) and the oracle's restatement (oracle/writer.py) against keys
written out by hand from those lines, then against each other on random
documents."""
import json
import random

import pytest

import cugraph_writer as W
from foundry_amd import _lib
from foundry_amd.restore import load_topology_key
from graph_json import doc_of, sample_nodes
from oracle import writer as OW


def kernel(kna=None, func_attrs=None):
    p = {"blockDimX": 1, "blockDimY": 1, "blockDimZ": 1, "gridDimX": 1, "gridDimY": 1, "gridDimZ": 1,
         "sharedMemBytes": 0, "function_name": "f", "kernel_source_binary_hash": 1, "kernelParams": [],
         "extra_argBuffer_hex": ""}
    if kna is not None:
        p["kernel_node_attrs"] = kna
    if func_attrs is not None:
        p["func_attrs"] = func_attrs
    return {"id": 0, "type": "KernelNode", "params": p}


def doc(nodes, **kw):
    d = {"nodes": nodes, "generators": []}
    d.update(kw)
    return json.dumps(d)


def cluster(x, y, z):
    return {"clusterDimX": x, "clusterDimY": y, "clusterDimZ": z}


HAND = [
    # no topology_key: recomputed from the nodes
    (doc([kernel(kna=cluster(2, 1, 1)), {"id": 1, "type": "MemsetNode", "params": {}},
          kernel(func_attrs={"required_cluster_width": 0, "required_cluster_height": 3}),
          kernel(kna=cluster(0, 5, 1), func_attrs={"required_cluster_width": 0}),
          {"id": 4, "type": "FooNode", "params": {}}, kernel()]),
     b"KernelNode:C2_1_1,MemsetNode,KernelNode:C0_3_0,KernelNode:C0_5_1,FooNode,KernelNode:0"),
    # an empty topology_key is recomputed too; common attrs fill x == 0
    (doc([kernel(), kernel(kna=cluster(8, 1, 1)), {"id": 2, "type": "EventRecordNode", "params": {"event_id": 0}},
          kernel(kna={"cooperative": 1}, func_attrs={"required_cluster_depth": 7})],
         topology_key="", common_kernel_node_attrs=cluster(4, 1, 2)),
     b"KernelNode:C4_1_2,KernelNode:C8_1_1,EventRecordNode,KernelNode:C4_1_2"),
    # common attrs without clusterDimX leave the required dims in charge
    (doc([kernel(func_attrs={"required_cluster_depth": 7})], common_kernel_node_attrs={"priority": 1}),
     b"KernelNode:C0_0_7"),
    # a saved key is used as it stands
    (doc([kernel()], topology_key="custom key"), b"custom key"),
    (doc([]), b""),
]


@pytest.mark.parametrize("i", range(len(HAND)))
def test_hand_written_keys(i):
    text, want = HAND[i]
    assert OW.load_topology_key(text) == want
    assert load_topology_key(text) == want


@pytest.mark.parametrize("bad", [
    doc([kernel(kna=cluster(-1, 1, 1))]),          # to_number<unsigned int> throws
    doc([kernel(kna={"clusterDimX": 2})]),           # clusterDimY missing
    doc([{"id": 0, "params": {}}]),                  # no type
    doc([kernel()], topology_key=5),                 # not a string
])
def test_documents_the_reference_cannot_key(bad):
    with pytest.raises(OW.WriterError):
        OW.load_topology_key(bad)
    with pytest.raises(_lib.FoundryError, match="FDY_E_FORMAT"):
        load_topology_key(bad)


@pytest.mark.parametrize("seed", range(8))
def test_random_documents(seed):
    rng = random.Random(seed)
    nodes = sample_nodes(rng, rng.randrange(0, 40))
    common = rng.choice([None, (4, 1, 1), (0, 2, 1)])
    d = doc_of(nodes, [], common=common)
    if rng.random() < 0.7:
        d["topology_key"] = rng.choice(["", d["topology_key"]])
        if rng.random() < 0.5:
            del d["topology_key"]
    text = json.dumps(d)
    assert load_topology_key(text) == OW.load_topology_key(text)
    # the archive the product restores such a graph from carries that key
    from tests import cugraph_reader as R
    assert R.read(OW.load_archive(text)).key() == OW.load_topology_key(text)
