"""Graphs saved as JSON documents alone: opening their .json paths finds no
valid .cugraph beside them and reads each document instead, as the
reference's load does (csrc/CUDAGraphParallel.cpp:1586-1617).  The restore
of such an archive is held to the oracle's restore of the archives the
oracle's writer makes from the same documents, and to the restore of the
same graphs opened from their .cugraph files."""
import json
import random

import numpy as np
import pytest

import cugraph_writer as W
from graph_json import doc_of, sample_nodes
from oracle import Restore
from oracle import writer as OW
from foundry_amd.restore import Archive, save_binary
from parity import assert_restore_parity

pytestmark = pytest.mark.gpu


def _documents(seed: int, count: int) -> list[str]:
    """`count` graphs of one topology: graph g > 0 changes a few param bytes."""
    rng = random.Random(seed)
    nodes = sample_nodes(rng, 48)
    texts = []
    for g in range(count):
        gnodes = []
        for n in nodes:
            if n.type == 0 and n.params and g:
                params = [bytes(b ^ (rng.randrange(256) if rng.random() < 0.1 else 0) for b in p) for p in n.params]
                n = W.Kernel(n.name, n.binary_hash, n.grid, n.block, params, n.arg, n.shmem, n.cluster, n.cooperative,
                             n.func_attrs, n.kna_ints)
            gnodes.append(n)
        texts.append(json.dumps(doc_of(gnodes, [(i, i + 1) for i in range(len(gnodes) - 1)],
                                       {"start_base_addr": 0, "events": []}, {"type": 0, "tensors": []})))
    return texts


def test_json_only_graphs_restore(tmp_path):
    texts = _documents(3, 6)
    bdir, jdir = tmp_path / "bin", tmp_path / "json"
    bdir.mkdir()
    jdir.mkdir()
    for i, t in enumerate(texts):
        save_binary(str(bdir / f"graph_{i}.cugraph"), t)
        (jdir / f"graph_{i}.json").write_text(t)
    # a .cugraph that is not a v1 archive is passed over for the document too
    (jdir / "graph_2.cugraph").write_bytes(b"NOTAGRPH" + bytes(120))
    print("json-only archive: 6 graphs x 48 nodes", flush=True)
    from_json = Archive.open([str(jdir / f"graph_{i}.json") for i in range(len(texts))])
    from_bin = Archive.open([str(bdir / f"graph_{i}.json") for i in range(len(texts))])
    from_json.restore()
    from_bin.restore()
    ref = Restore([OW.load_archive(t) for t in texts], None)
    assert_restore_parity(from_json, ref)
    for g in range(len(texts)):
        np.testing.assert_array_equal(from_json.param_image(g), from_bin.param_image(g))
        np.testing.assert_array_equal(from_json.overrides(g), from_bin.overrides(g))
    assert from_json.section(0, 8) == b'{"start_base_addr":0,"events":[]}'


def test_keyless_json_graphs_group_by_recomputed_keys(tmp_path):
    """JSON documents without a topology_key (or with an empty one) group by
    the key recomputed from their nodes (csrc/CUDAGraphParallel.cpp:
    1796-1840), not all under one empty key."""
    rng = random.Random(11)
    base = sample_nodes(rng, 30)
    alt = list(base)
    k = next(i for i, n in enumerate(alt) if n.type == 0)
    n0 = alt[k]
    alt[k] = W.Kernel(n0.name, n0.binary_hash, n0.grid, n0.block, n0.params, n0.arg, n0.shmem, (4, 1, 1),
                      n0.cooperative, n0.func_attrs, n0.kna_ints)
    short = sample_nodes(rng, 20)
    order = [base, alt, base, short, alt, base, short]
    texts = []
    for g, nodes in enumerate(order):
        d = doc_of(nodes, [], {"start_base_addr": 0, "events": []})
        if g % 2:
            d["topology_key"] = ""
        else:
            del d["topology_key"]
        texts.append(json.dumps(d))
    for i, t in enumerate(texts):
        (tmp_path / f"graph_{i}.json").write_text(t)
    keys = [OW.load_topology_key(t) for t in texts]
    assert len(set(keys)) == 3 and b"" not in keys
    print("key-less json archive: 7 graphs, 3 recomputed keys", flush=True)
    arch = Archive.open([str(tmp_path / f"graph_{i}.json") for i in range(len(texts))])
    try:
        arch.restore()
        assert arch.groups().tolist() == [0, 1, 0, 3, 1, 0, 3]
        for g in range(len(texts)):
            assert arch.section(g, 10) == keys[g]
        assert_restore_parity(arch, Restore([OW.load_archive(t) for t in texts], None))
    finally:
        arch.close()
