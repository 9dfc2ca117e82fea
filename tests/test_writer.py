"""The .cugraph writer: the archive CUDAGraph::save_binary writes for one
graph's JSON document (csrc/BinaryGraphIO.cpp:15-371).

The oracle (oracle/writer.py) is pinned against the test-side writer
(tests/cugraph_writer.py, written from the packed structs of
include/BinaryGraphFormat.h and sharing no code with either), against the
test-side reader, and against the closed-form layout; the product
(fdy_cugraph_from_json) is then held to the oracle byte for byte on seeded
documents, and on the documents either must refuse.  No device needed.
"""
from __future__ import annotations

import json
import os
import random
import struct

import pytest

import cugraph_reader as R
import cugraph_writer as W
from graph_json import compact, doc_of, sample_nodes
from foundry_amd import restore
from foundry_amd._lib import FoundryError
from oracle import writer as OW

FDY_E_FORMAT, FDY_E_UNSUPPORTED = -3, -11


# ---- the oracle, pinned ---------------------------------------------------------

@pytest.mark.parametrize("seed", range(12))
def test_oracle_matches_test_writer(seed):
    rng = random.Random(seed)
    nodes = sample_nodes(rng, rng.randrange(1, 40))
    deps = [(i, i + 1) for i in range(len(nodes) - 1)] if seed % 3 else []
    alloc = {"start_base_addr": 0x7F0000000000, "events": [{"alloc": 4096, "ptr": 0x7F0000200000}]}
    outputs = {"type": 1, "tensors": [{"data_ptr": 0x7F0000200000, "sizes": [2, 3], "strides": [3, 1], "dtype": 15,
                                       "device_type": 1, "device_index": 0, "requires_grad": False, "numel": 6,
                                       "element_size": 2}]}
    common = (2, 1, 1) if seed % 4 == 1 else None
    doc = doc_of(nodes, deps, alloc if seed % 2 else None, outputs if seed % 2 else None, common)
    want = W.write(nodes, deps, alloc_events=compact(alloc) if seed % 2 else b"",
                   output_tensors=compact(outputs) if seed % 2 else b"", common_cluster=common,
                   common_ints=(0, 0, 0, 0))
    assert OW.save_binary(json.dumps(doc)) == want


def test_oracle_layout_closed_form():
    """Header counts and flags, and section i at the 8-aligned running offset."""
    rng = random.Random(7)
    nodes = sample_nodes(rng, 30)
    doc = doc_of(nodes, [(0, 1), (1, 2)], {"events": []}, {"type": 0, "tensors": []})
    doc["generators"] = [{"id": 3, "seed": 99, "wholegraph_increment": 4}]
    img = OW.save_binary(json.dumps(doc))
    magic, ver, flags, nn, nd, ng, ns, nstr = struct.unpack_from("<8s7I", img, 0)
    assert (magic, ver, nn, nd, ng, ns) == (b"CUGRAPH\0", 1, 30, 2, 1, 11)
    assert flags == 2 | 4 | 8 | 16
    assert nstr == len({n.name for n in nodes if n.type == 0})
    off = 64 + 11 * 24
    for i in range(11):
        sid, pad, o, size = struct.unpack_from("<IIQQ", img, 64 + 24 * i)
        assert (sid, pad, o) == (i, 0, off)
        off += size + (-size % 8)
    assert off == len(img)
    sec = {i: struct.unpack_from("<QQ", img, 64 + 24 * i + 8) for i in range(11)}
    o, size = sec[7]
    assert img[o:o + size] == struct.pack("<3Q", 3, 99, 4)
    o, size = sec[8]
    assert img[o:o + size] == b'{"events":[]}'


def test_oracle_fields_through_reader():
    """The test-side reader sees every kernel's launch config, name, hash and param bytes."""
    rng = random.Random(11)
    nodes = sample_nodes(rng, 40)
    arc = R.read(OW.save_binary(json.dumps(doc_of(nodes, []))))
    for i, n in enumerate(nodes):
        assert arc.nodes[i].type == n.type and arc.nodes[i].node_id == i
        if n.type == 0:
            k = arc.nodes[i].kernel
            assert (k.block, k.grid, k.shmem, k.binary_hash, k.name) == (n.block, n.grid, n.shmem, n.binary_hash,
                                                                         n.name.encode())
            assert arc.param_bytes(i) == ([n.arg] if n.arg is not None else n.params)


def test_oracle_quirks():
    """Reference behaviours a restatement could plausibly get wrong."""
    base = {"nodes": [], "generators": []}
    # an unknown node type leaves a zero kernel entry with the id
    img = OW.save_binary(json.dumps({**base, "nodes": [{"id": 9, "type": "ConditionalNode"}]}))
    e = img[64 + 264 + 0:]
    arc = R.read(img)
    assert arc.nodes[0].node_id == 9 and arc.nodes[0].type == 0 and arc.nodes[0].raw[8:] == bytes(160)
    del e
    # odd-length hex: size is len // 2 but the final character still becomes a byte
    k = {"id": 0, "type": "KernelNode", "params": {
        "blockDimX": 1, "blockDimY": 1, "blockDimZ": 1, "gridDimX": 1, "gridDimY": 1, "gridDimZ": 1,
        "sharedMemBytes": 0, "function_name": "f", "kernel_source_binary_hash": 1,
        "kernelParams": [{"value_hex": "abc"}, {"value_hex": "0d"}]}}
    arc = R.read(OW.save_binary(json.dumps({**base, "nodes": [k]})))
    assert arc.nodes[0].kernel.params == [("PDATA", 0, 1), ("PDATA", 2, 1)]
    assert arc.section("PDATA") == b"\xab\x0c\x0d"
    # strtoul pairs: leading space, sign, trailing junk
    assert OW.hex_decode(b" 1-1+f1g") == bytes([1, 0xFF, 15, 1])
    with pytest.raises(OW.WriterError):
        OW.hex_decode(b"zz")
    # func_attrs optional members default to 0; metadata-only params keep offset/size
    k["params"]["func_attrs"] = {"max_dynamic_shared_size_bytes": 5, "preferred_shared_memory_carveout": -1}
    k["params"]["kernelParams"] = [{"offset": 16, "size": 8}]
    arc = R.read(OW.save_binary(json.dumps({**base, "nodes": [k]})))
    assert arc.nodes[0].kernel.func_attrs == (5, -1, 0, 0, 0, 0)
    assert arc.nodes[0].kernel.params == [("PDATA", 16, 8)]
    # "dependencies": [] sets no flag; a present but empty extra buffer is "none"
    img = OW.save_binary(json.dumps({**base, "dependencies": []}))
    assert struct.unpack_from("<I", img, 12)[0] == 0


# ---- the product against the oracle --------------------------------------------

def product(text) -> bytes:
    return restore.cugraph_from_json(text)


def random_value(rng: random.Random, depth: int = 0, floats: bool = False):
    r = rng.random()
    if depth > 3 or r < 0.3:
        return rng.choice([0, -1, 1 << 63, (1 << 64) - 1, -(1 << 63), rng.getrandbits(40), True, False, None])
    if r < 0.5:
        alphabet = ['a', 'Z', '"', '\\', '/', '\n', '\t', '\x01', '\x1f', '\x7f', 'é', '€', '😀', ' ']
        return "".join(rng.choice(alphabet) for _ in range(rng.randrange(0, 8)))
    if floats and r < 0.55:
        return 1.5
    if r < 0.75:
        return [random_value(rng, depth + 1, floats) for _ in range(rng.randrange(0, 4))]
    suffixes = ["", "é", '"']
    return {"k%d%s" % (i, rng.choice(suffixes)): random_value(rng, depth + 1, floats) for i in range(rng.randrange(0, 4))}


def random_num(rng: random.Random, v: int):
    """The integer v, sometimes written as a whole float."""
    return float(v) if rng.random() < 0.05 and abs(v) < (1 << 52) else v


def random_kna(rng: random.Random) -> dict:
    o = {}
    if rng.random() < 0.3:
        o["attrQueryAvailable"] = rng.random() < 0.5
    if rng.random() < 0.3:
        o.update(clusterDimX=rng.randrange(0, 9), clusterDimY=rng.randrange(0, 3), clusterDimZ=1)
    if rng.random() < 0.2:
        o.update(preferredClusterDimX=4, preferredClusterDimY=rng.randrange(0, 3), preferredClusterDimZ=1)
    for key in ("clusterSchedulingPolicyPreference", "cooperative", "priority", "memSyncDomain"):
        if rng.random() < 0.2:
            o[key] = rng.randrange(-3, 3)
    if rng.random() < 0.2:
        o.update(memSyncDomainMapDefault=rng.randrange(-300, 300), memSyncDomainMapRemote=rng.randrange(0, 300))
    if rng.random() < 0.2:
        o["preferredSharedMemCarveout"] = rng.randrange(0, 101)
    return o


def random_doc(rng: random.Random) -> dict:
    nodes = []
    for i in range(rng.randrange(0, 25)):
        t = rng.choice(["KernelNode"] * 4 + ["MemsetNode", "MemcpyNode", "EventRecordNode", "EventWaitNode",
                                              "EmptyNode", "ConditionalNode"])
        nid = rng.choice([i, rng.getrandbits(32)])
        if t == "KernelNode":
            p = {k: random_num(rng, rng.randrange(0, 1 << 10)) for k in
                 ("blockDimX", "blockDimY", "blockDimZ", "gridDimX", "gridDimY", "gridDimZ", "sharedMemBytes")}
            p["function_name"] = rng.choice(["k0", "k1", "kernel_é", "k0", ""])
            p["kernel_source_binary_hash"] = rng.getrandbits(64)
            if rng.random() < 0.7:
                fa = {"max_dynamic_shared_size_bytes": rng.randrange(-5, 1 << 16),
                      "preferred_shared_memory_carveout": rng.randrange(-1, 101)}
                for key in ("cluster_scheduling_policy_preference", "required_cluster_width",
                            "required_cluster_height", "required_cluster_depth"):
                    if rng.random() < 0.5:
                        fa[key] = rng.randrange(0, 4)
                p["func_attrs"] = fa
            if rng.random() < 0.5:
                p["kernel_node_attrs"] = random_kna(rng)
            kps = []
            for j in range(rng.randrange(0, 6)):
                if rng.random() < 0.8:
                    n = rng.randrange(0, 24)
                    h = bytes(rng.randrange(256) for _ in range(n)).hex()
                    if rng.random() < 0.1:
                        h += rng.choice("0123456789abcdefABCDEF")
                    if rng.random() < 0.1 and h:
                        k = rng.randrange(len(h))
                        h = h[:k] + rng.choice(" +-g") + h[k + 1:]
                    kps.append({"index": j, "offset": 0, "size": n, "value_hex": h})
                else:
                    kps.append({"index": j, "offset": rng.randrange(0, 1 << 12), "size": rng.randrange(0, 64)})
            p["kernelParams"] = kps
            if rng.random() < 0.8:
                p["extra_argBuffer_hex"] = bytes(rng.randrange(256) for _ in range(rng.choice([0, 0, 16, 33]))).hex()
            nodes.append({"id": nid, "type": t, "params": p})
        elif t == "MemsetNode":
            nodes.append({"id": nid, "type": t, "params": {
                "dst": rng.getrandbits(64), "elementSize": rng.choice([1, 2, 4]), "height": rng.randrange(1, 9),
                "pitch": rng.getrandbits(20), "value": rng.getrandbits(32), "width": rng.getrandbits(30)}})
        elif t == "MemcpyNode":
            p = {k: rng.getrandbits(rng.choice([8, 48, 64])) for k in
                 ("Depth", "Height", "WidthInBytes", "dstDevice", "dstHeight", "dstLOD", "dstPitch", "dstXInBytes",
                  "dstY", "dstZ", "srcDevice", "srcHeight", "srcLOD", "srcPitch", "srcXInBytes", "srcY", "srcZ")}
            p["dstMemoryType"] = rng.randrange(-2, 5)
            p["srcMemoryType"] = rng.randrange(-2, 5)
            nodes.append({"id": nid, "type": t, "params": p})
        elif t in ("EventRecordNode", "EventWaitNode"):
            nodes.append({"id": nid, "type": t, "params": {"event_id": rng.randrange(-(1 << 31), 1 << 31)}})
        else:
            nodes.append({"id": nid, "type": t, "params": {}})
    doc = {"nodes": nodes, "generators": [
        {"id": rng.getrandbits(64), "seed": rng.getrandbits(64), "wholegraph_increment": rng.getrandbits(64)}
        for _ in range(rng.randrange(0, 3))]}
    if rng.random() < 0.8:
        doc["dependencies"] = [{"from": rng.getrandbits(32), "to": rng.getrandbits(32)} for _ in range(rng.randrange(0, 6))]
    if rng.random() < 0.8:
        doc["allocator_events"] = random_value(rng)
    if rng.random() < 0.8:
        doc["output_tensors"] = random_value(rng)
    if rng.random() < 0.8:
        doc["topology_key"] = ",".join(n["type"] for n in nodes) + rng.choice(["", "é"])
    if rng.random() < 0.2:
        doc["common_kernel_node_attrs"] = random_kna(rng)
    keys = list(doc)
    rng.shuffle(keys)
    return {k: doc[k] for k in keys}


def outcome(fn, text):
    try:
        return "ok", fn(text)
    except OW.Unsupported:
        return "unsupported", None
    except OW.WriterError:
        return "format", None
    except FoundryError as e:
        return {FDY_E_FORMAT: "format", FDY_E_UNSUPPORTED: "unsupported"}.get(e.code, e.code), None


@pytest.mark.parametrize("seed", range(8))
def test_product_matches_oracle(seed):
    rng = random.Random(1000 + seed)
    for _ in range(60):
        doc = random_doc(rng)
        text = json.dumps(doc, ensure_ascii=rng.random() < 0.5, indent=rng.choice([None, None, 1]))
        po, pv = outcome(product, text)
        oo, ov = outcome(OW.save_binary, text)
        assert po == oo, (po, oo, text[:300])
        assert pv == ov


def mutate(rng: random.Random, doc: dict) -> dict:
    """One change the reference's serialiser rejects, or one it accepts."""
    d = json.loads(json.dumps(doc))
    kernels = [n for n in d["nodes"] if n["type"] == "KernelNode"]
    choice = rng.randrange(9)
    if choice == 0 and kernels:
        del kernels[0]["params"][rng.choice(["blockDimX", "function_name", "kernelParams", "gridDimZ"])]
    elif choice == 1 and kernels:
        kernels[0]["params"]["blockDimX"] = rng.choice([-1, 1 << 32, 2.5, "64", None, True])
    elif choice == 2:
        d["nodes"].append({"id": -1, "type": "EmptyNode"})
    elif choice == 3:
        del d["generators"]
    elif choice == 4 and kernels:
        kernels[0]["params"]["kernelParams"] = [{"value_hex": "zz"}]
    elif choice == 5:
        d["allocator_events"] = {"a": [1, 2.0]}
    elif choice == 6 and kernels:
        kernels[0]["params"]["kernel_node_attrs"] = {"memSyncDomainMapDefault": 1}
    elif choice == 7:
        d["nodes"].append({"id": 1, "type": "MemsetNode", "params": {"dst": 0}})
    elif choice == 8:
        d["topology_key"] = 5
    return d


@pytest.mark.parametrize("seed", range(4))
def test_product_matches_oracle_on_refusals(seed):
    rng = random.Random(2000 + seed)
    seen = set()
    for _ in range(80):
        text = json.dumps(mutate(rng, random_doc(rng)))
        po, pv = outcome(product, text)
        oo, ov = outcome(OW.save_binary, text)
        assert po == oo, (po, oo, text[:300])
        assert pv == ov
        seen.add(po)
    assert {"format", "unsupported", "ok"} <= seen


@pytest.mark.parametrize("text", [
    b'{"nodes": [], "generators": [], "nodes": []}',            # duplicate key
    b'{"nodes": [], "generators": [01]}',                         # leading zero
    b'{"nodes": [], "generators": [], "topology_key": "\\ud800"}',  # lone surrogate
    b'{"nodes": [], "generators": [], "topology_key": "\xff"}',   # not UTF-8
    b'\xef\xbb\xbf{"nodes": [], "generators": []}',              # byte-order mark
    b'{"nodes": [], "generators": [], "output_tensors": NaN}',
    b'{"nodes": [], "generators": []} x',
    b'[1, 2]',
    b'{"nodes": [], "generators": [], "topology_key": "a\tb"}',   # raw control character
    b'{"nodes": [], "generators": [1.]}',
])
def test_malformed_documents_refused(text):
    assert outcome(product, text)[0] == "format"
    assert outcome(OW.save_binary, text)[0] == "format"


def test_serialised_members_escape_and_order():
    doc = {"generators": [], "nodes": [], "output_tensors": {"z": "a\"b\\c\u0001\u001f\u007f/é😀\n", "a": [-(1 << 63), (1 << 64) - 1]},
           "allocator_events": None}
    text = json.dumps(doc)
    img = product(text)
    assert img == OW.save_binary(text)
    arc = R.read(img)
    assert arc.section("OT") == '{"z":"a\\"b\\\\c\\u0001\\u001f\u007f/é😀\\n","a":[-9223372036854775808,18446744073709551615]}'.encode()
    assert arc.section("AE") == b"null" and arc.flags & 4


def test_capacity_and_save_binary(tmp_path):
    rng = random.Random(5)
    text = json.dumps(doc_of(sample_nodes(rng, 10), [(0, 1)]))
    img = product(text)
    path = tmp_path / "graph_0.cugraph"
    restore.save_binary(str(path), text)
    assert path.read_bytes() == img
    assert restore.cugraph_path("/a/graph_3.json") == "/a/graph_3.cugraph"
    assert restore.cugraph_path("/a/graph_3") == "/a/graph_3.cugraph"


def test_save_binary_unwritable_path_warns(tmp_path, capsys):
    text = json.dumps({"nodes": [], "generators": []})
    restore.save_binary(str(tmp_path / "missing_dir" / "g.cugraph"), text)
    assert "Failed to write binary graph" in capsys.readouterr().err
    assert not os.path.exists(tmp_path / "missing_dir")
