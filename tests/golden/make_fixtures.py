#!/usr/bin/env python3
"""Hand-assembled .cugraph fixtures with hand-derived expected values.

Writes tiny_{a,b,c,d}.cugraph and expected.json next to this script.  The
archives are packed field by field with struct, following the packed
structs of the reference's include/BinaryGraphFormat.h (FileHeader 65-76,
SectionEntry 78-84, BinKernelNode 110-143, BinMemsetNode 144-154,
BinMemcpyNode 155-165, BinEventNode 167-169, BinNodeEntry 171-185,
BinParamEntry 189-193, BinCommonKernelAttrs 197-212, BinDependency 223-227)
and the writer's section order, 8-byte alignment and string interning
(csrc/BinaryGraphIO.cpp:24-36, 291-368).  Every expected value in
expected.json is written out by hand below (topology keys per
csrc/CUDAGraph.cpp:1347-1385 and csrc/CUDAGraphParallel.cpp:1798-1841,
params per csrc/CUDAGraphParallel.cpp:1391-1409), not computed by the
product or the oracle.

Run from anywhere: python3 tests/golden/make_fixtures.py
"""
from __future__ import annotations

import json
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))

KNA_CLUSTER_DIM = 1
FLAG_COMMON, FLAG_DEPS = 1, 2
NONE = 0xFFFFFFFF


def kernel_entry(node_id, block, grid, bhash, name_off, name_len, req=(0, 0, 0), kna_flags=0, cluster=(0, 0, 0),
                 pio=0, npar=0, aoff=NONE, asize=0):
    arm = struct.pack("<7I", *block, *grid, 0)                 # block, grid, sharedMemBytes
    arm += struct.pack("<Q", bhash)                             # binary_hash (entry offset 36)
    arm += struct.pack("<II", name_off, name_len)
    arm += struct.pack("<6i", 0, -1, 0, *req)                   # func_attrs
    arm += struct.pack("<4I", kna_flags, *cluster)              # kna_flags, clusterDim
    arm += struct.pack("<3I", 0, 0, 0)                          # preferredClusterDim
    arm += struct.pack("<4i", -1, -1, -1, -1)                   # scheduling, cooperative, priority, memSyncDomain
    arm += struct.pack("<4B", 0, 0, 0, 0)                       # map default/remote, attrQueryAvailable, pad
    arm += struct.pack("<I", 0)                                 # preferredSharedMemCarveout
    arm += struct.pack("<4I", pio, npar, aoff, asize)
    assert len(arm) == 136
    return entry(node_id, 0, arm)


def entry(node_id, ntype, arm=b""):
    e = struct.pack("<IB3x", node_id, ntype) + arm
    return e.ljust(168, b"\0")


def memset_entry(node_id, dst, elem, height, pitch, value, width):
    return entry(node_id, 1, struct.pack("<QI4xQQI4xQ", dst, elem, height, pitch, value, width))


def memcpy_entry(node_id, dst, dst_type, src, src_type, width_bytes):
    arm = struct.pack("<3Q", 1, 1, width_bytes)                 # Depth, Height, WidthInBytes
    arm += struct.pack("<Q", dst) + struct.pack("<6Q", 0, 0, 0, 0, 0, 0) + struct.pack("<ii", dst_type, 0)
    arm += struct.pack("<Q", src) + struct.pack("<6Q", 0, 0, 0, 0, 0, 0) + struct.pack("<ii", src_type, 0)
    assert len(arm) == 152
    return entry(node_id, 2, arm)


def event_entry(node_id, ntype, event_id):
    return entry(node_id, ntype, struct.pack("<i", event_id))


def common_attrs(cluster):
    b = struct.pack("<4I", KNA_CLUSTER_DIM, *cluster) + struct.pack("<3I", 0, 0, 0)
    b += struct.pack("<4i", -1, -1, -1, -1) + struct.pack("<4B", 0, 0, 0, 0) + struct.pack("<I", 0)
    assert len(b) == 52
    return b


def archive(strings, nodes, deps, pidx, pdata, arg, common, key, num_strings):
    secs = [strings, b"".join(nodes), b"".join(struct.pack("<II", *d) for d in deps),
            b"".join(struct.pack("<II", *p) for p in pidx), pdata, arg, common or b"", b"", b"", b"", key]
    off = 64 + 11 * 24
    table, body = b"", b""
    for i, s in enumerate(secs):
        table += struct.pack("<IIQQ", i, 0, off, len(s))
        pad = (8 - len(s) % 8) % 8
        body += s + b"\0" * pad
        off += len(s) + pad
    flags = (FLAG_COMMON if common else 0) | (FLAG_DEPS if deps else 0)
    header = struct.pack("<8s7I28x", b"CUGRAPH\0", 1, flags, len(nodes), len(deps), 0, 11, num_strings)
    assert len(header) == 64
    return header + table + body


def le(v, n=8):
    return v.to_bytes(n, "little")


def main():
    strings = b"vec_add\0gemm_tile\0"          # "vec_add" at 0 (7 bytes), "gemm_tile" at 8 (9 bytes)
    expected = {}

    # tiny_a: KernelNode (16 B + 12 B params), MemsetNode, KernelNode (extra-style, 20 B arg buffer,
    # per-node cluster 2x1x1); chain 0 -> 1 -> 2.
    def build_ab(second_word, arg_mid):
        p0 = le(0x7F0000001000) + le(second_word)
        p1 = le(7, 4) + le(8, 4) + le(9, 4)
        pdata = p0 + p1
        arg = le(0x7F0000003000) + le(arg_mid) + le(6, 4)
        nodes = [
            kernel_entry(0, (128, 1, 1), (64, 1, 1), 0x1111222233334444, 0, 7, pio=0, npar=2),
            memset_entry(1, 0x7F0000002000, 4, 1, 0, 0, 256),
            kernel_entry(2, (256, 1, 1), (8, 1, 1), 0x5555666677778888, 8, 9, kna_flags=KNA_CLUSTER_DIM,
                         cluster=(2, 1, 1), pio=16, npar=2, aoff=0, asize=20),
        ]
        pidx = [(0, 16), (16, 12), (0, 8), (8, 12)]   # node 2's entries describe its arg buffer
        key = b"KernelNode:0,MemsetNode,KernelNode:C2_1_1"
        return archive(strings, nodes, [(0, 1), (1, 2)], pidx, pdata, arg, None, key, 2), (p0, p1, arg)

    a, (a_p0, a_p1, a_arg) = build_ab(42, 5)
    b, (b_p0, b_p1, b_arg) = build_ab(43, 77)

    # tiny_c: common attrs carry cluster 4x1x1; KernelNode (8 B pointer param), EventRecordNode,
    # MemcpyNode (device dst, host src), EmptyNode, KernelNode (8 B param); no dependencies.
    c_pdata = le(0x7F0000004000) + le(0x1234)
    c_nodes = [
        kernel_entry(0, (64, 1, 1), (4, 1, 1), 0x1111222233334444, 0, 7, pio=0, npar=1),
        event_entry(1, 3, 3),
        memcpy_entry(2, 0x7F0000005000, 2, 0x1234, 1, 64),
        entry(3, 5),
        kernel_entry(4, (64, 1, 1), (4, 1, 1), 0x1111222233334444, 0, 7, pio=8, npar=1),
    ]
    c_key = b"KernelNode:C4_1_1,EventRecordNode,MemcpyNode,EmptyNode,KernelNode:C4_1_1"
    c = archive(strings, c_nodes, [], [(0, 8), (8, 8)], c_pdata, b"", common_attrs((4, 1, 1)), c_key, 2)

    # tiny_d: no common attrs, required cluster (0, 2, 0) on its only KernelNode, and an empty saved
    # key (an archive saved without one: grouping then uses "").
    d_nodes = [kernel_entry(0, (32, 1, 1), (1, 1, 1), 0x9999AAAABBBBCCCC, 8, 9, req=(0, 2, 0), pio=0, npar=1)]
    d = archive(strings, d_nodes, [], [(0, 8)], le(0xDEADBEEF), b"", None, b"", 2)

    for name, img in (("tiny_a", a), ("tiny_b", b), ("tiny_c", c), ("tiny_d", d)):
        with open(os.path.join(HERE, name + ".cugraph"), "wb") as f:
            f.write(img)

    w = lambda bs: [int.from_bytes(bs[i:i + 8].ljust(8, b"\0"), "little") for i in range(0, len(bs), 8)]
    reloc_lo, reloc_hi, reloc_new = 0x7F0000000000, 0x7F0000010000, 0x7E0000000000
    expected["tiny_a"] = {
        "saved_key": "KernelNode:0,MemsetNode,KernelNode:C2_1_1",
        "recomputed_key": "KernelNode:0,MemsetNode,KernelNode:C2_1_1",
        "params": {"0": (a_p0 + a_p1).hex(), "1": "", "2": a_arg.hex()},
        # node 0: 2 words of p0, then p1 as a whole word (7 | 8 << 32) and a 4-byte tail (9);
        # node 2: the 20-byte arg buffer as 2 whole words and a 4-byte tail.
        "words": [0x7F0000001000, 42, 7 | (8 << 32), 9, 0x7F0000003000, 5, 6],
        "node_words": [4, 0, 3],
        "ragged_nodes": [0, 2],
    }
    expected["tiny_b"] = {"words": [0x7F0000001000, 43, 7 | (8 << 32), 9, 0x7F0000003000, 77, 6]}
    expected["a_b_group"] = {
        "template_of": [0, 0],
        # records (template word, node, value), canonical order
        "overrides_b": [[1, 0, 43], [5, 2, 77]],
    }
    expected["relocation"] = {
        "intervals": [[reloc_lo, reloc_hi, reloc_new]],
        "words_a": [0x7E0000001000, 42, 7 | (8 << 32), 9, 0x7E0000003000, 5, 6],
        "memset_dst_a": 0x7E0000002000,
        "memcpy_dst_c": 0x7E0000005000,   # device memory: relocated
        "memcpy_src_c": 0x1234,           # host memory: left alone
    }
    expected["tiny_c"] = {
        "saved_key": c_key.decode(),
        "recomputed_key": c_key.decode(),
        "params": {"0": le(0x7F0000004000).hex(), "4": le(0x1234).hex()},
        "words": [0x7F0000004000, 0x1234],
    }
    expected["tiny_d"] = {"saved_key": "", "recomputed_key": "KernelNode:C0_2_0", "words": [0xDEADBEEF]}
    expected["check"] = {"words_a_from_params": w(a_p0) + w(a_p1) + w(a_arg)}
    with open(os.path.join(HERE, "expected.json"), "w") as f:
        json.dump(expected, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
