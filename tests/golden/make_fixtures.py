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


# Launch-attribute flag bits (BinaryGraphFormat.h KNA_*) and the 52-byte
# attribute block shared by a kernel entry (entry bytes 76..128) and the
# common-attrs section (BinKernelNode 110-142, BinCommonKernelAttrs 197-212).
KNA_PREF, KNA_SCHED, KNA_COOP, KNA_PRIO, KNA_MSD, KNA_MAP, KNA_CARVE = 2, 4, 8, 16, 32, 64, 128
KNA_ALL = 255


def kna(flags=0, cluster=(0, 0, 0), pref=(0, 0, 0), sched=-1, coop=-1, prio=-1, msd=-1, mp=(0, 0), carve=0):
    b = struct.pack("<4I", flags, *cluster)                     # flags, clusterDim
    b += struct.pack("<3I", *pref)                              # preferredClusterDim
    b += struct.pack("<4i", sched, coop, prio, msd)             # scheduling, cooperative, priority, memSyncDomain
    b += struct.pack("<4B", mp[0], mp[1], 0, 0)                 # map default/remote, attrQueryAvailable, pad
    b += struct.pack("<I", carve)                               # preferredSharedMemCarveout
    assert len(b) == 52
    return b


def kernel_entry(node_id, block, grid, bhash, name_off, name_len, req=(0, 0, 0), kna_flags=0, cluster=(0, 0, 0),
                 pio=0, npar=0, aoff=NONE, asize=0, attrs=None):
    arm = struct.pack("<7I", *block, *grid, 0)                 # block, grid, sharedMemBytes
    arm += struct.pack("<Q", bhash)                             # binary_hash (entry offset 36)
    arm += struct.pack("<II", name_off, name_len)
    arm += struct.pack("<6i", 0, -1, 0, *req)                   # func_attrs
    arm += attrs if attrs is not None else kna(kna_flags, cluster)
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
    return kna(KNA_CLUSTER_DIM, cluster)


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


def archive_raw_pidx(strings, nodes, pidx_bytes, pdata, key, num_strings):
    """archive() with the param-index section given as raw bytes."""
    secs = [strings, b"".join(nodes), b"", pidx_bytes, pdata, b"", b"", b"", b"", b"", key]
    off = 64 + 11 * 24
    table, body = b"", b""
    for i, s in enumerate(secs):
        table += struct.pack("<IIQQ", i, 0, off, len(s))
        pad = (8 - len(s) % 8) % 8
        body += s + b"\0" * pad
        off += len(s) + pad
    header = struct.pack("<8s7I28x", b"CUGRAPH\0", 1, 0, len(nodes), 0, 0, 11, num_strings)
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

    # attr_t / attr_m: one template and one member whose launch attributes come
    # from conflicting sources.  attr_t's common attrs set every attribute;
    # its nodes override some of them per node (negative scalar values do
    # not override, csrc/CUDAGraphParallel.cpp:1362-1369) and node 1 has a
    # required cluster (0, 3, 0), which wins over both (1376-1385; zero dims
    # become 1).  attr_m has no common attrs and spells every attribute out
    # per node, so each of its nodes' effective attributes is the value
    # written.  The effective attributes below are derived by hand from
    # those rules; a node's DESC flag is set exactly where they differ
    # (everything else about the two nodes is equal).
    ct = dict(cluster=(4, 1, 1), pref=(8, 1, 1), sched=1, coop=1, prio=2, msd=1, mp=(1, 2), carve=50)

    def full(**kw):  # every attribute explicit: attr_t's common values, some replaced
        v = dict(ct)
        v.update(kw)
        return kna(KNA_ALL, **v)

    attr_cases = [  # (attr_t node's per-node block, its required cluster, attr_m node's block)
        (kna(KNA_CLUSTER_DIM, (2, 1, 1)), (0, 0, 0), full(cluster=(2, 1, 1))),
        (kna(KNA_CLUSTER_DIM, (2, 1, 1)), (0, 3, 0), full(cluster=(1, 3, 1))),
        (kna(KNA_SCHED | KNA_COOP | KNA_PRIO | KNA_MSD, sched=-1, coop=0, prio=-1, msd=3), (0, 0, 0),
         full(coop=0, msd=3)),
        (kna(KNA_PRIO, prio=5), (0, 0, 0), full(prio=5)),
        (kna(0, cluster=(9, 9, 9), prio=9), (0, 0, 0), full()),   # values without flags are not read
        (kna(0), (0, 0, 0), full(cluster=(2, 1, 1))),             # a real difference
        (kna(KNA_PREF | KNA_CARVE, pref=(3, 1, 1), carve=20), (0, 0, 0), full(pref=(3, 1, 1), carve=20)),
        (kna(KNA_PRIO, prio=7), (0, 0, 0), full(prio=2)),         # a real difference
        (kna(KNA_MAP, mp=(3, 0)), (0, 0, 0), full(mp=(3, 0))),
        (kna(KNA_COOP, coop=-5), (0, 0, 0), full()),
    ]
    # Effective attributes, in the order has_cluster, cx, cy, cz, has_pref,
    # px, py, pz, sched, coop, prio, msd, has_map, map_default, map_remote,
    # has_carveout, carveout.
    common_eff = [1, 4, 1, 1, 1, 8, 1, 1, 1, 1, 2, 1, 1, 1, 2, 1, 50]

    def eff(**kw):
        v = list(common_eff)
        for k, x in kw.items():
            at = {"c": 1, "p": 5, "sched": 8, "coop": 9, "prio": 10, "msd": 11, "map": 13, "carve": 16}[k]
            x = list(x) if isinstance(x, tuple) else [x]
            v[at:at + len(x)] = x
        return v

    eff_t = [eff(c=(2, 1, 1)), eff(c=(1, 3, 1)), eff(coop=0, msd=3), eff(prio=5), eff(), eff(),
             eff(p=(3, 1, 1), carve=20), eff(prio=7), eff(map=(3, 0)), eff()]
    eff_m = [eff(c=(2, 1, 1)), eff(c=(1, 3, 1)), eff(coop=0, msd=3), eff(prio=5), eff(), eff(c=(2, 1, 1)),
             eff(p=(3, 1, 1), carve=20), eff(prio=2), eff(map=(3, 0)), eff()]
    desc_m = [0, 0, 0, 0, 0, 1, 0, 1, 0, 0]
    # Cluster dims of the recomputed key: per-node, else common, else required.
    key_t = ",".join("KernelNode:C%d_%d_%d" % c for c in
                     [(2, 1, 1), (2, 1, 1)] + [(4, 1, 1)] * 8)
    key_m = ",".join("KernelNode:C%d_%d_%d" % c for c in
                     [(2, 1, 1), (1, 3, 1), (4, 1, 1), (4, 1, 1), (4, 1, 1), (2, 1, 1)] + [(4, 1, 1)] * 4)
    params_t = [0x100 * n + 1 for n in range(len(attr_cases))]
    params_m = list(params_t)
    params_m[7] = 0x7FF

    def attr_archive(side, common, params):
        nodes = []
        for n, case in enumerate(attr_cases):
            block, req = (case[0], case[1]) if side == "t" else (case[2], case[1])
            nodes.append(kernel_entry(n, (128, 1, 1), (32, 1, 1), 0x1111222233334444, 0, 7, req=req, pio=8 * n,
                                      npar=1, attrs=block))
        pidx = [(8 * n, 8) for n in range(len(nodes))]
        pdata = b"".join(le(v) for v in params)
        # Both carry attr_t's key, so they group together whatever they recompute.
        return archive(strings, nodes, [], pidx, pdata, b"", common, key_t.encode(), 2)

    attr_t = attr_archive("t", kna(KNA_ALL, **ct), params_t)
    attr_m = attr_archive("m", None, params_m)
    expected["attrs"] = {
        "effective_t": eff_t,
        "effective_m": eff_m,
        "desc_m": desc_m,
        "recomputed_key_t": key_t,
        "recomputed_key_m": key_m,
        "template_of": [0, 0],
        "status": [0, 1],                 # attr_m's recomputed node types differ: TYPE_MISMATCH
        "words_t": params_t,
        "words_m": params_m,
        "overrides_m": [[7, 7, 0x7FF]],
    }

    # tiny_e / tiny_f: param-index offsets that are not multiples of 8 (the
    # reference reads BinParamEntry at any byte offset, pack(1),
    # csrc/CUDAGraphParallel.cpp:1391-1394) and a node with 18 params.  The
    # param-index section is written byte by byte:
    #   [0, 4)     unreferenced bytes
    #   [4, 20)    node 0 (pio 4): (0, 8), (8, 12)
    #   [20, 21)   unreferenced
    #   [21, 29)   node 1 (pio 21): (24, 16)
    #   [29, 173)  node 3 (pio 29): (40 + 8j, 8) for j < 18
    # node 2 has no params.
    def build_ef(word1, p17):
        pidx = b"\xAA" * 4 + struct.pack("<II", 0, 8) + struct.pack("<II", 8, 12) + b"\xBB"
        pidx += struct.pack("<II", 24, 16)
        pidx += b"".join(struct.pack("<II", 40 + 8 * j, 8) for j in range(18))
        assert len(pidx) == 173
        pdata = le(0x7F0000001000) + le(word1) + le(0x2B, 4) + le(0xCCCCCCCC, 4) + le(0x7F0000002000) + le(0x77)
        pdata += b"".join(le(p17 if j == 17 else 0x100 + j) for j in range(18))
        assert len(pdata) == 184
        nodes = [
            kernel_entry(0, (64, 1, 1), (2, 1, 1), 0x1111222233334444, 0, 7, pio=4, npar=2),
            kernel_entry(1, (64, 1, 1), (2, 1, 1), 0x1111222233334444, 0, 7, pio=21, npar=1),
            kernel_entry(2, (64, 1, 1), (2, 1, 1), 0x1111222233334444, 0, 7, pio=0, npar=0),
            kernel_entry(3, (64, 1, 1), (2, 1, 1), 0x5555666677778888, 8, 9, pio=29, npar=18),
        ]
        key = b"KernelNode:0,KernelNode:0,KernelNode:0,KernelNode:0"
        return archive_raw_pidx(strings, nodes, pidx, pdata, key, 2)

    e_img = build_ef(0x2A, 0x111)
    f_img = build_ef(0x2C, 0x999)
    words_e = [0x7F0000001000, 0x2A, 0x2B, 0x7F0000002000, 0x77] + [0x100 + j for j in range(18)]
    words_e[-1] = 0x111
    words_f = list(words_e)
    words_f[1], words_f[22] = 0x2C, 0x999
    expected["unaligned_pidx"] = {
        "node_words": [3, 2, 0, 18],
        "ragged_nodes": [0],
        "words_e": words_e,
        "words_f": words_f,
        "template_of": [0, 0],
        "overrides_f": [[1, 0, 0x2C], [22, 3, 0x999]],
        # relocated by the same interval as the other fixtures
        "words_e_relocated": [0x7E0000001000, 0x2A, 0x2B, 0x7E0000002000, 0x77] + words_e[5:],
    }

    for name, img in (("tiny_a", a), ("tiny_b", b), ("tiny_c", c), ("tiny_d", d), ("attr_t", attr_t),
                      ("attr_m", attr_m), ("tiny_e", e_img), ("tiny_f", f_img)):
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
