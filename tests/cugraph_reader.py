"""A third, independent reading of the .cugraph layout (test infrastructure).

Written from the packed structs of the reference's
include/BinaryGraphFormat.h (FileHeader 64 B at lines 65-76, SectionEntry
24 B at 78-84, BinNodeEntry 168 B at 171-185 with the kernel arm at entry
offset 8 per BinKernelNode 110-143, BinMemsetNode 144-154, BinMemcpyNode
155-165, BinEventNode 167-169, BinParamEntry 189-193, BinCommonKernelAttrs
197-212, BinDependency 223-227).  It shares no code with the product
(foundry_amd/csrc) or the oracle (oracle/), so the tests can hold either
against a reading neither of them made.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

MAGIC = b"CUGRAPH\0"
SECTIONS = ("STRING", "NODE", "DEP", "PIDX", "PDATA", "ARG", "COMMON", "GEN", "AE", "OT", "KEY")
TYPE_NAMES = ("KernelNode", "MemsetNode", "MemcpyNode", "EventRecordNode", "EventWaitNode", "EmptyNode")
KNA_CLUSTER_DIM = 1
FLAG_HAS_COMMON = 1
NO_ARG_BUFFER = 0xFFFFFFFF


@dataclass
class Kernel:
    block: tuple
    grid: tuple
    shmem: int
    binary_hash: int
    name: bytes
    func_attrs: tuple          # max_dyn_shmem, carveout, sched_pref, req_w, req_h, req_d
    kna_flags: int
    kna_cluster: tuple
    params: list = field(default_factory=list)   # (section, offset, size)
    arg_offset: int = NO_ARG_BUFFER
    arg_size: int = 0


@dataclass
class Node:
    node_id: int
    type: int
    raw: bytes
    kernel: Kernel | None = None


@dataclass
class Archive:
    data: bytes
    flags: int
    sections: dict
    nodes: list
    deps: list

    def section(self, name: str) -> bytes:
        off, size = self.sections[name]
        return self.data[off:off + size]

    def key(self) -> bytes:
        return self.section("KEY")

    def common_cluster(self):
        """(flags, cx, cy, cz) of the common kernel attrs, or None."""
        if not (self.flags & FLAG_HAS_COMMON):
            return None
        b = self.section("COMMON")
        if len(b) < 52:
            return None
        return struct.unpack_from("<IIII", b, 0)

    def param_bytes(self, n: int) -> list[bytes]:
        k = self.nodes[n].kernel
        out = []
        for sec, off, size in k.params:
            blob = self.section(sec)
            out.append(blob[off:off + size])
        return out


def read(data: bytes) -> Archive:
    magic, version, flags, num_nodes, num_deps, num_gen, num_sections, num_strings = struct.unpack_from(
        "<8sIIIIIII", data, 0)
    assert magic == MAGIC and version == 1, "not a .cugraph v1 image"
    sections = {}
    for i in range(num_sections):
        st, _pad, off, size = struct.unpack_from("<IIQQ", data, 64 + 24 * i)
        sections[SECTIONS[st]] = (off, size)
    arc = Archive(data, flags, sections, [], [])
    strings = arc.section("STRING")
    node_tab = arc.section("NODE")
    pidx = arc.section("PIDX")
    for n in range(num_nodes):
        e = node_tab[168 * n:168 * (n + 1)]
        node_id, ntype = struct.unpack_from("<IB", e, 0)
        node = Node(node_id, ntype, e)
        if ntype == 0:
            b = e[8:]
            bx, by, bz, gx, gy, gz, shmem = struct.unpack_from("<7I", b, 0)
            (bhash,) = struct.unpack_from("<Q", b, 28)
            name_off, name_len = struct.unpack_from("<II", b, 36)
            fa = struct.unpack_from("<6i", b, 44)
            kna_flags, cx, cy, cz = struct.unpack_from("<4I", b, 68)
            pio, npar, aoff, asize = struct.unpack_from("<4I", b, 120)
            k = Kernel((bx, by, bz), (gx, gy, gz), shmem, bhash, strings[name_off:name_off + name_len], fa,
                       kna_flags, (cx, cy, cz), [], aoff, asize)
            if aoff != NO_ARG_BUFFER:
                k.params.append(("ARG", aoff, asize))
            else:
                for j in range(npar):
                    off, size = struct.unpack_from("<II", pidx, pio + 8 * j)
                    k.params.append(("PDATA", off, size))
            node.kernel = k
        arc.nodes.append(node)
    deps = arc.section("DEP")
    arc.deps = [struct.unpack_from("<II", deps, 8 * i) for i in range(num_deps)]
    return arc


def load_rule_cluster(arc: Archive, n: int) -> tuple:
    """Cluster dims of kernel node n as the LOAD fallback reads them
    (csrc/CUDAGraphParallel.cpp:1807-1833): per-node clusterDim, else the
    common attrs' clusterDim, else func_attrs required_cluster_*."""
    k = arc.nodes[n].kernel
    c = (0, 0, 0)
    if k.kna_flags & KNA_CLUSTER_DIM:
        c = k.kna_cluster
    if c[0] == 0:
        com = arc.common_cluster()
        if com is not None and com[0] & KNA_CLUSTER_DIM:
            c = com[1:4]
    if c[0] == 0:
        c = tuple(v & 0xFFFFFFFF for v in k.func_attrs[3:6])
    return c


def key_from_nodes(arc: Archive) -> bytes:
    parts = []
    for n, node in enumerate(arc.nodes):
        s = TYPE_NAMES[node.type]
        if node.type == 0:
            c = load_rule_cluster(arc, n)
            s += ":C%d_%d_%d" % c if any(c) else ":0"
        parts.append(s)
    return ",".join(parts).encode()


def param_image(arc: Archive, n: int):
    """Node n's words: each param from its first byte in 8-byte steps, a
    short tail zero-filled; returns (words, widths)."""
    words, widths = [], []
    for p in arc.param_bytes(n):
        for b in range(0, len(p), 8):
            chunk = p[b:b + 8]
            widths.append(len(chunk))
            words.append(int.from_bytes(chunk.ljust(8, b"\0"), "little"))
    return words, widths
