"""A `.cugraph` v1 writer for test archives with chosen nodes.

Field by field per the packed structs of the reference's
include/BinaryGraphFormat.h (FileHeader 65-76, SectionEntry 78-84,
BinKernelNode 110-143, BinMemsetNode 144-154, BinMemcpyNode 155-165,
BinEventNode 167-169, BinNodeEntry 171-185, BinParamEntry 189-193,
BinCommonKernelAttrs 197-212, BinDependency 223-227), with the writer's
section order, 8-byte section alignment and string interning
(csrc/BinaryGraphIO.cpp:24-36, 291-368).  The saved topology key follows
CUDAGraph::save (csrc/CUDAGraph.cpp:1347-1385): per-node cluster dims, else
the function's required cluster dims, else ":0".
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

NO_ARG = 0xFFFFFFFF
KNA_CLUSTER_DIM, KNA_COOPERATIVE = 1 << 0, 1 << 3
FLAG_COMMON, FLAG_DEPS = 1, 2
MEM_DEVICE = 2
TYPE_NAMES = ["KernelNode", "MemsetNode", "MemcpyNode", "EventRecordNode", "EventWaitNode", "EmptyNode"]


@dataclass
class Kernel:
    name: str
    binary_hash: int
    grid: tuple = (1, 1, 1)
    block: tuple = (64, 1, 1)
    params: list = field(default_factory=list)  # list of bytes, one per param
    arg: bytes | None = None                     # extra-style arg buffer instead of params
    shmem: int = 0
    cluster: tuple | None = None                 # per-node cluster dims
    cooperative: int | None = None
    func_attrs: tuple = (0, -1, 0, 0, 0, 0)      # max dyn shmem, carveout, sched pref, required cluster w/h/d
    kna_ints: tuple | None = None                # (sched, cooperative, priority, mem sync domain) as stored
    type = 0


@dataclass
class Memset:
    dst: int
    value: int
    width: int
    element_size: int = 4
    height: int = 1
    pitch: int = 0
    type = 1


@dataclass
class Memcpy:
    dst: int
    src: int
    width_bytes: int
    dst_type: int = MEM_DEVICE
    src_type: int = MEM_DEVICE
    type = 2


@dataclass
class EventRecord:
    event_id: int
    type = 3


@dataclass
class EventWait:
    event_id: int
    type = 4


@dataclass
class Empty:
    type = 5


def _entry(node_id: int, ntype: int, arm: bytes = b"") -> bytes:
    return (struct.pack("<IB3x", node_id, ntype) + arm).ljust(168, b"\0")


def _kernel_arm(k: Kernel, name_off: int, pio: int) -> bytes:
    kna = 0
    cl = (0, 0, 0)
    if k.cluster is not None:
        kna |= KNA_CLUSTER_DIM
        cl = k.cluster
    coop = -1
    if k.cooperative is not None:
        kna |= KNA_COOPERATIVE
        coop = k.cooperative
    npar = len(k.params)
    aoff, asize = (NO_ARG, 0) if k.arg is None else (None, len(k.arg))
    arm = struct.pack("<7I", *k.block, *k.grid, k.shmem)
    arm += struct.pack("<Q", k.binary_hash)
    arm += struct.pack("<II", name_off, len(k.name))
    arm += struct.pack("<6i", *k.func_attrs)
    arm += struct.pack("<4I", kna, *cl)
    arm += struct.pack("<3I", 0, 0, 0)
    arm += struct.pack("<4i", *(k.kna_ints if k.kna_ints is not None else (-1, coop, -1, -1)))
    arm += struct.pack("<4B", 0, 0, 0, 0) + struct.pack("<I", 0)
    return arm, npar, aoff, asize


def saved_key(nodes) -> bytes:
    parts = []
    for n in nodes:
        s = TYPE_NAMES[n.type]
        if n.type == 0:
            s += ":C%d_%d_%d" % n.cluster if n.cluster is not None and any(n.cluster) else ":0"
        parts.append(s)
    return ",".join(parts).encode()


FLAG_ALLOC_EVENTS, FLAG_OUTPUT_TENSORS, FLAG_GENERATORS = 4, 8, 16


def write(nodes, deps=(), node_ids=None, common_cluster=None, alloc_events: bytes = b"",
          output_tensors: bytes = b"", common_ints=(-1, -1, -1, -1), key: bytes | None = None,
          generators=()) -> bytes:
    """Archive bytes for `nodes` (Kernel/Memset/...); deps are (from_id, to_id).
    alloc_events / output_tensors are the JSON texts of those sections.
    `key` replaces the saved topology key CUDAGraph::save would write;
    `generators` are (id, seed, wholegraph_increment) rows of the GENERATORS
    section (BinGenerator, include/BinaryGraphFormat.h:214-219)."""
    ids = list(node_ids) if node_ids is not None else list(range(len(nodes)))
    strings = b""
    name_at = {}
    pdata, arg_data, pidx = b"", b"", []
    entries = []
    for nid, n in zip(ids, nodes):
        if n.type == 0:
            if n.name not in name_at:
                name_at[n.name] = len(strings)
                strings += n.name.encode() + b"\0"
            arm, npar, _, asize = _kernel_arm(n, name_at[n.name], 8 * len(pidx))
            pio = 8 * len(pidx)
            if n.arg is not None:
                aoff = len(arg_data)
                arg_data += n.arg
                while len(arg_data) % 8:
                    arg_data += b"\0"
                npar = 0
            else:
                aoff = NO_ARG
                for p in n.params:
                    pidx.append((len(pdata), len(p)))
                    pdata += p
            arm += struct.pack("<4I", pio, npar, aoff, asize)
            assert len(arm) == 136
            entries.append(_entry(nid, 0, arm))
        elif n.type == 1:
            entries.append(_entry(nid, 1, struct.pack("<QI4xQQI4xQ", n.dst, n.element_size, n.height, n.pitch,
                                                      n.value, n.width)))
        elif n.type == 2:
            arm = struct.pack("<3Q", 1, 1, n.width_bytes)
            arm += struct.pack("<Q", n.dst) + struct.pack("<6Q", 0, 0, 0, 0, 0, 0) + struct.pack("<ii", n.dst_type, 0)
            arm += struct.pack("<Q", n.src) + struct.pack("<6Q", 0, 0, 0, 0, 0, 0) + struct.pack("<ii", n.src_type, 0)
            entries.append(_entry(nid, 2, arm))
        elif n.type in (3, 4):
            entries.append(_entry(nid, n.type, struct.pack("<i", n.event_id)))
        else:
            entries.append(_entry(nid, 5))
    common = b""
    if common_cluster is not None:
        common = struct.pack("<4I", KNA_CLUSTER_DIM, *common_cluster) + struct.pack("<3I", 0, 0, 0)
        common += struct.pack("<4i", *common_ints) + struct.pack("<4B", 0, 0, 0, 0) + struct.pack("<I", 0)
    gens = b"".join(struct.pack("<3Q", *g) for g in generators)
    secs = [strings, b"".join(entries), b"".join(struct.pack("<II", *d) for d in deps),
            b"".join(struct.pack("<II", *p) for p in pidx), pdata, arg_data, common, gens, alloc_events,
            output_tensors, saved_key(nodes) if key is None else key]
    off = 64 + 11 * 24
    table, body = b"", b""
    for i, s in enumerate(secs):
        table += struct.pack("<IIQQ", i, 0, off, len(s))
        pad = (8 - len(s) % 8) % 8
        body += s + b"\0" * pad
        off += len(s) + pad
    flags = (FLAG_COMMON if common else 0) | (FLAG_DEPS if deps else 0)
    flags |= (FLAG_ALLOC_EVENTS if alloc_events else 0) | (FLAG_OUTPUT_TENSORS if output_tensors else 0)
    flags |= FLAG_GENERATORS if generators else 0
    header = struct.pack("<8s7I28x", b"CUGRAPH\0", 1, flags, len(nodes), len(deps), len(generators), 11,
                         len(name_at))
    return header + table + body


def le(v: int, n: int = 8) -> bytes:
    return (v & ((1 << (8 * n)) - 1)).to_bytes(n, "little")
