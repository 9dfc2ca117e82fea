"""Archives of runnable graphs for the group-graph tests, and what running
them must produce.

Every kernel is one of tests/native/probe_kernels.hip; every pointer a graph
saves lies in the saved region [SAVED, SAVED + BUF_BYTES), which the tests
relocate onto a real device buffer.  `expected_image` restates the param
image the restore must produce (params in node order, each padded to
8 bytes, full words inside the saved region relocated), so a GPU test can
check every pointer before anything is launched.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field, replace

import cugraph_writer as W
from cugraph_writer import le

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE_CO = os.path.join(HERE, "native", "_build", "probe.co")

SAVED = 0x7F0000000000   # saved base of the output buffer
BUF_BYTES = 16384
CAP = 128                # u64 result slots at the start of the buffer
FILL_OFF, COPY_OFF = 4096, 8192
M64 = (1 << 64) - 1


def mix(h: int, v: int) -> int:
    h = (h ^ v) & M64
    h = (h * 0x9E3779B97F4A7C15) & M64
    return h ^ (h >> 29)


def mix_expect(a: int, b: int, grid_x: int, block_x: int) -> int:
    h = mix(mix(0x243F6A8885A308D3, a), b)
    return mix(mix(h, grid_x), block_x)


def blob_expect(words) -> int:
    h = 0x13198A2E03707344
    for w in words:
        h = mix(h, w)
    return h


@dataclass(frozen=True)
class Spec:
    """The values one graph of the group varies."""
    a0: int = 0x1111
    b0: int = 0x2222
    blob: tuple = tuple(0x100 + i for i in range(8))
    layout_mix: bool = False       # node 1 runs probe_mix (5 params) instead of probe_blob (4)
    a1: int = 0x5151
    b1: int = 0x5252
    slot_a: int = 0x3333
    slot_b: int = 0x4444
    slot_pad: int = 0x77
    count_v: int = 3
    count_grid: int = 4
    count_block: int = 64
    fill_value: int = 0xA5A5A5A5
    fill_words: int = 64
    copy_bytes: int = 256
    event_id: int = 7
    extra_empty: bool = False      # one more node: another topology key, another group


NODE_IDS_BASE = 100
# (from, to) by node position; stored as node ids NODE_IDS_BASE + position.
EDGES = [(0, 9), (9, 10), (4, 5), (6, 7), (3, 8), (8, 10)]


def nodes_of(s: Spec, bhash: int):
    out = le(SAVED)
    n = []
    n.append(W.Kernel("probe_mix", bhash, grid=(2, 1, 1), block=(64, 1, 1),
                      params=[out, le(0, 4), le(CAP, 4), le(s.a0), le(s.b0)]))
    if s.layout_mix:
        n.append(W.Kernel("probe_mix", bhash, params=[out, le(1, 4), le(CAP, 4), le(s.a1), le(s.b1)]))
    else:
        n.append(W.Kernel("probe_blob", bhash, params=[out, le(1, 4), le(CAP, 4), b"".join(le(w) for w in s.blob)]))
    n.append(W.Kernel("probe_mix_slot", bhash, arg=le(2, 4) + le(s.slot_pad, 4) + le(s.slot_a) + le(s.slot_b)))
    n.append(W.Kernel("probe_count", bhash, grid=(s.count_grid, 1, 1), block=(s.count_block, 1, 1),
                      params=[out, le(3, 4), le(CAP, 4), le(s.count_v)]))
    n.append(W.Memset(dst=SAVED + FILL_OFF, value=s.fill_value, width=s.fill_words, element_size=4))
    n.append(W.Memcpy(dst=SAVED + COPY_OFF, src=SAVED + FILL_OFF, width_bytes=s.copy_bytes))
    n.append(W.EventRecord(s.event_id))
    n.append(W.EventWait(s.event_id))
    n.append(W.Empty())
    n.append(W.Kernel("probe_chain", bhash, params=[out, le(9, 4), le(CAP, 4), le(0, 4)]))
    n.append(W.Kernel("probe_chain", bhash, params=[out, le(10, 4), le(CAP, 4), le(9, 4)]))
    if s.extra_empty:
        n.append(W.Empty())
    return n


def image_of(s: Spec, bhash: int) -> bytes:
    nodes = nodes_of(s, bhash)
    ids = [NODE_IDS_BASE + i for i in range(len(nodes))]
    deps = [(NODE_IDS_BASE + a, NODE_IDS_BASE + b) for a, b in EDGES]
    return W.write(nodes, deps, ids)


# The archive: group A = graphs 0-4 (template 0), group B = graph 5.
SPECS = [
    Spec(),                                                           # 0: template
    Spec(a0=0x1112, blob=(0x100, 0x101, 0x102, 0xBEEF, 0x104, 0x105, 0x106, 0x107), count_v=5),  # words
    Spec(count_grid=8, fill_value=0x01020304, copy_bytes=128, event_id=9),  # descriptors only
    Spec(layout_mix=True, a0=0x1999),                                 # layout of node 1 + words of node 0
    Spec(slot_a=0x3334),                                              # extra-style arg buffer words
    Spec(extra_empty=True),                                           # another group
]
GROUP_A = [0, 1, 2, 3, 4]


def images(bhash: int) -> list[bytes]:
    return [image_of(s, bhash) for s in SPECS]


def reloc(w: int, base: int) -> int:
    return (w - SAVED + base) & M64 if SAVED <= w < SAVED + BUF_BYTES else w


def expected_image(s: Spec, bhash: int, base: int) -> list[int]:
    """The relocated param image of the graph (kernel nodes' params in order)."""
    words = []
    for n in nodes_of(s, bhash):
        if n.type != 0:
            continue
        for p in ([n.arg] if n.arg is not None else n.params):
            for i in range(0, len(p), 8):
                chunk = p[i:i + 8]
                w = int.from_bytes(chunk.ljust(8, b"\0"), "little")
                words.append(reloc(w, base) if len(chunk) == 8 else w)
    return words


def expected_pointers(s: Spec, base: int) -> list[int]:
    """Relocated memset dst / memcpy dst, src per node (0 elsewhere)."""
    out = []
    for n in nodes_of(s, 0):
        if n.type == 1:
            out += [reloc(n.dst, base), 0]
        elif n.type == 2:
            out += [reloc(n.dst, base), reloc(n.src, base)]
        else:
            out += [0, 0]
    return out


def expected_buffer(s: Spec) -> tuple[dict, bytes, bytes]:
    """(result slots, fill region, copy region) after one launch on a zeroed buffer."""
    slots = {0: mix_expect(s.a0, s.b0, 2, 64)}
    slots[1] = mix_expect(s.a1, s.b1, 1, 64) if s.layout_mix else blob_expect(s.blob)
    slots[3] = (s.count_v * s.count_grid * s.count_block) & M64
    slots[9] = mix(slots[0], 9)
    slots[10] = mix(slots[9], 10)
    fill = le(s.fill_value, 4) * s.fill_words
    copy = fill[:s.copy_bytes]
    return slots, fill, copy


def expected_slot2(s: Spec) -> int:
    return mix_expect(s.slot_a, s.slot_b, 1, 64) ^ s.slot_pad


def own_nodes(s: Spec, t: Spec) -> set:
    """Nodes whose descriptor or layout differs between graph s and template t."""
    out = set()
    if s.count_grid != t.count_grid or s.count_block != t.count_block:
        out.add(3)
    if s.layout_mix != t.layout_mix:
        out.add(1)
    if s.fill_value != t.fill_value or s.fill_words != t.fill_words:
        out.add(4)
    if s.copy_bytes != t.copy_bytes:
        out.add(5)
    if s.event_id != t.event_id:
        out |= {6, 7}
    return out


__all__ = ["Spec", "SPECS", "GROUP_A", "replace", "field"]
