"""CPU restatement of CUDAGraph::save_binary (csrc/BinaryGraphIO.cpp:15-371):
the .cugraph v1 archive of one graph's JSON document.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker, never by the
product.  Pure Python over small documents.

Followed step by step:
  - string table: function names interned in first-use order, NUL after
    each (BinaryGraphIO.cpp:24-36); header num_strings = distinct names (336)
  - node entries, 168 B each, zero-filled, per type (149-264); an unknown
    type string leaves type 0 with a zero body (149-153: the entry starts as {})
  - kernel params: value_hex -> param data, size = len // 2, each 2-char
    chunk through strtoul base 16 (48-53, 186-196); otherwise offset/size
    (197-201); extra_argBuffer_hex -> arg data, else offset 0xFFFFFFFF (205-216)
  - kernel_node_attrs / common_kernel_node_attrs flag bits (55-137)
  - dependencies (266-272), generators (274-281)
  - allocator_events / output_tensors: the compact serialisation of those
    members (283-287)
  - section placement and 8-byte alignment (289-315), header flags (317-336),
    padded section writes (343-366)
Refused, as in the product: duplicate object keys (a graph save never
writes them) and non-integer numbers inside the two serialised members.
"""
from __future__ import annotations

import json
import struct

NO_ARG = 0xFFFFFFFF
HEADER_SIZE, SECTION_SIZE, NUM_SECTIONS, ENTRY_SIZE = 64, 24, 11, 168
KNA_CLUSTER_DIM, KNA_PREFERRED_CLUSTER_DIM, KNA_CLUSTER_SCHEDULING = 1, 2, 4
KNA_COOPERATIVE, KNA_PRIORITY, KNA_MEM_SYNC_DOMAIN = 8, 16, 32
KNA_MEM_SYNC_DOMAIN_MAP, KNA_SHARED_MEM_CARVEOUT, KNA_ATTR_QUERY_AVAILABLE = 64, 128, 256


class WriterError(ValueError):
    """The document cannot be serialised (the reference throws)."""


class Unsupported(WriterError):
    """A value the reference never writes into a serialised member."""


class _Float:
    """A JSON number with a fraction or exponent, kept as its text."""

    __slots__ = ("text",)

    def __init__(self, text: str):
        self.text = text


def _pairs(pairs):
    d = {}
    for k, v in pairs:
        if k in d:
            raise WriterError(f"duplicate key {k!r}")
        d[k] = v
    return d


def _bad_constant(name):
    raise WriterError(f"not JSON: {name}")


def _check_text(v) -> None:
    """Every string and key is well-formed Unicode (no lone surrogates)."""
    stack = [v]
    while stack:
        x = stack.pop()
        if isinstance(x, str):
            try:
                x.encode("utf-8")
            except UnicodeEncodeError:
                raise WriterError("lone surrogate") from None
        elif isinstance(x, list):
            stack.extend(x)
        elif isinstance(x, dict):
            stack.extend(x.keys())
            stack.extend(x.values())


def parse(text: bytes | str):
    """The document: UTF-8 text (no byte-order mark), standard JSON."""
    if isinstance(text, (bytes, bytearray)):
        try:
            text = bytes(text).decode("utf-8")
        except UnicodeDecodeError:
            raise WriterError("invalid UTF-8") from None
    try:
        root = json.loads(text, object_pairs_hook=_pairs, parse_float=_Float, parse_constant=_bad_constant)
    except json.JSONDecodeError as e:
        raise WriterError(str(e)) from None
    _check_text(root)
    return root


def _get(o, key):
    if not isinstance(o, dict):
        raise WriterError("not an object")
    if key not in o:
        raise WriterError(f"missing {key!r}")
    return o[key]


def _num(v, bits: int, signed: bool) -> int:
    """Boost.JSON to_number<T>: the integer, if T holds it exactly."""
    if isinstance(v, bool) or not isinstance(v, (int, _Float)):
        raise WriterError("not a number")
    if isinstance(v, _Float):
        d = float(v.text)
        if d != d or d in (float("inf"), float("-inf")) or d != int(d):
            raise WriterError("not exact")
        v = int(d)
    lo, hi = (-(1 << (bits - 1)), 1 << (bits - 1)) if signed else (0, 1 << bits)
    if not lo <= v < hi:
        raise WriterError("out of range")
    return v


def u32(v):
    return _num(v, 32, False)


def i32(v):
    return _num(v, 32, True)


def u64(v):
    return _num(v, 64, False)


def _str(v) -> bytes:
    if not isinstance(v, str):
        raise WriterError("not a string")
    try:
        return v.encode("utf-8")
    except UnicodeEncodeError:
        raise WriterError("lone surrogate") from None


def _arr(v):
    if not isinstance(v, list):
        raise WriterError("not an array")
    return v


def strtoul16(chunk: bytes) -> int:
    """strtoul(chunk, &end, 16) as C reads it, cast to uint8; no digits -> error."""
    i, n = 0, len(chunk)
    while i < n and chunk[i] in b" \t\n\v\f\r":
        i += 1
    neg = False
    if i < n and chunk[i] in b"+-":
        neg = chunk[i] == ord("-")
        i += 1
    if i + 2 < n and chunk[i:i + 2].lower() == b"0x" and chunk[i + 2:i + 3].lower() in b"0123456789abcdef":
        i += 2
    start, val = i, 0
    while i < n and chunk[i:i + 1].lower() in b"0123456789abcdef" and chunk[i] != 0:
        val = val * 16 + int(chunk[i:i + 1], 16)
        i += 1
    if i == start:
        raise WriterError(f"unreadable hex pair {chunk!r}")
    if neg:
        val = -val % (1 << 64)
    return val & 0xFF


def hex_decode(hexs: bytes) -> bytes:
    return bytes(strtoul16(hexs[j:j + 2].split(b"\0")[0]) for j in range(0, len(hexs), 2))


def _kna(o) -> tuple:
    """(flags, cluster[3], preferred[3], sched, coop, prio, domain, map_def, map_rem, query, carveout)."""
    if not isinstance(o, dict):
        raise WriterError("attrs not an object")
    f, cl, pc = 0, [0, 0, 0], [0, 0, 0]
    sched = coop = prio = dom = mdef = mrem = query = carve = 0
    if "attrQueryAvailable" in o:
        f |= KNA_ATTR_QUERY_AVAILABLE
        if not isinstance(o["attrQueryAvailable"], bool):
            raise WriterError("attrQueryAvailable not a bool")
        query = 1 if o["attrQueryAvailable"] else 0
    if "clusterDimX" in o:
        f |= KNA_CLUSTER_DIM
        cl = [u32(_get(o, "clusterDim" + a)) for a in "XYZ"]
    if "preferredClusterDimX" in o:
        f |= KNA_PREFERRED_CLUSTER_DIM
        pc = [u32(_get(o, "preferredClusterDim" + a)) for a in "XYZ"]
    if "clusterSchedulingPolicyPreference" in o:
        f |= KNA_CLUSTER_SCHEDULING
        sched = i32(o["clusterSchedulingPolicyPreference"])
    if "cooperative" in o:
        f |= KNA_COOPERATIVE
        coop = i32(o["cooperative"])
    if "priority" in o:
        f |= KNA_PRIORITY
        prio = i32(o["priority"])
    if "memSyncDomain" in o:
        f |= KNA_MEM_SYNC_DOMAIN
        dom = i32(o["memSyncDomain"])
    if "memSyncDomainMapDefault" in o:
        f |= KNA_MEM_SYNC_DOMAIN_MAP
        mdef = i32(o["memSyncDomainMapDefault"]) & 0xFF
        mrem = i32(_get(o, "memSyncDomainMapRemote")) & 0xFF
    if "preferredSharedMemCarveout" in o:
        f |= KNA_SHARED_MEM_CARVEOUT
        carve = u32(o["preferredSharedMemCarveout"])
    return f, cl, pc, sched, coop, prio, dom, mdef, mrem, query, carve


def _kna_bytes(k) -> bytes:
    f, cl, pc, sched, coop, prio, dom, mdef, mrem, query, carve = k
    return struct.pack("<7I4i4BI", f, *cl, *pc, sched, coop, prio, dom, mdef, mrem, query, 0, carve)


def _serialise(v) -> str:
    def check(x):
        if isinstance(x, _Float):
            raise Unsupported(f"non-integer number {x.text}")
        if isinstance(x, bool) or x is None or isinstance(x, str):
            return
        if isinstance(x, int):
            if not -(1 << 63) <= x < (1 << 64):
                raise Unsupported(f"integer {x} beyond 64 bits")
        elif isinstance(x, list):
            for y in x:
                check(y)
        elif isinstance(x, dict):
            for y in x.values():
                check(y)

    check(v)
    return json.dumps(v, ensure_ascii=False, separators=(",", ":"))


def save_binary(text: bytes | str, key_override: bytes | None = None) -> bytes:
    """The archive bytes; key_override, if given, is written as the topology
    key instead of the document's."""
    root = parse(text)
    if not isinstance(root, dict):
        raise WriterError("document is not an object")
    nodes = _arr(_get(root, "nodes"))
    deps = _arr(root["dependencies"]) if "dependencies" in root else []
    gens = _arr(_get(root, "generators"))

    strings, interned = bytearray(), {}

    def intern(s: bytes) -> int:
        if s not in interned:
            interned[s] = len(strings)
            strings.extend(s + b"\0")
        return interned[s]

    key = _str(root["topology_key"]) if "topology_key" in root else b""
    if key_override is not None:
        key = key_override
    has_common = "common_kernel_node_attrs" in root
    common = _kna_bytes(_kna(root["common_kernel_node_attrs"])) if has_common else b""

    entries, pindex, pdata, adata = [], bytearray(), bytearray(), bytearray()
    for no in nodes:
        nid = u32(_get(no, "id"))
        t = _get(no, "type")
        if not isinstance(t, str):
            raise WriterError("type not a string")
        if t == "KernelNode":
            p = _get(no, "params")
            if not isinstance(p, dict):
                raise WriterError("params not an object")
            dims = [u32(_get(p, n)) for n in ("blockDimX", "blockDimY", "blockDimZ", "gridDimX", "gridDimY", "gridDimZ",
                                              "sharedMemBytes")]
            fn = _str(_get(p, "function_name"))
            name_off = intern(fn)
            bh = u64(_get(p, "kernel_source_binary_hash"))
            fa = [0] * 6
            if "func_attrs" in p:
                a = p["func_attrs"]
                fa = [i32(_get(a, "max_dynamic_shared_size_bytes")), i32(_get(a, "preferred_shared_memory_carveout"))]
                for n in ("cluster_scheduling_policy_preference", "required_cluster_width", "required_cluster_height",
                          "required_cluster_depth"):
                    fa.append(i32(a[n]) if isinstance(a, dict) and n in a else 0)
            kna = _kna(p["kernel_node_attrs"]) if "kernel_node_attrs" in p else _kna({})
            pio = len(pindex)
            kps = _arr(_get(p, "kernelParams"))
            for kp in kps:
                if not isinstance(kp, dict):
                    raise WriterError("param not an object")
                if "value_hex" in kp:
                    h = _str(kp["value_hex"])
                    pindex += struct.pack("<II", len(pdata) & 0xFFFFFFFF, len(h) // 2)
                    pdata += hex_decode(h)
                else:
                    pindex += struct.pack("<II", u32(_get(kp, "offset")), u32(_get(kp, "size")))
            extra = _str(p["extra_argBuffer_hex"]) if "extra_argBuffer_hex" in p else b""
            if extra:
                aoff, asz = len(adata), len(extra) // 2
                adata += hex_decode(extra)
            else:
                aoff, asz = NO_ARG, 0
            body = struct.pack("<7IQII6i", *dims, bh, name_off, len(fn), *fa) + _kna_bytes(kna)
            body += struct.pack("<4I", pio, len(kps), aoff, asz)
            assert len(body) == 136
            entries.append(struct.pack("<IB3x", nid, 0) + body)
        elif t == "MemcpyNode":
            p = _get(no, "params")
            g = lambda n: u64(_get(p, n))  # noqa: E731
            body = struct.pack("<10Q", g("Depth"), g("Height"), g("WidthInBytes"), g("dstDevice"), g("dstHeight"),
                               g("dstLOD"), g("dstPitch"), g("dstXInBytes"), g("dstY"), g("dstZ"))
            body += struct.pack("<ii", i32(_get(p, "dstMemoryType")), 0)
            body += struct.pack("<7Q", g("srcDevice"), g("srcHeight"), g("srcLOD"), g("srcPitch"), g("srcXInBytes"),
                                g("srcY"), g("srcZ"))
            body += struct.pack("<ii", i32(_get(p, "srcMemoryType")), 0)
            entries.append(struct.pack("<IB3x", nid, 2) + body)
        elif t == "MemsetNode":
            p = _get(no, "params")
            body = struct.pack("<QI4xQQI4xQ", u64(_get(p, "dst")), u32(_get(p, "elementSize")), u64(_get(p, "height")),
                               u64(_get(p, "pitch")), u32(_get(p, "value")), u64(_get(p, "width")))
            entries.append(struct.pack("<IB3x", nid, 1) + body)
        elif t in ("EventRecordNode", "EventWaitNode"):
            ev = i32(_get(_get(no, "params"), "event_id"))
            entries.append(struct.pack("<IB3xi", nid, 3 if t == "EventRecordNode" else 4, ev))
        elif t == "EmptyNode":
            entries.append(struct.pack("<IB3x", nid, 5))
        else:
            entries.append(struct.pack("<IB3x", nid, 0))
    entries = [e.ljust(ENTRY_SIZE, b"\0") for e in entries]

    dep_bytes = b"".join(struct.pack("<II", u32(_get(d, "from")), u32(_get(d, "to"))) for d in deps)
    gen_bytes = b"".join(struct.pack("<3Q", u64(_get(g, "id")), u64(_get(g, "seed")), u64(_get(g, "wholegraph_increment")))
                         for g in gens)
    events = _serialise(root["allocator_events"]).encode() if "allocator_events" in root else b""
    outputs = _serialise(root["output_tensors"]).encode() if "output_tensors" in root else b""

    secs = [bytes(strings), b"".join(entries), dep_bytes, bytes(pindex), bytes(pdata), bytes(adata), common,
            gen_bytes, events, outputs, key]
    off = HEADER_SIZE + NUM_SECTIONS * SECTION_SIZE
    table, body = b"", b""
    for i, s in enumerate(secs):
        table += struct.pack("<IIQQ", i, 0, off, len(s))
        pad = -len(s) % 8
        body += s + b"\0" * pad
        off += len(s) + pad
    flags = (1 if has_common else 0) | (2 if deps else 0) | (4 if events else 0) | (8 if outputs else 0) | \
            (16 if gens else 0)
    header = struct.pack("<8s7I28x", b"CUGRAPH\0", 1, flags, len(entries), len(deps), len(gens), NUM_SECTIONS,
                         len(interned))
    return header + table + body


def load_topology_key(text: bytes | str) -> bytes:
    """The key start_graph_builds groups a graph read from its JSON document
    by (csrc/CUDAGraphParallel.cpp:1791-1841), restated line by line:
    topology_key when present and non-empty (1796-1797); otherwise, per node,
    the type string (1802-1806), and for a KernelNode the cluster dims from
    kernel_node_attrs when it contains clusterDimX (1809-1816), else from
    common_kernel_node_attrs when x is still 0 (1817-1824), else each
    required_cluster_* field func_attrs contains, when x is still 0
    (1825-1832); ":C<x>_<y>_<z>" if any is nonzero, ":0" otherwise
    (1833-1838).  Numbers as to_number<unsigned int>."""
    root = parse(text)
    if not isinstance(root, dict):
        raise WriterError("document is not an object")
    if "topology_key" in root and _str(root["topology_key"]) != b"":
        return _str(root["topology_key"])
    parts = []
    for no in _arr(_get(root, "nodes")):
        t = _str(_get(no, "type"))
        if t != b"KernelNode":
            parts.append(t)
            continue
        cdx = cdy = cdz = 0
        p = _get(no, "params")
        if not isinstance(p, dict):
            raise WriterError("params not an object")
        if "kernel_node_attrs" in p:
            kna = p["kernel_node_attrs"]
            if not isinstance(kna, dict):
                raise WriterError("kernel_node_attrs not an object")
            if "clusterDimX" in kna:
                cdx, cdy, cdz = (u32(_get(kna, k)) for k in ("clusterDimX", "clusterDimY", "clusterDimZ"))
        if cdx == 0 and "common_kernel_node_attrs" in root:
            ck = root["common_kernel_node_attrs"]
            if not isinstance(ck, dict):
                raise WriterError("common_kernel_node_attrs not an object")
            if "clusterDimX" in ck:
                cdx, cdy, cdz = (u32(_get(ck, k)) for k in ("clusterDimX", "clusterDimY", "clusterDimZ"))
        if cdx == 0 and "func_attrs" in p:
            fa = p["func_attrs"]
            if not isinstance(fa, dict):
                raise WriterError("func_attrs not an object")
            if "required_cluster_width" in fa:
                cdx = u32(fa["required_cluster_width"])
            if "required_cluster_height" in fa:
                cdy = u32(fa["required_cluster_height"])
            if "required_cluster_depth" in fa:
                cdz = u32(fa["required_cluster_depth"])
        parts.append(t + (b":C%d_%d_%d" % (cdx, cdy, cdz) if (cdx or cdy or cdz) else b":0"))
    return b",".join(parts)


def load_archive(text: bytes | str) -> bytes:
    """The archive the product restores a graph read from its JSON document
    from: save_binary's, with load_topology_key's key as the topology key
    (the reference keeps that key beside the parsed document)."""
    return save_binary(text, key_override=load_topology_key(text))
