"""Graph documents in the reference's JSON form (the object CUDAGraph::save
builds, csrc/CUDAGraph.cpp:1010-1491) for nodes of the test-side writer
(tests/cugraph_writer.py), so that the same graph exists as a JSON document
and as an archive written without the product or the oracle."""
from __future__ import annotations

import json
import random

import cugraph_writer as W


def kernel_json(k: W.Kernel, nid: int) -> dict:
    p = {
        "blockDimX": k.block[0], "blockDimY": k.block[1], "blockDimZ": k.block[2],
        "gridDimX": k.grid[0], "gridDimY": k.grid[1], "gridDimZ": k.grid[2],
        "sharedMemBytes": k.shmem, "function_name": k.name, "kernel_source_binary_hash": k.binary_hash,
        "func_attrs": dict(zip(("max_dynamic_shared_size_bytes", "preferred_shared_memory_carveout",
                                "cluster_scheduling_policy_preference", "required_cluster_width",
                                "required_cluster_height", "required_cluster_depth"), k.func_attrs)),
    }
    kna = {}
    if k.cluster is not None:
        kna.update(clusterDimX=k.cluster[0], clusterDimY=k.cluster[1], clusterDimZ=k.cluster[2])
    if k.cooperative is not None:
        kna["cooperative"] = k.cooperative
    if kna:
        p["kernel_node_attrs"] = kna
    p["kernelParams"] = [{"index": i, "offset": 0, "size": len(b), "value_hex": b.hex()} for i, b in enumerate(k.params)]
    p["extra_argBuffer_hex"] = k.arg.hex() if k.arg is not None else ""
    return {"id": nid, "type": "KernelNode", "params": p}


def node_json(n, nid: int) -> dict:
    if n.type == 0:
        return kernel_json(n, nid)
    if n.type == 1:
        return {"id": nid, "type": "MemsetNode", "params": {"dst": n.dst, "elementSize": n.element_size,
                                                             "height": n.height, "pitch": n.pitch, "value": n.value,
                                                             "width": n.width}}
    if n.type == 2:
        z = dict.fromkeys(("dstHeight", "dstLOD", "dstPitch", "dstXInBytes", "dstY", "dstZ", "srcHeight", "srcLOD",
                           "srcPitch", "srcXInBytes", "srcY", "srcZ"), 0)
        return {"id": nid, "type": "MemcpyNode", "params": {"Depth": 1, "Height": 1, "WidthInBytes": n.width_bytes,
                                                             "dstDevice": n.dst, "dstMemoryType": n.dst_type,
                                                             "srcDevice": n.src, "srcMemoryType": n.src_type, **z}}
    if n.type in (3, 4):
        return {"id": nid, "type": W.TYPE_NAMES[n.type], "params": {"event_id": n.event_id}}
    return {"id": nid, "type": "EmptyNode", "params": {}}


def sample_nodes(rng: random.Random, count: int) -> list:
    """Nodes the test writer and the JSON form both express (attribute ints
    as the JSON path stores them: zero unless present)."""
    names = ["gemm_bf16", "rmsnorm", "rope_q", "attn_decode", "silu_mul"]
    out = []
    for _ in range(count):
        t = rng.choice([0, 0, 0, 1, 2, 3, 4, 5])
        if t == 0:
            params = [bytes(rng.randrange(256) for _ in range(rng.choice([4, 8, 12, 16, 24, 64])))
                      for _ in range(rng.randrange(0, 5))]
            arg = bytes(rng.randrange(256) for _ in range(rng.choice([8, 40]))) if rng.random() < 0.2 else None
            cluster = (2, 1, 1) if rng.random() < 0.2 else None
            coop = rng.choice([None, None, 1])
            k = W.Kernel(rng.choice(names), rng.getrandbits(64), (rng.randrange(1, 999), 1, 2), (256, 1, 1),
                         [] if arg is not None else params, arg, rng.choice([0, 1024]), cluster, coop,
                         func_attrs=(rng.randrange(0, 9000), -1, 0, 0, 0, 0),
                         kna_ints=(0, coop if coop is not None else 0, 0, 0))
            out.append(k)
        elif t == 1:
            out.append(W.Memset(rng.getrandbits(48), rng.getrandbits(32), rng.randrange(1, 1 << 20)))
        elif t == 2:
            out.append(W.Memcpy(rng.getrandbits(48), rng.getrandbits(48), rng.randrange(1, 1 << 20)))
        elif t in (3, 4):
            ev = rng.randrange(0, 50)
            out.append(W.EventRecord(ev) if t == 3 else W.EventWait(ev))
        else:
            out.append(W.Empty())
    return out


def doc_of(nodes, deps, alloc=None, outputs=None, common=None) -> dict:
    doc = {"nodes": [node_json(n, i) for i, n in enumerate(nodes)],
           "dependencies": [{"from": a, "to": b} for a, b in deps], "generators": []}
    if alloc is not None:
        doc["allocator_events"] = alloc
    if outputs is not None:
        doc["output_tensors"] = outputs
    doc["topology_key"] = W.saved_key(nodes).decode()
    if common is not None:
        doc["common_kernel_node_attrs"] = {"clusterDimX": common[0], "clusterDimY": common[1], "clusterDimZ": common[2]}
    return doc


def compact(v) -> bytes:
    return json.dumps(v, separators=(",", ":")).encode()


