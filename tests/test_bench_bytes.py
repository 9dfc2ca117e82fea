"""The bench's algorithmic byte count for grouping + node passes, on images
the oracle's writer makes from documents whose node, dependency and kernel
name counts are known: 168 B per node entry, 8 B per dependency, 8 B plus the
name per kernel node, 24 B per graph.  No device needed."""
from __future__ import annotations

import json
import random

import numpy as np
import pytest

import bench
from graph_json import doc_of, sample_nodes
from oracle import writer as OW


@pytest.mark.parametrize("seed", range(4))
def test_image_hash_bytes_closed_form(seed):
    rng = random.Random(seed)
    nodes = sample_nodes(rng, 20 + 13 * seed)
    deps = [(i, i + 1) for i in range(0, len(nodes) - 1, 2)]
    img = OW.save_binary(json.dumps(doc_of(nodes, deps)))
    kernels = [n for n in nodes if n.type == 0]
    assert kernels and len(kernels) < len(nodes), "the sample mixes kernel and other nodes"
    want = 168 * len(nodes) + 8 * len(deps) + sum(8 + len(n.name.encode()) for n in kernels) + 24
    assert bench._image_hash_bytes(lambda off, n: img[off:off + n], np) == want
