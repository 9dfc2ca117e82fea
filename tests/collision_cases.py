"""Archives whose saved topology keys collide under CRC-64/XZ (equal digest
and length, other bytes), built with tests/refcrc.forge_collision.  The
reference partitions graphs by exact key string (csrc/CUDAGraphParallel.cpp:
1788-1851), so colliding keys form separate groups."""
import cugraph_writer as W
from cugraph_writer import le
from refcrc import crc64_xz, forge_collision

KEY = b"KernelNode:0,KernelNode:C2_1_1,KernelNode:0"
FORGED = forge_collision(KEY)
OTHER = b"KernelNode:0,KernelNode:0,KernelNode:0"
KEYS = [KEY, FORGED, KEY, FORGED, OTHER]
# Hand-derived: graphs 0/2 and 1/3 pair up by exact bytes; 1 and 3 each
# pass graph 0's colliding key on the way to their template (status bit 0x08).
TEMPLATE_OF = [0, 1, 0, 1, 4]
STATUS = [0, 8, 0, 8, 0]


def images():
    assert crc64_xz(FORGED) == crc64_xz(KEY) and len(FORGED) == len(KEY) and FORGED != KEY
    out = []
    for g, key in enumerate(KEYS):
        nodes = [W.Kernel("k_a", 0x1234, params=[le(0x7F0000001000 + 8 * n), le(g + n)]) for n in range(3)]
        out.append(W.write(nodes, key=key))
    return out
