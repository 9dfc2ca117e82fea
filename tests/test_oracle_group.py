"""Oracle grouping: key grouping against brute force, manifest grouping
against the rules of csrc/CUDAGraphParallel.cpp:1727-1786 written out by
hand."""
import json
import random

import oracle

NONE = 0xFFFFFFFF


def brute_force(keys):
    # template_for[i] = lowest index with the same key (1844-1850)
    return [min(j for j in range(len(keys)) if keys[j] == keys[i]) for i in range(len(keys))]


def test_key_grouping_brute_force():
    rng = random.Random(7)
    alphabet = [b"", b"KernelNode:0", b"KernelNode:0,MemsetNode", b"KernelNode:C2_1_1", b"KernelNode:0,"]
    for _ in range(300):
        keys = [rng.choice(alphabet) for _ in range(rng.randrange(1, 13))]
        assert oracle.group_by_keys(keys).tolist() == brute_force(keys)


def test_key_grouping_is_exact_string_equality():
    keys = [b"KernelNode:0", b"KernelNode:0 ", b"kernelnode:0", b"KernelNode:0"]
    assert oracle.group_by_keys(keys).tolist() == [0, 1, 2, 0]


def manifest(groups):
    return json.dumps({"topology_groups": groups}).encode()


NAMES = [f"graph_{i}.json" for i in range(6)]


def test_manifest_groups():
    m = manifest([
        {"topology_key": "k0", "template": "graph_0.json", "members": ["graph_0.json", "graph_2.json", "graph_4.json"]},
        {"topology_key": "k1", "template": "graph_1.json", "members": ["graph_1.json", "graph_3.json"]},
    ])
    # members point at their template; templates and unlisted graphs build their own exec
    assert oracle.group_manifest(m, NAMES).tolist() == [NONE, NONE, 0, 1, 0, NONE]


def test_manifest_unknown_template_skips_group():
    m = manifest([{"template": "graph_9.json", "members": ["graph_9.json", "graph_2.json"]},
                  {"template": "graph_1.json", "members": ["graph_5.json", "graph_nope.json"]}])
    assert oracle.group_manifest(m, NAMES).tolist() == [NONE, NONE, NONE, NONE, NONE, 1]


def test_manifest_later_group_wins_and_template_can_be_a_member():
    m = manifest([
        {"template": "graph_0.json", "members": ["graph_1.json", "graph_2.json"]},
        {"template": "graph_1.json", "members": ["graph_2.json", "graph_3.json"]},
    ])
    # graph_1 stays a member of group 0 although it templates group 1;
    # graph_2 is reassigned by the later group.
    assert oracle.group_manifest(m, NAMES).tolist() == [NONE, 0, 1, 1, NONE, NONE]


def test_manifest_parse_failures_fall_back():
    bad = [b"{", b"[]", b"{}", manifest([{"members": []}]), manifest([{"template": "graph_0.json"}]),
           manifest([{"template": 3, "members": []}]), manifest([{"template": "graph_0.json", "members": [1]}]),
           manifest(["graph_0.json"])]
    for m in bad:
        assert oracle.group_manifest(m, NAMES) is None, m


def test_manifest_empty_groups_list():
    assert oracle.group_manifest(manifest([]), NAMES).tolist() == [NONE] * 6


def test_manifest_unknown_template_is_skipped_before_its_members_are_read():
    # csrc/CUDAGraphParallel.cpp:1752-1760: the template lookup `continue`s before
    # group.at("members") is reached, so a bad members entry there does not throw.
    m = manifest([{"template": "graph_9.json", "members": 7},
                  {"template": "graph_0.json", "members": ["graph_3.json"]}])
    assert oracle.group_manifest(m, NAMES).tolist() == [NONE, NONE, NONE, 0, NONE, NONE]


def test_digest_collisions_group_by_exact_bytes():
    """Two keys with equal CRC-64/XZ and length but other bytes stay apart,
    and the graph that met a colliding lower key is flagged (0x08)."""
    import collision_cases as CC

    r = oracle.Restore(CC.images())
    assert r.groups().tolist() == CC.TEMPLATE_OF
    assert r.status().tolist() == CC.STATUS
    d = r.digests()
    assert d[0, 0] == d[1, 0]  # the forged key really collides
