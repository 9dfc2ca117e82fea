"""The allocation region as a planning region (placement arithmetic, no device): the
reference's cursor rules (csrc/hook.cpp:2272-2291, 2424, 2705-2721), the
saved event format (3354-3392) and the replay (3394-3492), checked against
hand-computed sequences and against the oracle's restatement."""
import json
import random

import numpy as np
import pytest

import oracle
from foundry_amd import _lib
from foundry_amd.region import MiB, Region

B1 = 0x500000000000  # the reference's default region base (csrc/hook.cpp:201)
B2 = 0x6A0000000000
GiB = 1 << 30


def _dry(base=B1, size=GiB):
    return Region.plan(base, base, size)


def test_placements_follow_the_cursor_rule():
    r = _dry()
    r.record(True)
    a = r.alloc(100)            # at the cursor; cursor -> align_up(ptr + 100, 2 MiB)
    b = r.alloc(3 * MiB)        # next 2 MiB boundary
    c = r.reserve(16 * MiB, 8 * MiB)   # carved at the next 8 MiB boundary
    d = r.alloc(2 * MiB)
    assert [x - B1 for x in (a, b, c, d)] == [0, 2 * MiB, 8 * MiB, 24 * MiB]
    assert r.offset == 26 * MiB
    r.free(b)
    assert r.alloc(1) - B1 == 26 * MiB  # the cursor never moves back into freed space
    info = r.info()
    assert info["live_allocations"] == 3 and info["num_events"] == 6  # reserves are not allocations


def test_saved_event_text_is_the_reference_format():
    r = _dry()
    r.record(True)
    a = r.alloc(100)
    c = r.reserve(4 * MiB, 2 * MiB)
    r.free(a)
    text = r.events_json()
    assert text == (
        '{"start_base_addr":%d,"events":[{"type":"alloc","size":100,"ptr":%d},'
        '{"type":"reserve","size":%d,"ptr":%d,"alignment":%d},{"type":"free","ptr":%d}]}'
        % (B1, a, 4 * MiB, c, 2 * MiB, a)
    )
    assert json.loads(text)["events"][1]["alignment"] == 2 * MiB


def test_replay_at_another_base_keeps_offsets_and_gives_the_intervals():
    src = _dry()
    src.alloc(7 * MiB)              # allocations before recording (model weights)
    src.record(True)
    p1 = src.alloc(5000)
    p2 = src.reserve(6 * MiB, 4 * MiB)
    p3 = src.alloc(64 * MiB)
    src.free(p1)
    text = src.events_json()

    dst = Region.plan(B1, B2, GiB)  # saved at B1, placed at B2
    dst.alloc(7 * MiB)
    dst.replay(text)
    lo, hi, nlo = dst.intervals(per_allocation=True)
    rows = [tuple(int(x) for x in t) for t in zip(lo, hi, nlo)]
    assert rows == [
        (B1, B1 + 7 * MiB, B2),
        (p1, p1 + 5000, p1 - B1 + B2),
        (p2, p2 + 6 * MiB, p2 - B1 + B2),
        (p3, p3 + 64 * MiB, p3 - B1 + B2),
    ]
    assert p2 - B1 == 12 * MiB  # 8 MiB + 2 MiB rounded to the 4 MiB alignment
    lo, hi, nlo = dst.intervals()
    assert (lo.tolist(), hi.tolist(), nlo.tolist()) == ([B1], [B1 + GiB], [B2])
    assert dst.info()["live_allocations"] == 2  # p1 was freed by the replay


def test_replay_refuses_what_the_reference_aborts_on():
    src = _dry()
    src.record(True)
    src.alloc(MiB)
    text = src.events_json()
    dst = _dry()
    dst.alloc(3 * MiB)  # more was allocated before the graph than at SAVE
    with pytest.raises(_lib.FoundryError, match="FDY_E_MISMATCH"):
        dst.replay(text)
    d = json.loads(text)
    d["events"][0]["ptr"] += 2 * MiB  # saved at another offset than the rule places it
    with pytest.raises(_lib.FoundryError, match="FDY_E_MISMATCH"):
        _dry().replay(json.dumps(d))
    with pytest.raises(_lib.FoundryError, match="FDY_E_FORMAT"):
        _dry().replay('{"events":[{"type":"alloc","ptr":1}]}')
    with pytest.raises(_lib.FoundryError, match="FDY_E_FORMAT"):
        _dry().replay('{"start_base_addr":')


def test_reference_text_with_whitespace_and_free_of_unknown_pointer():
    text = """{ "start_base_addr": %d,
               "events": [ {"type": "alloc", "size": 4096, "ptr": %d},
                           {"type": "free", "ptr": 12345} ] }""" % (B1 + 2 * MiB, B1 + 2 * MiB)
    r = _dry()
    r.replay(text)  # the unknown free is skipped, as the reference reports and continues
    assert r.offset == 4 * MiB


def test_preallocation_places_identically_without_new_mappings():
    r, q = _dry(), _dry()
    r.preallocate(32 * MiB)
    sizes = [1, 3 * MiB, 100, 5 * MiB, 9 * MiB]
    assert [r.alloc(s) for s in sizes] == [q.alloc(s) for s in sizes]
    info = r.info()
    assert info["prealloc_end"] - info["prealloc_begin"] == 32 * MiB
    # inside the preallocation nothing else is mapped (the last alloc ends at 23 MiB)
    assert info["mapped_bytes"] == 32 * MiB
    with pytest.raises(_lib.FoundryError, match="FDY_E_NOMEM"):
        r.alloc(40 * MiB)  # would start inside (at 24 MiB) and run past the end
    assert r.offset == 24 * MiB  # a refused allocation leaves the cursor
    last = r.alloc(8 * MiB)  # exactly fills the rest
    after = r.alloc(MiB)     # wholly past the preallocation: a mapping of its own
    assert last - B1 == 24 * MiB and after - B1 == 32 * MiB
    assert r.info()["mapped_bytes"] == 32 * MiB + 2 * MiB
    with pytest.raises(_lib.FoundryError, match="FDY_E_STATE"):
        r.free_preallocated()  # allocations still live inside it


def test_cursor_rules_and_errors():
    r = _dry(size=64 * MiB)
    r.offset = 10 * MiB
    with pytest.raises(_lib.FoundryError, match="FDY_E_INVALID"):
        r.offset = 4 * MiB  # never backward
    with pytest.raises(_lib.FoundryError, match="FDY_E_RANGE"):
        r.offset = 65 * MiB
    with pytest.raises(_lib.FoundryError, match="FDY_E_NOMEM"):
        r.alloc(60 * MiB)
    with pytest.raises(_lib.FoundryError, match="FDY_E_RANGE"):
        r.free(B1 + 12345)
    with pytest.raises(_lib.FoundryError, match="FDY_E_INVALID"):
        r.reserve(MiB, 3 * MiB)  # alignment not a power of two
    big = _dry(size=8 * GiB)
    with pytest.raises(_lib.FoundryError, match="FDY_E_UNSUPPORTED"):
        big.reserve(2 * GiB, 2 * MiB)
    with pytest.raises(_lib.FoundryError, match="FDY_E_INVALID"):
        Region.plan(B1 + 4096, B1, GiB)  # base not 2 MiB aligned


def test_oracle_replay_matches_hand_placements():
    """Pins the oracle: the placements of the hand sequence above."""
    text = ('{"start_base_addr":%d,"events":[{"type":"alloc","size":100,"ptr":%d},'
            '{"type":"alloc","size":%d,"ptr":%d},{"type":"reserve","size":%d,"ptr":%d,"alignment":%d},'
            '{"type":"alloc","size":%d,"ptr":%d}]}'
            % (B1, B1, 3 * MiB, B1 + 2 * MiB, 16 * MiB, B1 + 8 * MiB, 8 * MiB, 2 * MiB, B1 + 24 * MiB))
    rows, cur = oracle.region_replay(text, B1, B2, GiB, B2)
    assert cur == B2 + 26 * MiB
    assert [tuple(int(x) for x in r) for r in rows] == [
        (B1, B1 + 100, B2), (B1 + 2 * MiB, B1 + 5 * MiB, B2 + 2 * MiB),
        (B1 + 8 * MiB, B1 + 24 * MiB, B2 + 8 * MiB), (B1 + 24 * MiB, B1 + 26 * MiB, B2 + 24 * MiB)]
    bad = text.replace('"ptr":%d}' % (B1 + 2 * MiB), '"ptr":%d}' % (B1 + 4 * MiB))
    assert oracle.region_replay(bad, B1, B2, GiB, B2)[0] == -2
    assert oracle.region_replay(text, B1, B2, GiB, B2 + 2 * MiB)[0] == -2  # cursor ahead of the saved start
    assert oracle.region_replay("{", B1, B2, GiB, B2)[0] == -1


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5])
def test_random_sequences_agree_with_the_oracle(seed):
    rng = random.Random(seed)
    src = _dry(size=64 * GiB)
    src.alloc(rng.randrange(1, 50 * MiB))
    src.record(True)
    live = []
    for _ in range(200):
        k = rng.random()
        if k < 0.6:
            live.append(src.alloc(rng.choice([rng.randrange(1, 4096), rng.randrange(1, 64 * MiB)])))
        elif k < 0.75:
            src.reserve(rng.randrange(1, 32 * MiB), 1 << rng.randrange(21, 27))
        elif live:
            src.free(live.pop(rng.randrange(len(live))))
    text = src.events_json()
    rows, cur = oracle.region_replay(text, B1, B2, 64 * GiB, B2)
    assert not isinstance(rows, int)
    # The product replays the same text on a planning region saved at B1 and
    # placed at B2, and must place everything where the oracle does.
    dst = Region.plan(B1, B2, 64 * GiB)
    dst.replay(text)
    lo, hi, nlo = dst.intervals(per_allocation=True)
    got = np.stack([lo, hi, nlo], axis=1)
    np.testing.assert_array_equal(got, rows.astype(np.uint64))
    assert dst.offset == cur - B2
