"""The oracle's CRC-64/XZ against the textbook check value and a bit-serial
restatement (tests/refcrc.py)."""
import random

import oracle
from tests.refcrc import crc64_xz


def test_check_value():
    assert crc64_xz(b"123456789") == 0x995DC9BBDF1939FA
    assert oracle.crc64(b"123456789") == 0x995DC9BBDF1939FA


def test_empty_and_single_bytes():
    assert oracle.crc64(b"") == crc64_xz(b"") == 0
    for b in range(256):
        assert oracle.crc64(bytes([b])) == crc64_xz(bytes([b]))


def test_random_inputs():
    rng = random.Random(0x5EED)
    for _ in range(40):
        data = bytes(rng.getrandbits(8) for _ in range(rng.randrange(1, 700)))
        assert oracle.crc64(data) == crc64_xz(data)


def test_long_run():
    data = bytes(range(256)) * 64 + b"\0" * 1000
    assert oracle.crc64(data) == crc64_xz(data)
