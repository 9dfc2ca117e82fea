"""CRC-64/XZ one bit at a time, from its textbook definition (test
infrastructure): width 64, polynomial 0x42F0E1EBA9EA3693 processed
reflected (0xC96C5795D7870F42), initial value and final xor all ones; the
catalogue check value is crc(b"123456789") = 0x995DC9BBDF1939FA.  It is the
hash of the reference's csrc/hook.cpp:315-321 (Boost crc_optimal<64,
0x42F0E1EBA9EA3693, ~0, ~0, true, true>) and shares no table or code with
the oracle's or the product's CRC."""

POLY_REFLECTED = 0xC96C5795D7870F42
MASK = (1 << 64) - 1


def crc64_xz(data: bytes) -> int:
    crc = MASK
    for byte in data:
        crc ^= byte
        for _ in range(8):
            crc = (crc >> 1) ^ (POLY_REFLECTED if crc & 1 else 0)
    return crc ^ MASK
