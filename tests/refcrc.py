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


def forge_collision(data: bytes, change_at: int = 0) -> bytes:
    """Another message of the same length and the same CRC-64/XZ: byte
    `change_at` is flipped, then the last 8 bytes are solved for.  For a
    fixed length the CRC is affine in the message bits, crc(p || s) =
    A s xor crc(p || 0), and A (64 x 64 over GF(2)) is invertible, so
    s = A^-1 (crc(data) xor crc(p || 0)) by Gaussian elimination."""
    assert len(data) >= 9 and change_at < len(data) - 8
    target = crc64_xz(data)
    prefix = bytearray(data[:-8])
    prefix[change_at] ^= 0xFF
    base = crc64_xz(bytes(prefix) + bytes(8))
    cols = [crc64_xz(bytes(prefix) + (1 << k).to_bytes(8, "little")) ^ base for k in range(64)]
    # Solve sum over k of s_k * cols[k] = target ^ base: rows are CRC bits.
    rows = []
    for bit in range(64):
        r = 0
        for k in range(64):
            r |= ((cols[k] >> bit) & 1) << k
        rows.append([r, ((target ^ base) >> bit) & 1])
    piv = 0
    where = [-1] * 64
    for k in range(64):
        sel = next((i for i in range(piv, 64) if (rows[i][0] >> k) & 1), None)
        if sel is None:
            continue
        rows[piv], rows[sel] = rows[sel], rows[piv]
        for i in range(64):
            if i != piv and (rows[i][0] >> k) & 1:
                rows[i][0] ^= rows[piv][0]
                rows[i][1] ^= rows[piv][1]
        where[k] = piv
        piv += 1
    assert piv == 64, "singular system"
    sol = sum(rows[where[k]][1] << k for k in range(64))
    out = bytes(prefix) + sol.to_bytes(8, "little")
    assert crc64_xz(out) == target and out != data
    return out
