"""Archives in which a member's word differs from its template's raw word
but equals it once relocated (the member holds the already relocated
pointer).  Such a word is a compared candidate of the member pass but makes
no override record, so the record bounds the search pass places records by
leave gaps that the finishing pass closes.  Test infrastructure."""
from __future__ import annotations

import struct

import numpy as np

import cugraph_reader as cr
import oracle


def image_word_positions(arc):
    """(image word index, byte offset in the file, param width) of every
    full 8-byte word of every PARAM_DATA param, in image order."""
    pd_off = arc.sections["PDATA"][0]
    out, w = [], 0
    for node in arc.nodes:
        if node.kernel is None:
            continue
        for sec, off, size in node.kernel.params:
            for b in range(0, size, 8):
                if sec == "PDATA" and size - b >= 8:
                    out.append((w, pd_off + off + b))
                w += 1
    return out


def plant_equal_after_relocation(images, iv, member, template, tiles, per_tile=2):
    """Rewrite words of graph `member` so that each equals the relocated
    value of its template's word (a pointer whose relocated value lies in no
    interval): `per_tile` words in each 4096-word tile listed in `tiles`
    (negative: from the last tile).  Returns the new images and the image
    word indices rewritten."""
    lo, hi, new_lo = iv
    mg = cr.read(images[member])
    tg = cr.read(images[template])
    pos_m = image_word_positions(mg)
    pos_t = dict(image_word_positions(tg))
    ntiles = (pos_m[-1][0] // 4096) + 1
    want = sorted({t % ntiles for t in tiles})
    data = bytearray(images[member])
    timg = images[template]
    planted = []
    for tile in want:
        n = 0
        for w, off in pos_m:
            if w // 4096 != tile or w not in pos_t:
                continue
            (raw_t,) = struct.unpack_from("<Q", timg, pos_t[w])
            (raw_m,) = struct.unpack_from("<Q", data, off)
            r = oracle.relocate_word(raw_t, lo, hi, new_lo)
            if r == raw_t or oracle.relocate_word(r, lo, hi, new_lo) != r or raw_m == r:
                continue
            struct.pack_into("<Q", data, off, r)
            planted.append(w)
            n += 1
            if n == per_tile:
                break
    out = list(images)
    out[member] = bytes(data)
    return out, planted
