"""Writes tests/golden/hostile_headers.json: the malformed updates the reference's own tests feed its
parser (the reference's tests/test_roundtrip.py:109-135), as data.

Each is one tensor "w" of 100 elements (checksum 0) behind a table section; the cases differ in the
table section and in what follows the tensor's checksum.  They are built here field by field from the
format (magic "CRXS", version 2, LEB128 varints; a table is exponent, symbol count, then (symbol,
code length) pairs; a group is exponent, change count, Rice parameter), not run from the reference.
Usage:  python tests/golden/make_hostile.py
"""

from __future__ import annotations

import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def varint(v: int) -> bytes:
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        out.append(b | (0x80 if v else 0))
        if not v:
            return bytes(out)


def tables(*specs) -> bytes:
    """specs: (exponent, [(symbol, code length), ...])"""
    out = varint(len(specs))
    for exp, codes in specs:
        out += bytes([exp]) + varint(len(codes))
        for sym, length in codes:
            out += varint(sym) + bytes([length])
    return out


def groups(*specs) -> bytes:
    """specs: (exponent, count, rice parameter)"""
    out = varint(len(specs))
    for exp, count, rice in specs:
        out += bytes([exp]) + varint(count) + bytes([rice])
    return out


def update(table_section: bytes, after_checksum: bytes) -> bytes:
    return b"CRXS\x02" + table_section + varint(1) + varint(1) + b"w" + varint(100) + bytes(8) + after_checksum


ONE = tables((0, [(2, 1)]))  # exponent 0: symbol 2 with a 1-bit code
CASES = [
    ("one table whose symbol count is a ten-byte varint of at least 2^63", b"\x01\x00" + b"\xff" * 9 + b"\x7f", b""),
    # (read as a header, these bytes are one group of one change followed by the bytes of varint(2^62)
    # where the block table and the payload belong)
    ("one group of one change, then varint(2^62) for block table and payload", ONE,
     groups((0, 1, 0)) + varint(1 << 62) + b"\x00"),
    ("Rice parameter 31", ONE, groups((0, 5, 31))),
    ("no groups", ONE, groups()),
    ("two 1-bit codes and nothing after the header", tables((0, [(1, 1), (2, 1)])), b""),
    ("two groups of exponent 0", ONE, groups((0, 5, 0), (0, 5, 0))),
    ("a group of exponent 7, which has no table", ONE, groups((7, 5, 0))),
]


def main():
    out = {"source": "the reference's tests/test_roundtrip.py:109-135 (test_hostile_headers_fail_fast)",
           "cases": [{"what": what, "hex": update(t, rest).hex()} for what, t, rest in CASES]}
    with open(os.path.join(HERE, "hostile_headers.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
