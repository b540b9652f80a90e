"""A CPU model of the apply's decoder and local-index pass on corrupted updates, under AddressSanitizer
and UBSan.

tests/sanitize/decode_model.cpp restates k_decode (decode_blocks in crukx-sync_amd/csrc/kernels.hip)
and k_local_fix, with the decoding tables built as engine.cpp's apply() builds them, and checks every
array access.  It is fed single-byte flips (three values each) of every header byte, both ends of every
block-table entry, the payload length and random payload bytes of a three-tensor update.  For every
flip the host parser accepts, the model must decode without an out-of-bounds access, and whenever it
raises no error flag the positions it produces must lie below 2^32 and increase strictly within each
group: the select pass (modelled in tests/select_model.py) then sees an ordinary update.
"""

from __future__ import annotations

import os
import random
import shutil
import struct
import subprocess

import numpy as np
import pytest
import torch

import oracle
import scenarios
from crukx_sync import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "crukx-sync_amd", "csrc")
pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++ with AddressSanitizer")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("decode_model") / "decode_model")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", f"-I{CSRC}", os.path.join(CSRC, "format.cpp"),
           os.path.join(ROOT, "tests", "sanitize", "decode_model.cpp"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out


def _varint_len(v: int) -> int:
    n = 1
    while v >= 0x80:
        v >>= 7
        n += 1
    return n


def test_corrupted_updates_decode_within_bounds(model, tmp_path):
    old, new = {}, {}
    for i, n in enumerate([60_000, 45_001, 4_097]):
        a, b = scenarios.rl_pair(n, lr=4e-6, seed=60 + i)
        old[f"t{i}"], new[f"t{i}"] = a, b
    upd = oracle.encode_update(old, new)
    sizes = np.zeros((len(old), 256), np.uint32)
    for t, v in enumerate(old.values()):
        sizes[t] = np.bincount((v.view(torch.int16).numpy().astype(np.int32) >> 7) & 0xFF, minlength=256)
    u = _native.lib()
    import ctypes
    h, err = ctypes.c_void_p(), ctypes.create_string_buffer(512)
    assert u.crx_parse(upd, len(upd), ctypes.byref(h), err, 512) == 0
    n_blocks, pay, pay_len = u.crx_update_n_blocks(h.value), u.crx_update_payload_offset(h.value), u.crx_update_payload_len(h.value)
    u.crx_update_free(h.value)
    bt = pay - _varint_len(pay_len) - 4 * n_blocks
    rnd = random.Random(3)
    offsets = list(range(bt))
    for b in range(n_blocks):
        offsets += [bt + 4 * b, bt + 4 * b + 3]
    offsets += list(range(bt + 4 * n_blocks, pay))
    offsets += rnd.sample(range(pay, len(upd)), min(2000, len(upd) - pay))
    inputs = [upd]
    for i in offsets:
        for x in (0x01, 0x80, 0xFF):
            d = bytearray(upd)
            d[i] ^= x
            inputs.append(bytes(d))
    path = tmp_path / "batch.bin"
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(old)))
        f.write(sizes.tobytes())
        for d in inputs:
            f.write(struct.pack("<Q", len(d)))
            f.write(d)
    r = subprocess.run([model, str(path)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    out = [int(x) for x in r.stdout.split()]
    assert len(out) == len(inputs)
    assert out[0] == 0  # the clean update: in-range, ordered positions
    assert -2 not in out, [offsets[(j - 1) // 3] for j, v in enumerate(out) if v == -2][:5]
    assert not any(v > 0 and v & (8 | 16) for v in out)
    decoded = sum(1 for v in out[1:] if v == 0)
    assert decoded > 0 and sum(1 for v in out if v == -1) > 0  # both kinds are exercised
