"""The library's own kernels and host code on the CPU, under AddressSanitizer and UBSan.

tests/model/ builds crukx-sync_amd/csrc (kernels.hip, engine.cpp, format.cpp) as plain C++ against a
host stand-in for the HIP runtime and a wave64 emulator (tests/model/simt.cpp): every work-item is a
fiber, the lanes of a wavefront meet at each ballot, lane read, shuffle and fence, and every memory
access of the kernels is checked.  tests/model/run.py drives crukx_sync's unchanged Python layer on it,
with device memory in host memory that starts as all ones.  These tests need no GPU:

- the model's bytes equal the oracle's on every small scenario (encode and the device-resident form),
  and its applies are exact: the emulator runs the kernels as the GPU does;
- updates that the decoder rejects, on multi-slab tensors with warm caches, raise and leave the receiver
  as it was, with no access outside any buffer.  Before the undo pass was fixed this faulted: it read
  the record offsets that the locate pass does not write for an update already rejected, and all-ones
  offsets wrapped its 32-bit range start (the GPU fault of the four-tensor corruption test);
- the group-size check covers tensors of more than codec._SLAB elements, as in the reference.

The whole four-tensor corruption sequence (`run.py small4_flips`, about 13,500 flips) takes hours on the
model and is run outside the suite.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model")
sys.path.insert(0, HERE)
import run  # noqa: E402

pytestmark = pytest.mark.skipif(not os.path.exists(run.CLANG) or shutil.which("make") is None,
                                reason="needs ROCm's clang++ (host build with AddressSanitizer)")


@pytest.fixture(scope="module")
def model():
    return run.build()


def _run(lib: str, scenario: str) -> str:
    r = subprocess.run([sys.executable, os.path.join(HERE, "run.py"), scenario], env=run.env(lib),
                       capture_output=True, text=True, timeout=1500)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-6000:])
    return r.stdout


def test_model_bytes_and_applies_match_the_oracle(model):
    out = _run(model, "parity")
    assert out.count("parity ") >= 25


def test_updates_rejected_by_the_decoder_write_nothing(model):
    out = _run(model, "rejected_early")
    assert "updates rejected, the receiver unchanged each time" in out


def test_group_size_check_follows_the_slab_knob(model):
    out = _run(model, "group_message")
    assert "group has more changes than elements" in out


def test_device_resident_update_read_in_place_at_any_offset(model):
    """The decoder reads a device-resident payload in place from its aligned words when the update's
    allocation covers them (the model's allocations are the sanitizer's, so a read past one is
    reported), and from a copy when not."""
    out = _run(model, "device_offsets")
    assert "device offsets: 12 applies exact" in out


def test_part_wise_encode_and_apply_match_the_oracle(model):
    """CRX_PART_ELEMENTS splits updates into parts of one to three tensors: the bytes are the oracle's
    single-pass bytes, chained applies with both caches are exact, and a corruption in the last part is
    rejected by the verification of the whole update with every tensor unchanged."""
    out = _run(model, "parts")
    assert out.count("chained applies exact") == 2 and out.count("rejected by the device passes") == 2
