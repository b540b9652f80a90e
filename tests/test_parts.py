"""Updates encoded and applied part by part, on the GPU.

An update of 2^32 or more changes is split into parts of consecutive tensors (at most 2^31 elements
each, a larger tensor alone): encode ranks each part for the whole update's symbol counts, builds the
tables, then codes each part at its bit offset in the one payload (the reference packs batches of
changes the same way, codec.py:214,337-341,394-410); apply verifies every part without writing, takes
the verdict on the whole update, then writes part by part.  CRX_PART_ELEMENTS makes the library split
any update larger than it, so these tests check the part-wise path against the reference's own bytes
(the golden vectors) at small sizes; test_full_sizes.py holds the update of more than 2^32 changes.
"""

import hashlib

import pytest
import torch

import crukx_sync
import scenarios
from crukx_sync import CorruptUpdate

pytestmark = pytest.mark.gpu


def _dev(state: dict) -> dict:
    return {k: v.to("cuda") for k, v in state.items()}


def _equal(x: dict, y: dict) -> bool:
    return all(torch.equal(x[k].view(torch.int16), y[k].view(torch.int16)) for k in y)


def _sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


@pytest.mark.parametrize("name,part", [("many_tensors", 60_000), ("three_tensors", 60_000), ("three_tensors", 1),
                                       ("sweep_rho0.01_p0.87", 1_000_000), ("edges", 1_000_000)])
def test_part_wise_bytes_are_the_reference_bytes(golden, monkeypatch, name, part):
    """Parts of one to three tensors (part=1: every tensor alone): the bytes of encode_update and
    encode_update_device are the reference's, and both apply exactly."""
    monkeypatch.setenv("CRX_PART_ELEMENTS", str(part))
    old, new = (_dev(s) for s in scenarios.single_scenarios()[name])
    want = golden["updates"]["single"][name]["update"]["sha256"]
    upd = crukx_sync.encode_update(old, new)
    assert _sha(upd) == want
    dev = crukx_sync.encode_update_device(old, new)
    assert _sha(bytes(dev.cpu().numpy())) == want
    for u in (upd, dev):
        w = {k: v.clone() for k, v in old.items()}
        crukx_sync.apply_update(w, u)
        assert _equal(w, new)


def test_part_wise_chain_with_caches_and_a_corrupted_last_part(golden, monkeypatch):
    """The four-tensor chain in two parts (the 16.8M-element tensor, then the other three): every step's
    bytes are the reference's with the sender's cache, applies with both caches (checksums and the
    receiver's exponent counts) are exact, and a byte flipped in the last part's payload is rejected
    with all four tensors unchanged: the verdict is taken before any part is written."""
    monkeypatch.setenv("CRX_PART_ELEMENTS", "17000000")
    rec = golden["updates"]["chains"]["small4_chain"]
    states = [_dev(s) for s in scenarios.chain_small4(3)]
    send, rc = {}, {}
    w = {k: v.clone() for k, v in states[0].items()}
    for s in range(1, len(states)):
        upd = crukx_sync.encode_update(states[s - 1], states[s], send)
        assert _sha(upd) == rec["steps"][s - 1]["update"]["sha256"], s
        assert send == rec["steps"][s - 1]["sender_checksums"], s
        rejected = 0
        for k in (2, 3, 5, 9):  # bytes near the payload's end: blocks of the last part
            bad = bytearray(upd)
            bad[-k] ^= 0x10
            try:
                crukx_sync.apply_update(w, bytes(bad), rc)
            except CorruptUpdate:
                rejected += 1
            else:  # a harmless flip applies exactly; go back
                assert _equal(w, states[s])
                for n in w:
                    w[n].copy_(states[s - 1][n])
                rc.clear()
            assert _equal(w, states[s - 1]), (s, k)
        assert rejected >= 3
        crukx_sync.apply_update(w, upd, rc)
        assert _equal(w, states[s]), s
    assert send == {k: v[0] for k, v in rc.items()}
