"""The torch-CPU restatement of the reference's CPU path (oracle/torch_cpu.py), which bench.py times
as its CPU baseline, is checked here before anything trusts its timings: its bytes equal the
reference's own bytes on every golden scenario and over the chained 26.6M-weight steps with caches,
it applies them exactly, and its slab size (the reference's _SLAB) never changes the bytes.
"""

import hashlib

import pytest
import torch

import oracle
import scenarios
import torch_cpu


_SC = {}


def _scen():
    if not _SC:
        _SC.update(scenarios.single_scenarios())
    return _SC


def _sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


def _equal(x, y):
    return all(torch.equal(x[k].view(torch.int16), y[k].view(torch.int16)) for k in y)


@pytest.mark.parametrize("name", sorted(scenarios.single_scenarios().keys()))
def test_bytes_and_round_trip_equal_reference(golden, name):
    old, new = _scen()[name]
    rec = golden["updates"]["single"][name]
    chk = {}
    upd = torch_cpu.encode_update(old, new, chk)
    assert len(upd) == rec["update"]["len"] and _sha(upd) == rec["update"]["sha256"]
    assert chk == rec["sender_checksums"]
    w = {k: v.clone() for k, v in old.items()}
    assert torch_cpu.apply_update(w, upd) == oracle.apply_update({k: v.clone() for k, v in old.items()}, upd)
    assert _equal(w, new)


def test_chained_steps_with_caches(golden):
    rec = golden["updates"]["chains"]["small4_chain"]
    states = scenarios.chain_small4(3)
    send, recv = {}, {}
    w = {k: v.clone() for k, v in states[0].items()}
    for s in range(1, len(states)):
        upd = torch_cpu.encode_update(states[s - 1], states[s], send)
        assert _sha(upd) == rec["steps"][s - 1]["update"]["sha256"], s
        assert send == rec["steps"][s - 1]["sender_checksums"]
        torch_cpu.apply_update(w, upd, recv)
        assert _equal(w, states[s]), s
    assert send == recv


@pytest.mark.parametrize("slab", [128, 1000, 4096])
def test_slab_size_never_changes_bytes(golden, monkeypatch, slab):
    """Multi-slab ranking and selection (the reference's sorts are cut at 2^24 elements)."""
    monkeypatch.setattr(torch_cpu, "SLAB", slab)
    for name in ("slab_12293", "rl_200k", "edges", "every_element_arbitrary"):
        old, new = _scen()[name]
        upd = torch_cpu.encode_update(old, new)
        assert _sha(upd) == golden["updates"]["single"][name]["update"]["sha256"], name
        w = {k: v.clone() for k, v in old.items()}
        torch_cpu.apply_update(w, upd)
        assert _equal(w, new), name


def test_checksum_and_rejections():
    a, b = scenarios.rl_pair(30_000, seed=3)
    assert torch_cpu.checksum(b) == oracle.checksum(b)
    upd = bytearray(torch_cpu.encode_update({"w": a}, {"w": b}))
    for i in range(len(upd) - 1, len(upd) - 60, -3):  # payload flips: rejected with old kept, or exact
        bad = bytearray(upd)
        bad[i] ^= 0x20
        w = {"w": a.clone()}
        try:
            torch_cpu.apply_update(w, bytes(bad))
        except ValueError:
            assert torch.equal(w["w"].view(torch.int16), a.view(torch.int16))
        else:
            assert torch.equal(w["w"].view(torch.int16), b.view(torch.int16))
    w = {"w": a.clone()}
    with pytest.raises(ValueError):  # a wrong receiver cache
        torch_cpu.apply_update(w, bytes(upd), {"w": 12345})
    assert torch.equal(w["w"].view(torch.int16), a.view(torch.int16))


def test_shared_sorts_of_many_small_tensors():
    """Hundreds of small tensors ranked in shared sorts (groups cut by tensor count and by size), with
    a large tensor between them: the same bytes as the oracle, which ranks tensor by tensor, and an
    exact apply; the grouping never changes the bytes."""
    g = torch.Generator().manual_seed(7)
    old, new = {}, {}
    for i in range(300):
        n = int(torch.randint(1, 3000, (1,), generator=g)) if i != 150 else 70_000
        a = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
        b = a.clone()
        k = torch.randperm(n, generator=g)[:max(1, n // 50)]
        b.view(torch.int16)[k] += torch.randint(-3, 4, (k.numel(),), generator=g, dtype=torch.int16)
        old[f"t{i}"], new[f"t{i}"] = a, b
    want = oracle.encode_update(old, new)
    assert torch_cpu.encode_update(old, new) == want
    w = {k: v.clone() for k, v in old.items()}
    torch_cpu.apply_update(w, want)
    assert _equal(w, new)
    grouped = torch_cpu._small_groups([t.numel() for t in old.values()])
    assert len(grouped) >= 3 and all(len(x) <= torch_cpu.MAX_SEGS for x in grouped)
    saved = torch_cpu.MAX_SEGS, torch_cpu.SLAB
    try:
        torch_cpu.MAX_SEGS, torch_cpu.SLAB = 5, 20_000   # smaller groups, and the large tensor slab-wise
        assert torch_cpu.encode_update(old, new) == want
        w = {k: v.clone() for k, v in old.items()}
        torch_cpu.apply_update(w, want)
        assert _equal(w, new)
    finally:
        torch_cpu.MAX_SEGS, torch_cpu.SLAB = saved
