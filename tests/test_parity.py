"""Parity of the HIP path with the reference, on the GPU.

- Encode: for every golden scenario, the bytes from the gfx950 kernels equal the bytes the
  reference wrote (tests/golden/updates.json), and the sender checksums agree.
- Apply: the golden updates applied by the HIP path reproduce the new weights; results equal the
  oracle's on the same inputs, including rejections.
- Chained steps with both checksum caches (four tensors of 26.6M weights, three steps).
- Slab size (codec._SLAB) and the device-resident byte path never change the bytes.
- At sizes the oracle cannot check in seconds: size-independent properties (round trip exact,
  sender cache == receiver cache, checksum of the result equals a full recomputation).
"""

import hashlib

import pytest
import torch

import crukx_sync
import oracle
import scenarios
from crukx_sync import codec, workloads

pytestmark = pytest.mark.gpu

_SC = {}


def _scen():
    if not _SC:
        _SC.update(scenarios.single_scenarios())
    return _SC


def _cuda(d):
    return {k: v.to("cuda") for k, v in d.items()}


def _check(upd, rec):
    assert len(upd) == rec["len"]
    if "hex" in rec:
        assert upd.hex() == rec["hex"]
    assert hashlib.sha256(upd).hexdigest() == rec["sha256"]


@pytest.mark.parametrize("name", sorted(scenarios.single_scenarios().keys()))
def test_encode_bytes_equal_reference(golden, name):
    old, new = _scen()[name]
    rec = golden["updates"]["single"][name]
    assert scenarios.bits_sha(old) == rec["inputs_old"] and scenarios.bits_sha(new) == rec["inputs_new"]
    chk = {}
    upd = crukx_sync.encode_update(_cuda(old), _cuda(new), chk)
    _check(upd, rec["update"])
    assert chk == rec["sender_checksums"]


@pytest.mark.parametrize("name", sorted(scenarios.single_scenarios().keys()))
def test_apply_reference_bytes(golden, name):
    old, new = _scen()[name]
    rec = golden["updates"]["single"][name]
    upd = oracle.encode_update(old, new)  # the oracle's bytes equal the reference's (test_oracle)
    _check(upd, rec["update"])
    w = _cuda({k: v.clone() for k, v in old.items()})
    stats = crukx_sync.apply_update(w, upd)
    ref = {k: v.clone() for k, v in old.items()}
    n = oracle.apply_update(ref, upd)
    assert stats.changed == n
    for k in new:
        assert torch.equal(w[k].cpu().view(torch.int16), new[k].view(torch.int16)), k


def test_small4_chain_with_caches(golden):
    states = scenarios.chain_small4(3)
    rec = golden["updates"]["chains"]["small4_chain"]
    assert scenarios.bits_sha(states[0]) == rec["inputs_0"]
    send, recv = {}, {}
    w = _cuda(states[0])
    prev = _cuda(states[0])
    for s in range(1, len(states)):
        cur = _cuda(states[s])
        upd = crukx_sync.encode_update(prev, cur, send)
        _check(upd, rec["steps"][s - 1]["update"])
        assert send == rec["steps"][s - 1]["sender_checksums"]
        crukx_sync.apply_update(w, upd, recv)
        for k in w:
            assert torch.equal(w[k].view(torch.int16), cur[k].view(torch.int16))
        prev = cur
    assert send == {k: v[0] for k, v in recv.items()}


def test_cache_chain(golden):
    states = scenarios.chain_cache(5)
    rec = golden["updates"]["chains"]["cache_chain"]
    send, recv = {}, {}
    w = _cuda(states[0])
    for s in range(1, len(states)):
        upd = crukx_sync.encode_update(_cuda(states[s - 1]), _cuda(states[s]), send)
        _check(upd, rec["steps"][s - 1]["update"])
        crukx_sync.apply_update(w, upd, recv)
    assert torch.equal(w["w"].cpu().view(torch.int16), states[-1]["w"].view(torch.int16))


@pytest.mark.parametrize("slab", [128, 256, 4096, 1 << 17])
@pytest.mark.parametrize("name", ["rl_200k", "many_tensors", "slab_12293", "edges", "sweep_rho0.03_p0.7"])
def test_slab_size_never_changes_bytes(golden, monkeypatch, slab, name):
    monkeypatch.setattr(codec, "_SLAB", slab)
    old, new = _scen()[name]
    upd = crukx_sync.encode_update(_cuda(old), _cuda(new))
    _check(upd, golden["updates"]["single"][name]["update"])
    w = _cuda({k: v.clone() for k, v in old.items()})
    crukx_sync.apply_update(w, upd)
    for k in new:
        assert torch.equal(w[k].cpu().view(torch.int16), new[k].view(torch.int16))


def test_many_exponent_windows_per_slab(monkeypatch):
    """Slabs whose targets span all 256 exponents take four select windows each; with 128-element
    slabs there are more extra windows than the select pass's front blocks, so the overflow kernel
    runs too.  Every element changes to arbitrary bits; the result must equal the oracle's."""
    monkeypatch.setattr(codec, "_SLAB", 128)
    g = torch.Generator().manual_seed(31)
    a = torch.randint(-32768, 32768, (200_000,), generator=g, dtype=torch.int16)
    b = a ^ torch.randint(1, 32768, (200_000,), generator=g, dtype=torch.int16)
    old, new = {"w": a}, {"w": b}
    upd = crukx_sync.encode_update(_cuda(old), _cuda(new))
    assert upd == oracle.encode_update(old, new)
    w = _cuda({"w": a.clone()})
    assert crukx_sync.apply_update(w, upd).changed == 200_000
    assert torch.equal(w["w"].cpu(), b)


def test_device_resident_bytes_and_apply(golden):
    old, new = _scen()["three_tensors"]
    dev_upd = crukx_sync.encode_update_device(_cuda(old), _cuda(new))
    assert dev_upd.is_cuda and dev_upd.dtype == torch.uint8
    _check(dev_upd.cpu().numpy().tobytes(), golden["updates"]["single"]["three_tensors"]["update"])
    w = _cuda({k: v.clone() for k, v in old.items()})
    stats = crukx_sync.apply_update(w, dev_upd)
    assert stats.bytes == dev_upd.numel()
    for k in new:
        assert torch.equal(w[k].cpu().view(torch.int16), new[k].view(torch.int16))


def test_device_resident_update_at_every_byte_alignment_and_at_an_allocation_end():
    """A device-resident update is applied wherever its bytes sit: the decoder reads the payload in
    place from the 8-byte words around it (its first bit anywhere in a word), or from a padded copy
    when the words past the payload's end lie outside the allocation (here: the update placed at the
    very end of a tensor that has a device allocation of its own)."""
    a, b = scenarios.rl_pair(300_000, seed=21)
    upd = crukx_sync.encode_update_device({"w": a.cuda()}, {"w": b.cuda()})
    n = upd.numel()
    for shift in range(9):  # every offset of the payload within an aligned word, and one past
        buf = torch.zeros(n + shift + 40, dtype=torch.uint8, device="cuda")
        view = buf[shift:shift + n]
        view.copy_(upd)
        w = {"w": a.cuda()}
        assert crukx_sync.apply_update(w, view).changed == int((a.view(torch.int16) != b.view(torch.int16)).sum())
        assert torch.equal(w["w"].cpu().view(torch.int16), b.view(torch.int16)), shift
    # large tensors get a device allocation of exactly their (rounded) size: the update's last byte is
    # the allocation's last byte, so no aligned word past the payload may be read there
    big = torch.empty(16 << 20, dtype=torch.uint8, device="cuda")
    for cut in (0, 3, 5):
        view = big[big.numel() - n - cut:big.numel() - cut]
        view.copy_(upd)
        w = {"w": a.cuda()}
        crukx_sync.apply_update(w, view)
        assert torch.equal(w["w"].cpu().view(torch.int16), b.view(torch.int16)), cut


def test_device_resident_corruption_is_rejected():
    a, b = scenarios.rl_pair(20_000, seed=13)
    dev_upd = crukx_sync.encode_update_device({"w": a.cuda()}, {"w": b.cuda()})
    host = dev_upd.cpu().numpy().tobytes()
    for i in range(len(host) - 1, len(host) - 200, -7):  # payload bytes
        bad = dev_upd.clone()
        bad[i] ^= 0x10
        w = {"w": a.cuda()}
        try:
            crukx_sync.apply_update(w, bad)
        except crukx_sync.CorruptUpdate:
            assert torch.equal(w["w"].cpu().view(torch.int16), a.view(torch.int16))
        else:
            assert torch.equal(w["w"].cpu().view(torch.int16), b.view(torch.int16))


def test_checksum_matches_oracle():
    for n in (1, 2, 3, 255, 4097, 1 << 20, 3_000_001):
        t = torch.randint(-32768, 32768, (n,), dtype=torch.int16, generator=torch.Generator().manual_seed(n))
        assert codec.checksum(t.cuda()) == oracle.checksum(t)
        if n > 2:  # an odd 16-bit offset (not 32-bit aligned)
            assert codec.checksum(t.cuda()[1:]) == oracle.checksum(t[1:])


def test_corruptions_match_oracle_verdicts():
    """Random multi-byte corruptions: the HIP apply and the oracle agree on accept/reject, and the
    accepted results are identical."""
    a, b = scenarios.rl_pair(50_000, seed=21)
    upd = bytearray(crukx_sync.encode_update({"w": a.cuda()}, {"w": b.cuda()}))
    g = torch.Generator().manual_seed(3)
    for _ in range(200):
        bad = bytearray(upd)
        for i in torch.randint(0, len(upd), (3,), generator=g).tolist():
            bad[i] = int(torch.randint(0, 256, (1,), generator=g))
        bad = bytes(bad)
        w_hip, w_ref = {"w": a.cuda()}, {"w": a.clone()}
        hip_ok = ref_ok = True
        try:
            crukx_sync.apply_update(w_hip, bad)
        except ValueError:
            hip_ok = False
        try:
            oracle.apply_update(w_ref, bad)
        except ValueError:
            ref_ok = False
        assert hip_ok == ref_ok
        assert torch.equal(w_hip["w"].cpu().view(torch.int16), w_ref["w"].view(torch.int16))


def test_many_small_slabs_with_corruptions_in_the_last_tensor(monkeypatch):
    """Six tensors in 128-element slabs (over 7000 slabs).  Clean: the oracle's bytes, applied exactly.
    Corrupted in the payload of the last tensor: rejected, as by the oracle, with one of the
    reference's messages, and the weights as they were."""
    monkeypatch.setattr(codec, "_SLAB", 128)
    g = torch.Generator().manual_seed(5)
    names = [f"t{i}" for i in range(6)]
    old, new = {}, {}
    for i, n in enumerate(names):
        a, b = scenarios.rl_pair(150_000 + 37 * i, lr=3e-6, seed=40 + i)
        old[n], new[n] = a, b
    upd = crukx_sync.encode_update(_cuda(old), _cuda(new))
    assert upd == oracle.encode_update(old, new)
    w = _cuda({k: v.clone() for k, v in old.items()})
    crukx_sync.apply_update(w, upd)
    for k in names:
        assert torch.equal(w[k].cpu().view(torch.int16), new[k].view(torch.int16)), k
    tail = len(upd) // 6  # about the last tensor's share of the payload
    outcomes = set()
    for _ in range(60):
        bad = bytearray(upd)
        for i in torch.randint(len(upd) - tail, len(upd), (2,), generator=g).tolist():
            bad[i] ^= int(torch.randint(1, 256, (1,), generator=g))
        bad = bytes(bad)
        w_hip, w_ref = _cuda({k: v.clone() for k, v in old.items()}), {k: v.clone() for k, v in old.items()}
        hip = ref = None
        try:
            crukx_sync.apply_update(w_hip, bad)
        except ValueError as e:
            hip = str(e)
        try:
            oracle.apply_update(w_ref, bad)
        except ValueError as e:
            ref = str(e)
        assert (hip is None) == (ref is None)
        outcomes.add(hip)
        for k in names:
            assert torch.equal(w_hip[k].cpu().view(torch.int16), w_ref[k].view(torch.int16)), k
    assert None not in outcomes  # every corruption here is rejected
    assert all(m.startswith("update does not verify (checksum mismatch: [") or
               m == "payload positions outside their exponent groups" for m in outcomes), outcomes


def test_qwen_layer_sized_round_trip_properties():
    """One 7B-shaped decoder layer plus the final norm (233M weights), three chained steps with
    caches: exact round trips, sender cache == receiver cache == full checksums of the result."""
    shapes = [s for s in workloads.qwen25_shapes("qwen2.5-7b") if s[0].startswith("model.layers.0.")
              or s[0] == "model.norm.weight"]
    prev = workloads.make_weights(shapes, seed=3, device="cuda")
    recv = {k: v.clone() for k, v in prev.items()}
    send, rc = {}, {}
    for s in range(1, 4):
        cur = workloads.make_step(prev, s, rho=0.01, seed=3)
        crukx_sync.apply_update(recv, crukx_sync.encode_update(prev, cur, send), rc)
        for k in cur:
            assert torch.equal(recv[k].view(torch.int16), cur[k].view(torch.int16)), k
        prev = cur
    assert send == {k: v[0] for k, v in rc.items()}
    for k in ("model.layers.0.mlp.down_proj.weight", "model.norm.weight"):
        assert send[k] == codec.checksum(prev[k])


def test_receiver_exponent_counts_carried_across_updates():
    """apply keeps per-slab exponent counts of the receiver's weights between updates (used only
    with a checksum-cache hit): a chain with many binade crossings stays exact, an in-place edit of
    one tensor drops its counts, and a rejected update drops them too."""
    g = torch.Generator().manual_seed(7)
    shapes = [("a", (300, 4097)), ("b", (70001,)), ("c", (64, 1024))]
    cur = {n: (torch.randn(s, generator=g) * 0.02).to(torch.bfloat16) for n, s in shapes}
    cur["c"][:, :8] = 0  # zeros step to subnormals: exponent moves from 0
    recv = _cuda(cur)
    send_chk, recv_chk = {}, {}
    old_slab = codec._SLAB
    codec._SLAB = 4096  # many slabs per tensor
    try:
        for step in range(8):
            nxt = {}
            for n, t in cur.items():
                bits = t.view(torch.int16).clone()
                m = torch.rand(bits.shape, generator=g) < 0.05
                k = torch.randint(1, 300, bits.shape, generator=g, dtype=torch.int16)  # large steps: crossings
                bits[m] = bits[m] + k[m]
                nxt[n] = bits.view(torch.bfloat16)
            upd = crukx_sync.encode_update(_cuda(cur), _cuda(nxt), send_chk)
            crukx_sync.apply_update(recv, upd, recv_chk)
            for n in nxt:
                assert torch.equal(recv[n].cpu().view(torch.int16), nxt[n].view(torch.int16)), (step, n)
            if step == 3:  # edit one receiver tensor in place: its counts and checksum are stale
                recv["b"].add_(0)  # bumps the version, values unchanged
            cur = nxt
        assert send_chk == {k: v[0] for k, v in recv_chk.items()}
        # an update made against other old weights fails verification in the device pass: the weights
        # stay as they were and the counts of its tensors are forgotten
        alt = {n: t.clone() for n, t in cur.items()}
        alt["a"].view(torch.int16)[0, 0] += 1
        nxt = {n: (t.view(torch.int16) + 1).view(torch.bfloat16) for n, t in alt.items()}
        upd = crukx_sync.encode_update(_cuda(alt), _cuda(nxt), {})
        before = {n: t.clone() for n, t in recv.items()}
        with pytest.raises(crukx_sync.CorruptUpdate):
            crukx_sync.apply_update(recv, upd, recv_chk)
        for n in recv:
            assert torch.equal(recv[n], before[n])
            assert codec._hist_lookup(recv[n]) is None
    finally:
        codec._SLAB = old_slab


@pytest.mark.parametrize("name", ["rl_200k", "every_element_arbitrary", "three_tensors", "edges",
                                  "distinct_residuals_200k"])
def test_rejected_update_leaves_the_weights_as_they_were(name):
    """A receiver one mantissa bit away from the sender's old weights (same exponent counts, so every
    target is found and the select pass writes it through before the verdict): the update is rejected
    by the HIP path and by the oracle, and the weights come back bit for bit, in slabs streamed in one
    window and in slabs streamed in several (every_element_arbitrary)."""
    old, new = _scen()[name]
    upd = crukx_sync.encode_update(_cuda(old), _cuda(new), {})
    big = max(old, key=lambda k: old[k].numel())
    recv = {k: v.clone() for k, v in old.items()}
    flat = recv[big].view(-1).view(torch.int16)
    flat[flat.numel() // 2] ^= 1  # lowest mantissa bit: the exponent, and so every count, is unchanged
    ref = {k: v.clone() for k, v in recv.items()}
    with pytest.raises(oracle.OracleCorrupt):
        oracle.apply_update(ref, upd)
    dev = _cuda(recv)
    with pytest.raises(crukx_sync.CorruptUpdate):
        crukx_sync.apply_update(dev, upd)
    for k in recv:
        assert torch.equal(dev[k].cpu().view(torch.int16), recv[k].view(torch.int16)), k


@pytest.mark.parametrize("rho", [0.005, 0.02, 0.025, 0.1, 0.6, "mixed"])
def test_change_densities_across_target_list_sizes(rho):
    """Slabs with a few hundred to tens of thousands of changes (the select pass keeps up to a fixed
    number of a window's targets in LDS, more for denser updates, and reads larger lists from HBM):
    exact round trips and the oracle's bytes.  "mixed": one dense slab in a sparse update."""
    g = torch.Generator().manual_seed(7 if rho == "mixed" else int(rho * 1000))
    n = 400_003 if rho == "mixed" else 200_003
    a = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    bits = a.view(torch.int16).clone()
    if rho == "mixed":
        m = torch.rand(bits.shape, generator=g) < 0.002
        m[70_000:70_000 + 65_536] |= torch.rand(65_536, generator=g) < 0.06
    else:
        m = torch.rand(bits.shape, generator=g) < rho
    bits[m] = bits[m] + torch.randint(-3, 4, bits.shape, generator=g, dtype=torch.int16)[m]
    b = bits.view(torch.bfloat16)
    upd = crukx_sync.encode_update({"w": a.cuda()}, {"w": b.cuda()})
    assert upd == oracle.encode_update({"w": a}, {"w": b})
    got = {"w": a.cuda()}
    crukx_sync.apply_update(got, upd)
    assert torch.equal(got["w"].cpu().view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("n_large", [16_000, 60_000])
def test_many_large_residuals_bytes_equal_oracle(n_large):
    """Residuals of 16 ULP or more (zigzag symbols past the dense per-exponent table, counted in the
    rare list): fewer than the 16384 the encoder downloads with the symbol counts, and more, which
    take a second download.  Bytes equal the oracle's; the update applies exactly."""
    g = torch.Generator().manual_seed(n_large)
    n = 1 << 20
    a = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    bits = a.view(torch.int16).clone()
    idx = torch.randperm(n, generator=g)[:n_large]
    step = torch.randint(16, 2000, (n_large,), generator=g, dtype=torch.int16)
    step = torch.where(torch.rand(n_large, generator=g) < 0.5, -step, step)
    bits[idx] = bits[idx] + step  # magnitudes near 0.02: sign and exponent range stay finite
    b = bits.view(torch.bfloat16)
    assert torch.isfinite(b.float()).all()
    upd = crukx_sync.encode_update({"w": a.cuda()}, {"w": b.cuda()})
    assert upd == oracle.encode_update({"w": a}, {"w": b})
    got = {"w": a.cuda()}
    crukx_sync.apply_update(got, upd)
    assert torch.equal(got["w"].cpu().view(torch.int16), b.view(torch.int16))


def test_exponent_counts_are_not_reused_across_slab_sizes(monkeypatch):
    """Counts recorded with one slab size are recomputed, not reused, when the slab size changes
    between updates of the same receiver tensors (their layout differs)."""
    g = torch.Generator().manual_seed(9)
    cur = {"a": (torch.randn(200_003, generator=g) * 0.02).to(torch.bfloat16),
           "b": (torch.randn(96, 1024, generator=g) * 0.02).to(torch.bfloat16)}
    recv = _cuda(cur)
    send_chk, recv_chk = {}, {}
    for step, slab in enumerate((1 << 16, 4096, 1 << 14, 1 << 16, 4096)):
        monkeypatch.setattr(codec, "_SLAB", slab)
        nxt = {}
        for n, t in cur.items():
            bits = t.view(torch.int16).clone()
            m = torch.rand(bits.shape, generator=g) < 0.03
            bits[m] = bits[m] + torch.randint(1, 200, bits.shape, generator=g, dtype=torch.int16)[m]
            nxt[n] = bits.view(torch.bfloat16)
        crukx_sync.apply_update(recv, crukx_sync.encode_update(_cuda(cur), _cuda(nxt), send_chk), recv_chk)
        for n in nxt:
            assert torch.equal(recv[n].cpu().view(torch.int16), nxt[n].view(torch.int16)), (step, n)
            assert codec._hist_lookup(recv[n])[3] == slab
        cur = nxt


def test_verdict_messages_follow_the_reference():
    """apply's error messages and their priority are the reference's (codec.py:598-604,706-712):
    the group-size check of tensors over 2^24 elements first, then checksum mismatches naming up to
    three tensors as a Python list, then other inconsistencies."""
    names = ["x", "it's", 'q"t', "z"]
    g = torch.Generator().manual_seed(21)
    old = {n: (torch.randn(5000, generator=g) * 0.02).bfloat16() for n in names}
    new = {k: (v.float() + 3e-5 * torch.randn(v.shape, generator=g)).bfloat16() for k, v in old.items()}
    upd = crukx_sync.encode_update(_cuda(old), _cuda(new))
    recv = _cuda(old)
    wrong = {n: (12345, recv[n]._version) for n in names}
    with pytest.raises(crukx_sync.CorruptUpdate) as e:
        crukx_sync.apply_update(recv, upd, wrong)
    assert str(e.value) == f"update does not verify (checksum mismatch: {names[:3]})"
    for n in names:
        assert torch.equal(recv[n].cpu().view(torch.int16), old[n].view(torch.int16))

    # a group with more changes than the receiver has elements of its exponent
    n = (1 << 24) + 1000
    base = torch.full((n,), 0x3F80, dtype=torch.int16)
    sender = base.clone()
    sender[100:105] = 0x3C00  # five elements of exponent 120
    target = sender.clone()
    target[100:105] += 1
    upd = crukx_sync.encode_update({"w": sender.cuda()}, {"w": target.cuda()})
    short = base.clone()
    short[100:103] = 0x3C00  # the receiver has three
    with pytest.raises(crukx_sync.CorruptUpdate) as e:
        crukx_sync.apply_update({"w": short.cuda()}, upd)
    assert str(e.value) == "group has more changes than elements"


def test_group_size_check_follows_the_slab_knob(monkeypatch):
    """The group-size check covers tensors of more than codec._SLAB elements, as in the reference
    (codec.py:598-604): with _SLAB lowered to 4096 a 20,000-element tensor whose group outnumbers the
    receiver's elements of that exponent raises "group has more changes than elements"; with the
    default (2^24) the same update is refused by the verification instead."""
    n = 20_000
    base = torch.full((n,), 0x3F80, dtype=torch.int16)
    sender = base.clone()
    sender[100:105] = 0x3C00
    target = sender.clone()
    target[100:105] += 1
    upd = crukx_sync.encode_update({"w": sender.cuda()}, {"w": target.cuda()})
    short = base.clone()
    short[100:103] = 0x3C00
    with pytest.raises(crukx_sync.CorruptUpdate) as e:
        crukx_sync.apply_update({"w": short.cuda()}, upd)
    assert str(e.value) != "group has more changes than elements"
    monkeypatch.setattr(codec, "_SLAB", 4096)
    w = {"w": short.cuda()}
    with pytest.raises(crukx_sync.CorruptUpdate) as e:
        crukx_sync.apply_update(w, upd)
    assert str(e.value) == "group has more changes than elements"
    assert torch.equal(w["w"].cpu(), short)
