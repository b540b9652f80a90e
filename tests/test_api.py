"""The public API on the HIP implementation: round trips, rejected inputs, checksum caches, errors.

Organised by property, not by case:

- round trips: every named scenario (scenarios.single_scenarios) with the sender and receiver on the
  GPU, and a subset in every placement of sender and receiver (CPU tensors are staged through the
  GPU by the library); the statistics apply_update returns are checked against the inputs.
- rejected inputs: one table of hostile updates, each made by editing one field of a valid update
  (wire.Update re-serialised by wire.serialize) or its bytes, one per limit of the format's parser
  (the reference's src/crukx_sync/wire.py:126-212) and of apply (codec.py:598-604,703-712).  Each must
  be refused by the parser (a CPU test), by apply with the receiver unchanged, and by the oracle.
- caches and receivers: chained steps keep sender and receiver caches equal, and a cache that does
  not describe the receiver's weights leads to a rejection, never to wrong weights.

The behaviours are those the reference's API tests pin (its tests/test_roundtrip.py).
"""

from __future__ import annotations

import copy
import time

import pytest
import torch

import crukx_sync
import oracle
import scenarios
from crukx_sync import CorruptUpdate, apply_update, codec, encode_update, wire

gpu = pytest.mark.gpu
PLACEMENTS = [("cuda", "cuda"), ("cuda", "cpu"), ("cpu", "cuda"), ("cpu", "cpu")]  # (sender, receiver)
_SC = {}


def _scen(name):
    if not _SC:
        _SC.update(scenarios.single_scenarios())
    return _SC[name]


def _on(d, dev):
    return {k: v.clone().to(dev) for k, v in d.items()}


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def _same(a: dict, b: dict) -> bool:
    return a.keys() == b.keys() and all(torch.equal(_bits(a[k]), _bits(b[k])) for k in a)


def _diff(old, new):
    """(changed elements, tensors with a change)"""
    n = [int((_bits(old[k]) != _bits(new[k])).sum()) for k in old]
    return sum(n), sum(1 for x in n if x)


# ------------------------------------------------------------------ round trips

@gpu
@pytest.mark.parametrize("name", sorted(scenarios.single_scenarios()))
def test_round_trip_and_its_statistics(name):
    old, new = _scen(name)
    upd = encode_update(_on(old, "cuda"), _on(new, "cuda"))
    recv = _on(old, "cuda")
    stats = apply_update(recv, upd)
    assert _same(recv, new)
    changed, tensors = _diff(old, new)
    assert (stats.changed, stats.tensors, stats.bytes) == (changed, tensors, len(upd))


@gpu
@pytest.mark.parametrize("sender,receiver", PLACEMENTS)
@pytest.mark.parametrize("name", ["rl_200k", "many_tensors", "slab_4097_last", "extreme"])
def test_placements_of_sender_and_receiver(name, sender, receiver):
    old, new = _scen(name)
    upd = encode_update(_on(old, sender), _on(new, sender))
    assert upd == encode_update(_on(old, "cuda"), _on(new, "cuda"))  # the bytes do not depend on placement
    recv = _on(old, receiver)
    apply_update(recv, upd)
    assert all(v.device.type == receiver for v in recv.values()) and _same(recv, new)


@gpu
def test_an_optimizer_step_costs_under_one_and_a_half_bytes_per_change():
    old, new = _scen("rl_200k")
    changed, _ = _diff(old, new)
    assert 0 < changed < old["w"].numel()
    assert len(encode_update(_on(old, "cuda"), _on(new, "cuda"))) < 1.5 * changed


@gpu
def test_no_change_encodes_the_empty_container():
    a, _ = scenarios.rl_pair(1000)
    upd = encode_update({"w": a.cuda()}, {"w": a.clone().cuda()})
    assert upd == wire.serialize(wire.Update([], []))
    stats = apply_update({"w": a.cuda()}, upd)
    assert (stats.changed, stats.tensors) == (0, 0)


@gpu
@pytest.mark.parametrize("offset", [1, 2, 3])
def test_views_at_any_16_bit_offset(offset):
    """Receiver and sender tensors that are views into larger buffers, starting at any element
    (odd offsets are not 32-bit aligned): the writes land in the view only."""
    a, b = scenarios.rl_pair(10_001, seed=12)
    buf = torch.full((10_001 + offset + 5,), 7.0, dtype=torch.bfloat16, device="cuda")
    buf[offset:offset + 10_001] = a.cuda()
    guard = buf.clone()
    src = torch.zeros_like(buf)
    src[offset:offset + 10_001] = a.cuda()
    upd = encode_update({"w": src[offset:offset + 10_001]}, {"w": b.cuda()})
    assert upd == encode_update({"w": a.cuda()}, {"w": b.cuda()})
    apply_update({"w": buf[offset:offset + 10_001]}, upd)
    assert torch.equal(_bits(buf[offset:offset + 10_001]), _bits(b))
    assert torch.equal(_bits(buf[:offset]), _bits(guard[:offset]))
    assert torch.equal(_bits(buf[offset + 10_001:]), _bits(guard[offset + 10_001:]))


@gpu
@pytest.mark.parametrize("n", [4096, 4097, 3 * 4096 + 5])
@pytest.mark.parametrize("dev", ["cuda", "cpu"])
def test_slab_boundaries(monkeypatch, n, dev):
    """Tensors of one slab, one slab and one element, and three slabs and a few elements (4096-element
    slabs), with and without a change at the very last element."""
    monkeypatch.setattr(codec, "_SLAB", 4096)
    for name in (f"slab_{n}", f"slab_{n}_last"):
        old, new = _scen(name)
        recv = _on(old, dev)
        apply_update(recv, encode_update(_on(old, dev), _on(new, dev)))
        assert _same(recv, new)


@gpu
def test_a_long_zero_run_keeps_the_rice_parameter_small():
    """2000 changes at the start and one at the end of a 2^20-element group: the gaps are mostly 0,
    so the Rice parameter is small and the last gap is one unary run far longer than a 64-bit word."""
    old, new = _scen("long_unary")
    upd = encode_update(_on(old, "cuda"), _on(new, "cuda"))
    assert wire.parse(upd).tensors[0].groups[0].rice_r < 10
    recv = _on(old, "cuda")
    apply_update(recv, upd)
    assert _same(recv, new)


# ------------------------------------------------------------------ hostile updates

NAME = "w" * 11  # the tensor's name: unique in the bytes (name_not_utf8 overwrites it)


def _base():
    """A valid update (one step of size 2e-5 over 4000 weights: several exponent groups and blocks)
    as plain, editable fields, with its inputs."""
    a, b = scenarios.rl_pair(4000, lr=2e-5, seed=6)
    p = wire.parse(oracle.encode_update({NAME: a}, {NAME: b}))
    u = wire.Update(copy.deepcopy(p.tables), copy.deepcopy(p.tensors), list(p.block_bits), bytes(p.payload))
    return u, a, b


def _big_table(u):
    return max(u.tables, key=lambda t: len(t.symbols))


def _edit(fn):
    def make():
        u, a, b = _base()
        fn(u)
        return wire.serialize(u), a
    return make


def _raw(fn):
    def make():
        u, a, b = _base()
        return fn(wire.serialize(u)), a
    return make


def _unused_exponent(u):
    used = {t.exponent for t in u.tables}
    return next(e for e in range(256) if e not in used)


def _move_bits(u):  # the same total, but the first block gets fewer bits than its symbols need
    g = u.tensors[0].groups[0]
    need = min(wire.BLOCK, g.count) * (2 + g.rice_r)
    pair = u.block_bits[0] + u.block_bits[1]
    u.block_bits[0], u.block_bits[1] = need - 1, pair - (need - 1)


def _blocks_claim_nothing():
    """A 2^22-element receiver and a group claiming every element with zero-bit blocks: refused from
    the block table alone, before anything is sized by the count."""
    n = 1 << 22
    g = wire.Group(0, n, 0)
    u = wire.Update([wire.Table(0, [0], [1])], [wire.TensorHeader("w", n, 0, [g])], [0] * wire.n_blocks(n), b"")
    return wire.serialize(u), torch.zeros(n, dtype=torch.int16)


def _endless_unary():
    """2^18 changes whose payload is all one bits (every gap an endless unary run) with block sizes
    that pass the structural checks: the decoder must give up quickly."""
    n, count = 1 << 20, 1 << 18
    g = wire.Group(0x7F, count, 0)
    blocks = [512] * wire.n_blocks(count)
    u = wire.Update([wire.Table(0x7F, [2], [1])], [wire.TensorHeader("w", n, 0, [g])], blocks,
                    b"\xff" * (sum(blocks) // 8))
    return wire.serialize(u), torch.full((n,), 0x3F80, dtype=torch.int16)


HOSTILE = {
    # container
    "magic": _raw(lambda s: b"XRXS" + s[4:]),
    "version": _raw(lambda s: s[:4] + bytes([wire.VERSION + 1]) + s[5:]),
    "varint_beyond_64_bits": _raw(lambda s: s[:5] + b"\xff" * 10 + b"\x01" + s[6:]),
    "truncated": _raw(lambda s: s[:-1]),
    "trailing_byte": _raw(lambda s: s + b"\x00"),
    # tables
    "table_exponent_twice": _edit(lambda u: u.tables.append(copy.deepcopy(u.tables[0]))),
    "table_symbol_twice": _edit(lambda u: _big_table(u).symbols.__setitem__(1, _big_table(u).symbols[0])),
    "table_symbol_beyond_max": _edit(lambda u: _big_table(u).symbols.__setitem__(0, wire.MAX_SYMBOL + 1)),
    "code_length_zero": _edit(lambda u: _big_table(u).lengths.__setitem__(0, 0)),
    "code_length_beyond_max": _edit(lambda u: _big_table(u).lengths.__setitem__(0, wire.MAX_CODE_LEN + 1)),
    "code_lengths_oversubscribed": _edit(lambda u: _big_table(u).lengths.__setitem__(
        slice(None), [1] * len(_big_table(u).lengths))),
    "table_nobody_uses": _edit(lambda u: u.tables.append(wire.Table(_unused_exponent(u), [0], [1]))),
    # tensors and groups
    "name_not_utf8": _raw(lambda s: s.replace(NAME.encode(), b"\xff" * len(NAME))),
    "tensor_twice": _edit(lambda u: u.tensors.append(copy.deepcopy(u.tensors[0]))),
    "no_groups": _edit(lambda u: u.tensors[0].groups.clear()),
    "group_exponent_without_table": _edit(lambda u: setattr(u.tensors[0].groups[0], "exponent", _unused_exponent(u))),
    "group_exponent_twice": _edit(lambda u: u.tensors[0].groups.append(copy.deepcopy(u.tensors[0].groups[0]))),
    "group_count_zero": _edit(lambda u: setattr(u.tensors[0].groups[0], "count", 0)),
    "group_count_beyond_numel": _edit(lambda u: setattr(u.tensors[0].groups[0], "count", u.tensors[0].numel + 1)),
    "group_count_near_2_63": _edit(lambda u: setattr(u.tensors[0].groups[0], "count", (1 << 62) + 1)),
    "rice_beyond_max": _edit(lambda u: setattr(u.tensors[0].groups[0], "rice_r", wire.MAX_RICE + 1)),
    "changes_beyond_numel": _edit(lambda u: setattr(u.tensors[0], "numel", sum(g.count for g in u.tensors[0].groups) - 1)),
    # block table and payload
    "block_table_cut": _edit(lambda u: u.block_bits.pop()),
    "payload_longer_than_blocks": _edit(lambda u: setattr(u, "payload", u.payload + b"\x00")),
    "padding_bits_set": _edit(lambda u: (u.block_bits.__setitem__(-1, u.block_bits[-1] - 1),
                                         setattr(u, "payload", u.payload[:-1] + bytes([u.payload[-1] | 1])))),
    "block_shorter_than_its_symbols": _edit(_move_bits),
    # apply: verdicts that need the receiver
    "checksum_off_by_one": _edit(lambda u: setattr(u.tensors[0], "checksum", (u.tensors[0].checksum + 1) % (1 << 64))),
    "receiver_too_few_of_an_exponent": _edit(lambda u: None),  # the receiver is changed instead (_hostile)
}
PARSE_OK = {"checksum_off_by_one", "receiver_too_few_of_an_exponent"}  # well formed: apply rejects them
# the parser's message for each (the reference's, wire.py:126-212)
REASON = {
    "magic": "not a crukx-sync update", "version": "unsupported format version 3",
    "varint_beyond_64_bits": "varint out of range", "truncated": "update is truncated",
    "trailing_byte": "trailing bytes after the payload", "table_exponent_twice": "bad table header",
    "table_symbol_twice": "bad table symbols", "table_symbol_beyond_max": "bad table symbols",
    "code_length_zero": "bad Huffman code lengths", "code_length_beyond_max": "bad Huffman code lengths",
    "code_lengths_oversubscribed": "bad Huffman code lengths",
    "table_nobody_uses": "table unused or larger than its changes", "name_not_utf8": "tensor name is not valid UTF-8",
    "tensor_twice": "appears twice", "no_groups": "bad group count", "group_exponent_without_table": "bad group exponent",
    "group_exponent_twice": "bad group exponent", "group_count_zero": "bad group header",
    "group_count_beyond_numel": "bad group header", "group_count_near_2_63": "bad group header",
    "rice_beyond_max": "bad group header", "changes_beyond_numel": "more changes than elements",
    "block_table_cut": "trailing bytes after the payload",
    "payload_longer_than_blocks": "payload length does not match its block table",
    "padding_bits_set": "non-zero padding bits", "block_shorter_than_its_symbols": "block shorter than its symbols could be",
}


def _hostile(name):
    upd, recv = HOSTILE[name]()
    if name == "receiver_too_few_of_an_exponent":  # no element of the first group's exponent is left
        e = wire.parse(upd).tensors[0].groups[0].exponent
        bits = recv.view(torch.int16).clone()
        bits[((bits.int() >> 7) & 0xFF) == e] = 0x3F80 if e != 0x7F else 0x4000  # 1.0 (2.0): another exponent
        recv = bits.view(recv.dtype)
    return upd, recv


def test_hostile_updates_cover_the_format_limits():
    """Every case builds, differs from the valid update, and, but for the apply-level ones, is refused
    by the parser (which runs on the host) for its own reason."""
    base = wire.serialize(_base()[0])
    for name in HOSTILE:
        upd, _ = _hostile(name)
        if name != "receiver_too_few_of_an_exponent":
            assert upd != base, name
        if name in PARSE_OK:
            wire.parse(upd)
        else:
            with pytest.raises(CorruptUpdate, match=REASON[name]):
                wire.parse(upd)


@gpu
@pytest.mark.parametrize("name", sorted(HOSTILE))
def test_hostile_update_is_rejected_and_the_receiver_kept(name):
    upd, recv = _hostile(name)
    ref = {NAME: recv.clone()}
    with pytest.raises(oracle.OracleCorrupt):
        oracle.apply_update(ref, upd)
    for dev in ("cuda", "cpu"):
        w = {NAME: recv.clone().to(dev)}
        with pytest.raises(CorruptUpdate):
            apply_update(w, upd)
        assert torch.equal(_bits(w[NAME]), _bits(recv)), dev


@gpu
@pytest.mark.parametrize("make", [_blocks_claim_nothing, _endless_unary], ids=["blocks_claim_nothing", "endless_unary"])
def test_hostile_sizes_are_refused_quickly(make):
    upd, recv = make()
    w = {"w": recv.cuda()}
    t = time.time()
    with pytest.raises(CorruptUpdate):
        apply_update(w, upd)
    assert time.time() - t < 30
    assert torch.equal(_bits(w["w"]), _bits(recv))


@gpu
@pytest.mark.parametrize("dev", ["cuda", "cpu"])
def test_every_byte_of_an_update_is_guarded(dev):
    """Each byte of a small update XORed with 0x01, 0x80 and 0xFF: the result is either refused with
    the receiver unchanged (CorruptUpdate, or ValueError when the flip renames the tensor) or, if the
    flipped update still verifies, applied exactly."""
    a, b = scenarios.rl_pair(3000, seed=6)
    upd = encode_update({"w": a.to(dev)}, {"w": b.to(dev)})
    for i in range(len(upd)):
        for x in (0x01, 0x80, 0xFF):
            bad = bytearray(upd)
            bad[i] ^= x
            w = {"w": a.clone().to(dev)}
            try:
                apply_update(w, bytes(bad))
            except ValueError:  # CorruptUpdate, or a flipped name the receiver does not have
                assert torch.equal(_bits(w["w"]), _bits(a)), (i, x)
            else:
                assert torch.equal(_bits(w["w"]), _bits(b)), (i, x)


# ------------------------------------------------------------------ receivers, caches, argument errors

@gpu
def test_receivers_and_inputs_that_do_not_fit_are_argument_errors():
    a, b = scenarios.rl_pair(1000)
    a, b = a.cuda(), b.cuda()
    upd = encode_update({"w": a}, {"w": b})
    for recv in ({"v": a.clone()}, {"w": a[:999].clone()}, {"w": a.float()}):
        with pytest.raises(ValueError):
            apply_update(recv, upd)
    for old, new in (({"w": a}, {"w": b.float()}), ({"w": a}, {"v": b}), ({"w": a}, {"w": b[:999]}),
                     ({"w": a, "x": a.cpu()}, {"w": b, "x": b.cpu()})):
        with pytest.raises(ValueError):
            encode_update(old, new)


def _drift(n, steps, seed):
    """A weight vector and its bf16 snapshots after `steps` sign steps of 1e-6."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, generator=g) * 0.02
    out = [w.bfloat16()]
    for _ in range(steps):
        w = w + 1e-6 * torch.sign(torch.randn(w.shape, generator=g))
        out.append(w.bfloat16())
    return out


@gpu
@pytest.mark.parametrize("dev", ["cuda", "cpu"])
def test_caches_stay_equal_over_a_chain(dev):
    snaps = [s.to(dev) for s in _drift(300_000, 5, seed=7)]
    send, recv_chk = {}, {}
    recv = {"w": snaps[0].clone()}
    for prev, cur in zip(snaps, snaps[1:]):
        apply_update(recv, encode_update({"w": prev}, {"w": cur}, send), recv_chk)
        assert torch.equal(_bits(recv["w"]), _bits(cur))
    assert send == {k: v[0] for k, v in recv_chk.items()}


@gpu
@pytest.mark.parametrize("dev", ["cuda", "cpu"])
def test_a_cache_that_does_not_describe_the_receiver_leads_to_a_rejection(dev):
    s0, s1, s2 = (s.to(dev) for s in _drift(50_000, 2, seed=9))
    send, recv_chk = {}, {}
    # a cached checksum that is simply wrong, at the tensor's current version
    w = {"w": s0.clone()}
    with pytest.raises(CorruptUpdate):
        apply_update(w, encode_update({"w": s0}, {"w": s1}), {"w": (12345, w["w"]._version)})
    assert torch.equal(_bits(w["w"]), _bits(s0))
    # weights edited in place after a cached apply: the version moved, so the stale value is not used
    w = {"w": s0.clone()}
    apply_update(w, encode_update({"w": s0}, {"w": s1}, send), recv_chk)
    w["w"].view(torch.int16)[7] ^= 1
    before = w["w"].clone()
    with pytest.raises(CorruptUpdate):
        apply_update(w, encode_update({"w": s1}, {"w": s2}, send), recv_chk)
    assert torch.equal(_bits(w["w"]), _bits(before))


@gpu
def test_the_sender_cache_is_kept_when_serialising_fails(monkeypatch):
    a, b = scenarios.rl_pair(20_000, seed=10)
    cache = {}

    def fail(_):
        raise RuntimeError("serialize failed")
    monkeypatch.setattr(crukx_sync, "serialize", fail)
    with pytest.raises(RuntimeError):
        encode_update({"w": a.cuda()}, {"w": b.cuda()}, cache)
    assert cache == {}
