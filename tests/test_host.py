"""Host-side parts of the product, on CPU: the C ABI exports, the native parser (every limit of the
format), Huffman code lengths, canonical codes and the Rice choice against the reference's golden
vectors, and the oracle's parser on every single-byte flip of golden updates.
"""

import hashlib
import json
import os
import re

import numpy as np
import pytest
import torch

import crukx_sync
import oracle
from crukx_sync import _native, codec, wire

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    header = open(os.path.join(ROOT, "include", "crukx.h")).read()
    declared = set(re.findall(r"\b(crx_[a-z0-9_]+)\s*\(", header))
    declared.discard("crx_alloc_fn")
    L = _native.lib()
    missing = [s for s in sorted(declared) if not hasattr(L, s)]
    assert not missing, missing
    assert declared == set(_native.SIGNATURES), declared ^ set(_native.SIGNATURES)
    assert L.crx_abi_version() == _native.ABI_VERSION


def test_huffman_lengths_match_reference(golden):
    for c in golden["huffman"]["cases"]:
        assert codec.huffman_lengths(c["counts"]) == c["lengths"], c["counts"][:8]
        assert codec.canonical_codes(c["lengths"]) == c["codes"]
    for b in golden["huffman"]["big"]:
        cnt = [int(x) for x in np.random.default_rng(b["seed"]).integers(1, b["hi"], b["n"])]
        assert hashlib.sha256(json.dumps(codec.huffman_lengths(cnt)).encode()).hexdigest() == b["lengths_sha"]


def test_rice_choice_matches_reference(golden):
    for c in golden["rice"]["cases"]:
        g = np.array(c["gaps"], dtype=np.int64)
        r = codec.rice_parameter(len(g), int(g.sum()), lambda k: int((g >> k).sum()))
        assert r == c["rice"], c["gaps"][:5]


def test_rice_r0_agrees_with_fp64_log2():
    """The host r0 is the reference's fp64 form (codec.py:271-272); the device's exact integer form
    (largest k with count * 2^k <= sum) agrees with it on its domain, sum < 2^32."""
    import ctypes
    L = _native.lib()
    rng = np.random.default_rng(0)
    cases = [(c, s) for c in (1, 2, 3, 7, 1000, 123457) for s in (0, 1, c - 1, c, c + 1, 2 * c, 2 * c - 1)]
    cases += [(int(c), int(c) * (1 << k) + d) for c in rng.integers(1, 1 << 20, 50) for k in range(0, 31, 3)
              for d in (-1, 0, 1)]
    for count, gap_sum in cases:
        if gap_sum < 0:
            continue
        cand = (ctypes.c_int32 * 3)()
        L.crx_rice_candidates(count, gap_sum, cand)
        r0 = int(np.clip(np.floor(np.log2(max(gap_sum / count, 1.0))), 0, 30))
        assert cand[1] == r0, (count, gap_sum)
        if gap_sum < 1 << 32:
            k = 0
            while k < 30 and count << (k + 1) <= gap_sum:
                k += 1
            assert k == r0, (count, gap_sum)


def _golden_bytes(golden):
    return {n: bytes.fromhex(r["update"]["hex"]) for n, r in golden["updates"]["single"].items()
            if "hex" in r["update"]}


def test_parse_golden_updates_round_trip(golden):
    for name, data in _golden_bytes(golden).items():
        u = wire.parse(data)
        plain = wire.Update(u.tables, u.tensors, u.block_bits, u.payload)
        assert wire.serialize(plain) == data, name
        assert u.total_changes == sum(g.count for t in u.tensors for g in t.groups)


def test_hostile_headers_fail_in_parse():
    from test_oracle import hostile_updates
    for h in hostile_updates():
        with pytest.raises(crukx_sync.CorruptUpdate):
            wire.parse(h)
        a = torch.zeros(100, dtype=torch.int16)
        with pytest.raises(crukx_sync.CorruptUpdate):
            crukx_sync.apply_update({"w": a.clone()}, h)


def test_a_count_the_block_table_cannot_back_is_refused_by_the_parser():
    """A group claiming all 2^22 elements of a tensor, with zero-bit blocks: the block table alone
    refutes it (two bits per change at least), so nothing is sized by the count."""
    n = 1 << 22
    u = wire.Update([wire.Table(0, [0], [1])], [wire.TensorHeader("w", n, 0, [wire.Group(0, n, 0)])],
                    [0] * wire.n_blocks(n), b"")
    with pytest.raises(crukx_sync.CorruptUpdate, match="block shorter than its symbols could be"):
        crukx_sync.apply_update({"w": torch.zeros(n, dtype=torch.int16)}, wire.serialize(u))


def test_inputs_past_the_32_bit_limits_raise_before_device_work():
    """Tensors of 2^32 elements are refused with ValueError before any device work (this host has no
    device: device work would raise RuntimeError).  The big tensor is allocated and never touched.
    Updates of 2^32 or more changes are not refused: they are encoded and applied part by part."""
    big = torch.empty(1 << 32, dtype=torch.int16)
    one = wire.Update([wire.Table(0, [0], [1])], [wire.TensorHeader("w", 1 << 32, 0, [wire.Group(0, 1, 0)])],
                      [2], b"\x00")
    for call in (lambda: crukx_sync.apply_update({"w": big}, wire.serialize(one)),
                 lambda: crukx_sync.encode_update({"w": big}, {"w": big}),
                 lambda: codec.checksum(big)):
        with pytest.raises(ValueError, match=r"2\^32 or more elements"):
            call()


@pytest.mark.parametrize("name", ["rl_200k", "many_tensors", "slab_4097", "extreme", "three_tensors"])
def test_parser_agrees_with_oracle_on_every_byte_flip(golden, name):
    data = _golden_bytes(golden).get(name)
    if data is None:
        pytest.skip("not stored inline")
    for i in range(len(data)):
        for x in (0x01, 0x80, 0xFF):
            bad = bytearray(data)
            bad[i] ^= x
            bad = bytes(bad)
            try:
                oracle.parse_check(bad)
                ref_ok = True
            except oracle.OracleCorrupt:
                ref_ok = False
            try:
                wire.parse(bad)
                ok = True
            except crukx_sync.CorruptUpdate:
                ok = False
            assert ok == ref_ok, (name, i, x)


def test_varint_limits():
    out = bytearray()
    wire.write_varint(out, (1 << 63) - 1)
    assert len(out) == 9
    with pytest.raises(ValueError):
        wire.write_varint(bytearray(), 1 << 63)
    # non-canonical varints (trailing zero groups) are accepted, as in the reference's reader
    upd = b"CRXS\x02" + b"\x80\x00" + b"\x80\x80\x00" + b"\x00"
    u = wire.parse(upd)
    assert u.tensors == [] and u.tables == []
    # 10th byte carrying bit 63 is out of range
    with pytest.raises(crukx_sync.CorruptUpdate):
        wire.parse(b"CRXS\x02" + b"\x80" * 9 + b"\x01" + b"\x00\x00")


def test_empty_update_bytes():
    assert crukx_sync.encode_update({}, {}) == b"CRXS\x02\x00\x00\x00"
    assert crukx_sync.apply_update({}, b"CRXS\x02\x00\x00\x00").tensors == 0


def test_api_errors_before_any_device_work():
    a = torch.zeros(10, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        crukx_sync.encode_update({"w": a}, {"x": a})
    with pytest.raises(ValueError):
        crukx_sync.encode_update({"w": a}, {"w": a.float()})
    with pytest.raises(ValueError):
        crukx_sync.encode_update({"w": a}, {"w": torch.zeros(11, dtype=torch.bfloat16)})
    with pytest.raises(ValueError):
        crukx_sync.encode_update({"w": torch.zeros(4, 4, dtype=torch.bfloat16).t()},
                                 {"w": torch.zeros(4, 4, dtype=torch.bfloat16)})


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the behaviour without a HIP device")
def test_no_silent_cpu_fallback():
    a = torch.zeros(10, dtype=torch.bfloat16)
    b = a.clone()
    b[3] = 1.0
    with pytest.raises(RuntimeError, match="HIP"):
        crukx_sync.encode_update({"w": a}, {"w": b})


def test_tensor_metadata_helper_agrees_with_the_tensors():
    """The batched metadata helper (crukx_sync/crx_tensor_meta.so) returns what the tensors report one by
    one: address, element count, device, dtype/contiguity flags, version; and pairwise shape equality."""
    from array import array
    M = _native.tensor_meta()
    if M is None:
        pytest.skip("the helper is built by __graft_entry__.build()")
    base = torch.arange(100, dtype=torch.int16)
    ts = [torch.zeros(7, dtype=torch.bfloat16), base, base[3:50], base.view(10, 10).t(), torch.zeros(5),
          torch.ones(2, 3, dtype=torch.int16)]
    ts[1].add_(1)  # a version counter above zero
    ptr, numel, dev, flags, ver = M.meta(ts)
    ptr, numel, ver = array("Q", ptr), array("Q", numel), array("Q", ver)
    dev, flags = array("i", dev), array("i", flags)
    for i, t in enumerate(ts):
        assert ptr[i] == t.data_ptr() and numel[i] == t.numel() and dev[i] == t.get_device() and ver[i] == t._version
        assert flags[i] == (1 if t.dtype in (torch.bfloat16, torch.int16) else 0) | (2 if t.is_contiguous() else 0)
    assert array("Q", M.versions(ts)) == ver
    assert M.same_shapes(ts, [t.clone() for t in ts]) and not M.same_shapes(ts[:2], ts[1:3])
    ma, mb, same = M.meta_pair(ts, [t.clone() for t in ts])  # the encoder's combined call
    assert ma == M.meta(ts) and array("Q", mb[1]) == numel and same
    assert M.meta_pair(ts[:2], ts[1:3])[2] is False
    with pytest.raises(TypeError):
        M.meta([ts[0], None])
    with pytest.raises(TypeError):
        M.meta_pair([ts[0]], [None])


def test_parsed_update_fields_are_editable_like_the_reference_dataclass(golden):
    """The reference's Update is a plain mutable dataclass (wire.py:44-48).  An update parsed by the
    native library reads its fields lazily; assigning one turns it into plain data, so serialize()
    writes what was assigned."""
    rec = golden["updates"]["single"]["three_tensors"]["update"]
    sc = __import__("scenarios").single_scenarios()["three_tensors"]
    data = oracle.encode_update(*sc)
    assert hashlib.sha256(data).hexdigest() == rec["sha256"]
    u = wire.parse(data)
    assert not u.edited and wire.serialize(u) == data
    plain = wire.Update(u.tables, u.tensors, u.block_bits, u.payload)
    assert wire.serialize(plain) == data
    u.payload = u.payload[:-1] + bytes([u.payload[-1] ^ 0x80])
    assert u.edited
    edited = wire.serialize(u)
    assert len(edited) == len(data) and edited[:-1] == data[:-1] and edited[-1] == data[-1] ^ 0x80
    u.tables = u.tables[:1]
    assert wire.serialize(u) == wire.serialize(wire.Update(u.tables, u.tensors, u.block_bits, u.payload))
    with pytest.raises(crukx_sync.CorruptUpdate):  # the edited update, not the parsed one, is applied
        codec.apply({k: v.clone() for k, v in sc[0].items()}, u)
