"""Round trips at the workloads' full sizes, on the GPU: Qwen2.5-1.5B, -7B and -32B-shaped bf16
state dicts (1.54B, 7.62B and 32.8B weights), where the oracle would need hours.  Only
size-independent properties are checked:

- every chained step applies exactly (receiver == sender's new state, bit for bit);
- sender cache == receiver cache, and cached checksums equal a full recomputation;
- the change-density / step-size sweep (rho in {0.5, 1, 2, 3}%, P(|k| = 1) in {0.95, 0.87, 0.70});
- the 7B shape at rho = 1% and 2% over two chained steps;
- the four-tensor case: single-byte flips of every header byte, every block-table entry and 10,000
  payload bytes, each raising with the receiver unchanged or applying exactly; again with small
  slabs, slabs of several windows, an LDS-overflowing dense patch and flips inside those blocks;
- 32B shape with edge values (+-0, subnormals, +-max-finite) injected at 1e-4 density and smaller
  slabs: single-byte corruptions across the header, the block table and the payload either raise
  with the receiver unchanged or (if the flip happens to be harmless) apply exactly.
"""

import random

import pytest
import torch

import corruption
import crukx_sync
from crukx_sync import CorruptUpdate, _native, codec, wire, workloads

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _equal(x: dict, y: dict) -> bool:
    return all(torch.equal(x[k].view(torch.int16), y[k].view(torch.int16)) for k in x)


def _varint_len(v: int) -> int:
    n = 1
    while v >= 0x80:
        v >>= 7
        n += 1
    return n


@pytest.fixture(autouse=True)
def _free_memory():
    torch.cuda.empty_cache()
    yield
    torch.cuda.empty_cache()


def test_qwen25_1_5b_seven_chained_steps():
    """The 1.5B shape (tied embedding, 338 tensors), seven chained updates with both caches."""
    shapes = workloads.qwen25_shapes("qwen2.5-1.5b")
    assert workloads.numel(shapes) == 1_543_714_304
    prev = workloads.make_weights(shapes, seed=0, device="cuda")
    recv = {k: v.clone() for k, v in prev.items()}
    send, rc = {}, {}
    for s in range(1, 8):
        cur = workloads.make_step(prev, s, rho=0.01)
        upd = crukx_sync.encode_update(prev, cur, send)
        stats = crukx_sync.apply_update(recv, upd, rc)
        assert _equal(recv, cur), s
        assert stats.bytes == len(upd) and len(upd) / stats.changed < 1.5
        prev = cur
        _say(f"1.5b step {s}: {stats.changed} changes, {len(upd)} bytes")
    assert send == {k: v[0] for k, v in rc.items()}
    for k in ("model.embed_tokens.weight", "model.layers.27.mlp.down_proj.weight", "model.norm.weight"):
        assert send[k] == codec.checksum(prev[k]), k


@pytest.mark.parametrize("rho", [0.005, 0.01, 0.02, 0.03])
def test_qwen25_1_5b_density_and_step_size_sweep(rho):
    """One update per P(|k| = 1) at each density, from the same old weights; the receiver keeps its
    caches across the three (each is applied, then undone by applying the reverse update)."""
    shapes = workloads.qwen25_shapes("qwen2.5-1.5b")
    prev = workloads.make_weights(shapes, seed=1, device="cuda")
    recv = {k: v.clone() for k, v in prev.items()}
    rc = {}
    for j, p_one in enumerate((0.95, 0.87, 0.70)):
        cur = workloads.make_step(prev, 1 + j, rho=rho, p_one=p_one, seed=1)
        fwd = crukx_sync.encode_update(prev, cur)
        stats = crukx_sync.apply_update(recv, fwd, rc)
        assert _equal(recv, cur), (rho, p_one)
        changed = sum(int((prev[k].view(torch.int16) != cur[k].view(torch.int16)).sum()) for k in prev)
        assert stats.changed == changed
        assert abs(changed / workloads.numel(shapes) - rho) < 0.05 * rho
        crukx_sync.apply_update(recv, crukx_sync.encode_update(cur, prev), rc)
        assert _equal(recv, prev), (rho, p_one)
        _say(f"rho {rho} p_one {p_one}: {changed} changes, {len(fwd) / changed:.3f} bytes/change")
        del cur


@pytest.mark.parametrize("rho", [0.01, 0.02])
def test_qwen25_7b_chained(rho):
    """The 7B shape (the benchmark's workload at rho = 1%, and at 2%), two chained steps with both
    caches, device-resident bytes."""
    shapes = workloads.qwen25_shapes("qwen2.5-7b")
    assert workloads.numel(shapes) == 7_615_616_512 and len(shapes) == 339
    prev = workloads.make_weights(shapes, seed=0, device="cuda")
    recv = {k: v.clone() for k, v in prev.items()}
    send, rc = {}, {}
    for s in range(1, 3):
        cur = workloads.make_step(prev, s, rho=rho)
        buf = crukx_sync.encode_update_device(prev, cur, send)
        stats = crukx_sync.apply_update(recv, buf, rc)
        assert _equal(recv, cur), s
        assert abs(stats.changed / workloads.numel(shapes) - rho) < 0.02 * rho
        _say(f"7b rho {rho} step {s}: {stats.changed} changes, {buf.numel()} bytes")
        del prev
        prev = cur
    assert send == {k: v[0] for k, v in rc.items()}
    assert send["lm_head.weight"] == codec.checksum(prev["lm_head.weight"])


def test_update_of_more_than_2_32_changes():
    """Three tensors of 1.6e9 weights and one of 100,000, 97% of their elements changed by +-1 or +-2
    in their bit patterns: 4.66e9 changes, more than 2^32, so encode and apply go part by part (one
    tensor per part for the large ones).  The header counts each tensor's changes as torch counts them,
    a byte flipped in the last part's payload is rejected with every tensor unchanged (the first part
    included), and the update applies exactly, with both checksum caches equal to full checksums."""
    shapes = [(n, (1_600_000_000,), "linear") for n in ("a", "b", "c")] + [("d", (100_000,), "norm")]
    old = workloads.make_weights(shapes, seed=3, device="cuda")
    new, want = {}, {}
    g = torch.Generator(device="cuda").manual_seed(5)
    for k, t in old.items():
        r = torch.randint(0, 100, t.shape, generator=g, device="cuda", dtype=torch.int16)
        d = torch.where(r < 3, 0, (1 + (r & 1)) * (1 - 2 * ((r >> 1) & 1))).to(torch.int16)
        del r
        want[k] = int((d != 0).sum())
        new[k] = (t.view(torch.int16) + d).view(torch.bfloat16)
        del d
    total = sum(want.values())
    assert total > 1 << 32
    _say(f"2^32+: {total:,} changes")
    send, rc = {}, {}
    upd = crukx_sync.encode_update_device(old, new, send)
    u = wire.parse(upd)
    assert u.total_changes == total
    assert {t.name: sum(g.count for g in t.groups) for t in u.tensors} == want
    del u
    _say(f"2^32+: {upd.numel():,} bytes")
    recv = {k: v.clone() for k, v in old.items()}
    rejected = 0
    for k in (2, 3, 5):  # bytes near the payload's end: blocks of the last part
        upd[-k:upd.numel() - k + 1].bitwise_xor_(0x10)
        try:
            crukx_sync.apply_update(recv, upd, rc)
        except CorruptUpdate:
            rejected += 1
        upd[-k:upd.numel() - k + 1].bitwise_xor_(0x10)
        assert _equal(recv, old), k
    assert rejected == 3
    _say("2^32+: corrupted updates rejected, receiver unchanged")
    crukx_sync.apply_update(recv, upd, rc)
    assert _equal(recv, new)
    assert send == {k: v[0] for k, v in rc.items()}
    assert all(send[k] == codec.checksum(new[k]) for k in new)


def test_qwen25_32b_edge_values_and_corruptions(monkeypatch):
    """The 32B shape (771 tensors, 65.5 GB per copy) with edge values in both states and 16K-weight
    slabs.  A first update warms the receiver's caches; then single-byte flips of the second update
    (bytes before the block table, every 4-byte boundary of sampled block-table entries, random payload
    bytes) are applied to the receiver, which must stay equal to its old state whenever one raises."""
    monkeypatch.setattr(codec, "_SLAB", 1 << 14)
    shapes = workloads.qwen25_shapes("qwen2.5-32b")
    assert workloads.numel(shapes) == 32_763_876_352
    p0 = workloads.make_weights(shapes, seed=4, device="cuda")
    workloads.inject_edges(p0, 1e-4, seed=1)
    recv = {k: v.clone() for k, v in p0.items()}
    p1 = workloads.make_step(p0, 1, rho=0.01, seed=4)
    workloads.inject_edges(p1, 1e-4, seed=2)
    send, rc = {}, {}
    u1 = crukx_sync.encode_update_device(p0, p1, send)
    del p0
    crukx_sync.apply_update(recv, u1, rc)
    assert _equal(recv, p1)
    del u1
    chk1 = {k: v[0] for k, v in rc.items()}
    p2 = workloads.make_step(p1, 2, rho=0.01, seed=4)
    workloads.inject_edges(p2, 1e-4, seed=3)
    buf = crukx_sync.encode_update_device(p1, p2, send)
    _say(f"32b: update of {buf.numel()} bytes")

    u, L = wire.parse(buf), _native.lib()
    n_blocks = L.crx_update_n_blocks(u.handle)
    pay, pay_len = L.crx_update_payload_offset(u.handle), L.crx_update_payload_len(u.handle)
    bt = pay - _varint_len(pay_len) - 4 * n_blocks
    del u
    rnd = random.Random(5)
    offsets = list(range(64)) + rnd.sample(range(64, bt), 136)                      # header
    for b in rnd.sample(range(n_blocks), 50):                                       # block table
        offsets += [bt + 4 * b, bt + 4 * b + 3]
    offsets += list(range(bt + 4 * n_blocks, pay))                                  # payload_len
    offsets += [pay, pay + pay_len - 1] + rnd.sample(range(pay + 1, pay + pay_len - 1), 200)
    rejected = 0
    for j, i in enumerate(offsets):
        x = (0x01, 0x80, 0xFF)[j % 3]
        buf[i:i + 1].bitwise_xor_(x)
        try:
            crukx_sync.apply_update(recv, buf, rc)
        except (CorruptUpdate, ValueError):
            rejected += 1
        else:  # a harmless flip: the result must be exact; start over from the old state
            assert _equal(recv, p2), (i, x)
            for k in recv:
                recv[k].copy_(p1[k])
            rc.update({k: (chk1[k], recv[k]._version) for k in recv})
        buf[i:i + 1].bitwise_xor_(x)
        if j % 25 == 24 or j == len(offsets) - 1:
            assert _equal(recv, p1), f"a write after one of the flips at offsets {offsets[j - 24:j + 1]}"
            _say(f"32b: {j + 1} flips, {rejected} rejected")
    assert rejected >= 0.9 * len(offsets)
    crukx_sync.apply_update(recv, buf, rc)
    assert _equal(recv, p2)
    assert send == {k: v[0] for k, v in rc.items()}


def test_small4_every_header_byte_every_block_boundary_and_10k_payload_flips():
    """The four-tensor case (26.6M weights, receiver caches warm): single-byte flips of every header
    byte, both ends of every block-table entry, the payload length and 10,000 random payload bytes.
    Each flip either raises with the receiver unchanged or (a harmless flip) applies exactly."""
    rejected, applied = corruption.run("cuda", False, _say)
    assert rejected >= 0.9 * (rejected + applied)


def test_small4_widened_flips_with_small_slabs(monkeypatch):
    """The same flips with 16,384-element slabs (every tensor takes the group-size check; many slabs
    per tensor), edge values whose exponent-0 changes put slabs across several 64-exponent windows, a
    dense patch whose windows overflow the select pass's LDS list, the receiver's caches warm, and
    2,000 more payload flips inside the blocks of those slabs."""
    monkeypatch.setattr(codec, "_SLAB", 1 << 14)
    rejected, applied = corruption.run("cuda", True, _say)
    assert rejected >= 0.9 * (rejected + applied)
