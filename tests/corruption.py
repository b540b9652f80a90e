"""Single-byte corruption sequences over the four-tensor case (small4, 26,611,713 weights), shared by the
GPU tests (tests/test_full_sizes.py) and the CPU model of the library (tests/model/run.py), so that both
run exactly the same updates and flips in the same order.

Reference behaviour: every corrupted update raises, with the weights untouched
(tests/test_roundtrip.py:92-106, codec.py:709-712); a flip that leaves a valid update with the same
meaning (a harmless flip) applies exactly.
"""

from __future__ import annotations

import random

import torch

import crukx_sync
from crukx_sync import CorruptUpdate, _native, wire, workloads

DENSE_TENSOR = "layer.proj.weight"
DENSE_AT, DENSE_LEN, DENSE_FRAC = 3_000_000, 40_000, 0.3


def equal(x, y) -> bool:
    return all(torch.equal(x[k].view(torch.int16), y[k].view(torch.int16)) for k in x)


def _varint_len(v: int) -> int:
    n = 1
    while v >= 0x80:
        v >>= 7
        n += 1
    return n


def states(device, widened: bool):
    """p0 -> p1 -> p2 of small4 (weights seed 7, 1% steps).  Widened: edge values (+-0, subnormals,
    +-max-finite) at density 2e-5 in p0, whose exponent-0 elements change at every step (targets at
    exponent 0 beside the bulk near the median exponent: slabs of several 64-exponent windows), and a
    dense patch in p2 (30% of 40,000 consecutive elements of one tensor changed by one bit-pattern step:
    windows with more targets than the select pass keeps in LDS)."""
    shapes = workloads.small4_shapes()
    p0 = workloads.make_weights(shapes, seed=7, device=device)
    if widened:
        workloads.inject_edges(p0, 2e-5, seed=8)
    p1 = workloads.make_step(p0, 1, rho=0.01, seed=7)
    p2 = workloads.make_step(p1, 2, rho=0.01, seed=7)
    if widened:
        g = torch.Generator(device="cpu").manual_seed(9)
        b = p2[DENSE_TENSOR].view(torch.int16).view(-1)
        sel = torch.nonzero(torch.rand(DENSE_LEN, generator=g) < DENSE_FRAC).view(-1) + DENSE_AT
        step = torch.where(torch.rand(sel.numel(), generator=g) < 0.5, 1, -1).to(torch.int16)
        sel, step = sel.to(b.device), step.to(b.device)
        b[sel] = b[sel] + step
    return p0, p1, p2


def offsets(buf: torch.Tensor, widened: bool) -> tuple[list[int], str]:
    """The byte offsets to flip, in order: every header byte, both ends of every block-table entry,
    every byte of the payload length, the payload's first and last bytes and 10,000 random payload
    bytes; widened, also 1,000 bytes of the blocks of exponents below 64 (their changes lie in slabs of
    several windows) and 1,000 of the dense tensor's blocks."""
    u, L = wire.parse(buf), _native.lib()
    n_blocks = L.crx_update_n_blocks(u.handle)
    pay, pay_len = L.crx_update_payload_offset(u.handle), L.crx_update_payload_len(u.handle)
    bt = pay - _varint_len(pay_len) - 4 * n_blocks
    rnd = random.Random(11)
    out = list(range(bt))
    for b in range(n_blocks):
        out += [bt + 4 * b, bt + 4 * b + 3]
    out += list(range(bt + 4 * n_blocks, pay))
    out += [pay, pay + pay_len - 1] + rnd.sample(range(pay + 1, pay + pay_len - 1), 10_000)
    note = f"{bt} header bytes, {n_blocks} blocks, {pay_len} payload bytes"
    if widened:
        bits = u.block_bits
        starts = [0]
        for v in bits:
            starts.append(starts[-1] + v)
        far, dense = [], []
        b = 0
        for t in u.tensors:
            for gr in t.groups:
                nb = wire.n_blocks(gr.count)
                lo, hi = pay + starts[b] // 8, pay + (starts[b + nb] + 7) // 8
                if gr.exponent < 64:
                    far += range(lo, hi)
                if t.name == DENSE_TENSOR:
                    dense += range(lo, hi)
                b += nb
        assert far and dense
        out += rnd.sample(far, min(1000, len(far))) + rnd.sample(dense, min(1000, len(dense)))
        note += f", {len(far)} payload bytes in blocks of exponents below 64"
    del u
    return out, note


def run(device, widened: bool, say, first: int = 0, count: int = -1, every: int = 1, check_every: int = 500,
        verbose: bool = False, only=None) -> tuple[int, int]:
    """Encodes p0 -> p1 (applied, caches warm on both sides) and p1 -> p2 as a device-resident update,
    then flips each chosen offset by 0x01, 0x80 or 0xFF in turn and applies: a flip either raises with the
    receiver unchanged or applies exactly (then the receiver goes back to p1).  Flips [first, first +
    count) every `every`-th, or the indices in `only`.  Ends by applying the intact update.  Returns
    (rejected, applied)."""
    p0, p1, p2 = states(device, widened)
    send, rc = {}, {}
    recv = {k: v.clone() for k, v in p0.items()}
    crukx_sync.apply_update(recv, crukx_sync.encode_update_device(p0, p1, send), rc)
    assert equal(recv, p1)
    chk1 = {k: v[0] for k, v in rc.items()}
    buf = crukx_sync.encode_update_device(p1, p2, send)
    offs, note = offsets(buf, widened)
    tag = "small4 widened" if widened else "small4"
    say(f"{tag}: {len(offs)} flips ({note})")
    end = len(offs) if count < 0 else min(len(offs), first + count)
    order = list(range(first, end, every)) if only is None else list(only)
    rejected = applied = 0
    for n, j in enumerate(order):
        i, x = offs[j], (0x01, 0x80, 0xFF)[j % 3]
        if verbose:
            say(f"{tag}: flip {j}: byte {i} ^ {x:#x}")
        buf[i:i + 1].bitwise_xor_(x)
        try:
            crukx_sync.apply_update(recv, buf, rc)
        except (CorruptUpdate, ValueError):
            rejected += 1
        else:  # a harmless flip: the result must be exact; start over from the old state
            applied += 1
            assert equal(recv, p2), (j, i, x)
            for k in recv:
                recv[k].copy_(p1[k])
            rc.update({k: (chk1[k], recv[k]._version) for k in recv})
        buf[i:i + 1].bitwise_xor_(x)
        if n % check_every == check_every - 1 or n == len(order) - 1:
            assert equal(recv, p1), f"a write after one of the flips {order[max(0, n - check_every + 1)]}..{j}"
            say(f"{tag}: flip {j} ({n + 1} of {len(order)}): {rejected} rejected, {applied} applied")
    crukx_sync.apply_update(recv, buf, rc)
    assert equal(recv, p2)
    assert send == {k: v[0] for k, v in rc.items()}
    return rejected, applied
