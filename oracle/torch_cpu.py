"""A torch-CPU restatement of the reference's CPU path, for timing it beside the GPU.

TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it on the host cores, and tests/ check
its bytes against the golden vectors the reference wrote; the product (crukx-sync_amd/) never
imports it.

It runs the algorithm the reference runs on CPU tensors (src/crukx_sync/codec.py), in whole-tensor
torch operations, as the wire format (docs/FORMAT.md) and the reference's call structure lay it out:
- encode ranks the changes of each tensor by a stable argsort of the old exponents per slab of at
  most 2^24 elements (codec.py:124-147), orders them by (exponent, rank), derives gaps and zigzag
  residuals, picks Rice parameters (codec.py:268-275), builds one canonical Huffman table per
  exponent on the host with a binary heap (codec.py:71-111) and packs all codes with scatter-adds
  into 32-bit words (codec.py:218-257);
- apply parses the header in Python with the per-block length check (wire.py:126-212), decodes all
  blocks together in at most 256 vectorised steps (codec.py:504-536; unary runs longer than a
  64-bit window continue window by window, codec.py:539-575), finds each change's position by the
  same slab sorts of the receiver's weights (codec.py:654-694), verifies the checksums (full ones
  through 2^24-element chunks, codec.py:61-68) and writes with index_put_ (codec.py:713-714).
Tensors of at most 2^22 elements are ranked, in encode and in apply, by shared stable sorts on
(tensor, exponent) keys over groups of at most 127 tensors and 2^24 elements, as the reference batches
them (codec.py:150-194, 659-678).
"""

from __future__ import annotations

import heapq
import struct

import numpy as np
import torch

SLAB = 1 << 24       # elements per stable sort
SMALL_TENSOR = 1 << 22  # tensors up to this size share sorts with others
MAX_SEGS = 127       # tensors per shared sort: (tensor, exponent) keys fit int16
CHUNK = 1 << 24      # elements per checksum chunk
BLOCK = 256
MAX_LEN = 17
MAX_RICE = 30
SYM_SPACE = 131071   # zigzag residuals are 0 .. 131070
MASK64 = (1 << 64) - 1


class Corrupt(ValueError):
    pass


# ---------------------------------------------------------------- 64-bit helpers (int64 tensors wrap)

def _signed(v: int) -> int:
    v &= MASK64
    return v - (1 << 64) if v >> 63 else v


_G, _M1, _M2 = _signed(0x9E3779B97F4A7C15), _signed(0xBF58476D1CE4E5B9), _signed(0x94D049BB133111EB)


def _shr(x: torch.Tensor, k: int) -> torch.Tensor:
    """Logical right shift of int64 bit patterns."""
    return (x >> k) & ((1 << (64 - k)) - 1)


def _w(idx: torch.Tensor) -> torch.Tensor:
    """splitmix64(i) | 1 as int64 bit patterns (docs/FORMAT.md, Integrity)."""
    z = (idx + 1) * _G
    z = (z ^ _shr(z, 30)) * _M1
    z = (z ^ _shr(z, 27)) * _M2
    return (z ^ _shr(z, 31)) | 1


def checksum(t: torch.Tensor) -> int:
    flat = t.reshape(-1).view(torch.int16)
    s = 0
    for lo in range(0, flat.numel(), CHUNK):
        hi = min(flat.numel(), lo + CHUNK)
        u = flat[lo:hi].to(torch.int64) & 0xFFFF
        s += int((u * _w(torch.arange(lo, hi, dtype=torch.int64))).sum())
    return s & MASK64


def _delta(pos: torch.Tensor, old_u: torch.Tensor, new_u: torch.Tensor) -> int:
    return int(((new_u - old_u) * _w(pos)).sum()) & MASK64


# ---------------------------------------------------------------- tables

def huffman_lengths(counts: list[int]) -> list[int]:
    """Code lengths of at most MAX_LEN bits: a heap of (count, id), leaves 0..n-1 first and merged
    nodes numbered on from n; if the deepest leaf is too deep, counts become max(1, c >> 2) and the
    tree is built again (up to 8 times), else all codes get the same length."""
    n = len(counts)
    c = list(counts)
    for _ in range(8):
        if n == 1:
            return [1]
        heap = [(v, i) for i, v in enumerate(c)]
        heapq.heapify(heap)
        up = [0] * (2 * n - 1)
        nid = n
        while len(heap) > 1:
            a, b = heapq.heappop(heap), heapq.heappop(heap)
            up[a[1]] = up[b[1]] = nid
            heapq.heappush(heap, (a[0] + b[0], nid))
            nid += 1
        depth = [0] * (2 * n - 1)
        for node in range(2 * n - 3, -1, -1):
            depth[node] = depth[up[node]] + 1
        lens = depth[:n]
        if max(lens) <= MAX_LEN:
            return lens
        c = [max(1, v >> 2) for v in c]
    return [max(1, (n - 1).bit_length())] * n


def canonical_codes(lengths: list[int]) -> list[int]:
    order = sorted(range(len(lengths)), key=lambda i: (lengths[i], i))
    codes = [0] * len(lengths)
    code, prev = 0, lengths[order[0]]
    for k, i in enumerate(order):
        if k:
            code = (code + 1) << (lengths[i] - prev)
        codes[i] = code
        prev = lengths[i]
    return codes


def _varint(out: bytearray, v: int) -> None:
    while v >= 0x80:
        out.append((v & 0x7F) | 0x80)
        v >>= 7
    out.append(v)


# ---------------------------------------------------------------- ranking

def _exp(bits: torch.Tensor) -> torch.Tensor:
    """Old exponents (bits >> 7) & 0xFF of int16 bit patterns, as uint8."""
    return ((bits >> 7) & 0xFF).to(torch.uint8)


def _ranks_of_changes(e: torch.Tensor, changed: torch.Tensor):
    """For the changed elements of one tensor, in (exponent, position) order: their positions,
    exponents and ranks among all elements of their exponent (stable), via slab sorts."""
    n = e.numel()
    before = torch.zeros(256, dtype=torch.int64)
    pos_l, exp_l, rank_l = [], [], []
    for lo in range(0, n, SLAB):
        hi = min(n, lo + SLAB)
        key = e[lo:hi]
        order = torch.sort(key, stable=True).indices
        cnt = torch.bincount(key, minlength=256)
        start = torch.cumsum(cnt, 0) - cnt
        j = torch.nonzero(changed[lo:hi][order]).view(-1)  # sorted slots holding a change
        if j.numel():
            p = order[j]
            k = key[p].to(torch.int64)
            pos_l.append(p + lo)
            exp_l.append(k)
            rank_l.append(j - start[k] + before[k])
        before += cnt
    if not pos_l:
        z = torch.zeros(0, dtype=torch.int64)
        return z, z, z, before
    pos, ex, rank = torch.cat(pos_l), torch.cat(exp_l), torch.cat(rank_l)
    o = torch.argsort((ex << 40) + rank)  # (exponent, rank) across slabs
    return pos[o], ex[o], rank[o], before


def _small_groups(sizes: list[int]) -> list[list[int]]:
    """Indices of the tensors of at most SMALL_TENSOR (and SLAB) elements, in order, grouped so that
    each group holds at most SLAB elements and MAX_SEGS tensors (codec.py:154-168)."""
    groups, cur, total = [], [], 0
    for i, n in enumerate(sizes):
        if n > min(SMALL_TENSOR, SLAB):
            continue
        if cur and (total + n > SLAB or len(cur) == MAX_SEGS):
            groups.append(cur)
            cur, total = [], 0
        cur.append(i)
        total += n
    if cur:
        groups.append(cur)
    return groups


def _shared_sort(es: list[torch.Tensor]):
    """One stable sort of several tensors' exponents on (tensor, exponent) keys: the sort order (indices
    into the concatenation), each tensor's offset there, and where each key starts in the order
    ([len(es) * 256 + 1])."""
    sizes = torch.tensor([e.numel() for e in es], dtype=torch.int64)
    seg = torch.repeat_interleave(torch.arange(len(es), dtype=torch.int16), sizes)
    key = (seg << 8) | torch.cat(es).to(torch.int16)
    order = torch.sort(key, stable=True).indices
    cnt = torch.bincount(key.to(torch.int64), minlength=len(es) * 256)
    starts = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(cnt, 0)])
    offs = torch.cumsum(sizes, 0) - sizes
    return order, offs, starts


def _ranks_of_changes_many(es: list[torch.Tensor], changed: list[torch.Tensor]):
    """_ranks_of_changes for several small tensors with one shared sort (codec.py:171-194)."""
    order, offs, starts = _shared_sort(es)
    j = torch.nonzero(torch.cat(changed)[order]).view(-1)   # sorted slots holding a change
    p = order[j]
    t = torch.searchsorted(offs, p, right=True) - 1           # tensor of each change
    k = ((t << 8) | torch.cat(es).to(torch.int64)[p])
    rank = j - starts[k]
    pos = p - offs[t]
    # rows are tensor-major, then (exponent, position) within a tensor: (exponent, rank) order
    per = torch.bincount(t, minlength=len(es)).tolist()
    return [(p_, k_ & 255, r_) for p_, k_, r_ in zip(pos.split(per), k.split(per), rank.split(per))]


# ---------------------------------------------------------------- encode

def _rice(gaps: torch.Tensor, seg: torch.Tensor, counts: torch.Tensor) -> list[int]:
    """Per group: r0 = floor(log2(max(mean gap, 1))) in float64, clamped to [0, 30], then the cheapest
    of r0 - 1, r0, r0 + 1 (clamped) by bit cost sum((gap >> r) + 1 + r), first minimum."""
    ng = counts.numel()
    gsum = torch.zeros(ng, dtype=torch.int64).index_add_(0, seg, gaps)
    mean = gsum.to(torch.float64) / counts.to(torch.float64)
    r0 = torch.floor(torch.log2(torch.clamp(mean, min=1.0))).to(torch.int64).clamp(0, MAX_RICE)
    cand = torch.stack([(r0 - 1).clamp(min=0), r0, (r0 + 1).clamp(max=MAX_RICE)])  # [3, groups]
    cost = torch.stack([torch.zeros(ng, dtype=torch.int64).index_add_(0, seg, gaps >> cand[k][seg])
                        + counts * (1 + cand[k]) for k in range(3)])
    best = torch.argmin(cost, 0)  # first minimum on ties
    return cand.gather(0, best.view(1, -1)).view(-1).tolist()


def _place(words: torch.Tensor, off: torch.Tensor, val: torch.Tensor, ln: torch.Tensor) -> None:
    """OR codes (val < 2^62, ln <= 62 bits, none overlapping) into 32-bit big-endian-bit words at bit
    offsets `off`, with three scatter-adds."""
    w = off >> 5
    s = off & 31
    room = 32 - s                         # bits left in the first word
    first_shift = ln - room               # >0: the code continues into the next word
    a = torch.where(first_shift >= 0, val >> first_shift.clamp(min=0), val << (-first_shift).clamp(min=0))
    words.index_add_(0, w, a)
    rest = first_shift                    # bits after the first word
    m = rest > 0
    if bool(m.any()):
        v1, r1, w1 = val[m], rest[m], w[m] + 1
        b = torch.where(r1 >= 32, (v1 >> (r1 - 32).clamp(min=0)) & 0xFFFFFFFF, (v1 << (32 - r1).clamp(min=0)) & 0xFFFFFFFF)
        words.index_add_(0, w1, b)
        m2 = r1 > 32
        if bool(m2.any()):
            v2, r2 = v1[m2], r1[m2] - 32
            words.index_add_(0, w1[m2] + 1, (v2 << (32 - r2)) & 0xFFFFFFFF)


def encode_update(old: dict, new: dict, checksums: dict | None = None) -> bytes:
    """encode_update on CPU tensors; `checksums` (name -> int) is the sender cache, updated once the
    bytes exist."""
    names = list(old)
    todo = []  # (name, old bits, new bits, changed) of the tensors with a change
    for name in names:
        a = old[name].reshape(-1).view(torch.int16)
        b = new[name].reshape(-1).view(torch.int16)
        if a.numel() != b.numel():
            raise ValueError(f"{name}: old and new differ in shape")
        changed = a != b
        if bool(changed.any()):
            todo.append((name, a, b, changed))
    ranked = {}
    for grp in _small_groups([a.numel() for _, a, _, _ in todo]):
        res = _ranks_of_changes_many([_exp(todo[i][1]) for i in grp], [todo[i][3] for i in grp])
        ranked.update(zip(grp, res))
    tensors = []  # (name, numel, pos, exp, rank, old_u, new_u)
    for i, (name, a, b, changed) in enumerate(todo):
        pos, ex, rank = ranked[i] if i in ranked else _ranks_of_changes(_exp(a), changed)[:3]
        tensors.append((name, a.numel(), pos, ex, rank, a[pos].to(torch.int64) & 0xFFFF,
                        b[pos].to(torch.int64) & 0xFFFF))
    new_chk = {}
    if not tensors:
        return b"CRXS\x02\x00\x00\x00"
    # per tensor: groups (exponent runs), gaps, residual symbols
    per = []
    for name, numel, pos, ex, rank, ou, nu in tensors:
        head = torch.ones(ex.numel(), dtype=torch.bool)
        head[1:] = ex[1:] != ex[:-1]
        starts = torch.nonzero(head).view(-1)
        counts = torch.diff(torch.cat([starts, torch.tensor([ex.numel()])]))
        seg = torch.cumsum(head.to(torch.int64), 0) - 1
        prev = torch.empty_like(rank)
        prev[0] = -1
        prev[1:] = rank[:-1]
        prev[head] = -1
        gaps = rank - prev - 1
        d = (nu.to(torch.int16).to(torch.int64)) - (ou.to(torch.int16).to(torch.int64))
        zz = torch.where(d >= 0, 2 * d, -2 * d - 1)
        rice = _rice(gaps, seg, counts)
        gexp = ex[starts].tolist()
        cached = None if checksums is None else checksums.get(name)
        if cached is not None:
            new_chk[name] = (cached + _delta(pos, ou, nu)) & MASK64
        else:
            new_chk[name] = checksum(new[name])
        per.append((name, numel, gexp, counts, seg, gaps, zz, torch.tensor(rice, dtype=torch.int64), ex))
    # one table per exponent over all tensors: symbols ascending, canonical codes
    keys = torch.cat([p[8] * SYM_SPACE + p[6] for p in per])
    ukeys, ucnt = torch.unique(keys, sorted=True, return_counts=True)
    uk, uc = ukeys.tolist(), ucnt.tolist()
    code_of = [0] * len(uk)
    len_of = [0] * len(uk)
    tables = []
    i = 0
    while i < len(uk):
        e = uk[i] // SYM_SPACE
        j = i
        while j < len(uk) and uk[j] // SYM_SPACE == e:
            j += 1
        lens = huffman_lengths(uc[i:j])
        codes = canonical_codes(lens)
        code_of[i:j], len_of[i:j] = codes, lens
        tables.append((e, [k % SYM_SPACE for k in uk[i:j]], lens))
        i = j
    code_t, len_t = torch.tensor(code_of, dtype=torch.int64), torch.tensor(len_of, dtype=torch.int64)
    # every change's code pieces, in update order: the unary run of gap >> r ones, then the tail
    # (a zero, the r low bits, the Huffman code)
    bit_lens, ones_l, tail_l, tail_v, blk_l = [], [], [], [], []
    nblk = 0
    for name, numel, gexp, counts, seg, gaps, zz, rice, ex in per:
        r = rice[seg]
        ki = torch.searchsorted(ukeys, ex * SYM_SPACE + zz)
        hl, hc = len_t[ki], code_t[ki]
        q = gaps >> r
        tl = 1 + r + hl
        tail_v.append(((gaps & ((1 << r) - 1)) << hl) | hc)
        tail_l.append(tl)
        ones_l.append(q)
        bit_lens.append(q + tl)
        gstart = torch.cumsum(counts, 0) - counts
        gblk = torch.cumsum((counts + BLOCK - 1) // BLOCK, 0) - (counts + BLOCK - 1) // BLOCK
        idx_in_group = torch.arange(gaps.numel()) - gstart[seg]
        blk_l.append(nblk + gblk[seg] + (idx_in_group >> 8))
        nblk += int(((counts + BLOCK - 1) // BLOCK).sum())
    L = torch.cat(bit_lens)
    off = torch.cumsum(L, 0) - L
    total_bits = int(L.sum())
    block_bits = torch.zeros(nblk, dtype=torch.int64).index_add_(0, torch.cat(blk_l), L)
    if bool((block_bits >= 1 << 32).any()):
        raise ValueError("a block exceeds 2^32 bits")
    words = torch.zeros(total_bits // 32 + 3, dtype=torch.int64)
    q = torch.cat(ones_l)
    tl = torch.cat(tail_l)
    short = (q > 0) & (q <= 62)
    _place(words, off[short], (1 << q[short]) - 1, q[short])
    for o, n1 in zip(off[q > 62].tolist(), q[q > 62].tolist()):  # long unary runs, bit by bit
        for bit in range(o, o + n1):
            words[bit >> 5] |= 1 << (31 - (bit & 31))
    _place(words, off + q, torch.cat(tail_v), tl)
    payload = words.to(torch.int32).numpy().astype(">u4").tobytes()[:(total_bits + 7) // 8]
    # serialize (docs/FORMAT.md grammar)
    out = bytearray(b"CRXS\x02")
    _varint(out, len(tables))
    for e, syms, lens in tables:
        out.append(e)
        _varint(out, len(syms))
        for s, ln in zip(syms, lens):
            _varint(out, s)
            out.append(ln)
    _varint(out, len(per))
    for name, numel, gexp, counts, seg, gaps, zz, rice, ex in per:
        nb = name.encode()
        _varint(out, len(nb))
        out += nb
        _varint(out, numel)
        out += struct.pack("<Q", new_chk[name])
        _varint(out, len(gexp))
        for e, c, r in zip(gexp, counts.tolist(), rice.tolist()):
            out.append(e)
            _varint(out, c)
            out.append(r)
    out += block_bits.to(torch.int32).numpy().astype("<u4").tobytes()
    _varint(out, len(payload))
    out += payload
    if checksums is not None:
        checksums.update(new_chk)
    return bytes(out)


# ---------------------------------------------------------------- apply

class _Reader:
    def __init__(self, data: bytes):
        self.d, self.p = data, 0

    def take(self, n):
        if self.p + n > len(self.d):
            raise Corrupt("truncated update")
        b = self.d[self.p:self.p + n]
        self.p += n
        return b

    def u8(self):
        return self.take(1)[0]

    def varint(self):
        v = sh = 0
        while True:
            b = self.u8()
            v |= (b & 0x7F) << sh
            if not b & 0x80:
                break
            sh += 7
            if sh > 63:
                raise Corrupt("varint too long")
        if v >= 1 << 63:
            raise Corrupt("varint out of range")
        return v


def _parse(data: bytes):
    r = _Reader(data)
    if r.take(4) != b"CRXS" or r.u8() != 2:
        raise Corrupt("not a version-2 update")
    tables = {}
    for _ in range(r.varint()):
        e, n = r.u8(), r.varint()
        if e in tables or n < 1 or n > SYM_SPACE:
            raise Corrupt("bad table")
        syms, lens = [], []
        for _ in range(n):
            syms.append(r.varint())
            lens.append(r.u8())
        if max(syms) > SYM_SPACE - 1 or len(set(syms)) != n or min(lens) < 1 or max(lens) > MAX_LEN:
            raise Corrupt("bad table")
        if sum(1 << (MAX_LEN - ln) for ln in lens) > 1 << MAX_LEN:
            raise Corrupt("table violates the Kraft inequality")
        tables[e] = (syms, lens)
    tensors = []
    for _ in range(r.varint()):
        name = r.take(r.varint()).decode()
        numel = r.varint()
        chk = struct.unpack("<Q", r.take(8))[0]
        groups = []
        for _ in range(r.varint()):
            e, c, rr = r.u8(), r.varint(), r.u8()
            if e not in tables or c < 1 or c > numel or rr > MAX_RICE:
                raise Corrupt("bad group")
            groups.append((e, c, rr))
        if not groups or sum(g[1] for g in groups) > numel:
            raise Corrupt("bad tensor")
        tensors.append((name, numel, chk, groups))
    counts = [g for t in tensors for g in t[3]]
    nblk = sum((c + BLOCK - 1) // BLOCK for _, c, _ in counts)
    bb = np.frombuffer(r.take(4 * nblk), dtype="<u4").astype(np.int64)
    plen = r.varint()
    payload = r.take(plen)
    if r.p != len(data) or plen != (int(bb.sum()) + 7) // 8:
        raise Corrupt("payload length")
    k = 0
    for _, c, rr in counts:  # every block at least changes x (2 + rice) bits
        for b in range(0, c, BLOCK):
            if bb[k] < min(BLOCK, c - b) * (2 + rr):
                raise Corrupt("block too short")
            k += 1
    return tables, tensors, bb, payload


def _msb64(x: torch.Tensor) -> torch.Tensor:
    """Index of the highest set bit of nonzero int64 bit patterns (exact: 32-bit halves via frexp)."""
    hi = _shr(x, 32)
    lo = x & 0xFFFFFFFF
    part = torch.where(hi != 0, hi, lo).to(torch.float64)
    return torch.frexp(part).exponent.to(torch.int64) - 1 + torch.where(hi != 0, 32, 0)


def _decode(tables, groups, bb, payload):
    """All blocks at once, one change per block per step.  Returns (gap, zz) per change in update
    order; raises Corrupt when a block does not decode exactly to its length."""
    tix = {e: i for i, e in enumerate(sorted(tables))}
    T = len(tix)
    first = torch.zeros(T, MAX_LEN + 1, dtype=torch.int64)
    ncode = torch.zeros(T, MAX_LEN + 1, dtype=torch.int64)
    base = torch.zeros(T, MAX_LEN + 1, dtype=torch.int64)
    sym_all = []
    for e, i in tix.items():  # canonical tables: first code, count and symbol base per length
        syms, lens = tables[e]
        order = sorted(range(len(syms)), key=lambda k: (lens[k], k))
        code, b0 = 0, len(sym_all)
        for ln in range(1, MAX_LEN + 1):
            n_l = sum(1 for k in order if lens[k] == ln)
            first[i, ln], ncode[i, ln], base[i, ln] = code, n_l, b0
            code = (code + n_l) << 1
            b0 += n_l
        sym_all += [syms[k] for k in order]
    sym_t = torch.tensor(sym_all, dtype=torch.int64)
    # per block: its group's table, rice, changes, first change; bit ranges from the block table
    b_tbl, b_rice, b_cnt, b_eb = [], [], [], []
    eb = 0
    for e, c, rr in groups:
        for b in range(0, c, BLOCK):
            b_tbl.append(tix[e])
            b_rice.append(rr)
            b_cnt.append(min(BLOCK, c - b))
            b_eb.append(eb + b)
        eb += c
    tbl, rice, cnt, ebase = (torch.tensor(v, dtype=torch.int64) for v in (b_tbl, b_rice, b_cnt, b_eb))
    bbt = torch.from_numpy(bb)
    end = torch.cumsum(bbt, 0)
    cur = end - bbt
    pw = np.frombuffer(payload + b"\x00" * (16 - len(payload) % 4), dtype=">u4").astype(np.int64)
    W = torch.from_numpy(pw)
    nW = W.numel()

    def read64(p):  # 64 bits of the stream from bit p (zeros past the end)
        w, s = p >> 5, p & 31
        x0, x1, x2 = (W[(w + k).clamp(max=nW - 1)] * (w + k < nW) for k in range(3))
        return (x0 << (32 + s)) | (x1 << s) | torch.where(s > 0, x2 >> (32 - s).clamp(max=31), torch.zeros_like(x2))

    gaps = torch.zeros(eb, dtype=torch.int64)
    zz = torch.zeros(eb, dtype=torch.int64)
    lens = torch.arange(1, MAX_LEN + 1, dtype=torch.int64).view(-1, 1)
    for s in range(BLOCK):
        act = torch.nonzero(cnt > s).view(-1)
        if act.numel() == 0:
            break
        c, e_ = cur[act], end[act]
        r = rice[act]
        x = read64(c)
        ones = ~x
        q = torch.where(ones != 0, 63 - _msb64(torch.where(ones != 0, ones, torch.ones_like(ones))), 64)
        run = q == 64
        while bool(run.any()):  # unary runs past one window: continue window by window
            ix = torch.nonzero(run).view(-1)
            y = ~read64(c[ix] + q[ix])
            more = torch.where(y != 0, 63 - _msb64(torch.where(y != 0, y, torch.ones_like(y))), 64)
            q[ix] += more
            stop = (more < 64) | (c[ix] + q[ix] >= e_[ix])
            run[ix[stop]] = False
        after = c + q + 1
        y = read64(after)
        rem = torch.where(r > 0, _shr(y, 1) >> (63 - r), 0)
        peek = _shr(y << r, 64 - MAX_LEN)
        tb = tbl[act]
        code = peek.view(1, -1) >> (MAX_LEN - lens)                       # [17, blocks]
        idx = code - first[tb].t()[1:]
        ok = (idx >= 0) & (idx < ncode[tb].t()[1:])
        has = ok.any(0)
        L = torch.argmax(ok.to(torch.int8), 0)                             # shortest matching length - 1
        si = base[tb, L + 1] + idx.gather(0, L.view(1, -1)).view(-1)
        bad = (~has) | (after > e_)
        if bool(bad.any()):
            raise Corrupt("payload does not decode")
        slot = ebase[act] + s
        gaps[slot] = (q << r) | rem
        zz[slot] = sym_t[si.clamp(max=sym_t.numel() - 1)]
        cur[act] = after + r + L + 1
    if not bool((cur == end).all()):
        raise Corrupt("a block does not decode to its length")
    return gaps, zz


def apply_update(weights: dict, update: bytes, checksums: dict | None = None) -> int:
    """apply_update on CPU tensors, in place; `checksums` (name -> int) is the receiver cache."""
    tables, tensors, bb, payload = _parse(update)
    groups = [g for t in tensors for g in t[3]]
    gaps, zz = _decode(tables, groups, bb, payload)
    work = []  # per tensor: (weights as int16, name, checksum, group exponents and counts, locals, exponents, zz)
    at = 0
    for name, numel, chk, tg in tensors:
        a = weights[name].reshape(-1).view(torch.int16)
        if a.numel() != numel:
            raise ValueError(f"{name}: numel mismatch")
        n = sum(c for _, c, _ in tg)
        g_, z_ = gaps[at:at + n], zz[at:at + n]
        gexp = torch.tensor([e for e, _, _ in tg], dtype=torch.int64)
        gcnt = torch.tensor([c for _, c, _ in tg], dtype=torch.int64)
        seg = torch.repeat_interleave(torch.arange(len(tg)), gcnt)
        step = g_ + 1
        cs = torch.cumsum(step, 0)
        gstart = torch.cumsum(gcnt, 0) - gcnt
        local = cs - (cs[gstart] - step[gstart])[seg] - 1   # group-local index of each change
        work.append((a, name, chk, gexp, gcnt, local, gexp[seg], z_))
        at += n
    positions = {}
    # small tensors: one shared sort per group on (tensor, exponent) keys (codec.py:659-678)
    for grp in _small_groups([w[0].numel() for w in work]):
        order, offs, starts = _shared_sort([_exp(work[i][0]) for i in grp])
        for si, i in enumerate(grp):
            a, name, chk, gexp, gcnt, local, ex, z_ = work[i]
            size = starts[si * 256 + 1:si * 256 + 257] - starts[si * 256:si * 256 + 256]
            if bool((gcnt > size[gexp]).any()) or bool((local >= size[ex]).any()):
                raise Corrupt("a change lies outside its exponent group")
            positions[i] = order[starts[si * 256 + ex] + local] - offs[si]
    plans = []
    for i, (a, name, chk, gexp, gcnt, local, ex, z_) in enumerate(work):
        numel = a.numel()
        pos = positions.get(i)
        if pos is None:
            # the receiver's stable exponent order, slab by slab: which slab holds each change, then
            # its place in that slab's sorted order
            e_all = _exp(a)
            nsl = (numel + SLAB - 1) // SLAB
            cnts = torch.stack([torch.bincount(e_all[lo:lo + SLAB], minlength=256)
                                for lo in range(0, numel, SLAB)])      # [slabs, 256]
            incl = torch.cumsum(cnts, 0)
            size = incl[-1]
            if bool((gcnt > size[gexp]).any()) or bool((local >= size[ex]).any()):
                raise Corrupt("a change lies outside its exponent group")
            flat = (incl.t() + torch.arange(256).view(-1, 1) * (numel + 1)).reshape(-1)  # ascending
            sl = torch.searchsorted(flat, ex * (numel + 1) + local, right=True) - ex * nsl
            pos = torch.empty_like(local)
            for s in range(nsl):
                m = torch.nonzero(sl == s).view(-1)
                if m.numel() == 0:
                    continue
                lo = s * SLAB
                key = e_all[lo:lo + SLAB]
                order = torch.sort(key, stable=True).indices
                start = torch.cumsum(cnts[s], 0) - cnts[s]
                before = incl[s] - cnts[s]
                k = ex[m]
                pos[m] = lo + order[start[k] + local[m] - before[k]]
        ou = a[pos].to(torch.int64) & 0xFFFF
        d = torch.where(z_ & 1 == 1, -((z_ + 1) >> 1), z_ >> 1)
        nu = (ou + d) & 0xFFFF
        old_chk = checksums.get(name) if checksums is not None else None
        if old_chk is None:
            old_chk = checksum(weights[name])
        if (old_chk + _delta(pos, ou, nu)) & MASK64 != chk:
            raise Corrupt(f"update does not verify (checksum mismatch: [{name!r}])")
        plans.append((a, pos, nu, name, chk))
    changed = 0
    for a, pos, nu, name, chk in plans:  # every tensor verified: write
        a.index_put_((pos,), nu.to(torch.int16))
        changed += pos.numel()
        if checksums is not None:
            checksums[name] = chk
    return changed
