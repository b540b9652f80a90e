"""A lane-level CPU model of the apply's select pass (k_locate + k_select in
crukx-sync_amd/csrc/kernels.hip), for tests only.

It follows the kernels' arithmetic lane by lane: k_locate's lower-bound searches, record regions and
extra windows; per window, the target list, the per-lane state (next target, change index, end), the
running counts in kSelCopies lane-replicated copies plus spare counters, the rows as two 16-bit halves
(lane l holds elements l and l + 64), the first pass over the exponents with a target in the row
(ballot + mbcnt over one half) and the second (publish by in-row rank, take one per lane).  Every LDS
array (counters, target list, publish slots) and the record buffer is bounds-checked, every loop is
bounded, and at the end every change must have been recorded exactly once, at its true position with
its old bits.  The window size, copy count and list capacities are read from the kernel sources, so
the model runs the configuration the kernels are built with.
"""

from __future__ import annotations

import os
import re

import numpy as np

_CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "crukx-sync_amd", "csrc")
FAR = 0x40000000  # kFar: no target left
M32 = 0xFFFFFFFF


def kernel_constants() -> dict:
    src = open(os.path.join(_CSRC, "kernels.hip")).read() + open(os.path.join(_CSRC, "kernels.h")).read()

    def num(name):
        return int(re.search(rf"\b{name}\s*=\s*(\d+)", src).group(1))
    return {"win": num("kSelWin"), "copies": num("kSelCopies"), "cap_sparse": num("kTgtCapSparse"),
            "cap_dense": num("kTgtCapDense"), "dense_targets": num("kSelectDenseTargets")}


class Lds:
    """A bounds-checked array."""

    def __init__(self, n, name, fill=0):
        self.a = [fill] * n
        self.name = name

    def __getitem__(self, i):
        if not 0 <= i < len(self.a):
            raise IndexError(f"{self.name}[{i}] outside [0, {len(self.a)})")
        return self.a[i]

    def __setitem__(self, i, v):
        if not 0 <= i < len(self.a):
            raise IndexError(f"{self.name}[{i}] = ... outside [0, {len(self.a)})")
        self.a[i] = v


def _changes(old, new):
    """Exponent of every element, and the changes in update order (exponent, then rank within the
    tensor's elements of that exponent): their group-local indices and positions."""
    e = (old >> 7) & 0xFF
    rank = np.zeros(old.size, np.int64)
    for k in np.unique(e):
        idx = np.nonzero(e == k)[0]
        rank[idx] = np.arange(idx.size)
    chg = np.nonzero(old != new)[0]
    order = sorted(chg.tolist(), key=lambda i: (e[i], rank[i]))
    local = np.array([rank[i] for i in order], np.int64)
    gstart, gcnt = {}, {}
    for j, i in enumerate(order):
        k = int(e[i])
        gstart.setdefault(k, j)
        gcnt[k] = gcnt.get(k, 0) + 1
    return e, local, np.array(order, np.int64), gstart, gcnt


def run(old: np.ndarray, new: np.ndarray, slab: int, win=None, copies=None, cap=None) -> dict:
    """Models the select pass over one tensor (uint16 bit patterns) cut into `slab`-element slabs.
    Raises IndexError on an out-of-bounds access, AssertionError on any wrong or missing record."""
    kc = kernel_constants()
    win = win or kc["win"]
    copies = copies or kc["copies"]
    old = old.astype(np.int64) & 0xFFFF
    new = new.astype(np.int64) & 0xFFFF
    n = old.size
    e, local, truth, gstart, gcnt = _changes(old, new)
    C = local.size
    tiles = (n + slab - 1) // slab
    if cap is None:
        cap = kc["cap_dense"] if C > kc["dense_targets"] * tiles else kc["cap_sparse"]
    pre = np.zeros((tiles + 1, 256), np.int64)
    for t in range(tiles):
        pre[t + 1] = pre[t] + np.bincount(e[t * slab:min(n, (t + 1) * slab)], minlength=256)
    # k_locate
    lb = np.full((tiles + 1, 256), -1, np.int64)
    rstart = np.zeros(tiles + 1, np.int64)
    more = []
    for tau in range(tiles):
        last = tau + 1 == tiles
        before, has = 0, np.zeros(256, bool)
        for k, g0 in gstart.items():
            gend = g0 + gcnt[k]
            lo = g0 + int(np.searchsorted(local[g0:gend], pre[tau][k], side="left"))
            lb[tau][k] = lo
            has[k] = lo < gend and (last or local[lo] < pre[tau + 1][k])
            before += lo - g0
        rstart[tau] = before
        if last:
            rstart[tiles] = C
        first_at = lambda frm: next((k for k in range(frm, 256) if has[k]), 256)  # noqa: E731
        kb = first_at(0)
        while kb < 256 - win:
            kb = first_at(kb + win)
            if kb < 256:
                more.append((tau, kb))
    assert len(more) <= (256 // win - 1) * tiles
    rec = Lds(C, "rec", -1)
    written = np.zeros(C, np.int64)
    unplaced = False
    for tau, kfirst in [(t, 256) for t in range(tiles)] + more:
        unplaced |= _window(old, local, pre, lb, rstart, gstart, gcnt, tau, tiles, kfirst, slab, win, copies, cap,
                            rec, written)
    assert not unplaced, "targets left unplaced"
    assert (written == 1).all(), f"records per change: {np.bincount(written)}"
    for tau in range(tiles):
        for i in range(int(rstart[tau]), int(rstart[tau + 1])):
            r = rec[i]
            ci, off, bits = r & M32, (r >> 32) & 0xFFFF, (r >> 48) & 0xFFFF
            assert tau * slab + off == truth[ci], (tau, i, ci, tau * slab + off, truth[ci])
            assert bits == int(old[tau * slab + off])
    return {"changes": C, "slabs": tiles, "extra_windows": len(more), "cap": cap}


def _window(old, local, pre, lb, rstart, gstart, gcnt, tau, tiles, kfirst, slab, win, copies, cap, rec, written):
    """One select_window + select_slab; True if targets were left unplaced."""
    n = old.size
    last = tau + 1 == tiles
    n4 = np.zeros(256, np.int64)
    for k, g0 in gstart.items():
        je = g0 + gcnt[k] if last else lb[tau + 1][k]
        n4[k] = max(0, je - lb[tau][k])
    ks = np.nonzero(n4)[0]
    kbase = kfirst if kfirst < 256 else (int(ks[0]) if ks.size else 256)
    if kbase >= 256:
        return False
    jbase = int(rstart[tau]) + int(n4[:kbase].sum())
    nw = np.array([n4[k] if 0 <= k - kbase < win else 0 for k in range(256)], np.int64)
    total = int(nw.sum())
    wend = jbase + total
    in_lds = total <= cap
    info = [(0, 0, 0, 0)] * 64  # per lane: list begin, end, change index - list index, count before the slab
    off = 0
    for k in range(256):
        c = k - kbase
        if 0 <= c < win:
            info[c] = (off, off + int(nw[k]), int(lb[tau][k]) - off, int(pre[tau][k]))
        off += int(nw[k])
    lst = Lds(cap, "list")
    if in_lds:
        for c in range(win):
            x0, x1, z, w = info[c]
            for x in range(x0, x1):
                lst[x] = int(local[z + x]) - w

    def target(c, jo, pr):
        return lst[c - jo] if in_lds else int(local[c]) - pr

    lanes = np.arange(64)
    nxt = np.full(64, FAR, np.int64)
    ci, cend, jofs, prek = (np.zeros(64, np.int64) for _ in range(4))
    for ln in range(64):
        x, y, z, w = info[ln]
        if x < y:
            nxt[ln] = target(x + z, z, w)
        ci[ln], cend[ln], jofs[ln], prek[ln] = x + z, y + z, z, w
    cnt = Lds((win + 64 // copies) * copies, "cnt")
    sp = (win + lanes // copies) << 7  # the lane's spare key (window index << 7)
    lo_el, f_hi = tau * slab, min(n, (tau + 1) * slab) - tau * slab
    row_el = lambda f: int(old[lo_el + f]) if f < f_hi else 0  # noqa: E731
    j, prev = jbase, np.zeros(64, np.int64)
    for r in range((f_hi + 127) // 128):
        f = r * 128 + lanes
        vlo = np.array([row_el(x) for x in f])
        vhi = np.array([row_el(x + 64) for x in f])
        c0 = np.where(f >= f_hi, sp, np.minimum(((vlo & 0x7F80) - (kbase << 7)) & 0xFFFF, sp))
        c1 = np.where(f + 64 >= f_hi, sp, np.minimum(((vhi & 0x7F80) - (kbase << 7)) & 0xFFFF, sp))
        for half in (c0, c1):  # the two atomics: counter (key >> 7) copy (lane % copies)
            for ln in range(64):
                a = (int(half[ln]) >> 7) * copies + ln % copies
                cnt[a] = cnt[a] + 1
        s = np.array([sum(cnt[copies * ln + q] for q in range(copies)) for ln in range(64)], np.int64)
        seen, prev = prev, s
        hit = s > nxt
        if not hit.any():
            continue
        w0 = f | (vlo << 16)
        w1 = (f + 64) | (vhi << 16)
        q = (nxt - seen) & M32
        for k in np.nonzero(hit)[0]:  # exactly one element per exponent with a target in the row
            qk, ck = int(q[k]), int(ci[k])
            m0 = [ln for ln in range(64) if c0[ln] == (k << 7)]
            if qk < len(m0):
                lane, hw = m0[qk], w0
            else:
                m1 = [ln for ln in range(64) if c1[ln] == (k << 7)]
                assert qk - len(m0) < len(m1), ("no element holds the target", tau, r, k, qk)
                lane, hw = m1[qk - len(m0)], w1
            assert jbase <= j < wend and rec[j] == -1, ("record outside the window or written twice", j)
            rec[j] = ck | (int(hw[lane]) << 32)
            written[ck] += 1
            j += 1
        for ln in np.nonzero(hit)[0]:
            ci[ln] += 1
            nxt[ln] = target(int(ci[ln]), int(jofs[ln]), int(prek[ln])) if ci[ln] < cend[ln] else FAR
        for k in np.nonzero(s > nxt)[0]:  # more targets of one exponent in the row
            after, seen_k, ke, jo, pr, ck = int(s[k]), int(seen[k]), int(cend[k]), int(jofs[k]), int(prek[k]), int(ci[k])
            slot = Lds(256, "slot")
            m0 = [ln for ln in range(64) if c0[ln] == (k << 7)]
            m1 = [ln for ln in range(64) if c1[ln] == (k << 7)]
            for ln in range(64):
                slot[m0.index(ln) if ln in m0 else 128 + ln] = int(w0[ln])
            for ln in range(64):
                slot[len(m0) + m1.index(ln) if ln in m1 else 128 + ln] = int(w1[ln])
            for _ in range(4096):
                c = ck + lanes
                tl = np.array([target(int(x), jo, pr) if x < ke else FAR for x in c])
                take = (c < ke) & (tl < after)
                taken = int(take.sum())
                assert take[:taken].all(), "the takers are not a prefix of the lanes"
                for ln in range(taken):
                    assert jbase <= j + ln < wend and rec[j + ln] == -1, ("record outside the window or twice", j + ln)
                    rec[j + ln] = int(c[ln]) | (slot[int(tl[ln]) - seen_k] << 32)
                    written[int(c[ln])] += 1
                j += taken
                ck += taken
                if taken != 64:
                    break
            else:
                raise AssertionError("unbounded take loop")
            nxt[k], ci[k] = int(tl[taken]) if taken < 64 else FAR, ck
    return bool((ci < cend).any())
