"""Encode and apply updates on an MI355X (gfx950) through the native library.

Mirrors the reference's codec module (src/crukx_sync/codec.py): `encode`, `apply`, `checksum`,
`bits16`, `exponents`, `huffman_lengths`, `canonical_codes` and the `_SLAB` knob keep their names
and meaning. The work runs in hand-written HIP kernels (crukx-sync_amd/csrc); this module only
checks arguments, resolves names to tensors, manages checksum caches and device memory.

Tensors may live on a HIP device or on the CPU; CPU tensors are staged through the current HIP
device (there is no CPU implementation in the product, and without a HIP device the calls fail).
"""

from __future__ import annotations

import ctypes
from array import array
import threading
import weakref
from collections.abc import Mapping

import numpy as np
import torch

from . import _native
from .wire import (BLOCK, MAX_CODE_LEN, MAX_RICE, MAX_SYMBOL, CorruptUpdate, Group, NativeUpdate,  # noqa: F401
                   ParsedUpdate, Table, TensorHeader, Update, new_bytes, parse, serialize)

_MASK64 = (1 << 64) - 1
# The reference's knob (codec.py:30), with its default: tensors of more than _SLAB elements get their
# group sizes checked against the receiver's exponent counts before decoding ("group has more changes
# than elements", codec.py:598-604).  The reference also sorts at most _SLAB elements at once; here one
# wavefront ranks min(_SLAB, 65536) elements (rounded down to a multiple of 128), and the per-slab
# exponent histograms are scanned afterwards.  It never changes the bytes.
_SLAB = 1 << 24


# ---------------------------------------------------------------- shared helpers

def bits16(name: str, t: torch.Tensor) -> torch.Tensor:
    """Flat int16 view of a bf16 (or int16 bit-pattern) tensor (codec.py:35-41)."""
    if not isinstance(t, torch.Tensor) or t.dtype not in (torch.bfloat16, torch.int16):
        raise ValueError(f"{name}: expected a bfloat16 or int16 torch tensor, got {getattr(t, 'dtype', type(t))}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    return t.view(torch.int16).view(-1)


_DTYPES16 = (torch.bfloat16, torch.int16)
# The kernels index a tensor's elements and an update's changes in 32 bits: larger inputs are refused
# with ValueError before any device work (the reference has no such limit).
_LIMIT = 1 << 32
_TOO_LONG = "tensors of 2^32 or more elements are not supported"


def _check16(name: str, t) -> torch.Tensor:
    """bits16's checks without the views: the kernels take the storage address and element count."""
    if type(t) is not torch.Tensor and not isinstance(t, torch.Tensor) or t.dtype not in _DTYPES16:
        raise ValueError(f"{name}: expected a bfloat16 or int16 torch tensor, got {getattr(t, 'dtype', type(t))}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    return t


def exponents(a: torch.Tensor) -> torch.Tensor:
    return ((a >> 7) & 0xFF).long()


def _hip_device(dev: torch.device) -> torch.device:
    if dev.type == "cuda":
        return dev
    if not torch.cuda.is_available():
        raise RuntimeError("crukx_sync needs a HIP (ROCm) device: the codec runs only in its gfx950 kernels")
    return torch.device("cuda", torch.cuda.current_device())


def checksum(a: torch.Tensor) -> int:
    """sum(u_i * w_i) mod 2^64 over the uint16 bits u_i, w_i = splitmix64(i) | 1 (codec.py:61-68)."""
    a = bits16("tensor", a)
    if a.numel() >= _LIMIT:
        raise ValueError(_TOO_LONG)
    dev = _hip_device(a.device)
    if a.device != dev:
        a = a.to(dev)
    L = _native.lib()
    ws = _native.Workspace(dev)
    out = ctypes.c_uint64()
    err = _native.errbuf()
    with torch.cuda.device(dev):
        rc = L.crx_checksum(a.data_ptr(), a.numel(), _native.stream_of(dev), ws.fn, None, ctypes.byref(out), err, 512)
    ws.check()
    _native.raise_for(rc, err)
    return out.value


def huffman_lengths(counts: list[int]) -> list[int]:
    """Huffman code lengths limited to MAX_CODE_LEN (codec.py:71-78), computed natively."""
    n = len(counts)
    c = (ctypes.c_uint64 * n)(*counts)
    out = (ctypes.c_int32 * n)()
    _native.raise_for(_native.lib().crx_huffman_lengths(c, n, out), None)
    return list(out)


def canonical_codes(lengths: list[int]) -> list[int]:
    """Canonical codes, assigned in order of (length, position in the table) (codec.py:101-111)."""
    n = len(lengths)
    L = (ctypes.c_int32 * n)(*lengths)
    out = (ctypes.c_uint32 * n)()
    _native.raise_for(_native.lib().crx_canonical_codes(L, n, out), None)
    return list(out)


def rice_parameter(count: int, gap_sum: int, shifted_sums) -> int:
    """The Rice parameter of one group from its sums (codec.py:268-275): `shifted_sums(r)` must
    return sum(gap >> r) over the group's gaps."""
    L = _native.lib()
    cand = (ctypes.c_int32 * 3)()
    L.crx_rice_candidates(count, gap_sum, cand)
    sh = (ctypes.c_uint64 * 3)(*[shifted_sums(c) for c in cand])
    return L.crx_rice_choose(count, cand, sh)


# ---------------------------------------------------------------- encoder

# The tensor names of recent encodes as the library takes them (UTF-8 bytes, a C array of pointers to
# them, their lengths), keyed by the names: a run encodes the same tensors at every step, and building
# the pointer array costs about 0.07 ms for 339 names.  Each entry holds the bytes its array points to.
_name_cache: dict = {}
_name_lock = threading.Lock()


def _names_c(names: list[str]):
    key = tuple(names)
    with _name_lock:
        hit = _name_cache.get(key)
    if hit is None:
        enc = [n.encode() for n in names]
        hit = (enc, (ctypes.c_char_p * max(len(enc), 1))(*enc), _native.u64_array([len(n) for n in enc]))
        with _name_lock:
            if len(_name_cache) >= 8:
                _name_cache.clear()
            _name_cache[key] = hit
    return hit


class EncodedUpdate(NativeUpdate):
    """An update encoded on the device: header on the host, block table and payload in HBM."""

    def __init__(self, handle, names: list[str], device, workspace):
        self._h = handle
        self._free = _native.lib().crx_encoded_free
        self._names, arr, lens = _names_c(names)
        self._nargs = (arr, lens)
        self._device = device
        self._ws = workspace  # keeps the device buffers alive
        self._tensors = None

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._free(h)

    def _name_args(self):
        return self._nargs

    def nbytes(self) -> int:
        arr, lens = self._name_args()
        return _native.lib().crx_encoded_size(self._h, arr, lens)

    def _serialize_native(self) -> bytes:
        n = self.nbytes()
        data, addr = new_bytes(n)
        self._write(addr, False)
        return data

    def to_device(self) -> torch.Tensor:
        """The serialized update as a uint8 tensor on the encoding device."""
        if self.edited:
            return torch.frombuffer(bytearray(serialize(self)), dtype=torch.uint8).to(self._device)
        out = torch.empty(self.nbytes(), dtype=torch.uint8, device=self._device)
        self._write(out.data_ptr(), True)
        return out

    def _write(self, addr: int, on_device: bool) -> None:
        arr, lens = self._name_args()
        err = _native.errbuf()
        with torch.cuda.device(self._device):
            rc = _native.lib().crx_encoded_write(self._h, arr, lens, addr, 1 if on_device else 0,
                                                 _native.stream_of(self._device), err, 512)
        _native.raise_for(rc, err)

    def _read_tensors(self) -> list[TensorHeader]:
        if self._tensors is None:
            L = _native.lib()
            e, cnt, r = ctypes.c_int32(), ctypes.c_uint64(), ctypes.c_int32()
            out = []
            for t, name in enumerate(self._names):
                if not L.crx_encoded_present(self._h, t):
                    continue
                groups = []
                for g in range(L.crx_encoded_n_groups(self._h, t)):
                    L.crx_encoded_group(self._h, t, g, ctypes.byref(e), ctypes.byref(cnt), ctypes.byref(r))
                    groups.append(Group(e.value, cnt.value, r.value))
                out.append(TensorHeader(name.decode(), self._numels[t], L.crx_encoded_checksum(self._h, t), groups))
            self._tensors = out
        return self._tensors

    def _read_tables(self) -> list[Table]:
        L = _native.lib()
        e, n = ctypes.c_int32(), ctypes.c_int64()
        out = []
        for i in range(L.crx_encoded_n_tables(self._h)):
            L.crx_encoded_table(self._h, i, ctypes.byref(e), ctypes.byref(n), None, None)
            syms, lens = (ctypes.c_uint32 * n.value)(), (ctypes.c_uint8 * n.value)()
            L.crx_encoded_table(self._h, i, ctypes.byref(e), ctypes.byref(n), syms, lens)
            out.append(Table(e.value, list(syms), list(lens)))
        return out

    def _read_block_bits(self) -> list[int]:
        L = _native.lib()
        n = L.crx_encoded_n_blocks(self._h)
        arr = (ctypes.c_uint32 * max(n, 1))()
        with torch.cuda.device(self._device):
            _native.raise_for(L.crx_encoded_block_bits(self._h, arr, _native.stream_of(self._device)), None)
        return list(arr[:n])

    def _read_payload(self) -> bytes:
        L = _native.lib()
        n = L.crx_encoded_payload_len(self._h)
        data, addr = new_bytes(n)
        with torch.cuda.device(self._device):
            _native.raise_for(L.crx_encoded_payload(self._h, addr, _native.stream_of(self._device)), None)
        return data


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """32-bit aligned storage: the kernels read pairs of bf16 as one word."""
    return t if t.data_ptr() % 4 == 0 else t.clone()


def encode(old: Mapping[str, torch.Tensor], new: Mapping[str, torch.Tensor],
           checksums: dict[str, int] | None = None) -> tuple[Update, dict[str, int]]:
    """The update, and the new checksums for the caller to commit once the update is serialized
    (codec.py:278-420)."""
    names = list(old)
    if not names:
        return Update([], []), {}
    fast = _encode_inputs(names, old, new, checksums)
    if fast is not None:
        A, B, numels, pa, pb, has, vals, dev = fast
        return _encode_call(names, A, B, numels, pa, pb, has, vals, dev)
    # one pass over the tensors: checks, element counts, devices, pointers and cached checksums
    A, B = [], []
    numels, pa, pb, vals = array("Q"), array("Q"), array("Q"), array("Q")
    has = array("i")
    devs = set()
    T16 = torch.Tensor
    cg = checksums.get if checksums is not None else None
    for name in names:
        a, b = old[name], new[name]
        if (type(a) is not T16 or type(b) is not T16 or a.dtype not in _DTYPES16 or b.dtype not in _DTYPES16
                or not a.is_contiguous() or not b.is_contiguous()):
            a, b = _check16(name, a), _check16(name, b)  # raise, or pass tensor subclasses
        if a.shape != b.shape:
            raise ValueError(f"{name}: old and new differ in shape")
        k = a.numel()
        if k >= _LIMIT:
            raise ValueError(f"{name}: {_TOO_LONG}")
        A.append(a)
        B.append(b)
        numels.append(k)
        devs.add(a.get_device())
        devs.add(b.get_device())
        pa.append(a.data_ptr())
        pb.append(b.data_ptr())
        c = cg(name) if cg is not None else None
        has.append(0 if c is None else 1)
        vals.append(0 if c is None else c & _MASK64)
    if len(devs) == 1 and next(iter(devs)) >= 0:  # all on one GPU
        src = dev = A[0].device
    else:
        src = _device_of(A + B, "all tensors must be on one device")
        dev = _hip_device(src)
    if src != dev:
        A, B = [a.to(dev) for a in A], [b.to(dev) for b in B]
        pa, pb = array("Q", [a.data_ptr() for a in A]), array("Q", [b.data_ptr() for b in B])
    return _encode_call(names, A, B, numels, pa, pb, has, vals, dev)


def _encode_inputs(names, old, new, checksums):
    """The encoder's inputs from the batched metadata helper, when every tensor is regular (bf16 or
    int16, contiguous, shapes equal, under the size limit, all on one GPU); None otherwise, and the
    checks then run tensor by tensor to raise their exact errors."""
    M = _native.tensor_meta()
    if M is None:
        return None
    # `names` is list(old); plain dicts give their values in that order (and new's too when its keys
    # come in the same order)
    A = list(old.values()) if type(old) is dict else [old[n] for n in names]
    B = list(new.values()) if type(new) is dict and list(new) == names else [new[n] for n in names]
    try:
        ma, mb, same = M.meta_pair(A, B)
    except (TypeError, RuntimeError):  # not all tensors
        return None
    n = len(names)
    fa, fb, numels = array("i", ma[3]), array("i", mb[3]), array("Q", ma[1])
    if not same or fa.count(3) != n or fb.count(3) != n or max(numels) >= _LIMIT:
        return None
    devs = set(array("i", ma[2])) | set(array("i", mb[2]))
    if len(devs) != 1 or next(iter(devs)) < 0:
        return None
    if checksums is None:
        has, vals = array("i", bytes(4 * n)), array("Q", bytes(8 * n))
    else:
        cached = list(map(checksums.get, names))
        has = array("i", [0 if c is None else 1 for c in cached])
        vals = array("Q", [0 if c is None else c & _MASK64 for c in cached])
    return A, B, numels, array("Q", ma[0]), array("Q", mb[0]), has, vals, A[0].device


def _encode_call(names, A, B, numels, pa, pb, has, vals, dev):
    """crx_encode on checked inputs (A, B: the tensors on `dev`; pa, pb, numels, has, vals: packed arrays)."""
    if (int(np.bitwise_or.reduce(np.frombuffer(pa, np.uint64))) |
            int(np.bitwise_or.reduce(np.frombuffer(pb, np.uint64)))) & 3:  # the kernels read 32-bit words
        A = [a if a.data_ptr() & 3 == 0 else a.clone() for a in A]
        B = [b if b.data_ptr() & 3 == 0 else b.clone() for b in B]
        pa, pb = array("Q", [a.data_ptr() for a in A]), array("Q", [b.data_ptr() for b in B])
    n = len(names)
    L = _native.lib()
    ws = _native.Workspace(dev)
    err = _native.errbuf()
    h = ctypes.c_void_p()
    with torch.cuda.device(dev):
        rc = L.crx_encode(n, _native.view_ptr(pa), _native.view_ptr(pb), _native.view_u64(numels),
                          _native.view_i32(has), _native.view_u64(vals), int(_SLAB),
                          _native.stream_of(dev), ws.fn, None, ctypes.byref(h), err, 512)
    ws.check()
    _native.raise_for(rc, err)
    upd = EncodedUpdate(h.value, names, dev, ws)
    upd._numels = list(numels)
    present, chk = (ctypes.c_int32 * n)(), (ctypes.c_uint64 * n)()
    L.crx_encoded_checksums(h.value, present, chk)
    new_checksums = {name: chk[t] for t, name in enumerate(names) if present[t]}
    return upd, new_checksums


# ---------------------------------------------------------------- apply

# Whether apply keeps the receiver's exponent counts across updates (below).  The reference has no such
# cache (its apply re-sorts the receiver's weights every time); turning it off gives the reference's
# semantics exactly: only the checksum cache carries over between updates.
_COUNT_CACHE = True

# Receiver-side exponent counts per slab, kept on the device across updates of the same tensors:
# id(tensor) -> (weakref, _version after our last write, device buffer, slab size, device, buffer
# address).  They are used only with the same slab size and a checksum-cache hit for the tensor (the
# same trust rule), and let apply skip its full read of those weights (crx_apply_cached).
_hist = {}
# Guards _hist across threads.  Reentrant: a weakref callback that drops an entry can run inside a
# locked region when a garbage collection happens there.
_hist_lock = threading.RLock()


def _hist_lookup(t):
    with _hist_lock:
        e = _hist.get(id(t))
    if e is None or e[0]() is not t:
        return None
    return e


def _hist_forget(key):
    with _hist_lock:
        _hist.pop(key, None)


def _apply_inputs(names, numels, weights, checksums):
    """The receiver's tensors, versions and trusted cached checksums from the batched metadata helper,
    when every tensor is present and regular (bf16 or int16, contiguous, the update's element count,
    under the size limit, all on one GPU); None otherwise, and the checks then run tensor by tensor to
    raise their exact errors."""
    M = _native.tensor_meta()
    if M is None or not isinstance(weights, dict):
        return None
    get = weights.get
    targets = [get(n) for n in names]
    try:
        m = M.meta(targets)
    except (TypeError, RuntimeError):  # a missing name (None) or not a tensor
        return None
    n = len(names)
    if array("i", m[3]).count(3) != n or array("Q", m[1]) != array("Q", numels) or max(numels) >= _LIMIT:
        return None
    devs = set(array("i", m[2]))
    if len(devs) != 1 or next(iter(devs)) < 0:
        return None
    vers, ptrs = array("Q", m[4]), array("Q", m[0])
    if checksums is None:
        return targets, vers, array("i", bytes(4 * n)), array("Q", bytes(8 * n)), ptrs
    hits = list(map(checksums.get, names))
    ok = [isinstance(h, tuple) and h[1] == v for h, v in zip(hits, vers)]
    return (targets, vers, array("i", [1 if o else 0 for o in ok]),
            array("Q", [h[0] & _MASK64 if o else 0 for h, o in zip(hits, ok)]), ptrs)


def _hist_store(t, buf, slab, dev):
    """Record counts for t (the caller holds _hist_lock)."""
    key = id(t)
    e = _hist.get(key)
    ref = e[0] if e is not None and e[0]() is t else weakref.ref(t, lambda _r, key=key: _hist_forget(key))
    _hist[key] = (ref, t._version, buf, slab, dev, buf.data_ptr())


def _cache_get(checksums, name, t):
    """A cached checksum, trusted only if the tensor was not modified since it was recorded
    (codec.py:457-460)."""
    hit = checksums.get(name) if checksums is not None else None
    return hit[0] if isinstance(hit, tuple) and hit[1] == t._version else None


def _device_of(ts: list, what: str) -> torch.device:
    """The one device of all tensors in `ts` (ValueError naming `what` otherwise)."""
    idx = {t.get_device() for t in ts}
    if len(idx) == 1 and next(iter(idx)) >= 0:  # all on one GPU
        return ts[0].device
    src = ts[0].device
    if any(t.device != src for t in ts):
        raise ValueError(what)
    return src


def apply(weights: Mapping[str, torch.Tensor], u: Update, checksums: dict | None = None) -> int:
    """Verify `u` against `weights`, then write the new values in place. Returns elements changed
    (codec.py:578-717)."""
    if not isinstance(u, ParsedUpdate) or u.edited:
        u = parse(serialize(u))
    names, numels, header_chk = u.headers()
    if not names:
        return 0
    fast = _apply_inputs(names, numels, weights, checksums)
    ptrs = None
    if fast is not None:
        targets, vers, has, vals, ptrs = fast
        devs = {targets[0].get_device()}
    else:  # one pass over the receiver's tensors: checks, devices, versions and trusted cached checksums
        targets, vers, devs = [], [], set()
        has, vals = array("i"), array("Q")
        get = weights.get if isinstance(weights, dict) else None
        cg = checksums.get if checksums is not None else None
        T16 = torch.Tensor
        for name, numel in zip(names, numels):
            t = get(name) if get is not None else (weights[name] if name in weights else None)
            if t is None:
                raise ValueError(f"update has tensor {name!r} that the receiver does not have")
            if type(t) is not T16 or t.dtype not in _DTYPES16 or not t.is_contiguous():
                t = _check16(name, t)  # raises, or passes a tensor subclass
            if t.numel() != numel:
                raise ValueError(f"{name}: update is for {numel} elements, receiver has {t.numel()}")
            if numel >= _LIMIT:
                raise ValueError(f"{name}: {_TOO_LONG}")
            targets.append(t)
            devs.add(t.get_device())
            v = t._version
            vers.append(v)
            hit = cg(name) if cg is not None else None
            ok = isinstance(hit, tuple) and hit[1] == v
            has.append(1 if ok else 0)
            vals.append(hit[0] & _MASK64 if ok else 0)
    if len(devs) == 1 and next(iter(devs)) >= 0:  # all on one GPU
        src = dev = targets[0].device
    else:
        src = _device_of(targets, "all updated tensors must be on one device")
        dev = _hip_device(src)
    staged = [a.to(dev) for a in targets] if src != dev else targets
    n = len(names)
    L = _native.lib()
    payload_dev = 0
    if u._dev_bytes is not None:  # the whole update in device memory: payload and block table read there
        db = u._dev_bytes
        if db.device != dev:
            db = db.to(dev)
        payload_dev = db.data_ptr() + L.crx_update_payload_offset(u.handle)
    ws = _native.Workspace(dev)
    err = _native.errbuf()
    changed = ctypes.c_uint64()
    # exponent counts carried across updates: only for tensors updated in place with a trusted cache
    keep = checksums is not None and staged is targets and _COUNT_CACHE
    slab = int(_SLAB)
    hist_in, hist_out, bufs = [], [], []
    if keep:
        # an entry is used for the same tensor object, unmodified since, with the same slab size and
        # device, when the tensor's checksum is trusted too (one pass over the tensors)
        fresh = []
        with _hist_lock:
            hg = _hist.get
            for i, (a, c, v) in enumerate(zip(targets, has, vers)):
                e = hg(id(a)) if c else None
                if e is not None and e[1] == v and e[3] == slab and e[4] == dev and e[0]() is a:
                    bufs.append(e[2])
                    hist_in.append(e[5])
                else:
                    bufs.append(None)
                    hist_in.append(0)
                    fresh.append(i)
        hist_out = list(hist_in)
        # tensors without usable counts: one allocation, sliced per tensor
        fresh = [(i, L.crx_apply_hist_words(targets[i].numel(), slab)) for i in fresh]
        if fresh:
            block = torch.empty(sum(w for _, w in fresh), dtype=torch.int32, device=dev)
            at, base = 0, block.data_ptr()
            for i, w in fresh:
                bufs[i] = block[at:at + w]
                hist_out[i] = base + 4 * at
                at += w
    with torch.cuda.device(dev):
        if ptrs is None or staged is not targets:
            ptrs = array("Q", [a.data_ptr() for a in staged])
        rc = L.crx_apply_cached(u.handle, payload_dev or None, _native.view_ptr(ptrs),
                                _native.view_u64(array("Q", numels)), _native.view_i32(has), _native.view_u64(vals),
                                _native.view_ptr(array("Q", hist_in)) if keep else None,
                                _native.view_ptr(array("Q", hist_out)) if keep else None,
                                slab, _native.stream_of(dev), ws.fn, None, ctypes.byref(changed), err, 512)
    ws.check()
    ws.release()
    if rc != _native.OK:
        with _hist_lock:
            for a in targets:  # their counts may be half-updated
                _hist.pop(id(a), None)
        if rc == _native.DEVICE and staged is targets:
            # a runtime error may come after the verified writes were enqueued: the weights may have
            # changed, so cached checksums of them must no longer be trusted (a new _version does that)
            torch.autograd.graph.increment_version(targets)
    _native.raise_for(rc, err)
    if staged is targets:
        torch.autograd.graph.increment_version(targets)  # in place, like index_put_: bumps _version
    else:
        for a, s in zip(targets, staged):
            a.copy_(s)  # an in-place op: bumps the tensor's version
    M = _native.tensor_meta()
    after = array("Q", M.versions(targets)) if M is not None else [t._version for t in targets]
    if keep:
        with _hist_lock:
            hg = _hist.get
            for a, buf, v in zip(targets, bufs, after):
                e = hg(id(a))
                if e is not None and e[2] is buf and e[0]() is a:  # the same counts: a new version only
                    _hist[id(a)] = (e[0], v, buf, slab, dev, e[5])
                else:
                    _hist_store(a, buf, slab, dev)
    if checksums is not None:  # record the version after our own write
        checksums.update({name: (c, v) for name, c, v in zip(names, header_chk, after)})
    return changed.value
