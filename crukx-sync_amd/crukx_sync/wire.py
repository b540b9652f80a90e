"""The update container (format version 2): plain data, serialisation and bounds-checked parsing.

Mirrors the reference's wire module (src/crukx_sync/wire.py): the same constants, CorruptUpdate,
dataclasses, write_varint, serialize and parse. Parsing and the serialisation of encoded updates
run in the native library (include/crukx.h: crx_parse, crx_encoded_write); every limit of the
format is checked there in the reference's order (wire.py:126-212).
"""

from __future__ import annotations

import ctypes
import struct
import threading
from dataclasses import dataclass, field

MAGIC = b"CRXS"
VERSION = 2
MAX_CODE_LEN = 17   # a 16-bit difference has 131071 zigzag values: a code of 17 bits can name each
MAX_SYMBOL = 131070
MAX_RICE = 30
BLOCK = 256


class CorruptUpdate(ValueError):
    """Raised for bytes that break the format, end early, or decode to weights whose checksum is not
    the one the update carries."""


@dataclass
class Table:
    """The code of one exponent's residuals: symbols and their canonical Huffman code lengths."""
    exponent: int
    symbols: list[int]
    lengths: list[int]


@dataclass
class Group:
    exponent: int
    count: int
    rice_r: int


@dataclass
class TensorHeader:
    name: str
    numel: int
    checksum: int
    groups: list[Group]


@dataclass
class Update:
    tables: list[Table]
    tensors: list[TensorHeader]
    block_bits: list[int] = field(default_factory=list)
    payload: bytes = b""


def n_blocks(count: int) -> int:
    return -(-count // BLOCK)


def write_varint(out: bytearray, v: int) -> None:
    if not 0 <= v < 1 << 63:
        raise ValueError(f"varint out of range: {v}")
    while v >= 0x80:
        out.append((v & 0x7F) | 0x80)
        v >>= 7
    out.append(v)


def _serialize_plain(u: Update) -> bytes:
    """Format version 2 from plain Python data (for hand-built Update objects)."""
    out = bytearray(MAGIC)
    out.append(VERSION)
    write_varint(out, len(u.tables))
    for t in u.tables:
        out.append(t.exponent)
        write_varint(out, len(t.symbols))
        for s, L in zip(t.symbols, t.lengths):
            write_varint(out, s)
            out.append(L)
    write_varint(out, len(u.tensors))
    for t in u.tensors:
        raw = t.name.encode()
        write_varint(out, len(raw))
        out += raw
        write_varint(out, t.numel)
        out += struct.pack("<Q", t.checksum)
        write_varint(out, len(t.groups))
        for g in t.groups:
            out.append(g.exponent)
            write_varint(out, g.count)
            out.append(g.rice_r)
    out += struct.pack(f"<{len(u.block_bits)}I", *u.block_bits)
    write_varint(out, len(u.payload))
    out += u.payload
    return bytes(out)


def serialize(u: Update) -> bytes:
    """Bytes of an update: natively for updates produced by encode, else from the plain fields."""
    native = getattr(u, "_serialize_native", None)
    if native is not None and not u.edited:
        return native()
    return _serialize_plain(u)


# ------------------------------------------------------------------ parsed updates

_PyBytes_FromStringAndSize = ctypes.pythonapi.PyBytes_FromStringAndSize
_PyBytes_FromStringAndSize.restype = ctypes.py_object
_PyBytes_FromStringAndSize.argtypes = [ctypes.c_void_p, ctypes.c_ssize_t]
_PyBytes_AsString = ctypes.pythonapi.PyBytes_AsString
_PyBytes_AsString.restype = ctypes.c_void_p
_PyBytes_AsString.argtypes = [ctypes.py_object]


def new_bytes(n: int) -> tuple[bytes, int]:
    """A fresh bytes object of length n and the address of its buffer, for the native writer to
    fill before anything else sees the object."""
    b = _PyBytes_FromStringAndSize(None, n)
    return b, _PyBytes_AsString(b)


class NativeUpdate(Update):
    """An update whose fields live in the native library until read.  Assigning a field first reads all
    four into plain Python data; from then on the object behaves as the reference's mutable Update
    (wire.py:44-48): serialize() and apply use the edited fields."""

    _FIELDS = ("tables", "tensors", "block_bits", "payload")

    @property
    def edited(self) -> bool:
        return self.__dict__.get("_fields") is not None

    def _materialise(self) -> dict:
        f = self.__dict__.get("_fields")
        if f is None:
            f = {name: getattr(self, "_read_" + name)() for name in self._FIELDS}
            self.__dict__["_fields"] = f
        return f


def _field(name):
    def fget(self):
        f = self.__dict__.get("_fields")
        return f[name] if f is not None else getattr(self, "_read_" + name)()

    def fset(self, v):
        self._materialise()[name] = v

    return property(fget, fset)


for _n in NativeUpdate._FIELDS:
    setattr(NativeUpdate, _n, _field(_n))
del _n


# The tensor names of the last update parsed, decoded: (their UTF-8 bytes, their ends, the list).  A run
# sends the same tensors in every update, and decoding 339 names costs about 0.02 ms.  Replaced whole.
_names_memo = None


class ParsedUpdate(NativeUpdate):
    """An update parsed by the native library; fields are materialised on first access."""

    def __init__(self, handle, source, dev_bytes=None):
        # `source` keeps the parsed buffer alive: the native handle reads the payload from it;
        # `dev_bytes`: the whole update in device memory (apply reads payload and block table there)
        from . import _native
        self._free = _native.lib().crx_update_free
        self._h = handle
        self._source = source
        self._dev_bytes = dev_bytes
        self._tensors = None
        self._tables = None

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._free(h)

    @property
    def handle(self):
        return self._h

    def headers(self) -> tuple[list[str], list[int], list[int]]:
        """(names, numels, checksums) of the update's tensors, in order, from one native call."""
        if getattr(self, "_headers", None) is None:
            from . import _native
            L = _native.lib()
            n = L.crx_update_n_tensors(self._h)
            need = ctypes.c_uint64()
            L.crx_update_headers(self._h, None, 0, ctypes.byref(need), None, None, None)
            names = ctypes.create_string_buffer(max(need.value, 1))
            ends, numels, chks = ((ctypes.c_uint64 * max(n, 1))() for _ in range(3))
            _native.raise_for(L.crx_update_headers(self._h, names, need.value, ctypes.byref(need), ends, numels,
                                                   chks), None)
            raw, cut = names.raw, bytes(ends)
            memo = _names_memo
            if memo is not None and memo[0] == raw and memo[1] == cut:  # the same names as the last update
                out = memo[2]
            else:
                out, start = [], 0
                for i in range(n):
                    out.append(raw[start:ends[i]].decode("utf-8"))
                    start = ends[i]
                globals()["_names_memo"] = (raw, cut, out)
            self._headers = (out, list(numels[:n]), list(chks[:n]))
        return self._headers

    def _read_tensors(self) -> list[TensorHeader]:
        if self._tensors is None:
            from . import _native
            L = _native.lib()
            out = []
            name_p, name_len, numel, chk, ng = (ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_uint64(),
                                                ctypes.c_uint64(), ctypes.c_int32())
            e, cnt, r = ctypes.c_int32(), ctypes.c_uint64(), ctypes.c_int32()
            for i in range(L.crx_update_n_tensors(self._h)):
                L.crx_update_tensor(self._h, i, ctypes.byref(name_p), ctypes.byref(name_len), ctypes.byref(numel),
                                    ctypes.byref(chk), ctypes.byref(ng))
                name = ctypes.string_at(name_p, name_len.value).decode("utf-8")
                groups = []
                for g in range(ng.value):
                    L.crx_update_group(self._h, i, g, ctypes.byref(e), ctypes.byref(cnt), ctypes.byref(r))
                    groups.append(Group(e.value, cnt.value, r.value))
                out.append(TensorHeader(name, numel.value, chk.value, groups))
            self._tensors = out
        return self._tensors

    def _read_tables(self) -> list[Table]:
        if self._tables is None:
            from . import _native
            L = _native.lib()
            out = []
            e, n = ctypes.c_int32(), ctypes.c_int64()
            for i in range(L.crx_update_n_tables(self._h)):
                L.crx_update_table(self._h, i, ctypes.byref(e), ctypes.byref(n), None, None)
                syms = (ctypes.c_uint32 * n.value)()
                lens = (ctypes.c_uint8 * n.value)()
                L.crx_update_table(self._h, i, ctypes.byref(e), ctypes.byref(n), syms, lens)
                out.append(Table(e.value, list(syms), list(lens)))
            self._tables = out
        return self._tables

    def _read_block_bits(self) -> list[int]:
        from . import _native
        L = _native.lib()
        n = L.crx_update_n_blocks(self._h)
        arr = (ctypes.c_uint32 * max(n, 1))()
        L.crx_update_block_bits(self._h, arr)
        return list(arr[:n])

    def _read_payload(self) -> bytes:
        from . import _native
        L = _native.lib()
        off, n = L.crx_update_payload_offset(self._h), L.crx_update_payload_len(self._h)
        if self._dev_bytes is not None:
            return self._dev_bytes[off:off + n].cpu().numpy().tobytes()
        return bytes(memoryview(self._source)[off:off + n])

    @property
    def total_changes(self) -> int:
        from . import _native
        return _native.lib().crx_update_total_changes(self._h)


def _as_buffer(data):
    if isinstance(data, (bytes, bytearray)):
        return bytes(data) if isinstance(data, bytearray) else data
    if isinstance(data, memoryview):
        return data.tobytes()
    raise TypeError(f"an update is bytes or a uint8 torch tensor, got {type(data).__name__}")


def parse(data) -> ParsedUpdate:
    """Parse and structurally validate an update (limits of the format, wire.py:126-212 of the
    reference). `data` is bytes-like, or a uint8 tensor (its payload may stay on the GPU)."""
    from . import _native
    L = _native.lib()
    err = _native.errbuf()
    h = ctypes.c_void_p()
    try:
        import torch
        is_tensor = isinstance(data, torch.Tensor)
    except ImportError:  # pragma: no cover
        is_tensor = False
    if is_tensor:
        return _parse_tensor(data, L, err)
    buf = _as_buffer(data)
    rc = L.crx_parse(ctypes.c_char_p(buf) if buf else None, len(buf), ctypes.byref(h), err, 512)
    _native.raise_for(rc, err)
    return ParsedUpdate(h.value, buf)


# header bytes the last device-resident parse of this thread needed (updates of a run have headers of
# about the same size): a hint, kept per thread so concurrent callers do not share it
_prefix_hint = threading.local()


def _parse_tensor(t, L, err):
    import torch
    from . import _native
    if t.dtype != torch.uint8 or t.dim() != 1 or not t.is_contiguous():
        raise TypeError("an update tensor must be a contiguous 1-D uint8 tensor")
    if t.device.type != "cuda":
        return parse(t.numpy().tobytes())
    total = t.numel()
    if total == 0:
        return parse(b"")
    have = min(total, max(1 << 16, getattr(_prefix_hint, "n", 0)))
    while True:
        # the leading bytes and the last byte, through pinned host memory
        host = torch.empty(have + 1, dtype=torch.uint8, pin_memory=True)
        host[:have].copy_(t[:have], non_blocking=True)
        host[have:].copy_(t[total - 1:], non_blocking=True)
        torch.cuda.current_stream(t.device).synchronize()  # one wait for both copies
        h = ctypes.c_void_p()
        need = ctypes.c_uint64()
        rc = L.crx_parse_prefix(ctypes.c_void_p(host.data_ptr()), have, total, int(host[have]), ctypes.byref(h),
                                ctypes.byref(need), err, 512)
        if rc == _native.INVALID and need.value > have:
            have = min(total, max(need.value + 64, 2 * have))
            continue
        _native.raise_for(rc, err)
        _prefix_hint.n = have
        return ParsedUpdate(h.value, host, dev_bytes=t)
