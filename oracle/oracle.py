"""ctypes front end of the CPU oracle (crx_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker for the MI355X implementation. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module; the product
(crukx-sync_amd/) never imports, loads or calls it.

The functions mirror the reference's public API (src/crukx_sync/__init__.py:38-57) on host
arrays: numpy uint16/int16 arrays or CPU torch tensors (bf16 / int16), viewed as uint16 bits.
Receiver caches here are plain {name: checksum} dicts (no tensor versions on host arrays).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

OK, CORRUPT, VALUE, NOMEM = 0, 1, 2, 3


class OracleCorrupt(ValueError):
    """The oracle rejects the update (CorruptUpdate in the reference)."""


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u64, i64, i32, vp = ctypes.c_uint64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
        L.orc_weight.restype = u64
        L.orc_weight.argtypes = [u64]
        L.orc_checksum.restype = u64
        L.orc_checksum.argtypes = [vp, u64]
        L.orc_huffman_lengths.restype = i32
        L.orc_huffman_lengths.argtypes = [vp, i64, vp]
        L.orc_canonical_codes.restype = i32
        L.orc_canonical_codes.argtypes = [vp, i64, vp]
        L.orc_rice_param.restype = i32
        L.orc_rice_param.argtypes = [vp, i64]
        L.orc_encode.restype = i32
        L.orc_encode.argtypes = [i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_char_p, u64]
        L.orc_apply.restype = i32
        L.orc_apply.argtypes = [vp, u64, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_char_p, u64]
        L.orc_parse_check.restype = i32
        L.orc_parse_check.argtypes = [vp, u64, ctypes.c_char_p, u64]
        L.orc_free.restype = None
        L.orc_free.argtypes = [vp]
        _lib = L
    return _lib


def _u16(x) -> np.ndarray:
    """Flat uint16 view (shares memory) of a numpy array or a CPU torch tensor."""
    if isinstance(x, np.ndarray):
        if x.dtype not in (np.uint16, np.int16):
            raise ValueError(f"expected 16-bit data, got {x.dtype}")
        return np.ascontiguousarray(x).reshape(-1).view(np.uint16)
    import torch
    if x.dtype not in (torch.bfloat16, torch.int16):
        raise ValueError(f"expected a bfloat16 or int16 tensor, got {x.dtype}")
    if not x.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return x.detach().view(torch.int16).reshape(-1).cpu().numpy().view(np.uint16)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def weight(i: int) -> int:
    return lib().orc_weight(i)


def checksum(x) -> int:
    u = _u16(x)
    return lib().orc_checksum(_ptr(u), u.size)


def huffman_lengths(counts) -> list[int]:
    c = np.asarray(counts, dtype=np.uint64)
    out = np.zeros(len(c), dtype=np.int32)
    if lib().orc_huffman_lengths(_ptr(c), len(c), _ptr(out)) != OK:
        raise MemoryError
    return out.tolist()


def canonical_codes(lengths) -> list[int]:
    L = np.asarray(lengths, dtype=np.int32)
    out = np.zeros(len(L), dtype=np.uint32)
    if lib().orc_canonical_codes(_ptr(L), len(L), _ptr(out)) != OK:
        raise MemoryError
    return out.tolist()


def rice_param(gaps) -> int:
    g = np.asarray(gaps, dtype=np.int64)
    return lib().orc_rice_param(_ptr(g), len(g))


def parse_check(data: bytes) -> None:
    err = ctypes.create_string_buffer(256)
    buf = np.frombuffer(data, dtype=np.uint8) if len(data) else np.zeros(1, np.uint8)
    rc = lib().orc_parse_check(_ptr(buf), len(data), err, 256)
    if rc == CORRUPT:
        raise OracleCorrupt(err.value.decode())
    if rc != OK:
        raise RuntimeError(rc)


def _names(keys):
    raw = [k.encode() for k in keys]
    arr = (ctypes.c_char_p * max(len(raw), 1))(*raw)
    lens = np.array([len(r) for r in raw] or [0], dtype=np.uint64)
    return raw, arr, lens


def encode_update(old, new, checksums: dict | None = None) -> bytes:
    """encode_update (src/crukx_sync/__init__.py:38-48) on host arrays."""
    if old.keys() != new.keys():
        raise ValueError("old and new differ in tensor names")
    keys = list(old.keys())
    A = [_u16(old[k]) for k in keys]
    B = [_u16(new[k]) for k in keys]
    for k, a, b in zip(keys, A, B):
        if a.size != b.size:
            raise ValueError(f"{k}: old and new differ in shape")
    n = len(keys)
    raw, names, name_lens = _names(keys)
    olds = np.array([_ptr(a) for a in A] or [0], dtype=np.uint64)
    news = np.array([_ptr(b) for b in B] or [0], dtype=np.uint64)
    numels = np.array([a.size for a in A] or [0], dtype=np.uint64)
    has = np.array([1 if checksums is not None and k in checksums else 0 for k in keys] or [0], dtype=np.int32)
    vals = np.array([checksums[k] if h else 0 for k, h in zip(keys, has)] or [0], dtype=np.uint64)
    out = ctypes.c_void_p()
    out_len = ctypes.c_uint64()
    new_chk = np.zeros(max(n, 1), dtype=np.uint64)
    present = np.zeros(max(n, 1), dtype=np.int32)
    err = ctypes.create_string_buffer(256)
    rc = lib().orc_encode(n, ctypes.cast(names, ctypes.c_void_p), _ptr(name_lens), _ptr(olds), _ptr(news),
                          _ptr(numels), _ptr(has), _ptr(vals), ctypes.byref(out), ctypes.byref(out_len),
                          _ptr(new_chk), _ptr(present), err, 256)
    if rc == VALUE:
        raise ValueError(err.value.decode())
    if rc != OK:
        raise MemoryError
    data = ctypes.string_at(out, out_len.value)
    lib().orc_free(out)
    if checksums is not None:
        for i, k in enumerate(keys):
            if present[i]:
                checksums[k] = int(new_chk[i])
    return data


def apply_update(weights, update: bytes, checksums: dict | None = None) -> int:
    """apply_update (src/crukx_sync/__init__.py:51-57) on host arrays, in place; returns the
    number of changed elements. The receiver cache maps name -> checksum."""
    keys = list(weights.keys())
    W = [_u16(weights[k]) for k in keys]
    raw, names, name_lens = _names(keys)
    datas = np.array([_ptr(w) for w in W] or [0], dtype=np.uint64)
    numels = np.array([w.size for w in W] or [0], dtype=np.uint64)
    has = np.array([1 if checksums is not None and k in checksums else 0 for k in keys] or [0], dtype=np.int32)
    vals = np.array([checksums[k] if h else 0 for k, h in zip(keys, has)] or [0], dtype=np.uint64)
    buf = np.frombuffer(update, dtype=np.uint8) if len(update) else np.zeros(1, np.uint8)
    changed = ctypes.c_uint64()
    n_t = ctypes.c_int32()
    cap = len(update) + 1
    tgt = np.zeros(cap, dtype=np.int32)
    chk = np.zeros(cap, dtype=np.uint64)
    err = ctypes.create_string_buffer(256)
    rc = lib().orc_apply(_ptr(buf), len(update), len(keys), ctypes.cast(names, ctypes.c_void_p), _ptr(name_lens),
                         _ptr(datas), _ptr(numels), _ptr(has), _ptr(vals), ctypes.byref(changed), ctypes.byref(n_t),
                         _ptr(tgt), _ptr(chk), err, 256)
    if rc == CORRUPT:
        raise OracleCorrupt(err.value.decode())
    if rc == VALUE:
        raise ValueError(err.value.decode())
    if rc != OK:
        raise MemoryError
    if checksums is not None:
        for i in range(n_t.value):
            checksums[keys[tgt[i]]] = int(chk[i])
    return changed.value
