"""ctypes binding of libcrukx_hip.so (the gfx950 implementation, C ABI in include/crukx.h).

The library is loaded after torch so that it binds to the HIP runtime torch already loaded. There
is no fallback: if the library is missing the import of the codec fails with instructions to build
it, and every tensor operation runs on a HIP device.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

from .wire import CorruptUpdate

# the in-tree build, or another build of the library named by CRX_LIBRARY (e.g. to compare versions)
LIB_PATH = os.environ.get("CRX_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcrukx_hip.so")
ABI_VERSION = 1
OK, CORRUPT, INVALID, DEVICE, NOMEM = 0, 1, 2, 3, 4

ALLOC_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64)

_lib = None
_lock = threading.Lock()
_meta = None
_meta_tried = False

# name -> (restype, argtypes), exactly the declarations of include/crukx.h
_u8p, _u32p, _u64p, _i32p, _i64p = (ctypes.POINTER(t) for t in
                                    (ctypes.c_uint8, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32, ctypes.c_int64))
_vp, _cp = ctypes.c_void_p, ctypes.c_char_p
_i32, _i64, _u64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64
SIGNATURES = {
    "crx_abi_version": (_i32, []),
    "crx_parse": (_i32, [_vp, _u64, ctypes.POINTER(_vp), _cp, _u64]),
    "crx_parse_prefix": (_i32, [_vp, _u64, _u64, ctypes.c_uint8, ctypes.POINTER(_vp), _u64p, _cp, _u64]),
    "crx_update_free": (None, [_vp]),
    "crx_update_n_tables": (_i64, [_vp]),
    "crx_update_table": (_i32, [_vp, _i64, _i32p, _i64p, _vp, _vp]),
    "crx_update_n_tensors": (_i64, [_vp]),
    "crx_update_tensor": (_i32, [_vp, _i64, ctypes.POINTER(_vp), _u64p, _u64p, _u64p, _i32p]),
    "crx_update_group": (_i32, [_vp, _i64, _i32, _i32p, _u64p, _i32p]),
    "crx_update_headers": (_i32, [_vp, _vp, _u64, _u64p, _vp, _vp, _vp]),
    "crx_update_n_blocks": (_u64, [_vp]),
    "crx_update_block_bits": (_i32, [_vp, _vp]),
    "crx_update_payload_offset": (_u64, [_vp]),
    "crx_update_payload_len": (_u64, [_vp]),
    "crx_update_total_changes": (_u64, [_vp]),
    "crx_apply": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, ALLOC_FN, _vp, _u64p, _cp, _u64]),
    "crx_apply_cached": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, ALLOC_FN, _vp, _u64p, _cp, _u64]),
    "crx_apply_hist_words": (_u64, [_u64, _i32]),
    "crx_encode": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp, ALLOC_FN, _vp, ctypes.POINTER(_vp), _cp, _u64]),
    "crx_encoded_present": (_i32, [_vp, _i32]),
    "crx_encoded_checksum": (_u64, [_vp, _i32]),
    "crx_encoded_checksums": (None, [_vp, _vp, _vp]),
    "crx_encoded_total_changes": (_u64, [_vp]),
    "crx_encoded_size": (_u64, [_vp, _vp, _vp]),
    "crx_encoded_write": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _cp, _u64]),
    "crx_encoded_n_tables": (_i64, [_vp]),
    "crx_encoded_table": (_i32, [_vp, _i64, _i32p, _i64p, _vp, _vp]),
    "crx_encoded_n_groups": (_i32, [_vp, _i32]),
    "crx_encoded_group": (_i32, [_vp, _i32, _i32, _i32p, _u64p, _i32p]),
    "crx_encoded_n_blocks": (_u64, [_vp]),
    "crx_encoded_block_bits": (_i32, [_vp, _vp, _vp]),
    "crx_encoded_payload_len": (_u64, [_vp]),
    "crx_encoded_payload": (_i32, [_vp, _vp, _vp]),
    "crx_encoded_free": (None, [_vp]),
    "crx_checksum": (_i32, [_vp, _u64, _vp, ALLOC_FN, _vp, _u64p, _cp, _u64]),
    "crx_checksum_noalloc": (_i32, [_vp, _u64, _vp, _u64p, _cp, _u64]),
    "crx_huffman_lengths": (_i32, [_vp, _i64, _vp]),
    "crx_canonical_codes": (_i32, [_vp, _i64, _vp]),
    "crx_rice_candidates": (None, [_u64, _u64, _vp]),
    "crx_rice_choose": (_i32, [_u64, _vp, _vp]),
    "crx_timing_enable": (None, [_i32]),
    "crx_timing_only": (None, [_cp]),
    "crx_timing_reset": (None, []),
    "crx_timing_read": (_i32, [_cp, _u64]),
}


class NativeLibraryMissing(ImportError):
    pass


def lib():
    """The loaded library (built by __graft_entry__.build() / `make -C crukx-sync_amd/csrc`)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryMissing(
                    f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `make -C crukx-sync_amd/csrc` (hipcc, --offload-arch=gfx950)")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                f = getattr(L, name)
                f.restype = res
                f.argtypes = args
            if L.crx_abi_version() != ABI_VERSION:
                raise NativeLibraryMissing(f"{LIB_PATH}: ABI {L.crx_abi_version()}, expected {ABI_VERSION}")
            _lib = L
    return _lib


def raise_for(rc: int, err) -> None:
    if rc == OK:
        return
    msg = err.value.decode("utf-8", "replace") if err is not None else ""
    if rc == CORRUPT:
        raise CorruptUpdate(msg)
    if rc == INVALID:
        raise ValueError(msg)
    if rc == NOMEM:
        raise MemoryError(msg or "out of device memory")
    raise RuntimeError(f"HIP error: {msg}")


def errbuf():
    return ctypes.create_string_buffer(512)


class Workspace:
    """Device memory for one native call, handed out from torch's caching allocator."""

    def __init__(self, device: torch.device):
        self.device = device
        # the callback holds these, not the workspace: no reference cycle, so the buffers are freed as
        # soon as the workspace is dropped rather than at the next garbage collection
        tensors: list[torch.Tensor] = []
        errors: list[BaseException] = []
        self.tensors = tensors
        self._errors = errors

        def _alloc(_ctx, nbytes):
            try:
                t = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
            except BaseException as e:  # noqa: BLE001  (re-raised after the native call returns)
                errors.append(e)
                return None
            tensors.append(t)
            return t.data_ptr()

        self.fn = ALLOC_FN(_alloc)

    def check(self):
        if self._errors:
            e = self._errors[0]
            self._errors.clear()
            raise e

    def release(self):
        self.tensors.clear()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def u64_array(values):
    return (ctypes.c_uint64 * max(len(values), 1))(*[v & 0xFFFFFFFFFFFFFFFF for v in values])


def tensor_meta():
    """The batched tensor-metadata helper (crx_tensor_meta.so next to this file, built with the library),
    or None: the Python layer then reads the same fields tensor by tensor."""
    global _meta, _meta_tried
    if not _meta_tried:
        with _lock:
            if not _meta_tried:
                path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "crx_tensor_meta.so")
                if os.path.exists(path):
                    import importlib.util
                    spec = importlib.util.spec_from_file_location("crx_tensor_meta", path)
                    mod = importlib.util.module_from_spec(spec)
                    spec.loader.exec_module(mod)
                    _meta = mod
                _meta_tried = True
    return _meta


def view_u64(arr):
    """A ctypes u64 array over an array.array('Q') (no copy; the array must not grow while in use)."""
    if not len(arr):
        arr.append(0)
    return (ctypes.c_uint64 * len(arr)).from_buffer(arr)


def view_ptr(arr):
    """A ctypes pointer array over an array.array('Q') of addresses (no copy)."""
    if not len(arr):
        arr.append(0)
    return (ctypes.c_void_p * len(arr)).from_buffer(arr)


def view_i32(arr):
    """A ctypes int32 array over an array.array('i') (no copy)."""
    if not len(arr):
        arr.append(0)
    return (ctypes.c_int32 * len(arr)).from_buffer(arr)


def i32_array(values):
    return (ctypes.c_int32 * max(len(values), 1))(*values)


def ptr_array(values):
    return (ctypes.c_void_p * max(len(values), 1))(*values)


def timing(enable: bool, only: list[str] | None = None) -> None:
    """Per-launch kernel timing on or off; `only` limits it to the named kernels."""
    lib().crx_timing_only(",".join(only).encode() if only else None)
    lib().crx_timing_enable(1 if enable else 0)


def timing_reset() -> None:
    lib().crx_timing_reset()


def timing_read() -> dict[str, tuple[int, float]]:
    """kernel name -> (launches, total milliseconds) since the last reset."""
    n = lib().crx_timing_read(None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    lib().crx_timing_read(buf, n + 1)
    out = {}
    for line in buf.value.decode().splitlines():
        name, calls, ms = line.split()
        out[name] = (int(calls), float(ms))
    return out
