"""crukx-sync on MI355X: the exact, compact bf16 weight-update codec, computed in gfx950 kernels.

    update = encode_update(prev, cur)   # trainer side: name -> bf16 tensor mappings in, bytes out
    apply_update(weights, update)       # worker side: the new values land in `weights`, in place

The names, arguments, errors, wire format (version 2) and all-or-nothing rule are those of the
reference (Crukx-dev/crukx-sync, src/crukx_sync/__init__.py): an update either decodes and matches
every tensor's checksum, or it raises and the weights keep their old values.

Checksum caches (optional, one dict per side, kept by the caller from one update to the next):
- With a cache the sender derives each new checksum from the old one plus the changed elements, and
  the receiver checks against a cached value instead of reading all of its weights again.
- A stale or wrong sender cache cannot corrupt a receiver: the update it yields fails to verify.
- The receiver trusts an entry only while the tensor's PyTorch `_version` equals the one recorded
  after this library's own write. In-place PyTorch ops move `_version`, so they are noticed; writes
  that go around PyTorch (raw device pointers, some communication libraries) are not, and callers
  that update weights that way should start from an empty receiver cache.

Device-resident variant (no host round trip of the bytes): `encode_update_device` returns the same
bytes as a uint8 tensor on the GPU, and `apply_update` accepts such a tensor.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass

import torch

from . import codec
from .wire import CorruptUpdate, parse, serialize

__all__ = ["encode_update", "apply_update", "UpdateStats", "CorruptUpdate", "encode_update_device"]


@dataclass
class UpdateStats:
    tensors: int
    changed: int
    bytes: int


def encode_update(old: Mapping[str, torch.Tensor], new: Mapping[str, torch.Tensor],
                  checksums: dict | None = None) -> bytes:
    """Bytes that turn `old` into `new` exactly. Same names and shapes; tensors are bf16 or int16."""
    if old.keys() != new.keys():
        raise ValueError(f"old and new differ in tensor names: {sorted(old.keys() ^ new.keys())[:5]}")
    with torch.no_grad():
        update, new_checksums = codec.encode(old, new, checksums)
    data = serialize(update)
    if checksums is not None:  # commit only once the update exists
        checksums.update(new_checksums)
    return data


def encode_update_device(old: Mapping[str, torch.Tensor], new: Mapping[str, torch.Tensor],
                         checksums: dict | None = None) -> torch.Tensor:
    """encode_update, with the bytes left in device memory as a uint8 tensor (on the tensors'
    device). The bytes are identical to encode_update's."""
    if old.keys() != new.keys():
        raise ValueError(f"old and new differ in tensor names: {sorted(old.keys() ^ new.keys())[:5]}")
    with torch.no_grad():
        update, new_checksums = codec.encode(old, new, checksums)
    if isinstance(update, codec.EncodedUpdate):
        data = update.to_device()
    else:
        dev = next(iter(old.values())).device if old else torch.device("cuda")
        data = torch.frombuffer(bytearray(serialize(update)), dtype=torch.uint8).to(
            dev if dev.type == "cuda" else torch.device("cuda"))
    if checksums is not None:
        checksums.update(new_checksums)
    return data


def apply_update(weights: Mapping[str, torch.Tensor], update, checksums: dict | None = None) -> UpdateStats:
    """Write the update into `weights` in place; on any error the weights end as they were. `update`
    is the bytes from encode_update or the uint8 tensor from encode_update_device. Most changes are
    written while they are located, before the update's checksums are verified, and put back if the
    update does not verify; the call returns once the last writes (or that undoing) are done, so
    later work on any stream sees all of the update or none of it."""
    u = parse(update)
    with torch.no_grad():
        changed = codec.apply(weights, u, checksums)
    n = update.numel() if isinstance(update, torch.Tensor) else len(update)
    return UpdateStats(len(u.headers()[0]), changed, n)
