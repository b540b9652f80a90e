"""crukx-sync on MI355X: exact, compact bf16 weight updates for RL weight sync.

    update = encode_update(prev, cur)   # trainer: dicts of name -> bf16 torch tensors
    apply_update(weights, update)       # worker: writes the new values into `weights` in place

Same public API, wire format (version 2) and all-or-nothing semantics as the reference
(Crukx-dev/crukx-sync, src/crukx_sync/__init__.py): nothing is written unless the whole update
decodes and every tensor's checksum verifies. The work runs in hand-written gfx950 kernels.

For per-step sync, pass a `checksums` dict on each side and keep it between steps: checksums are
then updated from the changed elements only instead of re-reading every tensor.
- Sender: a wrong cache produces an update the receiver rejects (CorruptUpdate), never wrong weights.
- Receiver: a cached checksum is used only while the tensor's `_version` is unchanged since this
  library last wrote it; any PyTorch in-place op bumps it and forces a full re-check. Writes that
  bypass PyTorch's version counter (raw pointers, some collective libraries) are not detected, so
  drop the receiver cache if weights can change that way.

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
    """Write the update into `weights` in place; on any error nothing is written. `update` is the
    bytes from encode_update or the uint8 tensor from encode_update_device. Errors are raised before
    anything is written; the writes themselves are ordered on the current stream, like any in-place
    torch operation on the weights."""
    u = parse(update)
    with torch.no_grad():
        changed = codec.apply(weights, u, checksums)
    n = update.numel() if isinstance(update, torch.Tensor) else len(update)
    return UpdateStats(len(u.headers()[0]), changed, n)
