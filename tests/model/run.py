"""Runs crukx_sync's Python layer on the CPU model of the library (tests/model/, libcrukx_model.so):
the library's own kernels and host code, built for the CPU under AddressSanitizer and UBSan, with
every kernel run by the wave64 emulator of simt.cpp.  Test infrastructure only.

The process must start with the sanitizer runtime preloaded (`env()` gives the environment); it then
binds crukx_sync to the model library and routes the few device-only pieces of the Python layer to
the CPU: tensors live in host memory, the "device" is the CPU, every stream is the null stream.  The
rest of the Python layer (argument checks, caches, the receiver's exponent counts and their
lifecycle) runs unchanged.

    python tests/model/run.py <scenario> [args]   (scenarios below)
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
LIB = os.path.join(HERE, "_build", "libcrukx_model.so")
CLANG = "/opt/rocm/llvm/bin/clang++"


def build() -> str:
    """Builds the model library (make in tests/model); returns its path."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def asan_runtime() -> str:
    out = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    if not os.path.isabs(path):  # this clang keeps it under its resource directory
        res = subprocess.run([CLANG, "-print-resource-dir"], capture_output=True, text=True).stdout.strip()
        path = os.path.join(res, "lib", "linux", "libclang_rt.asan-x86_64.so")
    return path


def env(lib: str | None = None) -> dict:
    """The environment of a model process: the sanitizer runtime first, leaks not reported (the
    interpreter keeps its own until exit), a sanitizer report ends the process with status 86."""
    e = dict(os.environ)
    e["LD_PRELOAD"] = asan_runtime()
    # every allocation filled with 0xFF: device memory that no kernel wrote reads as all ones (the
    # kernels' "none" value, and the value closest to wrapping in index arithmetic)
    e["ASAN_OPTIONS"] = ("detect_leaks=0:detect_stack_use_after_return=0:exitcode=86:abort_on_error=0:"
                         "malloc_fill_byte=255:max_malloc_fill_size=4294967295")
    e["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1:exitcode=86"
    e["CRX_LIBRARY"] = lib or LIB
    e["OMP_NUM_THREADS"] = "1"
    return e


def install():
    """Binds crukx_sync to the model library (CRX_LIBRARY) and routes its device plumbing to the CPU."""
    for p in (os.path.join(ROOT, "crukx-sync_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
        if p not in sys.path:
            sys.path.insert(0, p)
    assert os.environ.get("CRX_LIBRARY"), "start the process with run.env()"
    import torch

    import crukx_sync  # noqa: F401
    from crukx_sync import _native, codec, wire

    assert os.path.samefile(_native.LIB_PATH, os.environ["CRX_LIBRARY"])
    codec._hip_device = lambda dev: dev          # the model's device is the CPU
    _native.stream_of = lambda dev: 0            # the null stream
    torch.cuda.device = lambda d: contextlib.nullcontext()

    def parse_tensor(t, L, err):
        """wire._parse_tensor's device branch for a host tensor: the header and block table are parsed
        from a copy of the leading bytes, and apply reads the block table and payload from `t` itself."""
        if t.dtype != torch.uint8 or t.dim() != 1 or not t.is_contiguous():
            raise TypeError("an update tensor must be a contiguous 1-D uint8 tensor")
        total = t.numel()
        if total == 0:
            return wire.parse(b"")
        have = min(total, 1 << 16)
        while True:
            host = torch.empty(have + 1, dtype=torch.uint8)
            host[:have].copy_(t[:have])
            host[have:].copy_(t[total - 1:])
            h, need = ctypes.c_void_p(), ctypes.c_uint64()
            rc = L.crx_parse_prefix(ctypes.c_void_p(host.data_ptr()), have, total, int(host[have]), ctypes.byref(h),
                                    ctypes.byref(need), err, 512)
            if rc == _native.INVALID and need.value > have:
                have = min(total, max(need.value + 64, 2 * have))
                continue
            _native.raise_for(rc, err)
            return wire.ParsedUpdate(h.value, host, dev_bytes=t)

    wire._parse_tensor = parse_tensor


# ------------------------------------------------------------------ scenarios

def scenario_parity() -> None:
    """Encode (bytes and the device-resident form) and apply of the small scenarios against the oracle."""
    import torch

    import crukx_sync
    import oracle
    import scenarios
    sc = scenarios.single_scenarios()
    names = sorted(sc)
    for name in names:
        old, new = sc[name]
        upd = crukx_sync.encode_update(old, new)
        ref = oracle.encode_update(old, new)
        assert upd == ref, f"{name}: model bytes differ from the oracle ({len(upd)} vs {len(ref)})"
        dev = crukx_sync.encode_update_device(old, new)
        assert bytes(dev.numpy()) == ref, name
        for u in (upd, dev):
            w = {k: v.clone() for k, v in old.items()}
            crukx_sync.apply_update(w, u)
            for k in new:
                assert torch.equal(w[k].view(torch.int16), new[k].view(torch.int16)), (name, k)
        print(f"parity {name}: {len(upd)} bytes", flush=True)


def scenario_small4_flips(first: int = 0, count: int = -1, every: int = 1, widened: int = 0) -> None:
    """The four-tensor exhaustive corruption sequences of tests/test_full_sizes.py (tests/corruption.py),
    on the model: the same weights, steps, caches, device-resident update and flips in the same order.
    Flips [first, first + count) of the list are applied (every `every`-th; SMALL4_LIST: an explicit
    list of flip indices), starting from the warm state.  widened=1: the widened sequence, with
    16,384-element slabs."""
    import corruption
    from crukx_sync import codec

    if widened:
        codec._SLAB = 1 << 14
    only = [int(v) for v in os.environ["SMALL4_LIST"].split(",")] if os.environ.get("SMALL4_LIST") else None
    rejected, applied = corruption.run("cpu", bool(widened), lambda m: print(m, flush=True), first, count, every,
                                       check_every=1, verbose=bool(os.environ.get("SMALL4_VERBOSE")), only=only)
    print(f"small4 done: {rejected} rejected, {applied} applied", flush=True)


def scenario_rejected_early() -> None:
    """Updates the decoder rejects, applied to multi-slab tensors (4096-element slabs) while device
    memory starts as all ones: each raises CorruptUpdate and leaves the receiver as it was.  Two
    neighbouring block-table entries are moved by one bit in opposite directions (the header and the
    payload length still parse), so both blocks fail to decode and the update is rejected before its
    changes are located; the receivers' caches are warm, as in a training run.  The undo pass once
    took such an update's never-written record offsets (all ones) as a range to restore and walked
    past the record buffer."""
    import struct

    import torch

    import crukx_sync
    import scenarios
    from crukx_sync import CorruptUpdate, _native, codec, wire

    codec._SLAB = 4096
    old, new = {}, {}
    for i, n in enumerate([300_000, 50_001, 4_097]):
        a, b = scenarios.rl_pair(n, lr=4e-6, seed=80 + i)
        old[f"t{i}"], new[f"t{i}"] = a, b
    send, rc = {}, {}
    recv = {k: v.clone() for k, v in old.items()}
    crukx_sync.apply_update(recv, crukx_sync.encode_update(old, new, send), rc)  # caches warm
    old, new = new, old  # the updates below take the receiver back
    upd = bytearray(crukx_sync.encode_update(old, new, send))
    u = wire.parse(bytes(upd))
    L = _native.lib()
    n_blocks, pay = L.crx_update_n_blocks(u.handle), L.crx_update_payload_offset(u.handle)
    pay_len = L.crx_update_payload_len(u.handle)
    n = 1
    while pay_len >= 128 ** n:
        n += 1
    bt = pay - n - 4 * n_blocks
    bits = list(struct.unpack_from(f"<{n_blocks}I", upd, bt))
    rejected = 0
    for b in range(0, n_blocks - 1, max(1, n_blocks // 12)):
        bad = bytearray(upd)
        struct.pack_into("<II", bad, bt + 4 * b, bits[b] + 1, bits[b + 1] - 1)
        for form in (bytes(bad), torch.frombuffer(bytearray(bad), dtype=torch.uint8)):
            try:
                crukx_sync.apply_update(recv, form, rc)
            except CorruptUpdate:
                rejected += 1
            else:
                raise AssertionError(f"blocks {b}, {b + 1} moved by one bit: applied")
            for k in old:
                assert torch.equal(recv[k].view(torch.int16), old[k].view(torch.int16)), (b, k)
    crukx_sync.apply_update(recv, bytes(upd), rc)
    for k in new:
        assert torch.equal(recv[k].view(torch.int16), new[k].view(torch.int16)), k
    print(f"rejected early: {rejected} updates rejected, the receiver unchanged each time", flush=True)


def scenario_group_message() -> None:
    """The group-size check covers tensors of more than codec._SLAB elements (codec.py:598-604): a
    20,000-element tensor whose group outnumbers the receiver's elements of its exponent is refused by
    the verification with the default _SLAB, and with "group has more changes than elements" once
    _SLAB is 4096; the receiver is unchanged either way."""
    import torch

    import crukx_sync
    from crukx_sync import CorruptUpdate, codec

    n = 20_000
    base = torch.full((n,), 0x3F80, dtype=torch.int16)
    sender = base.clone()
    sender[100:105] = 0x3C00
    target = sender.clone()
    target[100:105] += 1
    upd = crukx_sync.encode_update({"w": sender}, {"w": target})
    short = base.clone()
    short[100:103] = 0x3C00
    msgs = []
    for slab in (1 << 24, 4096):
        codec._SLAB = slab
        w = {"w": short.clone()}
        try:
            crukx_sync.apply_update(w, upd)
        except CorruptUpdate as e:
            msgs.append(str(e))
        assert torch.equal(w["w"], short)
    assert len(msgs) == 2 and msgs[0] != msgs[1] and msgs[1] == "group has more changes than elements", msgs
    print(f"group message: {msgs}", flush=True)


def scenario_device_offsets() -> None:
    """A device-resident update applied from views at every byte offset within an 8-byte word (the
    decoder then reads the payload in place, from the aligned words around it) and from the end of an
    allocation of exactly its size (then from a padded copy, or in place when its last word ends
    there): every access stays inside the update's allocation, and every apply is exact."""
    import torch

    import crukx_sync
    import scenarios

    a, b = scenarios.rl_pair(70_000, seed=21)
    upd = crukx_sync.encode_update_device({"w": a}, {"w": b})
    n = upd.numel()
    views = []
    for shift in range(9):
        buf = torch.zeros(n + shift + 40, dtype=torch.uint8)
        views.append(buf[shift:shift + n])
    for cut in (0, 3, 5):
        buf = torch.empty(n + cut, dtype=torch.uint8)  # the update at the very end of its allocation
        views.append(buf[cut:])
    for view in views:
        view.copy_(upd)
        w = {"w": a.clone()}
        crukx_sync.apply_update(w, view)
        assert torch.equal(w["w"].view(torch.int16), b.view(torch.int16))
    print(f"device offsets: {len(views)} applies exact", flush=True)


def scenario_parts() -> None:
    """The part-wise encode and apply (CRX_PART_ELEMENTS=60000: parts of one to three tensors) on the
    multi-tensor scenarios: the bytes equal the oracle's single-pass bytes (also with the sender's
    checksum cache), two chained applies with both caches are exact (the receiver's exponent counts kept
    part by part), and a corruption in the last part is rejected with every tensor unchanged (the
    verdict is taken on the whole update before any part is written)."""
    import torch

    import crukx_sync
    import oracle
    import scenarios
    from crukx_sync import CorruptUpdate

    def equal(x, y):
        return all(torch.equal(x[k].view(torch.int16), y[k].view(torch.int16)) for k in y)

    os.environ["CRX_PART_ELEMENTS"] = "60000"
    sc = scenarios.single_scenarios()
    for name in ("many_tensors", "three_tensors"):
        old, new = sc[name]
        ref = oracle.encode_update(old, new)
        assert crukx_sync.encode_update(old, new) == ref, name
        assert bytes(crukx_sync.encode_update_device(old, new).numpy()) == ref, name
        send, rc = {}, {}
        w = {k: v.clone() for k, v in old.items()}
        crukx_sync.apply_update(w, crukx_sync.encode_update(old, new, send), rc)
        assert equal(w, new), name
        chk = dict(send)
        back = crukx_sync.encode_update(new, old, send)
        assert back == oracle.encode_update(new, old, dict(chk)), name
        # bytes near the payload's end (blocks of the last part), until one that parses is rejected by
        # the device passes
        found = None
        for k in range(2, 40):
            bad = bytearray(back)
            bad[-k] ^= 0x10
            try:
                crukx_sync.apply_update(w, bytes(bad), rc)
            except CorruptUpdate as e:
                if "verify" in str(e) or "outside" in str(e):
                    found = (k, str(e))
            else:
                raise AssertionError(f"{name}: a corrupted update applied")
            assert equal(w, new), (name, k)
            if found:
                break
        assert found, name
        print(f"parts {name}: byte -{found[0]} flipped, rejected by the device passes ({found[1]})", flush=True)
        crukx_sync.apply_update(w, back, rc)
        assert equal(w, old), name
        assert send == {k: v[0] for k, v in rc.items()}, name
        print(f"parts {name}: {len(ref)} bytes as the oracle's; chained applies exact", flush=True)


SCENARIOS = {"parity": scenario_parity, "small4_flips": scenario_small4_flips, "rejected_early": scenario_rejected_early,
             "group_message": scenario_group_message, "parts": scenario_parts,
             "device_offsets": scenario_device_offsets}

if __name__ == "__main__":
    install()
    SCENARIOS[sys.argv[1]](*[int(a) for a in sys.argv[2:]])
