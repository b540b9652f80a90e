"""Writes the golden vectors in tests/golden/ by running the reference implementation.

The reference (Crukx-dev/crukx-sync v0.2.0) is imported from its read-only checkout at
/root/reference/src, on CPU, in the build container only; it never travels with this repository.
It is run only for what no closed form pins: Huffman code lengths with their tie-breaks and
length limiting (codec.huffman_lengths, codec.py:71-98), canonical codes (codec.py:101-111), the
Rice parameter choice (codec._rice_params, codec.py:268-275), and the composed bytes of
encode_update (src/crukx_sync/__init__.py:38-48) on the inputs of tests/scenarios.py.

Outputs (data only): huffman.json, rice.json, checksum.json, updates.json.
Usage:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, "/root/reference/src")

import crukx_sync as ref  # noqa: E402  (the reference)
import crukx_sync.codec as ref_codec  # noqa: E402
import scenarios  # noqa: E402

assert os.path.abspath(ref.__file__).startswith("/root/reference/"), ref.__file__

INLINE = 16384  # updates up to this many bytes are stored whole, larger ones by SHA-256


def fib(n, scale=1):
    a, b, out = 1, 1, []
    for _ in range(n):
        out.append(a * scale)
        a, b = b, a + b
    return out


def huffman_cases():
    rng = np.random.default_rng(1234)
    cases = []
    for n in (1, 2, 3, 4, 5, 8, 13, 30, 100, 257, 1000):
        cases.append([int(x) for x in rng.integers(1, 1000, n)])
        cases.append([int(x) for x in rng.integers(1, 4, n)])
        cases.append([7] * n)
        cases.append([max(1, int(1e6 * 2.0 ** -(i % 40))) for i in range(n)])
    for n in (17, 18, 19, 20, 25, 30, 40, 60, 80, 90):
        cases.append(fib(n))
        cases.append(list(reversed(fib(n, 3))))
    cases.append(fib(80) + [1] * 500)                       # deep even after flattening: flat fallback
    cases.append([1 << 40, 1 << 39] + [1] * 3000)           # one flattening round is not enough
    cases.append([int(x) for x in rng.integers(1, 1 << 62, 50)])
    cases.append([0, 0, 5, 1, 0])                           # zero counts (never produced by encode)
    big = []
    for seed, n, hi in ((1, 5000, 100), (2, 70000, 3), (3, 131071, 2), (4, 20000, 1 << 30)):
        c = [int(x) for x in np.random.default_rng(seed).integers(1, hi, n)]
        big.append({"seed": seed, "n": n, "hi": hi, "counts_sha": hashlib.sha256(json.dumps(c).encode()).hexdigest(),
                    "lengths_sha": hashlib.sha256(json.dumps(ref_codec.huffman_lengths(c)).encode()).hexdigest()})
    out = []
    for c in cases:
        L = ref_codec.huffman_lengths(c)
        out.append({"counts": c, "lengths": L, "codes": ref_codec.canonical_codes(L)})
    return {"cases": out, "big": big}


def rice_cases():
    rng = np.random.default_rng(99)
    groups = []
    for mean in (0, 0.3, 1, 1.5, 2, 3, 7, 8, 9, 100, 1000, 1e5, 1e7):
        for n in (1, 2, 5, 64, 1000):
            groups.append([int(x) for x in rng.geometric(1.0 / (mean + 1), n) - 1])
    for k in range(0, 31):  # sum/count exactly 2^k, and just below / above
        c = 3
        groups.append([(1 << k) * c - 2, 1, 1])
        groups.append([(1 << k) * c - 3, 1, 1])
        groups.append([(1 << k) * c - 1, 1, 1])
    groups.append([0] * 4096)
    groups.append([(1 << 20) - 1])
    groups.append([0] * 2000 + [(1 << 20) - 2001])
    groups.append([1 << 40, 0, 0])
    out = []
    gaps = torch.tensor([g for grp in groups for g in grp], dtype=torch.long)
    counts = torch.tensor([len(grp) for grp in groups], dtype=torch.long)
    gid = torch.repeat_interleave(torch.arange(len(groups)), counts)
    r = ref_codec._rice_params(gaps, gid, counts).tolist()
    for grp, rr in zip(groups, r):
        out.append({"gaps": grp, "rice": int(rr)})
    return {"cases": out}


def checksum_cases():
    out = []
    arrays = {
        "single_3f81": np.array([0x3F81], dtype=np.uint16),
        "arange_65536": np.arange(65536, dtype=np.uint16),
        "zeros_1000": np.zeros(1000, dtype=np.uint16),
        "ffff_777": np.full(777, 0xFFFF, dtype=np.uint16),
    }
    for name, a in arrays.items():
        t = torch.from_numpy(a.view(np.int16).copy())
        out.append({"name": name, "u16": a.tolist() if a.size <= 16 else None,
                    "checksum": int(ref_codec.checksum(t))})
    rnd = np.random.default_rng(5).integers(0, 65536, 3_000_001).astype(np.uint16)
    out.append({"name": "random_3000001_seed5", "u16": None,
                "checksum": int(ref_codec.checksum(torch.from_numpy(rnd.view(np.int16).copy())))})
    weights = [int(ref_codec._weights(torch.tensor([i], dtype=torch.long))[0]) & ((1 << 64) - 1)
               for i in (0, 1, 2, 3, 1000, 1 << 20, (1 << 31) + 5, (1 << 40) + 7)]
    return {"cases": out, "weights": {"index": [0, 1, 2, 3, 1000, 1 << 20, (1 << 31) + 5, (1 << 40) + 7],
                                      "w": weights}}


def record(upd: bytes):
    rec = {"len": len(upd), "sha256": hashlib.sha256(upd).hexdigest()}
    if len(upd) <= INLINE:
        rec["hex"] = upd.hex()
    return rec


def update_cases():
    out = {}
    for name, (old, new) in scenarios.single_scenarios().items():
        chk = {}
        upd = ref.encode_update(old, new, None)
        upd_c = ref.encode_update(old, new, chk)  # full checksums recorded by the sender cache
        assert upd == upd_c
        out[name] = {"inputs_old": scenarios.bits_sha(old), "inputs_new": scenarios.bits_sha(new),
                     "update": record(upd), "sender_checksums": {k: int(v) for k, v in chk.items()}}
        print(name, len(upd), flush=True)
    chains = {}
    for cname, states in (("small4_chain", scenarios.chain_small4(3)), ("cache_chain", scenarios.chain_cache(5))):
        send = {}
        steps = []
        for s in range(1, len(states)):
            upd = ref.encode_update(states[s - 1], states[s], send)
            steps.append({"inputs_new": scenarios.bits_sha(states[s]), "update": record(upd),
                          "sender_checksums": {k: int(v) for k, v in send.items()}})
            print(cname, s, len(upd), flush=True)
        chains[cname] = {"inputs_0": scenarios.bits_sha(states[0]), "steps": steps}
    return {"single": out, "chains": chains}


def main():
    torch.manual_seed(0)
    meta = {"reference": "Crukx-dev/crukx-sync 0.2.0", "torch": torch.__version__, "numpy": np.__version__}
    for fname, fn in (("huffman.json", huffman_cases), ("rice.json", rice_cases),
                      ("checksum.json", checksum_cases), ("updates.json", update_cases)):
        data = fn()
        data["meta"] = meta
        with open(os.path.join(HERE, fname), "w") as f:
            json.dump(data, f, separators=(",", ":"))
        print("wrote", fname, flush=True)


if __name__ == "__main__":
    main()
