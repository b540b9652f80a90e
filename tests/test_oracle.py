"""The CPU oracle against the reference's golden vectors and against what the mathematics fixes.

The oracle is the parity checker for the HIP path, so it is pinned here first: SplitMix64's
published seed-0 outputs, the vectors the reference itself wrote (tests/golden/make_golden.py),
Kraft/prefix properties, the malformed updates of the reference's tests (as data, in
tests/golden/hostile_headers.json), and the single-byte-flip invariant.
"""

import hashlib
import json
import os

import numpy as np
import pytest
import torch

import oracle
import scenarios


def test_splitmix64_published_vectors():
    # SplitMix64 seeded with 0: the first outputs are splitmix64 of the counter 1, 2, 3, 4
    expect = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F5, 0x06C45D188009454F, 0xF88BB8A8724C81ED]
    assert [oracle.weight(i) for i in range(4)] == [w | 1 for w in expect]


def test_checksum_vectors(golden):
    C = golden["checksum"]
    assert [oracle.weight(i) for i in C["weights"]["index"]] == C["weights"]["w"]
    arrays = {"single_3f81": np.array([0x3F81], np.uint16), "arange_65536": np.arange(65536, dtype=np.uint16),
              "zeros_1000": np.zeros(1000, np.uint16), "ffff_777": np.full(777, 0xFFFF, np.uint16),
              "random_3000001_seed5": np.random.default_rng(5).integers(0, 65536, 3_000_001).astype(np.uint16)}
    for c in C["cases"]:
        assert oracle.checksum(arrays[c["name"]]) == c["checksum"], c["name"]
    # closed form: a single element u at index 0 contributes u * w_0
    assert oracle.checksum(np.array([0x3F81], np.uint16)) == (0x3F81 * oracle.weight(0)) % (1 << 64)


def test_huffman_lengths_and_codes(golden):
    for c in golden["huffman"]["cases"]:
        L = oracle.huffman_lengths(c["counts"])
        assert L == c["lengths"], c["counts"][:8]
        assert oracle.canonical_codes(L) == c["codes"]
        assert sum(2.0 ** -x for x in L) <= 1.0 + 1e-12 and max(L) <= 17


def test_huffman_large_tables(golden):
    for b in golden["huffman"]["big"]:
        cnt = [int(x) for x in np.random.default_rng(b["seed"]).integers(1, b["hi"], b["n"])]
        assert hashlib.sha256(json.dumps(cnt).encode()).hexdigest() == b["counts_sha"]
        L = oracle.huffman_lengths(cnt)
        assert hashlib.sha256(json.dumps(L).encode()).hexdigest() == b["lengths_sha"], b["n"]


def test_huffman_is_optimal_on_tiny_inputs():
    """Unlimited Huffman lengths minimise sum(count * length) over all prefix codes (brute force)."""
    import itertools
    rng = np.random.default_rng(3)
    for n in range(2, 6):
        for _ in range(20):
            counts = [int(x) for x in rng.integers(1, 50, n)]
            L = oracle.huffman_lengths(counts)
            best = min(sum(c * l for c, l in zip(counts, ls))
                       for ls in itertools.product(range(1, n), repeat=n) if sum(2.0 ** -x for x in ls) <= 1)
            assert sum(c * l for c, l in zip(counts, L)) == best


def test_canonical_codes_are_prefix_free():
    rng = np.random.default_rng(8)
    for n in (2, 3, 17, 100):
        L = oracle.huffman_lengths([int(x) for x in rng.integers(1, 1000, n)])
        codes = oracle.canonical_codes(L)
        words = [format(c, f"0{l}b") for c, l in zip(codes, L)]
        for i, a in enumerate(words):
            for j, b in enumerate(words):
                assert i == j or not b.startswith(a)


def test_rice_parameter_choice(golden):
    for c in golden["rice"]["cases"]:
        assert oracle.rice_param(c["gaps"]) == c["rice"], c["gaps"][:4]


def test_rice_choice_is_cheapest_of_three():
    rng = np.random.default_rng(4)
    for _ in range(50):
        g = rng.geometric(1 / (1 + rng.integers(1, 5000)), 200) - 1
        r = oracle.rice_param(g)
        cost = lambda k: int(((g >> k) + 1 + k).sum())  # noqa: E731
        r0 = int(np.clip(np.floor(np.log2(max(g.mean(), 1))), 0, 30))
        cands = [max(r0 - 1, 0), r0, min(r0 + 1, 30)]
        assert r in cands and cost(r) == min(cost(k) for k in cands)


@pytest.mark.parametrize("name", sorted(scenarios.single_scenarios().keys()))
def test_encode_matches_reference_bytes(golden, name):
    old, new = scenarios.single_scenarios()[name] if name not in _CACHE else _CACHE[name]
    rec = golden["updates"]["single"][name]
    assert scenarios.bits_sha(old) == rec["inputs_old"] and scenarios.bits_sha(new) == rec["inputs_new"]
    chk = {}
    upd = oracle.encode_update(old, new, chk)
    assert len(upd) == rec["update"]["len"]
    if "hex" in rec["update"]:
        assert upd.hex() == rec["update"]["hex"]
    assert hashlib.sha256(upd).hexdigest() == rec["update"]["sha256"]
    assert chk == rec["sender_checksums"]
    w = {k: v.clone() for k, v in old.items()}
    assert oracle.apply_update(w, upd) == sum(int((old[k].view(torch.int16) != new[k].view(torch.int16)).sum()) for k in old)
    for k in new:
        assert torch.equal(w[k].view(torch.int16), new[k].view(torch.int16)), k


_CACHE = {}


@pytest.fixture(scope="module", autouse=True)
def _scenarios_once():
    _CACHE.update(scenarios.single_scenarios())
    yield
    _CACHE.clear()


@pytest.mark.parametrize("chain", ["small4_chain", "cache_chain"])
def test_chained_updates_with_caches(golden, chain):
    states = scenarios.chain_small4(3) if chain == "small4_chain" else scenarios.chain_cache(5)
    rec = golden["updates"]["chains"][chain]
    assert scenarios.bits_sha(states[0]) == rec["inputs_0"]
    send, recv = {}, {}
    w = {k: v.clone() for k, v in states[0].items()}
    for s in range(1, len(states)):
        upd = oracle.encode_update(states[s - 1], states[s], send)
        assert hashlib.sha256(upd).hexdigest() == rec["steps"][s - 1]["update"]["sha256"]
        assert send == rec["steps"][s - 1]["sender_checksums"]
        oracle.apply_update(w, upd, recv)
        for k in w:
            assert torch.equal(w[k].view(torch.int16), states[s][k].view(torch.int16))
    assert send == recv


def hostile_updates():
    """The malformed updates of the reference's own tests, as data (tests/golden/hostile_headers.json)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hostile_headers.json")
    return [bytes.fromhex(c["hex"]) for c in json.load(open(path))["cases"]]


def test_hostile_headers_are_rejected():
    for h in hostile_updates():
        with pytest.raises(oracle.OracleCorrupt):
            oracle.parse_check(h)
        w = {"w": np.zeros(100, np.uint16)}
        with pytest.raises(oracle.OracleCorrupt):
            oracle.apply_update(w, h)
        assert not w["w"].any()


def test_every_single_byte_flip_is_rejected_or_exact(golden):
    old, new = scenarios.rl_pair(3000, seed=6)
    upd = oracle.encode_update({"w": old}, {"w": new})
    for i in range(len(upd)):
        for x in (0x01, 0x80, 0xFF):
            bad = bytearray(upd)
            bad[i] ^= x
            w = {"w": old.clone()}
            try:
                oracle.apply_update(w, bytes(bad))
            except ValueError:
                assert torch.equal(w["w"].view(torch.int16), old.view(torch.int16))
            else:
                assert torch.equal(w["w"].view(torch.int16), new.view(torch.int16))


def test_empty_and_unchanged():
    a = np.arange(10, dtype=np.uint16)
    assert oracle.encode_update({}, {}) == b"CRXS\x02\x00\x00\x00"
    assert oracle.encode_update({"w": a}, {"w": a.copy()}) == b"CRXS\x02\x00\x00\x00"
    assert oracle.apply_update({"w": a}, b"CRXS\x02\x00\x00\x00") == 0
