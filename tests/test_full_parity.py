"""Encode bytes of the HIP path equal the oracle's at the workloads' full tensor sizes, on the GPU.

A round trip cannot tell a different-but-valid Rice parameter, Huffman table or tie-break from the
reference's choice: the decoder reads those from the header.  So here the bytes themselves are
compared with the oracle's (the C restatement of the reference, pinned to the reference's own bytes
by tests/test_oracle.py), on the same inputs moved to the host in the same process:

- the first step of the Qwen2.5-1.5B-shaped chain, every tensor (1,543,714,304 weights), cold;
- Qwen2.5-7B-shaped embedding, decoder layer 0 and lm_head (1,323,052,544 weights): a cold step at
  rho = 1%, then a step at rho = 2% with the sender's checksum cache from the first;
- Qwen2.5-32B-shaped embedding and decoder layer 0 (1,266,172,928 weights) with edge values (+-0,
  subnormals, +-max-finite) at 1e-4 density in both states and 16K-element slabs.

These shapes hold the largest tensors of the workloads (the 545M- and 779M-weight embeddings), so
every size-dependent path runs here: many slabs per tensor, the rank pass's record regions, tens of
millions of changes per exponent in the dense and rare symbol counts, multi-window select slabs.
"""

import pytest
import torch

import crukx_sync
import oracle
from crukx_sync import codec, workloads

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(autouse=True)
def _free_memory():
    torch.cuda.empty_cache()
    yield
    torch.cuda.empty_cache()


def _host(d):
    return {k: v.cpu() for k, v in d.items()}


def _same_bytes_as_oracle(prev, cur, send_hip, send_orc, what):
    """HIP encode (bytes API and device-resident bytes) == oracle encode, and equal sender caches."""
    hip = crukx_sync.encode_update(prev, cur, send_hip)
    hp, hc = _host(prev), _host(cur)
    ref = oracle.encode_update(hp, hc, send_orc)
    assert len(hip) == len(ref), (what, len(hip), len(ref))
    if hip != ref:
        first = next(i for i, (x, y) in enumerate(zip(hip, ref)) if x != y)
        raise AssertionError(f"{what}: first differing byte at {first} of {len(ref)}")
    assert send_hip == send_orc, what
    _say(f"{what}: {len(hip):,} bytes identical to the oracle's")
    return hip


def _shapes(model, keep):
    out = [s for s in workloads.qwen25_shapes(model) if keep(s[0])]
    return out


def test_qwen25_1_5b_first_step_bytes_equal_oracle():
    shapes = workloads.qwen25_shapes("qwen2.5-1.5b")
    assert workloads.numel(shapes) == 1_543_714_304
    prev = workloads.make_weights(shapes, seed=0, device="cuda")
    cur = workloads.make_step(prev, 1, rho=0.01)
    _same_bytes_as_oracle(prev, cur, {}, {}, "1.5b step 1")


def test_qwen25_7b_largest_tensors_bytes_equal_oracle():
    shapes = _shapes("qwen2.5-7b", lambda n: n in ("model.embed_tokens.weight", "lm_head.weight")
                     or n.startswith("model.layers.0."))
    assert workloads.numel(shapes) == 1_323_052_544
    p0 = workloads.make_weights(shapes, seed=0, device="cuda")
    p1 = workloads.make_step(p0, 1, rho=0.01)
    send_hip, send_orc = {}, {}
    _same_bytes_as_oracle(p0, p1, send_hip, send_orc, "7b subset rho 1% (cold)")
    del p0
    p2 = workloads.make_step(p1, 2, rho=0.02)
    _same_bytes_as_oracle(p1, p2, send_hip, send_orc, "7b subset rho 2% (cached)")


def test_qwen25_32b_largest_tensors_with_edges_bytes_equal_oracle(monkeypatch):
    monkeypatch.setattr(codec, "_SLAB", 1 << 14)
    shapes = _shapes("qwen2.5-32b", lambda n: n == "model.embed_tokens.weight" or n.startswith("model.layers.0."))
    assert workloads.numel(shapes) == 1_266_172_928
    p0 = workloads.make_weights(shapes, seed=4, device="cuda")
    workloads.inject_edges(p0, 1e-4, seed=1)
    p1 = workloads.make_step(p0, 1, rho=0.01, seed=4)
    workloads.inject_edges(p1, 1e-4, seed=2)
    _same_bytes_as_oracle(p0, p1, {}, {}, "32b subset with edges, 16K slabs")
