"""Named input scenarios shared by the golden-vector writer and the parity tests.

Each scenario builds (old, new) dicts of CPU tensors deterministically from torch's CPU
generator (or from fixed values), so the vectors in tests/golden can be checked again anywhere
this torch version runs. Scenario recipes mirror the cases the reference's own tests exercise
(tests/test_roundtrip.py in the reference): an Adam-like RL step, many tensors with unchanged
ones, every element changed, one group with more residuals than 15-bit codes, Rice edge cases,
a single element, extreme residuals, long unary runs, slab boundaries, and chained steps.
"""

from __future__ import annotations

import hashlib
import importlib.util
import os

import torch

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# loaded by path: the workload generator depends on torch only, and this module is also used
# where another package named crukx_sync is importable
_spec = importlib.util.spec_from_file_location(
    "crx_workloads", os.path.join(_ROOT, "crukx-sync_amd", "crukx_sync", "workloads.py"))
workloads = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(workloads)


def rl_pair(n=200_000, lr=1e-6, seed=0):
    """bf16 weights and the next broadcast after one Adam-like step of size lr * U(0.5, 1.5)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, generator=g) * 0.02
    step = lr * torch.sign(torch.randn(n, generator=g)) * (0.5 + torch.rand(n, generator=g))
    return w.bfloat16(), (w + step).bfloat16()


def bits_sha(d: dict) -> str:
    h = hashlib.sha256()
    for k, v in d.items():
        h.update(k.encode())
        h.update(v.contiguous().view(torch.int16).numpy().tobytes())
    return h.hexdigest()


def single_scenarios():
    """name -> (old, new) for one-update scenarios."""
    out = {}
    a, b = rl_pair()
    out["rl_200k"] = ({"w": a.view(400, 500)}, {"w": b.view(400, 500)})
    a, b = rl_pair(50_000, seed=1)
    out["many_tensors"] = ({"a": a, "same": a.clone(), "c": a[:777].clone()},
                           {"a": b, "same": a.clone(), "c": b[:777].clone()})
    g = torch.Generator().manual_seed(2)
    a = torch.randint(-32768, 32768, (5000,), generator=g, dtype=torch.int16)
    b = a ^ torch.randint(1, 32768, (5000,), generator=g, dtype=torch.int16)
    out["every_element_arbitrary"] = ({"w": a}, {"w": b})
    a = torch.full((200_000,), 0x3C00, dtype=torch.int16)
    b = torch.randint(-32768, 32768, (200_000,), generator=torch.Generator().manual_seed(4), dtype=torch.int16)
    out["distinct_residuals_200k"] = ({"w": a}, {"w": b})
    a = torch.full((1 << 20,), 0x3F80, dtype=torch.int16)
    dense, tail = a.clone(), a.clone()
    dense[:4096] += 1
    tail[-1] += 1
    out["rice_dense"] = ({"w": a}, {"w": dense})
    out["rice_tail"] = ({"w": a.clone()}, {"w": tail})
    out["single"] = ({"w": torch.tensor([0x3F80], dtype=torch.int16)}, {"w": torch.tensor([0x3F81], dtype=torch.int16)})
    out["extreme"] = ({"w": torch.tensor([0x7FFF, -0x8000, 0, 0x7FFF], dtype=torch.int16)},
                      {"w": torch.tensor([-0x8000, 0x7FFF, 0x7FFF, 0], dtype=torch.int16)})
    a = torch.full((1 << 20,), 0x3F80, dtype=torch.int16)
    b = a.clone()
    b[:2000] += 1
    b[-1] += 1
    out["long_unary"] = ({"w": a}, {"w": b})
    for n in (4096, 4097, 3 * 4096 + 5):
        a, b = rl_pair(n, seed=n)
        out[f"slab_{n}"] = ({"w": a}, {"w": b})
        c = a.clone()
        if not torch.equal(a[-1:], b[-1:]):
            c[-1] = b[-1]
        else:
            c[-1] = (c[-1:].view(torch.int16) + 1).view(torch.bfloat16)[0]
        out[f"slab_{n}_last"] = ({"w": a}, {"w": c})
    g = torch.Generator().manual_seed(11)
    old = {f"t{i}": (torch.randn(n, generator=g) * 0.02).bfloat16() for i, n in enumerate([5000, 300_000, 77])}
    new = {k: (v.float() + 3e-5 * torch.randn(v.shape, generator=g)).bfloat16() for k, v in old.items()}
    out["three_tensors"] = (old, new)
    sh = [("q.weight", (1536, 1536), "linear"), ("k.weight", (256, 1536), "linear"),
          ("k.bias", (256,), "linear"), ("norm.weight", (1536,), "norm")]
    base = workloads.make_weights(sh, seed=5)
    for rho in (0.005, 0.01, 0.02, 0.03):
        for p1 in (0.95, 0.87, 0.70):
            out[f"sweep_rho{rho}_p{p1}"] = (base, workloads.make_step(base, 1, rho=rho, p_one=p1, seed=5))
    edge = {k: v.clone() for k, v in workloads.make_weights(sh, seed=6).items()}
    workloads.inject_edges(edge, 0.01, seed=6)
    out["edges"] = (edge, workloads.make_step(edge, 1, rho=0.01, seed=6))
    return out


def chain_small4(steps=3):
    """Four tensors (26.6M weights), `steps` chained 1% steps: [state_0, state_1, ...]."""
    sh = workloads.small4_shapes()
    states = [workloads.make_weights(sh, seed=0)]
    for s in range(1, steps + 1):
        states.append(workloads.make_step(states[-1], s, rho=0.01, seed=0))
    return states


def chain_cache(steps=5):
    """300k weights, `steps` chained steps of +-1e-6 (the receiver/sender cache scenario)."""
    g = torch.Generator().manual_seed(7)
    w = torch.randn(300_000, generator=g) * 0.02
    states = [{"w": w.bfloat16()}]
    for _ in range(steps):
        w = w + 1e-6 * torch.sign(torch.randn(w.shape, generator=g))
        states.append({"w": w.bfloat16()})
    return states
