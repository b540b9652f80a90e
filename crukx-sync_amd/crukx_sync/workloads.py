"""Synthetic bf16 state dicts and RL-like update steps (Qwen2.5-shaped), for tests and benchmarks.

Weights: linear weights, biases and embeddings ~ N(0, 0.02); norm weights ~ N(1, 0.05); rounded
to bf16 with round-to-nearest-even (torch's float32 -> bfloat16 cast).

Change model for one step, per tensor: let e be the 8-bit exponent field of the old bf16 bits and
m the tensor's median exponent. A weight changes with probability p_e = min(1, c * 2^(-(e-m)/2)),
c found by bisection so the expected changed fraction is rho. A change moves the 15-bit magnitude
by d = +-k (sign +-1 with probability 1/2), |k| = 1 with probability p_one, else 1 + G with G
geometric on {1, 2, ...} with success probability 1/2. A zero magnitude becomes magnitude 1 with a
random sign; a result at or above exponent 0xFF uses +-1 instead (-1 for max-finite); a result
below 0 uses magnitude - 1. The sign bit is kept.

Everything is torch tensor ops, so the same code runs on CPU (fixtures, small tests) and on the
GPU (large benchmarks). Random streams are per tensor and per step (seeded torch Generators); a
CPU run and a GPU run of the same seed draw different numbers.
"""

from __future__ import annotations

import math

import torch

_MIX = 0x9E3779B97F4A7C15


def _seed(*parts: int) -> int:
    """A 63-bit seed from integers (splitmix64 finaliser over a running mix)."""
    z = 0
    for p in parts:
        z = (z + (p & 0xFFFFFFFFFFFFFFFF) + _MIX) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        z ^= z >> 31
    return z & 0x7FFFFFFFFFFFFFFF


def _gen(device, *parts: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(_seed(*parts))
    return g


# ------------------------------------------------------------------ shapes

QWEN25 = {
    # name: (layers, hidden, kv_dim, intermediate, vocab, tied embedding)
    "qwen2.5-1.5b": (28, 1536, 256, 8960, 151936, True),
    "qwen2.5-7b": (28, 3584, 512, 18944, 152064, False),
    "qwen2.5-32b": (64, 5120, 1024, 27648, 152064, False),
}


def qwen25_shapes(model: str) -> list[tuple[str, tuple[int, ...], str]]:
    """(name, shape, kind) in Hugging Face Qwen2 state-dict order; kind is 'linear' or 'norm'."""
    layers, h, kv, inter, vocab, tied = QWEN25[model]
    out = [("model.embed_tokens.weight", (vocab, h), "linear")]
    for i in range(layers):
        p = f"model.layers.{i}."
        out += [
            (p + "self_attn.q_proj.weight", (h, h), "linear"),
            (p + "self_attn.q_proj.bias", (h,), "linear"),
            (p + "self_attn.k_proj.weight", (kv, h), "linear"),
            (p + "self_attn.k_proj.bias", (kv,), "linear"),
            (p + "self_attn.v_proj.weight", (kv, h), "linear"),
            (p + "self_attn.v_proj.bias", (kv,), "linear"),
            (p + "self_attn.o_proj.weight", (h, h), "linear"),
            (p + "mlp.gate_proj.weight", (inter, h), "linear"),
            (p + "mlp.up_proj.weight", (inter, h), "linear"),
            (p + "mlp.down_proj.weight", (h, inter), "linear"),
            (p + "input_layernorm.weight", (h,), "norm"),
            (p + "post_attention_layernorm.weight", (h,), "norm"),
        ]
    out.append(("model.norm.weight", (h,), "norm"))
    if not tied:
        out.append(("lm_head.weight", (vocab, h), "linear"))
    return out


def small4_shapes() -> list[tuple[str, tuple[int, ...], str]]:
    """Four tensors, 26,611,713 weights; the 1-D one is not a multiple of 256."""
    return [
        ("layer.proj.weight", (4096, 4096), "linear"),
        ("layer.down.weight", (4096, 1024), "linear"),
        ("layer.mlp.weight", (11008, 512), "linear"),
        ("layer.norm.weight", (4097,), "norm"),
    ]


def shapes_for(workload: str):
    if workload == "small4":
        return small4_shapes()
    return qwen25_shapes(workload)


# ------------------------------------------------------------------ weights

def make_weights(shapes, seed: int = 0, device="cpu") -> dict[str, torch.Tensor]:
    """bf16 state dict: linear ~ N(0, 0.02), norm ~ N(1, 0.05), round-to-nearest-even."""
    out = {}
    for i, (name, shape, kind) in enumerate(shapes):
        g = _gen(device, 1, seed, i)
        x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
        if kind == "norm":
            x.mul_(0.05).add_(1.0)
        else:
            x.mul_(0.02)
        out[name] = x.to(torch.bfloat16)
        del x
    return out


# ------------------------------------------------------------------ change model

def _median_exponent(hist: list[int], n: int) -> int:
    """Lower median of the exponent field (torch.median's convention)."""
    k, acc = (n - 1) // 2, 0
    for e, c in enumerate(hist):
        acc += c
        if acc > k:
            return e
    return 255


def change_probabilities(hist: list[int], rho: float) -> list[float]:
    """p_e = min(1, c * 2^(-(e-m)/2)) with c chosen so sum_e hist[e] * p_e = rho * n."""
    n = sum(hist)
    if n == 0 or rho <= 0:
        return [0.0] * 256
    m = _median_exponent(hist, n)
    f = [2.0 ** (-(e - m) / 2.0) for e in range(256)]
    target = min(rho, 1.0) * n

    def expected(c):
        return sum(h * min(1.0, c * fe) for h, fe in zip(hist, f) if h)

    lo, hi = 0.0, 1.0
    while expected(hi) < target and hi < 1e300:
        hi *= 2.0
    for _ in range(200):
        mid = 0.5 * (lo + hi)
        if expected(mid) < target:
            lo = mid
        else:
            hi = mid
    return [min(1.0, hi * fe) for fe in f]


def step_bits(bits: torch.Tensor, rho: float, p_one: float, g: torch.Generator) -> torch.Tensor:
    """One RL-like step on a flat int16 bit tensor; returns the new int16 bits."""
    n = bits.numel()
    x = bits.to(torch.int32)
    mag = x & 0x7FFF
    exp = mag >> 7
    hist = torch.bincount(exp.view(-1), minlength=256).tolist()
    p = torch.tensor(change_probabilities(hist, rho), dtype=torch.float32, device=bits.device)
    u = torch.rand(n, generator=g, device=bits.device)
    changed = u < p[exp]
    del u
    changed &= mag < 0x7F80  # never step inf/nan patterns
    idx = torch.nonzero(changed).view(-1)
    del changed
    c = idx.numel()
    if c == 0:
        return bits.clone()
    m = mag[idx]
    s = x[idx] & 0x8000
    v = torch.rand(c, generator=g, device=bits.device)
    w = 1.0 - torch.rand(c, generator=g, device=bits.device)          # (0, 1]
    sg = torch.rand(c, generator=g, device=bits.device) < 0.5
    geo = torch.floor(-torch.log2(w)).to(torch.int32) + 1              # 1, 2, ... with P = 2^-G
    k = torch.where(v < p_one, torch.ones_like(geo), 1 + geo)
    d = torch.where(sg, k, -k)
    nm = m + d
    pm1 = torch.where(d > 0, m + 1, m - 1)
    nm = torch.where(nm >= 0x7F80, torch.where(pm1 >= 0x7F80, m - 1, pm1), nm)
    nm = torch.where(nm < 0, m - 1, nm)
    zero = m == 0
    nm = torch.where(zero, torch.ones_like(nm), nm)
    s = torch.where(zero, torch.where(sg, 0, 0x8000), s)
    out = bits.clone()
    out[idx] = (s | nm).to(torch.int16)
    return out


def make_step(prev: dict[str, torch.Tensor], step: int, rho: float = 0.01, p_one: float = 0.87,
              seed: int = 0) -> dict[str, torch.Tensor]:
    """The next broadcast after one synthetic RL step: same names, shapes and dtypes as prev."""
    out = {}
    for i, (name, t) in enumerate(prev.items()):
        g = _gen(t.device, 2, seed, step, i)
        nb = step_bits(t.view(torch.int16).reshape(-1), rho, p_one, g)
        out[name] = nb.view(t.dtype).view(t.shape)
    return out


def inject_edges(state: dict[str, torch.Tensor], density: float, seed: int = 0) -> None:
    """In place: set a fraction of weights to +0, -0, a random subnormal or +-max-finite."""
    for i, (name, t) in enumerate(state.items()):
        g = _gen(t.device, 3, seed, i)
        b = t.view(torch.int16).view(-1)
        n = b.numel()
        sel = torch.nonzero(torch.rand(n, generator=g, device=t.device) < density).view(-1)
        if sel.numel() == 0:
            continue
        kind = torch.randint(0, 4, (sel.numel(),), generator=g, device=t.device)
        sub = torch.randint(1, 0x80, (sel.numel(),), generator=g, device=t.device, dtype=torch.int32)
        sgn = torch.randint(0, 2, (sel.numel(),), generator=g, device=t.device, dtype=torch.int32) << 15
        val = torch.where(kind == 0, torch.zeros_like(sub), torch.full_like(sub, 0x8000))
        val = torch.where(kind == 2, sgn | sub, val)
        val = torch.where(kind == 3, sgn | 0x7F7F, val)
        b[sel] = val.to(torch.int16)


def numel(shapes) -> int:
    return sum(math.prod(s) for _, s, _ in shapes)
