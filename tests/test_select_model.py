"""The select pass's lane-level model (tests/select_model.py) on CPU: with the kernels' own window size,
copy count and list capacities, every change is recorded exactly once at its true position, with no
LDS or record access out of bounds, over slab sizes from one row to one whole slab, updates whose
targets span every exponent (several windows per slab), dense ones (lists read from HBM), and the
edge values of the workload generator.  A configuration known to read past its counters (32-exponent
windows with 8 copies, counts read by every lane) must be caught."""

import numpy as np
import pytest
import torch

import scenarios
import select_model


def _bits(t):
    return t.reshape(-1).contiguous().view(torch.int16).numpy().astype(np.int64) & 0xFFFF


def _arbitrary(n, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-32768, 32768, (n,), generator=g, dtype=torch.int16)
    return a, a ^ torch.randint(1, 32768, (n,), generator=g, dtype=torch.int16)


def _dense(n, rho, seed):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16).view(torch.int16)
    b = a.clone()
    m = torch.rand(n, generator=g) < rho
    b[m] += torch.randint(1, 4, (n,), generator=g, dtype=torch.int16)[m]
    return a, b


CASES = {
    "every_element_arbitrary": lambda: tuple(t["w"] for t in scenarios.single_scenarios()["every_element_arbitrary"]),
    "slab_12293": lambda: tuple(t["w"] for t in scenarios.single_scenarios()["slab_12293"]),
    "extreme": lambda: tuple(t["w"] for t in scenarios.single_scenarios()["extreme"]),
    "edges_norm": lambda: tuple(t["norm.weight"] for t in scenarios.single_scenarios()["edges"]),
    "arbitrary_20k": lambda: _arbitrary(20_000, 31),
    "dense_60pct": lambda: _dense(30_000, 0.6, 600),
}


@pytest.mark.parametrize("slab", [128, 4096, 65536])
@pytest.mark.parametrize("name", sorted(CASES))
def test_model_places_every_change(name, slab):
    a, b = CASES[name]()
    out = select_model.run(_bits(a), _bits(b), slab)
    assert out["changes"] == int((a != b).sum())


def test_model_reads_lists_from_hbm_when_they_do_not_fit():
    a, b = _dense(30_000, 0.6, 601)
    out = select_model.run(_bits(a), _bits(b), 65536, cap=1024)  # one window of ~18000 targets: the HBM list
    assert out["changes"] > 1024


def test_model_catches_counters_read_past_their_array():
    a, b = CASES["every_element_arbitrary"]()
    with pytest.raises(IndexError, match="cnt"):
        select_model.run(_bits(a), _bits(b), 4096, win=32, copies=8)


def test_model_runs_the_kernels_configuration():
    kc = select_model.kernel_constants()
    assert kc["win"] in (32, 64) and kc["copies"] in (4, 8) and kc["cap_sparse"] % 1024 == 0
