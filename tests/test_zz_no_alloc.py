"""crx_checksum_noalloc (the allocation-free variant of crx_checksum) through the C ABI.

Its partial sums live in a static per-device array that every call reuses, so two calls in a row,
the second over fewer elements (fewer partial sums than the first left behind), must both equal
crx_checksum's result and the oracle's.
"""

import ctypes

import pytest
import torch

import oracle
from crukx_sync import _native


def _noalloc(t: torch.Tensor) -> int:
    out = ctypes.c_uint64(0xDEADBEEF)
    err = _native.errbuf()
    rc = _native.lib().crx_checksum_noalloc(t.data_ptr(), t.numel(), _native.stream_of(t.device),
                                           ctypes.byref(out), err, 512)
    _native.raise_for(rc, err)
    return out.value


def _with_alloc(t: torch.Tensor) -> int:
    ws = _native.Workspace(t.device)
    out = ctypes.c_uint64(0)
    err = _native.errbuf()
    rc = _native.lib().crx_checksum(t.data_ptr(), t.numel(), _native.stream_of(t.device), ws.fn, None,
                                    ctypes.byref(out), err, 512)
    ws.check()
    _native.raise_for(rc, err)
    return out.value


def test_rejects_sizes_beyond_the_limit_before_any_device_work():
    """n >= 2^32 is refused before the data pointer is touched (so no device is needed)."""
    buf = (ctypes.c_uint16 * 4)()
    out = ctypes.c_uint64(7)
    err = _native.errbuf()
    rc = _native.lib().crx_checksum_noalloc(ctypes.addressof(buf), 1 << 32, None, ctypes.byref(out), err, 512)
    assert rc == _native.INVALID and out.value == 0
    assert b"2^32" in err.value


@pytest.mark.gpu
def test_noalloc_checksum_equals_crx_checksum_on_consecutive_calls():
    g = torch.Generator().manual_seed(11)
    big = torch.randint(-32768, 32768, (150_000_001,), generator=g, dtype=torch.int16)
    small = torch.randint(-32768, 32768, (300_007,), generator=g, dtype=torch.int16)
    dbig, dsmall = big.cuda(), small.cuda()
    for t_dev, t_host in ((dbig, big), (dsmall, small)):  # the second call uses fewer partial sums
        got = _noalloc(t_dev)
        assert got == _with_alloc(t_dev)
        assert got == oracle.checksum(t_host)
    # odd 16-bit start (not 32-bit aligned), then a single element, then the large input again
    assert _noalloc(dsmall[1:]) == _with_alloc(dsmall[1:]) == oracle.checksum(small[1:])
    assert _noalloc(dsmall[5:6]) == oracle.checksum(small[5:6])
    assert _noalloc(dbig) == oracle.checksum(big)
