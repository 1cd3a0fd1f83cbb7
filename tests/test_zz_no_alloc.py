"""GPU test of the allocation-free prefill (sparkmv_vq_prefill_noalloc)
against the pooled one (sparkmv_vq_prefill), through the C-ABI.

Both run the same kernels with the same K split; only where the split's
partial sums live differs (the library's fixed scratch array instead of its
memory pool), so the outputs must be equal bit for bit. Two calls in a row,
the second smaller, both splitting K: the second must not see the first's
leftovers. A call whose split slices exceed the array is refused with the
byte count, before any launch."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _call(sm, fn, m, x, y, accumulate):
    pp, keep = m._stages()
    h = m.host
    return fn(pp, h.nstages, h.dim, h.nc, h.rows, h.cols, h.v3, x.data_ptr(), sm.X_BF16, x.stride(0), x.shape[0],
              y.data_ptr(), y.stride(0), int(accumulate), None)


def test_noalloc_prefill_equals_pooled(sm, dev):
    import torch
    L = sm.lib()
    rows, cols = 2560, 10240
    m = sm.DeviceContainer(sm.synth_container(0x7A11, rows, cols), dev)
    for ntok in (512, 192):
        xb = sm.synth_bf16(0x7A12 + ntok, ntok * cols).reshape(ntok, cols)
        x = torch.from_numpy(xb.view(np.int16).copy()).to(dev)
        want = torch.zeros(ntok, rows, device=dev)
        sm.check(_call(sm, L.sparkmv_vq_prefill, m, x, want, False), "pooled prefill")
        got = torch.full((ntok, rows), float("nan"), device=dev)
        sm.check(_call(sm, L.sparkmv_vq_prefill_noalloc, m, x, got, False), "no-allocation prefill")
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{ntok} tokens: the no-allocation prefill differs"
        # accumulate: y += W x on top of what is there
        base = torch.from_numpy(np.random.default_rng(ntok).standard_normal((ntok, rows)).astype(np.float32)).to(dev)
        want2, got2 = base.clone(), base.clone()
        sm.check(_call(sm, L.sparkmv_vq_prefill, m, x, want2, True), "pooled prefill")
        sm.check(_call(sm, L.sparkmv_vq_prefill_noalloc, m, x, got2, True), "no-allocation prefill")
        torch.cuda.synchronize()
        assert torch.equal(got2, want2), f"{ntok} tokens, accumulate: the no-allocation prefill differs"


def test_noalloc_prefill_refuses_oversize(sm, dev):
    """4096 tokens of the 2560 x 10240 matrix split K two ways: 84 MB of
    partial sums, more than the 32 MiB array. Refused before any launch."""
    import torch
    L = sm.lib()
    rows, cols, ntok = 2560, 10240, 4096
    m = sm.DeviceContainer(sm.synth_container(0x7A13, rows, cols), dev)
    x = torch.zeros(ntok, cols, dtype=torch.int16, device=dev)
    y = torch.zeros(ntok, rows, device=dev)
    assert _call(sm, L.sparkmv_vq_prefill_noalloc, m, x, y, False) == -1
    msg = sm.last_error()
    assert "bytes of scratch" in msg and "holds 33554432" in msg, msg
