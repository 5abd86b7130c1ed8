"""GPU test of the allocation-free entry point hif8_modln_quant_static, through the C ABI.

It must give, bit for bit, the x_q of the entry points it stands in for -- hif8_modln_amax and
hif8_modln_fake_quant with caller-owned statistics and state -- on two calls in a row, the
second with a smaller input (fewer rows, another width, per-batch modulation, the other qdq
semantics), so that whatever the first call left in the static workspace cannot leak into the
second.  Inputs above the workspace's row limit are refused before any work is enqueued.
"""
from __future__ import annotations

import ctypes

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
MAX_ROWS = 131072


def _inputs(rows, dim, batches, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = (torch.randn(rows, dim, generator=g, device=DEV) * 2 + 0.25)
    x[:, :4] *= 25
    x = x.to(torch.bfloat16)
    shift = (torch.randn(batches, dim, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    scale = (torch.randn(batches, dim, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    return x, shift, scale


def _with_buffers(pkg, x, shift, scale, rpb, sem):
    """x_q from hif8_modln_amax + hif8_modln_fake_quant with caller-owned stats and state."""
    L = pkg._lib.load()
    s = pkg._lib.stream_ptr(x.device)
    rows, dim = x.shape
    stats = torch.empty(rows * 2, dtype=torch.float32, device=x.device)
    st = pkg.QuantState(x.device)
    xq = torch.empty_like(x)
    pkg._lib.check(L.hif8_modln_amax(x.data_ptr(), shift.data_ptr(), scale.data_ptr(), rows, dim, rpb, 1e-6,
                                     stats.data_ptr(), 15.0, st.ptr, s), "hif8_modln_amax")
    pkg._lib.check(L.hif8_modln_fake_quant(x.data_ptr(), shift.data_ptr(), scale.data_ptr(), rows, dim, rpb,
                                           stats.data_ptr(), st.ptr, sem, xq.data_ptr(), None, s),
                   "hif8_modln_fake_quant")
    return xq


def _static(pkg, x, shift, scale, rpb, sem):
    L = pkg._lib.load()
    rows, dim = x.shape
    xq = torch.empty_like(x)
    rc = L.hif8_modln_quant_static(x.data_ptr(), shift.data_ptr(), scale.data_ptr(), rows, dim, rpb,
                                   ctypes.c_float(1e-6), ctypes.c_float(15.0), sem, xq.data_ptr(),
                                   pkg._lib.stream_ptr(x.device))
    pkg._lib.check(rc, "hif8_modln_quant_static")
    return xq


def test_static_entry_point_matches_caller_buffers(pkg):
    # call 1: the 14B 720P block's q/k/v input (80640 padded rows x 5120), one modulation row
    print("[no_alloc] call 1: 80640 x 5120, NPU semantics", flush=True)
    x, shift, scale = _inputs(80640, 5120, 1, seed=1)
    got = _static(pkg, x, shift, scale, 80640, pkg._lib.SEM_NPU)
    want = _with_buffers(pkg, x, shift, scale, 80640, pkg._lib.SEM_NPU)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # call 2: smaller -- 3000 rows of width 1536, three batches with their own modulation rows,
    # torch semantics
    print("[no_alloc] call 2: 3000 x 1536, 3 batches, torch semantics", flush=True)
    x2, shift2, scale2 = _inputs(3000, 1536, 3, seed=2)
    got2 = _static(pkg, x2, shift2, scale2, 1000, pkg._lib.SEM_TORCH)
    want2 = _with_buffers(pkg, x2, shift2, scale2, 1000, pkg._lib.SEM_TORCH)
    torch.cuda.synchronize()
    assert torch.equal(got2.view(torch.int16), want2.view(torch.int16))
    # and the Python wrapper on the first input again
    got3 = pkg.modulated_norm_quant_static(x.view(1, 80640, 5120), shift.view(1, 1, 5120), scale.view(1, 1, 5120))
    assert torch.equal(got3.view(-1, 5120).view(torch.int16), want.view(torch.int16))


def test_static_entry_point_refuses_more_rows_than_its_workspace(pkg):
    L = pkg._lib.load()
    x = torch.zeros(16, 512, dtype=torch.bfloat16, device=DEV)
    rc = L.hif8_modln_quant_static(x.data_ptr(), None, None, MAX_ROWS + 1, 512, MAX_ROWS + 1, ctypes.c_float(1e-6),
                                   ctypes.c_float(15.0), 0, x.data_ptr(), pkg._lib.stream_ptr(x.device))
    assert rc == -5 and b"static workspace" in L.hif8_strerror(rc)
