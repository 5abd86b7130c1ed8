"""GPU parity of the fp32-input operand route: ``_quant`` of an fp32 tensor (the
self-attention ``o`` input of the reference, osp_next.py:644 / attention.py:518) handed to the
bf16 GEMM as its autocast rounding (hif8_fake_quant_to_bf16), and the same for a bf16 tensor
quantised as x.float() would be (HIF8_DTYPE_BF16_AS_F32).  Every x_q and code is compared bit
for bit with the CPU oracle's fp32 _quant (hif8_ref.quant_f32), the linear within the linear
tolerance."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def f32_input(seed, n, scale=1.0, tiny=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, generator=g) * scale
    if tiny and n > 64:
        x[::37] *= 1e-7            # below 2^-22 after scaling: the two semantics' tails
        x[5] = 0.0
        x[11] = -0.0
    return x


def bits32(t):
    return t.detach().cpu().contiguous().view(torch.int32).numpy().view(np.uint32)


def bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("n", [4096 * 5, 1000003, 17])
@pytest.mark.parametrize("sem", ["npu", "torch"])
def test_f32_to_bf16_operand(pkg, R, n, sem):
    semc = pkg._lib.SEM_NPU if sem == "npu" else pkg._lib.SEM_TORCH
    x = f32_input(n, n, 3.0)
    xd = x.to(DEV)
    st = pkg.absmax_scale(xd, 15.0, pkg.QuantState(DEV))
    got = pkg.fake_quant_to_bf16(xd, st, semc)
    xq, s = R.quant_f32(x.numpy(), 15.0, sem)
    assert np.array_equal(bits16(got), R.f32_to_bf16(xq))
    # and the fp32 x_q the same state gives is the oracle's
    assert np.array_equal(bits32(pkg.fake_quant(xd, st, semc)), xq.view(np.uint32))


@pytest.mark.parametrize("n", [4096 * 5, 1000003, 17])
def test_bf16_quantised_as_f32(pkg, R, n):
    x = f32_input(n + 1, n, 2.0).to(torch.bfloat16)
    xd = x.to(DEV)
    st = pkg.absmax_scale(xd, 15.0, pkg.QuantState(DEV), as_f32=True)
    st_ref = pkg.absmax_scale(xd.float(), 15.0, pkg.QuantState(DEV))
    a, s = st.read()
    a_ref, s_ref = st_ref.read()
    assert a == a_ref and s == s_ref
    assert np.float32(s) == R.hif8_scale_f32(R.absmax_f32(x.float().numpy()), 15.0)
    xq, _ = R.quant_f32(x.float().numpy(), 15.0, "npu")
    assert np.array_equal(bits16(pkg.fake_quant_to_bf16(xd, st, as_f32=True)), R.f32_to_bf16(xq))
    codes = pkg.encode(xd, st, as_f32=True)
    assert torch.equal(codes, pkg.encode(xd.float(), st_ref))
    assert np.array_equal(bits32(pkg.decode(codes, st, torch.float32)), xq.view(np.uint32))


def test_degenerate_states(pkg, R):
    """amax 0 (scale from the 1e-8 clamp) and an Inf element (scale 0: the scalar route).  Where
    x * scale is NaN (Inf * 0) the Ascend kernel's select order gives -Inf
    (hif8_quant_op.h:143-150), and -Inf / 0 stays -Inf: the library follows it."""
    for x in (torch.zeros(1000), torch.tensor([1.0, float("inf"), -2.0] * 100)):
        xd = x.to(DEV)
        st = pkg.absmax_scale(xd, 15.0, pkg.QuantState(DEV))
        got = bits16(pkg.fake_quant_to_bf16(xd, st))
        xq, s = R.quant_f32(x.numpy(), 15.0, "npu")
        with np.errstate(all="ignore"):
            nan_in = np.isnan(x.numpy() * np.float32(s))
        want = R.f32_to_bf16(xq)
        nan = (want & 0x7FFF) > 0x7F80
        assert np.array_equal(got[~nan], want[~nan]) and np.all((got[nan] & 0x7FFF) > 0x7F80)
        assert np.all(got[nan_in] == 0xFF80)


def test_linear_fp32_input(pkg, R):
    """HIF8Linear with fp32 input: the fused bf16 GEMM on bf16(x_q); forward_f32_of_bf16 of a bf16
    tensor equals forward of its fp32 copy bit for bit."""
    M, K, N = 700, 512, 384
    g = torch.Generator().manual_seed(3)
    xb = torch.randn(M, K, generator=g).to(torch.bfloat16)
    lin = pkg.HIF8Linear(K, N, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16))
        lin.bias.copy_((torch.randn(N, generator=g) * 0.1).to(torch.bfloat16))
        y32 = lin(xb.to(DEV).float())
        y16 = lin.forward_f32_of_bf16(xb.to(DEV))
    assert torch.equal(y32.view(torch.int16), y16.view(torch.int16))
    xq, _ = R.quant_f32(xb.float().numpy(), 15.0, "npu")
    xq = R.bf16_to_f32(R.f32_to_bf16(xq)).astype(np.float64)
    wq = R.bf16_to_f32(R.quant_bf16(bits16(lin.weight), 15.0)[0]).astype(np.float64)
    yref = xq @ wq.T + R.bf16_to_f32(bits16(lin.bias)).astype(np.float64)
    err = np.abs(y32.float().cpu().numpy() - yref).max() / np.abs(yref).max()
    assert err < 1e-2, err
    # with autograd the forward result is the same, and the backward sees the fp32 x_q
    x = xb.to(DEV).float().requires_grad_(True)
    y = lin(x)
    assert torch.equal(y.detach().view(torch.int16), y32.view(torch.int16))
    y.float().sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all() and torch.isfinite(lin.weight.grad.float()).all()
