"""GPU parity of the FFN producer fusion (osp_next.py:873-877): the GELU + amax epilogue of
the up-projection, and HIF8FFN's fused forward.

- y = gelu_tanh(rnd(x_q w^T + b)) from the epilogue equals torch's bf16 GELU applied to the
  plain fused linear's output (the same accumulators) within one bf16 ulp; the GELU's tanh is
  the device library's, so exact equality is not guaranteed element by element.
- The amax folded into the state is exactly max|y| over the [M, N] output (padding rows and
  columns excluded) and its scale the reference rule's; the down-projection's quantisation
  with that state is bit-exact against a standalone _quant of y.
- HIF8FFN's fused forward matches the plain sequence within the linear tolerance."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def rel_errors(y, y_ref):
    y, y_ref = y.double(), y_ref.double()
    rms = y_ref.square().mean().sqrt()
    floor = torch.clamp(y_ref.abs(), min=1e-2 * float(rms))
    return float(((y - y_ref).abs() / floor).max()), float((y - y_ref).norm() / y_ref.norm())


def ulp_diff(a, b):
    """|bit distance| between two bf16 tensors of the same sign pattern (monotone encoding)."""
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    ai = torch.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = torch.where(bi < 0, -(bi & 0x7FFF), bi)
    return (ai - bi).abs()


@pytest.mark.parametrize("M,K,N", [(300, 256, 264), (777, 512, 1024), (2048, 1536, 8960), (1, 64, 8)])
def test_gelu_amax_epilogue(pkg, R, M, K, N):
    g = torch.Generator(device="cpu").manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    b = (torch.randn(N, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    packed = pkg.PackedWeight(w, 15.0)
    a, fmt, st = pkg.quantize_activation(x, 15.0, "bf16")
    y_st = pkg.QuantState(x.device)
    y = pkg.linear_fwd_gelu_amax(a, packed, b, y_st, 15.0)
    lin = pkg.linear_fwd(a, fmt, st, packed, b)
    want = torch.nn.functional.gelu(lin, approximate="tanh")
    d = ulp_diff(y, want)
    assert int(d.max()) <= 1 and float((d > 0).float().mean()) <= 1e-3, (int(d.max()), float((d > 0).float().mean()))
    # amax over exactly the [M, N] output, scale by the reference rule
    amax_bits, scale = y_st.read()
    assert amax_bits == int(y.view(torch.int16).cpu().numpy().view(np.uint16).__and__(0x7FFF).max())
    sb = R.hif8_scale_bf16(amax_bits, 15.0)
    assert np.float32(scale) == R.bf16_to_f32(np.array([sb], np.uint16))[0]
    # the down-projection's quantisation with this state is _quant(y)
    yq = pkg.fake_quant(y, y_st)
    yq_ref, _ = pkg._quant(y, 15.0)
    assert torch.equal(yq.view(torch.int16), yq_ref.view(torch.int16))


def test_state_reuse_across_calls(pkg):
    """The epilogue resets its accumulators: a second, smaller call leaves the second amax."""
    g = torch.Generator(device="cpu").manual_seed(7)
    w = (torch.randn(256, 128, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    packed = pkg.PackedWeight(w, 15.0)
    y_st = pkg.QuantState(DEV)
    for M, mult in ((1000, 8.0), (300, 1.0)):
        x = (torch.randn(M, 128, generator=g) * mult).to(torch.bfloat16).to(DEV)
        a, _, _ = pkg.quantize_activation(x, 15.0, "bf16")
        y = pkg.linear_fwd_gelu_amax(a, packed, None, y_st, 15.0)
        amax_bits, _ = y_st.read()
        assert amax_bits == int(y.view(torch.int16).cpu().numpy().view(np.uint16).__and__(0x7FFF).max())


@pytest.mark.parametrize("dim,ffn,M", [(512, 1536, 600), (1536, 8960, 2048)])
def test_hif8ffn_fused_forward(pkg, dim, ffn, M):
    torch.manual_seed(dim)
    mod = pkg.HIF8FFN(dim, ffn, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        for p in mod.parameters():
            p.normal_(0, 0.02)
    x = torch.randn(2, M // 2, dim, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        assert mod.fused_ok(x)
        y = mod(x)
        y_seq = torch.nn.Sequential.forward(mod, x)
    assert y.shape == (2, M // 2, dim) and y.dtype == torch.bfloat16
    elem, norm = rel_errors(y, y_seq)
    assert elem <= 1e-2 and norm <= 4e-3, (elem, norm)
    # and with autograd the module runs the plain sequence
    x.requires_grad_(True)
    assert not mod.fused_ok(x)
    mod(x).float().sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad.float()).all()
