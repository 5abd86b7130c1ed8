"""GPU parity of the QLinear API (ospnext/quant_cy_npu/layers/QLinear.py) and of the
packed-weight files.

QLinear applies the raw HiF8 qdq (no per-tensor scale) to x, W and the output
gradient; its quantised operands are checked bit for bit against the CPU restatement
and its products against fp32 torch on them.  Packed files must reproduce the
prepacked module's output bit for bit."""
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


def raw_qdq_bf16(R, t):
    """quant_dequant_float(t, QType('hif8'), force_fp32=True) for bf16 t: fp32 qdq, back to bf16."""
    bits = t.detach().cpu().view(torch.int16).numpy().view(np.uint16)
    q = R.f32_to_bf16(R.quant_hif8_npu(R.bf16_to_f32(bits)))
    return torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).reshape(t.shape)


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("quant_grad", [True, False])
def test_qlinear_forward_backward(pkg, R, fast, quant_grad):
    torch.manual_seed(0)
    lin = pkg.QLinear(256, 192, bias=True).to(DEV).to(torch.bfloat16)
    lin.assign_qparams("hif8")
    lin.set_quant_grad(quant_grad)
    lin._fast_forward = fast
    g = torch.Generator(device="cpu").manual_seed(1)
    x = (torch.randn(3, 50, 256, generator=g) * 4).to(torch.bfloat16).to(DEV).requires_grad_(True)
    y = lin(x)
    xq, wq = raw_qdq_bf16(R, x), raw_qdq_bf16(R, lin.weight)
    ref = xq.float() @ wq.float().t() + lin.bias.detach().cpu().float()
    elem, norm = rel_errors(y.cpu(), ref)
    assert elem <= 1e-2 and norm <= 4e-3, (elem, norm)
    gy = torch.randn(y.shape, generator=g).to(torch.bfloat16)
    y.backward(gy.to(DEV))
    gq = raw_qdq_bf16(R, gy) if quant_grad else gy
    gx = gq.float() @ wq.float()
    gw = gq.reshape(-1, 192).float().t() @ xq.reshape(-1, 256).float()
    gb = gy.reshape(-1, 192).float().sum(0)
    for got, want in ((x.grad, gx), (lin.weight.grad, gw), (lin.bias.grad, gb)):
        elem, norm = rel_errors(got.cpu(), want)
        assert norm <= 4e-3, norm


def test_replace_linear(pkg):
    net = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.GELU(), torch.nn.Linear(128, 64))
    net = net.to(DEV).to(torch.bfloat16)
    w0 = net[0].weight.detach().clone()
    pkg.replace_linear(net, "hif8", exclude_layers=["2"])
    assert isinstance(net[0], pkg.QLinear) and not isinstance(net[2], pkg.QLinear)
    assert torch.equal(net[0].weight.detach(), w0) and net[0].qparams.desc == "hif8"
    y = net(torch.randn(5, 64, device=DEV).to(torch.bfloat16))
    assert y.shape == (5, 64) and torch.isfinite(y.float()).all()


def test_packed_file_round_trip(pkg, tmp_path):
    torch.manual_seed(0)
    net = torch.nn.Sequential(pkg.HIF8Linear(512, 768, bias=True), torch.nn.GELU(),
                              pkg.HIF8Linear(768, 512, bias=False)).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        net[0].bias.normal_(0, 0.1)
    x = torch.randn(4, 100, 512, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        y_ref = net(x)
    path = str(tmp_path / "packed.safetensors")
    names = pkg.save_packed(net, path)
    assert names == ["0", "2"]
    fresh = torch.nn.Sequential(pkg.HIF8Linear(512, 768, bias=True), torch.nn.GELU(),
                                pkg.HIF8Linear(768, 512, bias=False)).to(DEV).to(torch.bfloat16)
    assert pkg.load_packed(fresh, path) == ["0", "2"]
    assert fresh[0].weight.numel() == 0                       # bf16 weight released
    with torch.no_grad():
        y = fresh(x)
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    # the stored codes are the encoder's, the decode table the weight's
    p0 = net[0]._packed_weight()
    assert torch.equal(fresh[0]._packed.codes, p0.codes)
    assert torch.equal(fresh[0]._packed.state.lut_bf16().view(torch.int16), p0.state.lut_bf16().view(torch.int16))


def test_pack_state_dict(pkg, tmp_path):
    torch.manual_seed(1)
    ref = pkg.HIF8Linear(384, 256, bias=True).to(DEV).to(torch.bfloat16)
    sd = {f"blk.{k}": v.detach().cpu() for k, v in ref.state_dict().items()}
    path = str(tmp_path / "sd.safetensors")
    pkg.pack_state_dict(sd, ["blk"], path)
    holder = torch.nn.Module()
    holder.blk = pkg.HIF8Linear(384, 256, bias=True).to(DEV).to(torch.bfloat16)
    assert pkg.load_packed(holder, path) == ["blk"]
    x = torch.randn(77, 384, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        assert torch.equal(holder.blk(x).view(torch.int16), ref(x).view(torch.int16))
