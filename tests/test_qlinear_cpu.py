"""CPU-side checks of the QLinear API and the packed-file reader (no GPU work)."""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")


def test_replace_linear_structure(pkg):
    net = torch.nn.Sequential(torch.nn.Linear(8, 16), torch.nn.ReLU(),
                              torch.nn.Sequential(torch.nn.Linear(16, 4, bias=False)))
    w = net[2][0].weight.detach().clone()
    pkg.replace_linear(net, "hif8", in_Q="hif8", quant_grad=False, exclude_layers=["0"])
    assert type(net[0]) is torch.nn.Linear
    q = net[2][0]
    assert isinstance(q, pkg.QLinear) and q.bias is None
    assert torch.equal(q.weight.detach(), w)
    assert q.qparams.desc == "hif8" and q.in_qparams.desc == "hif8" and q._quant_grad is False
    with pytest.raises(AssertionError):
        pkg.replace_linear(net, "hif8", exclude_layers="0")


def test_qlinear_requires_qparams(pkg):
    q = pkg.QLinear(4, 4)
    with pytest.raises(AssertionError):
        q(torch.zeros(1, 4))


def test_load_packed_rejects_foreign_files(pkg, tmp_path):
    from safetensors.torch import save_file
    path = str(tmp_path / "x.safetensors")
    save_file({"a": torch.zeros(2)}, path, metadata={"format": "something-else"})
    with pytest.raises(ValueError):
        pkg.load_packed(torch.nn.Module(), path)
