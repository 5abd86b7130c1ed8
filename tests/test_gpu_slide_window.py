"""GPU parity of ``quant_slide_window`` (QTensor.py:147-174) against the oracle.

The reference quantises, in place, everything outside a trailing window with the plain
(unscaled) HiF8 qdq of ``quant_dequant_float``: the last ``win`` columns (qdim -1), the last
``win`` rows of the last two dims (qdim -2), or everything outside the top-left
``[:-rows, :-cols]`` block for a pair.  Expected values are built on the CPU from the oracle's
qdq of exactly the quantised region, the window copied unchanged; bf16 and fp32, both qdq
semantics (``force_py``), positive qdim, and tensors no larger than the window (unchanged).
The gradient passes straight through."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _input(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * 3
    x.view(-1)[::37] *= 1e-6          # values near the tapered grid's small end
    x.view(-1)[::101] *= 3e3          # and beyond 40960 (Ascend: +-Inf)
    return x.to(dtype)


def _oracle(R, x_cpu: torch.Tensor, region, semantics: str) -> torch.Tensor:
    want = x_cpu.clone()
    part = x_cpu[region].float().contiguous().numpy()
    q = R.quant_hif8(part.reshape(-1), semantics).reshape(part.shape)
    want[region] = torch.from_numpy(q).to(x_cpu.dtype)
    return want


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    if a.dtype == torch.bfloat16:
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


CASES = [
    # (shape, qdim, win, region of the quantised part)
    ((2, 300, 260), -1, 128, (Ellipsis, slice(None, -128))),
    ((2, 300, 260), -2, 128, (Ellipsis, slice(None, -128), slice(None))),
    ((2, 300, 260), 2, 100, (Ellipsis, slice(None, -100))),                 # qdim 2 of 3 dims = -1
    ((2, 300, 260), 1, 64, (Ellipsis, slice(None, -64), slice(None))),      # qdim 1 of 3 dims = -2
    ((3, 4, 200, 136), -2, (64, 100), (Ellipsis, slice(None, -64), slice(None, -100))),
    ((3, 4, 200, 136), -1, [199, 8], (Ellipsis, slice(None, -199), slice(None, -8))),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("force_py", [False, True])
@pytest.mark.parametrize("shape,qdim,win,region", CASES)
def test_slide_window_matches_oracle(pkg, R, shape, qdim, win, region, dtype, force_py):
    x_cpu = _input(shape, dtype, seed=len(shape) * 11 + abs(qdim))
    want = _oracle(R, x_cpu, region, "torch" if force_py else "npu")
    x = x_cpu.to(DEV)
    ptr = x.data_ptr()
    out = pkg.quant_slide_window(x, pkg.QType("hif8"), force_py=force_py, qdim=qdim, win_size=win)
    torch.cuda.synchronize()
    assert out.data_ptr() == ptr and x.data_ptr() == ptr          # in place, x itself returned
    assert _same(x.cpu(), want)
    assert _same(out.cpu(), want)


@pytest.mark.parametrize("shape,qdim,win", [((4, 128, 64), -1, 64), ((4, 128, 64), -2, 128),
                                            ((4, 128, 64), -2, (128, 10)), ((4, 128, 64), -1, (10, 64))])
def test_slide_window_not_larger_than_window(pkg, shape, qdim, win):
    x = _input(shape, torch.bfloat16, 3).to(DEV)
    before = x.clone()
    pkg.quant_slide_window(x, pkg.QType("hif8"), qdim=qdim, win_size=win)
    assert torch.equal(x.view(torch.int16), before.view(torch.int16))


def test_slide_window_bad_dim_and_gradient(pkg):
    x = _input((2, 64, 300), torch.float32, 4).to(DEV)
    with pytest.raises(NotImplementedError):
        pkg.quant_slide_window(x, pkg.QType("hif8"), qdim=-3, win_size=16)
    leaf = _input((2, 64, 300), torch.float32, 5).to(DEV).requires_grad_(True)
    y = pkg.quant_slide_window(leaf * 1.0, pkg.QType("hif8"), qdim=-1, win_size=128)
    g = torch.randn(y.shape, device=DEV)
    y.backward(g)
    assert torch.equal(leaf.grad, g)                            # straight through
