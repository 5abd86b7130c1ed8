"""The DiT block's feed-forward network with producer fusion.

``HIF8FFN`` is ``nn.Sequential(HIF8Linear(dim, ffn_dim), nn.GELU(approximate="tanh"),
HIF8Linear(ffn_dim, dim))`` -- ``ospnext/modules/osp_next.py:873-877`` -- with the same
children and state-dict keys.  Without autograd, a bf16 input takes the fused route:

    up:    hif8_linear[_wq]_gelu_stat  y = x_q @ w_up^T + b_up, and max y, which settles
                                        amax|GELU(y)| and its scale (GELU increases on y >= 0)
    down:  hif8_gelu_fake_quant(y)      x_q = _quant(GELU(y)) with that scale, GELU applied on
                                        the way in; then the GEMM

which removes the GELU pass (read and write of y), the down-projection's amax pass and the GELU
evaluation from the up-projection's epilogue, where the matrix cores would wait for it.  If max
y does not settle the amax (no positive output large enough, or a non-finite one), the
quantisation runs the amax pass of GELU(y) first.  With autograd, or for inputs and shapes the
fused kernels do not take, it runs the plain sequence.
"""
from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor

from . import _lib
from .hif8_linear import (HIF8Linear, QuantState, fused_shape_ok, gelu_fake_quant, linear_any,
                          linear_fwd_gelu_stat, quantize_activation)


class HIF8FFN(nn.Sequential):
    def __init__(self, dim: int, ffn_dim: int, scale_max_forward: float = 15.0, scale_max_backward: float = 224.0,
                 bias: bool = True, device=None, dtype=None):
        super().__init__(
            HIF8Linear(dim, ffn_dim, bias=bias, scale_max_forward=scale_max_forward,
                       scale_max_backward=scale_max_backward, device=device, dtype=dtype),
            nn.GELU(approximate="tanh"),
            HIF8Linear(ffn_dim, dim, bias=bias, scale_max_forward=scale_max_forward,
                       scale_max_backward=scale_max_backward, device=device, dtype=dtype),
        )

    def fused_ok(self, x: Tensor) -> bool:
        up, down = self[0], self[2]
        grad = torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))
        return (not grad and x.dtype == torch.bfloat16 and x.is_cuda and up.a_format != "codes"
                and fused_shape_ok(up.out_features, up.in_features)
                and fused_shape_ok(down.out_features, down.in_features))

    def forward(self, x: Tensor) -> Tensor:
        if not self.fused_ok(x):
            return super().forward(x)
        K = x.shape[-1]
        a, _, _ = quantize_activation(x.reshape(-1, K).contiguous(), self[0].scale_max_forward, "bf16")
        return self._fused_from_xq(a).view(*x.shape[:-1], -1)

    def forward_quantized(self, x_q: Tensor) -> Tensor:
        """The FFN of an input already quantised with the up-projection's ``scale_max_forward``
        (``x_q = _quant(x)[0]``, e.g. from ``modulated_norm_quant``): equals ``forward(x)``.
        Inference only."""
        if not self.fused_ok(x_q):
            if torch.is_grad_enabled() and (x_q.requires_grad or any(p.requires_grad for p in self.parameters())):
                raise RuntimeError("forward_quantized has no autograd; call forward(x) when gradients are needed")
            return self[2](self[1](self[0].forward_quantized(x_q)))
        K = x_q.shape[-1]
        return self._fused_from_xq(x_q.reshape(-1, K).contiguous()).view(*x_q.shape[:-1], -1)

    def _fused_from_xq(self, a: Tensor) -> Tensor:
        """up with the GELU-statistic epilogue, the fake quant of GELU of its output, down."""
        up, down = self[0], self[2]
        y_st = QuantState(a.device)
        y = linear_fwd_gelu_stat(a, up._packed_weight(), up.bias, y_st, down.scale_max_forward)
        yq = gelu_fake_quant(y, y_st, down.scale_max_forward)
        return linear_any(yq, _lib.A_BF16, None, down._packed_weight(), down.bias)
