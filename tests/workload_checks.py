"""Checks shared by the GPU tests at the full BASELINE workloads (configs 3-5).

At these sizes the CPU oracle cannot run on whole tensors, so every check is one of:

- a row sample: x_q rows bit-exact against the oracle's ``_quant`` (hif8_linear.py:42-50)
  with the scale the oracle's rule gives for the full tensor's amax, the amax taken by torch
  on the GPU (a max is exact in any order); GEMM output rows against fp32 torch on the same
  (bit-exact) operands, within the north-star tolerance of tests/test_gpu_linear.py;
- a whole-tensor identity on the GPU: a producer's x_q equal, bit for bit, to the standalone
  ``_quant`` (absmax_scale + fake_quant) of the tensor it quantises.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

TOL_ELEM = 1e-2
TOL_NORM = 4e-3


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def sample_rows(M: int, seed: int, n: int = 384, tail: int = 80, device="cuda:0") -> torch.Tensor:
    """``n`` random rows plus the last ``tail`` rows (the GEMMs' ragged last tile)."""
    g = torch.Generator().manual_seed(seed)
    rows = torch.cat([torch.randint(0, M, (n,), generator=g), torch.arange(max(0, M - tail), M)])
    return rows.to(device)


def rel_errors(y: torch.Tensor, y_ref: torch.Tensor):
    """(max elementwise error relative to max(|ref|, 1e-2 rms(ref)), normwise error)."""
    y = y.double()
    y_ref = y_ref.double()
    rms = y_ref.square().mean().sqrt()
    floor = torch.clamp(y_ref.abs(), min=1e-2 * float(rms))
    return float(((y - y_ref).abs() / floor).max()), float((y - y_ref).norm() / y_ref.norm())


def check_scale(R, x: torch.Tensor, state, scale_max: float, as_f32: bool = False) -> float:
    """The state's scale equals the oracle's rule (hif8_linear.py:45-46) applied to torch's amax
    of the whole tensor; returns the scale."""
    _, s_got = state.read()
    if x.dtype == torch.bfloat16 and not as_f32:
        amax = int(bits(x.abs().max().reshape(1))[0])
        s_bits = R.hif8_scale_bf16(amax, scale_max)
        s_want = float(R.bf16_to_f32(np.array([s_bits], np.uint16))[0])
    else:
        amax = float(x.float().abs().max())
        s_want = float(R.hif8_scale_f32(amax, scale_max))
    assert np.float32(s_got) == np.float32(s_want), (s_got, s_want)
    return s_want


def oracle_xq_rows(R, x_rows: torch.Tensor, scale: float, as_f32: bool = False) -> np.ndarray:
    """bf16 bits of x_q for rows of x under the full tensor's scale: the oracle's _quant chain
    (bf16: x*s, fp32 qdq, cast, /s each rounded to bf16; fp32: all in fp32, then the bf16 cast
    of F.linear's autocast)."""
    if x_rows.dtype == torch.bfloat16 and not as_f32:
        s = np.float32(scale)
        xs = R.f32_to_bf16(R.bf16_to_f32(bits(x_rows)) * s)
        q = R.f32_to_bf16(R.quant_hif8_npu(R.bf16_to_f32(xs)))
        return R.f32_to_bf16(R.bf16_to_f32(q) / s)
    xf = x_rows.float().cpu().numpy()
    s = np.float32(scale)
    with np.errstate(all="ignore"):
        xq = (R.quant_hif8_npu((xf * s).astype(np.float32)) / s).astype(np.float32)
    return R.f32_to_bf16(xq)


def check_xq_rows(R, x: torch.Tensor, xq: torch.Tensor, state, scale_max: float, rows: torch.Tensor,
                  as_f32: bool = False) -> None:
    """Scale from the full tensor, then sampled rows of x_q bit-exact against the oracle."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    s = check_scale(R, x2, state, scale_max, as_f32)
    want = oracle_xq_rows(R, x2[rows], s, as_f32)
    got = bits(xq.reshape(-1, K)[rows])
    bad = np.nonzero(got != want)
    assert bad[0].size == 0, f"{bad[0].size} x_q values differ from the oracle, first at {bad[0][0]},{bad[1][0]}"


def standalone_quant(pkg, y: torch.Tensor, scale_max: float):
    """``_quant(y)[0]`` through the standalone codec (amax + scale pass, then fake quant)."""
    y2 = y.reshape(-1, y.shape[-1]).contiguous()
    st = pkg.absmax_scale(y2, scale_max, pkg.QuantState(y2.device))
    return pkg.fake_quant(y2, st), st


def check_linear_rows(a: torch.Tensor, w_q: torch.Tensor, b, y: torch.Tensor, rows: torch.Tensor,
                      gelu: bool = False):
    """Rows of a bf16 GEMM output against fp32 torch on the same operands: ``a`` the bf16 x_q
    [M, K], ``w_q`` the dequantised bf16 weight [N, K], ``b`` the bias or None; with ``gelu``
    the output is GELU(tanh) of the bf16 linear output.  Returns (elem, norm) errors."""
    K = a.shape[-1]
    ref = a.reshape(-1, K)[rows].float() @ w_q.float().t()
    if b is not None:
        ref = ref + b.float()
    got = y.reshape(-1, y.shape[-1])[rows]
    if gelu:
        # GELU's tail shrinks values much faster than their derivative: a one-unit bf16 change of
        # the pre-activation (accumulation order) is a large relative change of a tiny output.  The
        # bound is therefore GELU's variation over the pre-activation's own tolerance band
        # (two bf16 units plus 2^-12 rms) plus one bf16 unit of the output (both sides round).
        g = lambda t: F.gelu(t, approximate="tanh")  # noqa: E731
        d = ref.abs() * 2.0 ** -7 + float(ref.square().mean().sqrt()) * 2.0 ** -12
        mid = g(ref.to(torch.bfloat16).float())
        band = torch.maximum((g(ref + d) - mid).abs(), (g(ref - d) - mid).abs())
        bound = band + mid.abs() * 2.0 ** -7 + 1e-30
        err = (got.float() - mid).abs()
        assert bool((err <= bound).all()), float((err / bound).max())
        ref = mid
    elem, norm = rel_errors(got, ref)
    assert norm <= TOL_NORM and (gelu or elem <= TOL_ELEM), (elem, norm)
    return elem, norm


def check_attention_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_idx, key_count,
                         out: torch.Tensor, seed: int, n: int = 48):
    """Sampled queries of every batch of an attention output ([B, Nq, H, 128], as
    hif8_attention_fwd writes it) against softmax(q k^T / sqrt(128)) v in float32 over the keys
    the batch keeps: normwise <= 1e-2 and elementwise <= 2e-2 of the largest reference magnitude
    (the kernel rounds the probabilities and the output to bf16)."""
    B, Nq, H, D = q.shape
    g = torch.Generator().manual_seed(seed)
    for b in range(B):
        rows = torch.randint(0, Nq, (n,), generator=g).to(q.device)
        kb = k[b if k.shape[0] == B else 0]
        vb = v[b if v.shape[0] == B else 0]
        if key_count is not None:
            c = int(key_count[b])
            sel = key_idx[b, :c].long() if key_idx is not None else torch.arange(c, device=q.device)
            kb, vb = kb[sel], vb[sel]
        qs = q[b, rows].float().permute(1, 0, 2).contiguous()               # [H, n, D]
        s = torch.matmul(qs, kb.float().permute(1, 2, 0).contiguous()) / D ** 0.5
        ref = torch.matmul(torch.softmax(s, dim=-1), vb.float().permute(1, 0, 2).contiguous())
        got = out[b, rows].float().permute(1, 0, 2)
        err = float((got - ref).norm() / ref.norm().clamp_min(1e-30))
        mx = float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
        assert err <= 1e-2 and mx <= 2e-2, (b, err, mx)
