"""CPU restatement of Mote's RMSNorm with the fused-residual interface (test infrastructure only).

Follows mote/model/norm.py:26-59 of the reference (the pure-PyTorch path its fused Triton kernel
must match, tests/test_fused_norm.py of the reference): `rms_norm_ref` is the forward, and
`rms_norm_backward_ref` states its gradients in closed form. Nothing in the product imports this
module: it is the checker of mote_amd.norm.

Pins (tests/test_norm_oracle.py): the forward against torch.nn.functional.rms_norm in float64 and
the closed form of a constant row; the backward against autograd of the forward and against
central finite differences; the prenorm dtype rules of norm.py:50-55. Planted mistakes (eps outside
the root, a sum instead of a mean, a dropped weight, a dropped projection term, r^2 for r^3) are
injected through `_plant` and each must fail one of the pins. The reference's own tests hold no
fixtures for this path (they compare its Triton kernel with norm.py:46-59 on random inputs).
"""

from __future__ import annotations

from typing import Optional

import torch


def rms_norm_ref(x: torch.Tensor, weight: torch.Tensor, residual: Optional[torch.Tensor] = None,
                 prenorm: bool = False, residual_in_fp32: bool = True, eps: float = 1e-5,
                 compute_dtype: torch.dtype = torch.float32, _plant: Optional[str] = None):
    """norm.py:36-59: the residual added (in fp32 when residual_in_fp32), then
    y = s / sqrt(mean(s^2) + eps) * weight in the dtype of x; returns (y, s) when prenorm.
    `compute_dtype` float64 gives the exact reference for the pins."""
    out_dtype = x.dtype
    up = torch.float32 if compute_dtype == torch.float32 else compute_dtype   # fp32 stream (exact: f64)
    if residual is not None:                                           # norm.py:50-51
        s = (x.to(up) + residual.to(up)) if residual_in_fp32 else x + residual
    elif residual_in_fp32 and prenorm:                                 # norm.py:52-53
        s = x.to(up)
    else:
        s = x
    sf = s.to(compute_dtype)                                           # norm.py:33
    ms = sf.pow(2).mean(-1, keepdim=True)
    if _plant == "eps_outside":
        r = torch.rsqrt(ms) + eps
    elif _plant == "sum_not_mean":
        r = torch.rsqrt(sf.pow(2).sum(-1, keepdim=True) + eps)
    else:
        r = torch.rsqrt(ms + eps)                                      # norm.py:34
    w = torch.ones_like(weight) if _plant == "no_weight" else weight
    y = (sf * r * w.to(compute_dtype)).to(out_dtype if compute_dtype == torch.float32 else compute_dtype)
    return (y, s) if prenorm else y


def rms_norm_backward_ref(dy: torch.Tensor, s: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5,
                          dres_out: Optional[torch.Tensor] = None, _plant: Optional[str] = None):
    """Gradients of y = s r w, r = (mean(s^2) + eps)^(-1/2), in float64:
    ds = r g - (r^3 / D) s sum(g s) + dres_out with g = dy w, dw = sum over rows of dy s r."""
    s64, dy64, w64 = s.double(), dy.double(), weight.double()
    D = s64.shape[-1]
    r = torch.rsqrt(s64.pow(2).mean(-1, keepdim=True) + eps)
    g = dy64 * w64
    r3 = r ** 2 if _plant == "r_squared" else r ** 3
    proj = 0.0 if _plant == "no_proj" else (r3 / D) * s64 * (g * s64).sum(-1, keepdim=True)
    ds = r * g - proj
    if dres_out is not None:
        ds = ds + dres_out.double()
    dw = (dy64 * s64 * r).reshape(-1, D).sum(0)
    return ds, dw
