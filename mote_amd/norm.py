"""Fused residual add + RMSNorm on MI355X (mote/model/norm.py:26-59 of the reference).

`RMSNorm` keeps the reference's constructor, parameter and call signature:
forward(x, residual=None, prenorm=False, residual_in_fp32=True) adds the residual (in fp32 when
residual_in_fp32), normalises in fp32 and returns y in the dtype of x, and with prenorm also the new
residual stream (fp32 when residual_in_fp32). Underneath are the custom ops `mote::add_rms_norm` /
`mote::add_rms_norm_bwd` over the C ABI (mote_add_rms_norm_fwd / _bwd): one HIP launch forward, two
backward (the weight gradient is summed in a fixed order, so every gradient is reproducible). There is
no CPU path: CPU tensors raise.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib as L


def _sum_dtype(x: torch.Tensor, residual: Optional[torch.Tensor], prenorm: bool, residual_in_fp32: bool):
    """dtype of the summed stream s (norm.py:50-55): fp32 when residual_in_fp32 and a residual is
    added or prenorm; otherwise x + residual in torch's promotion, or x itself."""
    if residual is not None:
        return torch.float32 if residual_in_fp32 else torch.promote_types(x.dtype, residual.dtype)
    if residual_in_fp32 and prenorm:
        return torch.float32
    return x.dtype


def _rows(t: torch.Tensor) -> torch.Tensor:
    """[..., D] -> [rows, D] with unit element stride (a view when possible)."""
    t = t if t.stride(-1) == 1 else t.contiguous()
    try:
        return t.view(-1, t.shape[-1])
    except RuntimeError:
        return t.reshape(-1, t.shape[-1]).contiguous()


@torch.library.custom_op("mote::add_rms_norm", mutates_args=())
def _add_rms_norm(x: torch.Tensor, weight: torch.Tensor, residual: Optional[torch.Tensor], eps: float, prenorm: bool,
                  residual_in_fp32: bool) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    if not x.is_cuda:
        raise RuntimeError("mote::add_rms_norm needs the HIP library and an MI355X")
    shape, D = x.shape, x.shape[-1]
    x2 = _rows(x)
    rows = x2.shape[0]
    r2 = _rows(residual) if residual is not None else None
    sdt = _sum_dtype(x, residual, prenorm, residual_in_fp32)
    w = weight.detach().to(torch.float32).contiguous()
    y = torch.empty(rows, D, device=x.device, dtype=x.dtype)
    # the sum is materialised unless it is x itself (then x is what the backward saves)
    s = torch.empty(rows, D, device=x.device, dtype=sdt) if (residual is not None or sdt != x.dtype) else None
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
    a = L.NormArgs()
    a.dtype, a.out_dtype = L.dtype_code(x2), L.dtype_code(y)
    a.res_dtype = L.dtype_code(r2) if r2 is not None else a.dtype
    a.res_out_dtype = L.dtype_code(s) if s is not None else a.dtype
    a.rows, a.D, a.eps = rows, D, float(eps)
    a.x, a.x_sr = x2.data_ptr(), x2.stride(0)
    a.residual, a.res_sr = (r2.data_ptr(), r2.stride(0)) if r2 is not None else (None, 0)
    a.weight = w.data_ptr()
    a.y, a.y_sr = y.data_ptr(), D
    a.residual_out, a.res_out_sr = (s.data_ptr(), D) if s is not None else (None, 0)
    a.rstd = rstd.data_ptr()
    L.check(L.lib().mote_add_rms_norm_fwd(a, L.stream_of(x)), "mote_add_rms_norm_fwd")
    # s is x itself when it is not materialised: an empty tensor stands in (outputs may not alias x)
    return y.view(shape), (s.view(shape) if s is not None else x.new_empty(0)), rstd


@_add_rms_norm.register_fake
def _add_rms_norm_fake(x, weight, residual, eps, prenorm, residual_in_fp32):
    rows = x.numel() // x.shape[-1]
    sdt = _sum_dtype(x, residual, prenorm, residual_in_fp32)
    s = x.new_empty(x.shape, dtype=sdt) if (residual is not None or sdt != x.dtype) else x.new_empty(0)
    return x.new_empty(x.shape), s, x.new_empty((rows,), dtype=torch.float32)


@torch.library.custom_op("mote::add_rms_norm_bwd", mutates_args=())
def _add_rms_norm_bwd(dy: torch.Tensor, dres_out: Optional[torch.Tensor], s: torch.Tensor, rstd: torch.Tensor,
                      weight: torch.Tensor, x_dtype: torch.dtype, has_res: bool, res_dtype: torch.dtype
                      ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dx, dresidual, dweight); dresidual is empty when has_res is false."""
    shape, D = s.shape, s.shape[-1]
    dy2, s2 = _rows(dy), _rows(s)
    rows = s2.shape[0]
    dro2 = _rows(dres_out) if dres_out is not None else None
    w = weight.detach().to(torch.float32).contiguous()
    dx = torch.empty(rows, D, device=s.device, dtype=x_dtype)
    dres = torch.empty(rows, D, device=s.device, dtype=res_dtype) if has_res else None
    dw = torch.empty(D, device=s.device, dtype=torch.float32)
    a = L.NormBwdArgs()
    a.dtype, a.s_dtype, a.dx_dtype = L.dtype_code(dy2), L.dtype_code(s2), L.dtype_code(dx)
    a.dres_out_dtype = L.dtype_code(dro2) if dro2 is not None else a.dtype
    a.dres_dtype = L.dtype_code(dres) if dres is not None else a.dtype
    a.rows, a.D = rows, D
    a.dy, a.dy_sr = dy2.data_ptr(), dy2.stride(0)
    a.dres_out, a.dres_out_sr = (dro2.data_ptr(), dro2.stride(0)) if dro2 is not None else (None, 0)
    a.s, a.s_sr = s2.data_ptr(), s2.stride(0)
    a.rstd, a.weight = rstd.data_ptr(), w.data_ptr()
    a.dx, a.dx_sr = dx.data_ptr(), D
    a.dresidual, a.dres_sr = (dres.data_ptr(), D) if dres is not None else (None, 0)
    a.dweight = dw.data_ptr()
    ws = torch.empty(max(int(L.lib().mote_add_rms_norm_bwd_workspace(a)), 16), device=s.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    L.check(L.lib().mote_add_rms_norm_bwd(a, L.stream_of(s)), "mote_add_rms_norm_bwd")
    return dx.view(shape), (dres.view(shape) if dres is not None else s.new_empty(0, dtype=res_dtype)), dw


@_add_rms_norm_bwd.register_fake
def _add_rms_norm_bwd_fake(dy, dres_out, s, rstd, weight, x_dtype, has_res, res_dtype):
    return (s.new_empty(s.shape, dtype=x_dtype), s.new_empty(s.shape if has_res else 0, dtype=res_dtype),
            s.new_empty((s.shape[-1],), dtype=torch.float32))


def _setup(ctx, inputs, output):
    x, weight, residual, eps, prenorm, residual_in_fp32 = inputs
    _y, s, rstd = output
    ctx.s_is_x = s.shape != x.shape          # the empty stand-in: s is x itself
    ctx.save_for_backward(x if ctx.s_is_x else s, rstd, weight)
    ctx.x_dtype = x.dtype
    ctx.has_res = residual is not None
    ctx.res_dtype = residual.dtype if residual is not None else x.dtype
    ctx.w_dtype = weight.dtype


def _backward(ctx, dy, ds_out, _drstd):
    s, rstd, weight = ctx.saved_tensors
    if dy is None:
        dy = torch.zeros_like(s, dtype=ctx.x_dtype)
    if ctx.s_is_x or (ds_out is not None and ds_out.shape != s.shape):
        ds_out = None                       # the returned stream is x itself: autograd routes its gradient
    dx, dres, dw = _add_rms_norm_bwd(dy, ds_out, s, rstd, weight, ctx.x_dtype, ctx.has_res, ctx.res_dtype)
    return dx, dw.to(ctx.w_dtype), (dres if ctx.has_res else None), None, None, None


_add_rms_norm.register_autograd(_backward, setup_context=_setup)


def add_rms_norm(x: torch.Tensor, weight: torch.Tensor, residual: Optional[torch.Tensor] = None, eps: float = 1e-5,
                 prenorm: bool = False, residual_in_fp32: bool = True):
    """Functional form of RMSNorm.forward (norm.py:36-59)."""
    y, s, _ = _add_rms_norm(x, weight, residual, float(eps), bool(prenorm), bool(residual_in_fp32))
    if not prenorm:
        return y
    return y, (s if s.shape == x.shape else x)


class RMSNorm(nn.Module):
    """RMSNorm(dim, eps=1e-5) with the fused-residual call of mote/model/norm.py:26-59."""

    def __init__(self, dim: int, eps: float = 1e-5, device=None, dtype=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=dtype))

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None, prenorm: bool = False,
                residual_in_fp32: bool = True):
        return add_rms_norm(x, self.weight, residual, self.eps, prenorm, residual_in_fp32)
