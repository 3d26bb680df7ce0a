"""Chunk gather and EMA dechunk on MI355X (mote/model/dc.py:192-352 of the reference).

`ChunkLayer` and `DeChunkLayer` keep the reference's constructors, call signatures, return values and
dtypes; `DeChunkState` its decode state. Underneath are custom ops over the C ABI:

    mote::chunk_route(mask)                              -> (cum, perm, num, cu_seqlens)
    mote::chunk_gather(hidden, perm, num, mask, cum, M)  -> out            (autograd: chunk_gather_bwd)
    mote::dechunk(hidden, prob, perm, num, mask, cum, eps, init) -> (out, w)   (autograd: dechunk_bwd)

`chunk_pack` gives the packed varlen layout (rows of every sequence back to back plus cu_seqlens) that
`mote::relation_fwd_varlen` consumes. There is no CPU path: CPU tensors raise.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib as L


def _need_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what} needs the HIP library and an MI355X (got a {t.device} tensor)")


def _mask_u8(mask: torch.Tensor) -> torch.Tensor:
    m = mask if mask.dtype in (torch.bool, torch.uint8) else mask.bool()
    return m if m.stride(-1) == 1 else m.contiguous()


def _last_unit(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


# ------------------------------------------------------------------------------------------------
# route
# ------------------------------------------------------------------------------------------------
@torch.library.custom_op("mote::chunk_route", mutates_args=())
def chunk_route(mask: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per row of the boundary mask [B, L]: cum (int32 inclusive count), perm (int32: boundary
    positions in order, then the others), num (int32) and cu_seqlens (int32 [B + 1])."""
    _need_gpu(mask, "mote::chunk_route")
    m = _mask_u8(mask)
    B, Ln = m.shape
    cum = torch.empty(B, Ln, device=m.device, dtype=torch.int32)
    perm = torch.empty(B, Ln, device=m.device, dtype=torch.int32)
    num = torch.empty(B, device=m.device, dtype=torch.int32)
    cu = torch.empty(B + 1, device=m.device, dtype=torch.int32)
    a = L.ChunkRouteArgs()
    a.B, a.L = B, Ln
    a.mask, a.mask_sr = m.data_ptr(), m.stride(0)
    a.cum, a.perm, a.num, a.cu_seqlens = cum.data_ptr(), perm.data_ptr(), num.data_ptr(), cu.data_ptr()
    if B == 0:
        cu.zero_()
    L.check(L.lib().mote_chunk_route(a, L.stream_of(m)), "mote_chunk_route")
    return cum, perm, num, cu


@chunk_route.register_fake
def _chunk_route_fake(mask):
    B, Ln = mask.shape
    i = torch.int32
    return (mask.new_empty((B, Ln), dtype=i), mask.new_empty((B, Ln), dtype=i), mask.new_empty((B,), dtype=i),
            mask.new_empty((B + 1,), dtype=i))


# ------------------------------------------------------------------------------------------------
# gather
# ------------------------------------------------------------------------------------------------
def _gather_launch(hidden: torch.Tensor, perm: torch.Tensor, num: torch.Tensor, M: int,
                   cu: Optional[torch.Tensor], out: torch.Tensor) -> None:
    B, Ln, D = hidden.shape
    a = L.ChunkGatherArgs()
    a.dtype, a.B, a.L, a.M, a.D = L.dtype_code(hidden), B, Ln, M, D
    a.hidden, a.h_sb, a.h_sr = hidden.data_ptr(), hidden.stride(0), hidden.stride(1)
    a.perm, a.num = perm.data_ptr(), num.data_ptr()
    a.cu_seqlens = cu.data_ptr() if cu is not None else None
    a.out = out.data_ptr()
    if cu is not None:
        a.o_sb, a.o_sr = 0, out.stride(0)
    else:
        a.o_sb, a.o_sr = out.stride(0), out.stride(1)
    L.check(L.lib().mote_chunk_gather(a, L.stream_of(hidden)), "mote_chunk_gather")


@torch.library.custom_op("mote::chunk_gather", mutates_args=())
def chunk_gather(hidden: torch.Tensor, perm: torch.Tensor, num: torch.Tensor, mask: torch.Tensor,
                 cum: torch.Tensor, M: int) -> torch.Tensor:
    """out[b, m] = hidden[b, perm[b, m]], m < M (dc.py:214-216)."""
    _need_gpu(hidden, "mote::chunk_gather")
    h = _last_unit(hidden)
    out = torch.empty(h.shape[0], M, h.shape[2], device=h.device, dtype=h.dtype)
    _gather_launch(h, perm, num, M, None, out)
    return out


@chunk_gather.register_fake
def _chunk_gather_fake(hidden, perm, num, mask, cum, M):
    return hidden.new_empty((hidden.shape[0], M, hidden.shape[2]))


@torch.library.custom_op("mote::chunk_gather_bwd", mutates_args=())
def chunk_gather_bwd(dout: torch.Tensor, mask: torch.Tensor, cum: torch.Tensor, num: torch.Tensor,
                     L_len: int) -> torch.Tensor:
    """d hidden [B, L, D]: the gathered rows' gradients in place, zero elsewhere."""
    g = _last_unit(dout)
    B, M, D = g.shape
    m = _mask_u8(mask)
    dh = torch.empty(B, L_len, D, device=g.device, dtype=g.dtype)
    a = L.ChunkGatherBwdArgs()
    a.dtype, a.B, a.L, a.M, a.D = L.dtype_code(g), B, L_len, M, D
    a.dout, a.g_sb, a.g_sr = g.data_ptr(), g.stride(0), g.stride(1)
    a.mask, a.mask_sr, a.cum, a.num, a.cu_seqlens = m.data_ptr(), m.stride(0), cum.data_ptr(), num.data_ptr(), None
    a.dhidden, a.dh_sb, a.dh_sr = dh.data_ptr(), dh.stride(0), dh.stride(1)
    L.check(L.lib().mote_chunk_gather_bwd(a, L.stream_of(g)), "mote_chunk_gather_bwd")
    return dh


@chunk_gather_bwd.register_fake
def _chunk_gather_bwd_fake(dout, mask, cum, num, L_len):
    return dout.new_empty((dout.shape[0], L_len, dout.shape[2]))


def _gather_setup(ctx, inputs, output):
    hidden, perm, num, mask, cum, M = inputs
    ctx.save_for_backward(mask, cum, num)
    ctx.L = hidden.shape[1]


def _gather_backward(ctx, dout):
    mask, cum, num = ctx.saved_tensors
    return chunk_gather_bwd(dout, mask, cum, num, ctx.L), None, None, None, None, None


chunk_gather.register_autograd(_gather_backward, setup_context=_gather_setup)


def chunk_pack(hidden: torch.Tensor, boundary_mask: torch.Tensor):
    """The boundary rows of every sequence back to back: (packed [total, D], cu_seqlens int32 [B + 1],
    max_len) -- the layout of `mote::relation_fwd_varlen`. Reads num once on the host for the sizes."""
    _need_gpu(hidden, "chunk_pack")
    h = _last_unit(hidden)
    cum, perm, num, cu = chunk_route(boundary_mask)
    B, Ln, D = h.shape
    sizes = num.tolist()
    total, M = int(sum(sizes)), int(max(sizes)) if sizes else 0
    out = torch.empty(total, D, device=h.device, dtype=h.dtype)
    if total:
        _gather_launch(h, perm, num, M, cu, out)
    return out, cu, M


# ------------------------------------------------------------------------------------------------
# dechunk
# ------------------------------------------------------------------------------------------------
@torch.library.custom_op("mote::dechunk", mutates_args=())
def dechunk(hidden: torch.Tensor, prob: torch.Tensor, perm: torch.Tensor, num: torch.Tensor, mask: torch.Tensor,
            cum: torch.Tensor, eps: float, init: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """(out [B, L, D] in hidden's dtype, w [B, M, D] fp32 = hidden_m - z_{m-1}, kept for the backward) of
    DeChunkLayer.forward (dc.py:312-335); mask and cum (from mote::chunk_route) are kept for the backward."""
    _need_gpu(prob, "mote::dechunk")
    h = _last_unit(hidden)
    pr = _last_unit(prob)
    B, M, D = h.shape
    L_len = mask.shape[1]
    out = torch.empty(B, L_len, D, device=pr.device, dtype=h.dtype)
    w = torch.empty(B, M, D, device=pr.device, dtype=torch.float32)
    ini = init.detach().to(torch.float32).contiguous() if init is not None else None
    a = L.DechunkArgs()
    a.dtype, a.prob_dtype, a.out_dtype = L.dtype_code(h), L.dtype_code(pr), L.dtype_code(out)
    a.B, a.L, a.M, a.D, a.eps = B, L_len, M, D, float(eps)
    a.hidden, a.h_sb, a.h_sr = h.data_ptr(), h.stride(0), h.stride(1)
    a.prob, a.p_sb, a.p_sr = pr.data_ptr(), pr.stride(0), pr.stride(1)
    a.perm, a.num, a.cum = perm.data_ptr(), num.data_ptr(), cum.data_ptr()
    a.init = ini.data_ptr() if ini is not None else None
    a.out, a.o_sb, a.o_sr = out.data_ptr(), out.stride(0), out.stride(1)
    a.w = w.data_ptr()
    ws = torch.empty(max(int(L.lib().mote_dechunk_workspace(a)), 16), device=pr.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    L.check(L.lib().mote_dechunk_fwd(a, L.stream_of(pr)), "mote_dechunk_fwd")
    return out, w


@dechunk.register_fake
def _dechunk_fake(hidden, prob, perm, num, mask, cum, eps, init):
    B, M, D = hidden.shape
    return hidden.new_empty((B, mask.shape[1], D)), hidden.new_empty((B, M, D), dtype=torch.float32)


@torch.library.custom_op("mote::dechunk_bwd", mutates_args=())
def dechunk_bwd(dout: torch.Tensor, hidden: torch.Tensor, prob: torch.Tensor, perm: torch.Tensor, num: torch.Tensor,
                mask: torch.Tensor, cum: torch.Tensor, w: torch.Tensor, eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """(d hidden, d boundary_prob) of DeChunkLayer.forward without a carried value."""
    h, pr = _last_unit(hidden), _last_unit(prob)
    g = _last_unit(dout.to(h.dtype))
    m = _mask_u8(mask)
    B, M, D = h.shape
    Ln = g.shape[1]
    dh = torch.empty(B, M, D, device=h.device, dtype=h.dtype)
    dp = torch.empty(B, Ln, 2, device=h.device, dtype=pr.dtype)
    a = L.DechunkBwdArgs()
    a.dtype, a.prob_dtype, a.dout_dtype = L.dtype_code(h), L.dtype_code(pr), L.dtype_code(g)
    a.dx_dtype, a.dprob_dtype = L.dtype_code(dh), L.dtype_code(dp)
    a.B, a.L, a.M, a.D, a.eps = B, Ln, M, D, float(eps)
    a.dout, a.g_sb, a.g_sr = g.data_ptr(), g.stride(0), g.stride(1)
    a.hidden, a.h_sb, a.h_sr = h.data_ptr(), h.stride(0), h.stride(1)
    a.prob, a.p_sb, a.p_sr = pr.data_ptr(), pr.stride(0), pr.stride(1)
    a.perm, a.num, a.mask, a.mask_sr, a.cum = perm.data_ptr(), num.data_ptr(), m.data_ptr(), m.stride(0), cum.data_ptr()
    a.w = w.data_ptr()
    a.dhidden, a.dh_sb, a.dh_sr = dh.data_ptr(), dh.stride(0), dh.stride(1)
    a.dprob, a.dp_sb, a.dp_sr = dp.data_ptr(), dp.stride(0), dp.stride(1)
    ws = torch.empty(max(int(L.lib().mote_dechunk_bwd_workspace(a)), 16), device=h.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    L.check(L.lib().mote_dechunk_bwd(a, L.stream_of(h)), "mote_dechunk_bwd")
    return dh, dp


@dechunk_bwd.register_fake
def _dechunk_bwd_fake(dout, hidden, prob, perm, num, mask, cum, w, eps):
    return hidden.new_empty(hidden.shape), prob.new_empty((prob.shape[0], dout.shape[1], 2))


def _dechunk_setup(ctx, inputs, output):
    hidden, prob, perm, num, mask, cum, eps, init = inputs
    ctx.eps = eps
    ctx.has_init = init is not None
    ctx.save_for_backward(hidden, prob, perm, num, mask, cum, output[1])


def _dechunk_backward(ctx, dout, _dz):
    if ctx.has_init:
        raise RuntimeError("mote::dechunk has no backward with a carried value (the decode-state form)")
    hidden, prob, perm, num, mask, cum, w = ctx.saved_tensors
    dh, dp = dechunk_bwd(dout, hidden, prob, perm, num, mask, cum, w, ctx.eps)
    return dh, dp, None, None, None, None, None, None


dechunk.register_autograd(_dechunk_backward, setup_context=_dechunk_setup)


# ------------------------------------------------------------------------------------------------
# modules
# ------------------------------------------------------------------------------------------------
class ChunkLayer(nn.Module):
    """ChunkLayer(bucket=1) of dc.py:192-222: keep the boundary positions, compacted to the front of
    [B, M] (M rounded up to a multiple of `bucket`, capped at L), with the mask of real rows."""

    def __init__(self, bucket: int = 1):
        super().__init__()
        self.bucket = max(int(bucket), 1)

    def forward(self, hidden: torch.Tensor, boundary_mask: torch.Tensor, exact: bool = False):
        _need_gpu(hidden, "ChunkLayer")
        B, Ln, D = hidden.shape
        cum, perm, num, _ = chunk_route(boundary_mask)
        M = int(num.max()) if B > 0 else 0            # dc.py:210 reads the count on the host too
        if self.bucket > 1 and not exact:
            M = min(Ln, -(-M // self.bucket) * self.bucket)
        out = chunk_gather(hidden, perm, num, boundary_mask, cum, M)
        next_mask = torch.arange(M, device=hidden.device)[None, :] < num[:, None]
        return out, next_mask

    def step(self, hidden: torch.Tensor, boundary_mask: torch.Tensor) -> torch.Tensor:
        # hidden [B, 1, D] -> [B', 1, D] rows where a boundary fired (dc.py:220-222)
        return hidden[boundary_mask]


@dataclass
class DeChunkState:
    last_value: torch.Tensor  # [B, D]


class DeChunkLayer(nn.Module):
    """DeChunkLayer(d_model, headdim=32, block_size=256, prob_clamp=1e-4) of dc.py:225-352: EMA
    smoothing z_t = p_t x_t + (1 - p_t) z_{t-1} over the chunk outputs, expanded back to bytes."""

    def __init__(self, d_model: int, headdim: int = 32, block_size: int = 256, prob_clamp: float = 1e-4):
        super().__init__()
        self.d_model = d_model
        self.headdim = headdim
        self.block_size = block_size
        self.eps = prob_clamp
        assert d_model % headdim == 0
        self.nheads = d_model // headdim

    def allocate_inference_cache(self, batch_size: int, device, dtype=None) -> DeChunkState:
        return DeChunkState(last_value=torch.zeros(batch_size, self.d_model, device=device, dtype=dtype))

    def forward(self, hidden: torch.Tensor, boundary_mask: torch.Tensor, boundary_prob: torch.Tensor,
                state: Optional[DeChunkState] = None) -> torch.Tensor:
        _need_gpu(boundary_prob, "DeChunkLayer")
        B, Ln = boundary_mask.shape
        cum, perm, num, _ = chunk_route(boundary_mask)
        init = state.last_value if state is not None else None
        if init is None and hidden.shape[1] == 0:
            raise RuntimeError("DeChunkLayer: no chunk rows and no carried value")
        if init is not None and hidden.shape[1] == 0:
            hidden = hidden.new_empty(B, 0, hidden.shape[-1])
        out, _ = dechunk(hidden, boundary_prob, perm, num, boundary_mask, cum, float(self.eps), init)
        if state is not None:
            state.last_value.copy_(out[:, -1])
        return out

    def step(self, hidden: torch.Tensor, boundary_mask: torch.Tensor, boundary_prob: torch.Tensor,
             state: DeChunkState) -> torch.Tensor:
        # hidden: [B', 1, D] for rows with a boundary; boundary_mask [B]; boundary_prob [B, 2]
        last = state.last_value
        _need_gpu(last, "DeChunkLayer.step")
        B, D = last.shape
        m = _mask_u8(boundary_mask)
        pr = _last_unit(boundary_prob)
        h = _last_unit(hidden.reshape(hidden.shape[0], -1)) if hidden.shape[0] > 0 else None
        out = torch.empty(B, D, device=last.device, dtype=last.dtype)
        a = L.DechunkStepArgs()
        a.prob_dtype, a.state_dtype = L.dtype_code(pr), L.dtype_code(last)
        a.hidden_dtype = L.dtype_code(h) if h is not None else a.state_dtype
        a.B, a.D, a.eps = B, D, float(self.eps)
        a.mask, a.prob, a.p_sr = m.data_ptr(), pr.data_ptr(), pr.stride(0)
        a.hidden, a.h_sr = (h.data_ptr(), h.stride(0)) if h is not None else (None, 0)
        if last.stride(-1) != 1:
            raise RuntimeError("DeChunkLayer.step: the state must have unit stride along D")
        a.last_value, a.l_sr = last.data_ptr(), last.stride(0)
        a.out, a.o_sr = out.data_ptr(), out.stride(0)
        L.check(L.lib().mote_dechunk_step(a, L.stream_of(last)), "mote_dechunk_step")
        return out.unsqueeze(1)
