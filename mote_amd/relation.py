"""FullRelation on MI355X — the Relation token mixer behind mote/model/relation.py's interface.

Same constructor, parameter names and construction order (relation.py:97-157), same forward
signature and return convention (relation.py:184-268). What runs underneath:

    p1, p2, I~ = mote::qkv_rope(x, [w1; w2; wi])  HIP: one launch for the projections with RoPE on
                                                 p1/p2 and Givens on I~ in the epilogue (bf16,
                                                 dh 64 / 96 / 128, no QK-Norm); otherwise one
                                                 hipBLASLt GEMM and mote::rope_givens
    Y, g = mote::relation_fwd(p1, P2, I~)        HIP: the fused Relation core (any T, decode too)
    out = wo(Y [* sigmoid(wg x)])                 Y is token-major already, so no transpose copy

There is no materialized path: `USE_FLASH = False` raises, and so does a CPU tensor. The
materialized restatement lives in the test oracle.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib as L
from .arena import ArenaLayer
from .flash_relation import HAS_HIP, HAS_TRITON, flash_relation  # noqa: F401  (re-exported names)

RelationCache = Tuple[torch.Tensor, torch.Tensor]  # (P2 [B,H,S,dh], I~ [B,H,S,dh]) or an ArenaLayer
USE_FLASH = True   # the HIP path; the reference's materialized alternative is not part of this package
FLASH_MIN_T = 16   # kept for callers that read it; the HIP kernels serve every T, T = 1 included


def rope_inv_freq(dim: int, theta: float, device=None) -> torch.Tensor:
    """fp32 [dim/2] table 1 / theta^(2k/dim), computed with the same fp32 ops as relation.py:39 so
    the kernels' angles float(pos) * inv_freq[k] round exactly like the reference's tables. Built on
    the CPU and then moved: a last-ulp difference of the device's pow would grow by the position
    (one ulp of the angle at pos ~ 1000 is ~6e-5 rad)."""
    k2 = torch.arange(0, dim, 2, dtype=torch.float32)
    return (1.0 / (theta ** (k2 / dim))).to(device)


# ---- torch-level RoPE helpers (the names mote/model/relation.py:37-68 exports) ------------------
# The module's own forward runs RoPE inside the HIP prologue kernels; these helpers are for callers
# that rotate rows themselves (mote/infer/graph.py:39, 158-164). They round where the kernels round:
# tables cast to the operand dtype, then every product and sum in that dtype.
def _rope_cos_sin(positions: torch.Tensor, dim: int, theta: float, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    """positions [T] (integers) -> cos, sin [T, dim] in `dtype`: fp32 angles pos * inv_freq, the
    half-table repeated for the rotate-half convention (relation.py:37-42)."""
    inv = rope_inv_freq(dim, theta, positions.device)
    ang = positions.to(torch.float32)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


_ROPE_CPU_TABLES: "dict" = {}


def rope_tables(S: int, T: int, dim: int, theta: float, dtype: torch.dtype, device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos / sin for absolute positions S .. S+T-1, memoised per (S, T, dim, theta, dtype, device),
    at most 32 entries (relation.py:45-58)."""
    key = (int(S), int(T), int(dim), float(theta), dtype, str(torch.device(device) if device is not None else "cpu"))
    hit = _ROPE_CPU_TABLES.get(key)
    if hit is None:
        if len(_ROPE_CPU_TABLES) >= 32:
            _ROPE_CPU_TABLES.clear()
        hit = _rope_cos_sin(torch.arange(S, S + T, device=device), dim, theta, dtype)
        _ROPE_CPU_TABLES[key] = hit
    return hit


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    """(x1, x2) -> (-x2, x1) over the two halves of the last axis (relation.py:61-63)."""
    half = x.shape[-1] // 2
    return torch.cat([-x[..., half:], x[..., :half]], dim=-1)


def _apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, H, T, dh] rotated by tables [T, dh]: x cos + rotate_half(x) sin (relation.py:66-68)."""
    return x * cos[None, None] + _rotate_half(x) * sin[None, None]


# ---- mote::rope_givens ---------------------------------------------------------------------------
def _heads_out(B, T, H, D, like, dtype):
    return torch.empty(B, T, H, D, device=like.device, dtype=dtype).transpose(1, 2)


@torch.library.custom_op("mote::rope_givens", mutates_args=())
def _rope_givens(qkv: torch.Tensor, inv_freq: Optional[torch.Tensor], theta: Optional[torch.Tensor], n_heads: int,
                 parity: int, pos0: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, T, D3 = qkv.shape
    H = n_heads
    D = D3 // (3 * H)
    if not qkv.is_cuda:
        raise RuntimeError("mote::rope_givens needs the HIP library and an MI355X")
    qkv = qkv if qkv.stride(-1) == 1 else qkv.contiguous()
    p1 = _heads_out(B, T, H, D, qkv, qkv.dtype)
    p2 = _heads_out(B, T, H, D, qkv, qkv.dtype)
    info = _heads_out(B, T, H, D, qkv, qkv.dtype)
    a = L.RopeArgs()
    a.dtype = L.dtype_code(qkv)
    a.B, a.T, a.H, a.D, a.pos0, a.layer_parity = B, T, H, D, int(pos0), int(parity)
    inv = None if inv_freq is None else inv_freq.to(device=qkv.device, dtype=torch.float32).contiguous()
    th = None if theta is None else theta.detach().to(device=qkv.device, dtype=torch.float32).contiguous()
    a.inv_freq, a.theta = L.ptr(inv), L.ptr(th)
    a.qkv, a.qkv_sb, a.qkv_sr = qkv.data_ptr(), qkv.stride(0), qkv.stride(1)
    a.p1, a.p2, a.info = L.view(p1), L.view(p2), L.view(info)
    L.check(L.lib().mote_rope_givens_fwd(a, L.stream_of(qkv)), "mote_rope_givens_fwd")
    return p1, p2, info


@_rope_givens.register_fake
def _rope_givens_fake(qkv, inv_freq, theta, n_heads, parity, pos0):
    B, T, D3 = qkv.shape
    H = n_heads
    D = D3 // (3 * H)
    mk = lambda: qkv.new_empty((B, T, H, D)).transpose(1, 2)
    return mk(), mk(), mk()


@torch.library.custom_op("mote::rope_givens_bwd", mutates_args=())
def _rope_givens_bwd(dp1: torch.Tensor, dp2: torch.Tensor, dinfo: torch.Tensor, qkv: torch.Tensor,
                     inv_freq: Optional[torch.Tensor], theta: Optional[torch.Tensor], n_heads: int, parity: int,
                     pos0: int, info_only: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """(dqkv [B, T, 3 H dh], dtheta). qkv is the projection output, or with info_only its I~ part
    alone ([B, T, H dh]): the backward reads only the I~ columns (for dtheta)."""
    B, T, Dx = qkv.shape
    H = n_heads
    D = Dx // H if info_only else Dx // (3 * H)
    D3 = 3 * H * D
    qkv = qkv if qkv.stride(-1) == 1 else qkv.contiguous()
    dp1, dp2, dinfo = (t.to(qkv.dtype) if t.stride(-1) == 1 else t.to(qkv.dtype).contiguous() for t in (dp1, dp2, dinfo))
    dqkv = torch.empty(B, T, D3, device=qkv.device, dtype=qkv.dtype)
    # written whole by the kernel when theta is given
    dtheta = (torch.empty if theta is not None else torch.zeros)(max(H // 2, 1), device=qkv.device, dtype=torch.float32)
    a = L.RopeBwdArgs()
    a.dtype = L.dtype_code(qkv)
    a.B, a.T, a.H, a.D, a.pos0, a.layer_parity = B, T, H, D, int(pos0), int(parity)
    inv = None if inv_freq is None else inv_freq.to(device=qkv.device, dtype=torch.float32).contiguous()
    th = None if theta is None else theta.detach().to(device=qkv.device, dtype=torch.float32).contiguous()
    a.inv_freq, a.theta = L.ptr(inv), L.ptr(th)
    a.qkv, a.qkv_sb, a.qkv_sr = qkv.data_ptr(), qkv.stride(0), qkv.stride(1)
    a.qkv_info_only = int(bool(info_only))
    a.dp1, a.dp2, a.dinfo = L.view(dp1), L.view(dp2), L.view(dinfo)
    a.dqkv, a.dqkv_sb, a.dqkv_sr = dqkv.data_ptr(), dqkv.stride(0), dqkv.stride(1)
    a.dtheta = dtheta.data_ptr()
    nbytes = L.lib().mote_rope_givens_bwd_workspace(a)
    ws = torch.empty(max(int(nbytes), 16), device=qkv.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    L.check(L.lib().mote_rope_givens_bwd(a, L.stream_of(qkv)), "mote_rope_givens_bwd")
    return dqkv, dtheta


@_rope_givens_bwd.register_fake
def _rope_givens_bwd_fake(dp1, dp2, dinfo, qkv, inv_freq, theta, n_heads, parity, pos0, info_only=False):
    B, T, Dx = qkv.shape
    D3 = 3 * Dx if info_only else Dx
    return qkv.new_empty((B, T, D3)), qkv.new_empty((max(n_heads // 2, 1),), dtype=torch.float32)


def _rg_setup(ctx, inputs, output):
    qkv, inv_freq, theta, n_heads, parity, pos0 = inputs
    ctx.save_for_backward(qkv, inv_freq, theta)
    ctx.has_theta = theta is not None
    ctx.n_heads, ctx.parity, ctx.pos0 = n_heads, parity, pos0


def _rg_backward(ctx, dp1, dp2, dinfo):
    qkv, inv_freq, theta = ctx.saved_tensors
    B, T, D3 = qkv.shape
    H = ctx.n_heads
    D = D3 // (3 * H)
    z = lambda: torch.zeros(B, H, T, D, device=qkv.device, dtype=qkv.dtype)
    dp1 = z() if dp1 is None else dp1
    dp2 = z() if dp2 is None else dp2
    dinfo = z() if dinfo is None else dinfo
    dqkv, dtheta = _rope_givens_bwd(dp1, dp2, dinfo, qkv, inv_freq, theta, H, ctx.parity, ctx.pos0)
    return dqkv, None, (dtheta[: H // 2] if ctx.has_theta else None), None, None, None


_rope_givens.register_autograd(_rg_backward, setup_context=_rg_setup)


def rope_givens(qkv: torch.Tensor, n_heads: int, inv_freq: Optional[torch.Tensor], theta: Optional[torch.Tensor],
                layer_idx: int, pos0: int = 0):
    """[B, T, 3*H*dh] projections -> (p1, p2, I~) as [B, H, T, dh] views: RoPE at positions
    pos0.. on p1/p2 (relation.py:211-214), Givens on I~ (relation.py:215). Differentiable in qkv
    and theta."""
    return _rope_givens(qkv, inv_freq, theta, int(n_heads), int(layer_idx) % 2, int(pos0))


# ---- mote::qkv_rope (fused projection prologue) ----------------------------------------------------
USE_FUSED_PROLOGUE = True   # bf16 activations, head dim 64 / 96 / 128 (with or without QK-Norm): one
                            # launch for the projections, QK-Norm and RoPE / Givens, at every row count;
                            # the unfused path serves everything else. Against hipBLASLt's product plus
                            # the RoPE kernel at width 768 it measured 28.6 / 34.8 us at 4,964 rows
                            # (dh 96) and 365 / 414, 369 / 403, 407 / 406 us at 79,424 rows (dh 96,
                            # 128, 64).


# cos / sin tables of the fused prologue, memoised per (device, stream, inv_freq, T, pos0) the way
# the reference memoises its RoPE tables (at most 32 entries, relation.py:45-58): every layer of a
# step asks for the same positions. Keyed by stream as well, so a table is only reused behind the
# launch that wrote it. A graph capture reuses a table written before the capture began (on the
# capture stream) and pins it, since the graph keeps its address; a table missing at capture time
# is computed inside the graph on every replay and not memoised (its memory belongs to the graph).
_ROPE_TABLES: "dict" = {}          # key -> (inv_freq, its version, table)
_ROPE_TABLES_PINNED: "dict" = {}   # tables a captured graph reads, kept for the life of the process
_ROPE_TABLES_MAX = 32


def _rope_table_ws(a, x: torch.Tensor, inv: Optional[torch.Tensor], cacheable: bool) -> Tuple[torch.Tensor, int]:
    """Workspace for mote_qkv_rope_fwd and whether it already holds the table (table_ready).
    `cacheable`: inv is the caller's own frequency tensor (not a converted temporary)."""
    n = max(int(L.lib().mote_qkv_rope_workspace(a)), 16)
    if inv is None or not cacheable:
        return torch.empty(n, device=x.device, dtype=torch.uint8), 0
    key = (x.device, torch.cuda.current_stream(x.device).cuda_stream, inv.data_ptr(), a.T, a.pos0, a.D)
    hit = _ROPE_TABLES.get(key)
    # the entry holds the frequency tensor itself: its memory cannot be recycled for another tensor
    # while the entry lives, and an in-place change of it shows in its version counter
    valid = hit is not None and hit[0] is inv and hit[1] == inv._version
    if torch.cuda.is_current_stream_capturing():
        if valid:
            _ROPE_TABLES_PINNED[hit[2].data_ptr()] = hit[2]
            return hit[2], 1
        return torch.empty(n, device=x.device, dtype=torch.uint8), 0
    if valid:
        return hit[2], 1
    if hit is None and len(_ROPE_TABLES) >= _ROPE_TABLES_MAX:
        _ROPE_TABLES.pop(next(iter(_ROPE_TABLES)))  # a pinned table stays alive through the pin
    ws = torch.empty(n, device=x.device, dtype=torch.uint8)
    _ROPE_TABLES[key] = (inv, inv._version, ws)
    return ws, 0


@torch.library.custom_op("mote::qkv_rope", mutates_args=())
def _qkv_rope(x: torch.Tensor, w: torch.Tensor, inv_freq: Optional[torch.Tensor], theta: Optional[torch.Tensor],
              n_heads: int, parity: int, pos0: int, keep_info: bool, norm_w1: Optional[torch.Tensor] = None,
              norm_w2: Optional[torch.Tensor] = None, norm_eps: float = 1e-5
              ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(p1, p2, I~) as [B, H, T, dh] views of x [w1; w2; wi]^T after (QK-Norm,) RoPE / Givens, and for
    the backward (keep_info): the I~ projections before the rotation ([B, T, H dh]) and, with QK-Norm,
    the p1 | p2 projections before the norm ([B, T, 2 H dh]); empty otherwise."""
    if not x.is_cuda:
        raise RuntimeError("mote::qkv_rope needs the HIP library and an MI355X")
    B, T, K = x.shape
    H = n_heads
    D = K // H
    norm = norm_w1 is not None
    if norm != (norm_w2 is not None):
        raise ValueError("mote::qkv_rope: QK-Norm needs both gains")
    x = x.contiguous()
    w = w.contiguous()
    p1, p2, info = (_heads_out(B, T, H, D, x, x.dtype) for _ in range(3))
    iraw = torch.empty(B, T, K, device=x.device, dtype=x.dtype) if keep_info else x.new_empty(0)
    qkraw = torch.empty(B, T, 2 * K, device=x.device, dtype=x.dtype) if (keep_info and norm) else x.new_empty(0)
    a = L.QkvRopeArgs()
    a.B, a.T, a.H, a.D, a.pos0, a.layer_parity = B, T, H, D, int(pos0), int(parity)
    a.x, a.x_sb, a.x_sr = x.data_ptr(), x.stride(0), x.stride(1)
    a.w, a.w_sr = w.data_ptr(), w.stride(0)
    inv = None if inv_freq is None else inv_freq.to(device=x.device, dtype=torch.float32).contiguous()
    th = None if theta is None else theta.detach().to(device=x.device, dtype=torch.float32).contiguous()
    a.inv_freq, a.theta = L.ptr(inv), L.ptr(th)
    a.p1, a.p2, a.info = L.view(p1), L.view(p2), L.view(info)
    if keep_info:
        a.info_raw, a.ir_sb, a.ir_sr = iraw.data_ptr(), iraw.stride(0), iraw.stride(1)
    if norm:
        nw1 = norm_w1.detach().to(device=x.device, dtype=torch.float32).contiguous()
        nw2 = norm_w2.detach().to(device=x.device, dtype=torch.float32).contiguous()
        if nw1.numel() != D or nw2.numel() != D:
            raise ValueError("mote::qkv_rope: QK-Norm gains must have head-dim elements")
        a.norm_w1, a.norm_w2, a.norm_eps = nw1.data_ptr(), nw2.data_ptr(), float(norm_eps)
        if keep_info:
            a.qk_raw, a.qr_sb, a.qr_sr = qkraw.data_ptr(), qkraw.stride(0), qkraw.stride(1)
    ws, a.table_ready = _rope_table_ws(a, x, inv, inv is inv_freq)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    L.check(L.lib().mote_qkv_rope_fwd(a, L.stream_of(x)), "mote_qkv_rope_fwd")
    return p1, p2, info, iraw, qkraw


@_qkv_rope.register_fake
def _qkv_rope_fake(x, w, inv_freq, theta, n_heads, parity, pos0, keep_info, norm_w1=None, norm_w2=None, norm_eps=1e-5):
    B, T, K = x.shape
    D = K // n_heads
    mk = lambda: x.new_empty((B, T, n_heads, D)).transpose(1, 2)
    norm = norm_w1 is not None
    return (mk(), mk(), mk(), (x.new_empty((B, T, K)) if keep_info else x.new_empty(0)),
            (x.new_empty((B, T, 2 * K)) if (keep_info and norm) else x.new_empty(0)))


def _qr_setup(ctx, inputs, output):
    x, w, inv_freq, theta, n_heads, parity, pos0, keep_info, norm_w1, norm_w2, norm_eps = inputs
    ctx.save_for_backward(x, w, inv_freq, theta, output[3], norm_w1, norm_w2, output[4])
    ctx.has_theta = theta is not None
    ctx.norm = norm_w1 is not None
    ctx.keep = keep_info
    ctx.n_heads, ctx.parity, ctx.pos0, ctx.eps = n_heads, parity, pos0, norm_eps


@torch.library.custom_op("mote::head_rms_norm_bwd_", mutates_args=("dqkv",))
def _head_norm_bwd_(dqkv: torch.Tensor, qkraw: torch.Tensor, gain1: torch.Tensor, gain2: torch.Tensor, eps: float,
                    n_heads: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Backward of QK-Norm (relation.py:71-94) on p1 | p2 of the prologue, in place: the first 2 H dh
    columns of dqkv [B, T, 3 H dh] (gradients of the normalised projections) become the gradients
    of the raw projections qkraw [B, T, 2 H dh]; returns the two gains' gradients (fp32). One launch
    of mote_head_rms_norm_bwd (per head row g = dy gain, r = rsqrt(mean(x^2) + eps):
    dx = r g - r^3 x mean(g x), dgain = sum of dy x r)."""
    if not dqkv.is_cuda:
        raise RuntimeError("mote::head_rms_norm_bwd_ needs the HIP library and an MI355X")
    B, T, K3 = dqkv.shape
    K = K3 // 3
    D = K // n_heads
    if B * T == 0:
        z = torch.zeros(D, device=dqkv.device, dtype=torch.float32)
        return z, z.clone()
    if dqkv.stride(2) != 1 or qkraw.stride(2) != 1 or (B > 1 and (dqkv.stride(0) != T * dqkv.stride(1) or
                                                               qkraw.stride(0) != T * qkraw.stride(1))):
        raise ValueError("mote::head_rms_norm_bwd_: token rows must be back to back with unit column stride")
    g1 = gain1.detach().to(device=dqkv.device, dtype=torch.float32).contiguous()
    g2 = gain2.detach().to(device=dqkv.device, dtype=torch.float32).contiguous()
    dg1 = torch.empty(D, device=dqkv.device, dtype=torch.float32)
    dg2 = torch.empty(D, device=dqkv.device, dtype=torch.float32)
    a = L.HeadNormBwdArgs()
    a.dtype, a.rows, a.parts, a.H, a.D, a.eps = L.dtype_code(dqkv), B * T, 2, int(n_heads), D, float(eps)
    a.x, a.x_sr = qkraw.data_ptr(), qkraw.stride(1)
    a.dy, a.dy_sr = dqkv.data_ptr(), dqkv.stride(1)
    a.dx, a.dx_sr = dqkv.data_ptr(), dqkv.stride(1)
    a.gain0, a.gain1, a.dgain0, a.dgain1 = g1.data_ptr(), g2.data_ptr(), dg1.data_ptr(), dg2.data_ptr()
    ws = torch.empty(max(int(L.lib().mote_head_rms_norm_bwd_workspace(a)), 16), device=dqkv.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    L.check(L.lib().mote_head_rms_norm_bwd(a, L.stream_of(dqkv)), "mote_head_rms_norm_bwd")
    return dg1, dg2


@_head_norm_bwd_.register_fake
def _head_norm_bwd_fake(dqkv, qkraw, gain1, gain2, eps, n_heads):
    D = dqkv.shape[-1] // 3 // n_heads
    return dqkv.new_empty(D, dtype=torch.float32), dqkv.new_empty(D, dtype=torch.float32)


# ---- mote::wgrad (weight gradient of the projections) -------------------------------------------
USE_WGRAD = True  # bf16 rows, both widths multiples of 128: mote_wgrad; else the GEMM library


@torch.library.custom_op("mote::wgrad", mutates_args=())
def _wgrad(a: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """bf16 dW [N, K] = a^T x for a [M, N], x [M, K], fp32 sums (operands whose rows are not unit-stride
    and 16-byte aligned are copied first)."""
    if not a.is_cuda:
        raise RuntimeError("mote::wgrad needs the HIP library and an MI355X")
    ok = lambda t: t.stride(1) == 1 and (t.stride(0) * 2) % 16 == 0 and t.data_ptr() % 16 == 0
    a = a if ok(a) else a.contiguous()
    x = x if ok(x) else x.contiguous()
    M, N = a.shape
    K = x.shape[1]
    dw = torch.empty(N, K, device=a.device, dtype=a.dtype)
    args = L.WgradArgs()
    args.dtype, args.M, args.N, args.K = L.dtype_code(a), M, N, K
    args.a, args.a_sr = a.data_ptr(), a.stride(0)
    args.x, args.x_sr = x.data_ptr(), x.stride(0)
    args.dw, args.dw_sr = dw.data_ptr(), dw.stride(0)
    nbytes = int(L.lib().mote_wgrad_workspace(args))
    ws = torch.empty(max(nbytes, 16), device=a.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    L.check(L.lib().mote_wgrad(args, L.stream_of(a)), "mote_wgrad")
    return dw


@_wgrad.register_fake
def _wgrad_fake(a, x):
    return a.new_empty((a.shape[1], x.shape[1]))


def weight_grad(a: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """a^T x over the token rows of a [..., N] and x [..., K]: the weight gradient of y = x W^T.
    mote_wgrad for bf16 on the GPU with N, K multiples of 128; the GEMM library otherwise."""
    N, K = a.shape[-1], x.shape[-1]
    a2, x2 = a.reshape(-1, N), x.reshape(-1, K)
    if (USE_WGRAD and a2.is_cuda and a2.dtype == torch.bfloat16 and x2.dtype == torch.bfloat16
            and N % 128 == 0 and K % 128 == 0):
        return _wgrad(a2, x2)
    return torch.matmul(a2.t(), x2)


class _LinearWgrad(torch.autograd.Function):
    """y = x W^T on the GEMM library; backward dx = dy W on the library and dW = dy^T x on
    mote_wgrad (the library runs that product with its reduction over the token rows)."""

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return F.linear(x, w)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx = torch.matmul(dy, w) if ctx.needs_input_grad[0] else None
        dw = weight_grad(dy, x) if ctx.needs_input_grad[1] else None
        return dx, dw


def linear_wgrad(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """F.linear(x, w) whose weight gradient runs on mote_wgrad: bf16 x and w on the GPU (or bf16
    autocast, which casts both as F.linear would) with both widths multiples of 128; F.linear otherwise."""
    if torch.is_autocast_enabled() and torch.get_autocast_dtype("cuda") == torch.bfloat16 and x.is_cuda:
        x, w = x.to(torch.bfloat16), w.to(torch.bfloat16)
    if (USE_WGRAD and x.is_cuda and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
            and w.shape[0] % 128 == 0 and w.shape[1] % 128 == 0):
        return _LinearWgrad.apply(x, w)
    return F.linear(x, w)


def _qr_backward(ctx, dp1, dp2, dinfo, _diraw, _dqkraw):
    x, w, inv_freq, theta, iraw, norm_w1, norm_w2, qkraw = ctx.saved_tensors
    if (ctx.has_theta or ctx.norm) and not ctx.keep:
        raise RuntimeError("mote::qkv_rope: the backward needs keep_info=True with theta or QK-Norm")
    B, T, K = x.shape
    H = ctx.n_heads
    D = K // H
    z = lambda: torch.zeros(B, H, T, D, device=x.device, dtype=x.dtype)
    dp1 = z() if dp1 is None else dp1
    dp2 = z() if dp2 is None else dp2
    dinfo = z() if dinfo is None else dinfo
    src = iraw if ctx.keep else x.new_empty(B, T, K)  # read only for dtheta
    dqkv, dtheta = _rope_givens_bwd(dp1, dp2, dinfo, src, inv_freq, theta, H, ctx.parity, ctx.pos0, True)
    dn1 = dn2 = None
    if ctx.norm:  # gradients of the normalised p1 / p2 back through QK-Norm, in place in dqkv
        dn1, dn2 = _head_norm_bwd_(dqkv, qkraw, norm_w1, norm_w2, ctx.eps, H)
        dn1, dn2 = dn1.to(norm_w1.dtype), dn2.to(norm_w2.dtype)
    dx = torch.matmul(dqkv, w)                                        # [B, T, 3K] x [3K, K]
    dw = weight_grad(dqkv, x)                                        # [3K, K]
    return (dx, dw, None, (dtheta[: H // 2] if ctx.has_theta else None), None, None, None, None, dn1, dn2, None)


_qkv_rope.register_autograd(_qr_backward, setup_context=_qr_setup)


def qkv_rope(x: torch.Tensor, w: torch.Tensor, n_heads: int, inv_freq: Optional[torch.Tensor],
             theta: Optional[torch.Tensor], layer_idx: int, pos0: int = 0,
             norm: Optional[Tuple[torch.Tensor, torch.Tensor, float]] = None):
    """The fused prologue: bf16 x [B, T, H dh] and w = [w1; w2; wi] [3 H dh, H dh] -> (p1, p2, I~),
    the same as rope_givens(F.linear(x, w), ...) (relation.py:199-215); `norm` = (p1 gain, p2 gain,
    eps) applies QK-Norm to p1 / p2 first (relation.py:208-210). Differentiable in x, w, theta and
    the gains."""
    n1, n2, eps = norm if norm is not None else (None, None, 1e-5)
    keep = torch.is_grad_enabled() and (theta is not None or norm is not None)
    p1, p2, info, _, _ = _qkv_rope(x, w, inv_freq, theta, int(n_heads), int(layer_idx) % 2, int(pos0), keep,
                                   n1, n2, float(eps))
    return p1, p2, info


# ---- mote::out_gate (the output gate of _out) ----------------------------------------------------
@torch.library.custom_op("mote::out_gate", mutates_args=())
def _out_gate(x: torch.Tensor, wg: torch.Tensor, y: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 (z, s): z = y * sigmoid(x wg^T) and s = the sigmoid, [B, T, D] (relation.py:179-181)."""
    if not x.is_cuda:
        raise RuntimeError("mote::out_gate needs the HIP library and an MI355X")
    B, T, D = x.shape
    x2 = x.reshape(B * T, D).contiguous()
    y2 = y.reshape(B * T, D).contiguous()
    wc = wg.contiguous()
    z = torch.empty(B, T, D, device=x.device, dtype=x.dtype)
    s = torch.empty(B, T, D, device=x.device, dtype=x.dtype)
    a = L.GateProductArgs()
    a.B, a.T, a.D = 1, B * T, D
    a.x, a.x_sr = x2.data_ptr(), x2.stride(0)
    a.w, a.w_sr = wc.data_ptr(), wc.stride(0)
    a.y, a.y_sr = y2.data_ptr(), y2.stride(0)
    a.z, a.s, a.z_sr = z.data_ptr(), s.data_ptr(), D
    L.check(L.lib().mote_gate_product(a, L.stream_of(x)), "mote_gate_product")
    return z, s


@_out_gate.register_fake
def _out_gate_fake(x, wg, y):
    return x.new_empty(x.shape), x.new_empty(x.shape)


def _og_setup(ctx, inputs, output):
    x, wg, y = inputs
    ctx.save_for_backward(x, wg, y, output[1])


def _og_backward(ctx, dz, _ds):
    """z = y s, s = sigmoid(g), g = x wg^T: dy = dz s, dg = dz y s (1 - s), dx = dg wg, dwg = dg^T x."""
    x, wg, y, s = ctx.saved_tensors
    dzf, sf = dz.float(), s.float()
    dy = (dzf * sf).to(y.dtype)
    dg = (dzf * y.float() * sf * (1.0 - sf)).to(x.dtype)
    D = x.shape[-1]
    dx = torch.matmul(dg, wg)
    dwg = weight_grad(dg, x)
    return dx, dwg, dy


_out_gate.register_autograd(_og_backward, setup_context=_og_setup)
USE_FUSED_GATE = True  # bf16 and a width that is a multiple of 128: the gate product kernel


def out_gate(x: torch.Tensor, wg: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """y * sigmoid(x wg^T) in one launch (bf16 x, wg, y [B, T, D]); differentiable in all three."""
    return _out_gate(x, wg, y)[0]


class HeadRMSNorm(nn.Module):
    """QK-Norm over the head dim with a learnable gain (relation.py:71-94); fp32 math."""

    def __init__(self, dim: int, eps: float = 1e-5, device=None, dtype=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class FullRelation(nn.Module):
    def __init__(self, d_model: int, n_heads: int, layer_idx: int, tau_s: float = 2.0, lambda_init: float = 0.5,
                 rope_theta: float = 10000.0, givens: bool = True, qk_norm: bool = False, out_gate: bool = False,
                 rope: bool = True, device=None, dtype=None):
        super().__init__()
        assert d_model % n_heads == 0, "d_model must be divisible by n_heads"
        assert n_heads % 2 == 0, "Givens pairing needs an even number of heads"
        fk = {"device": device, "dtype": dtype}
        self.d_model, self.n_heads, self.d_head = d_model, n_heads, d_model // n_heads
        assert self.d_head % 2 == 0, "head dim must be even for RoPE"
        self.layer_idx = layer_idx
        self.tau_s = tau_s
        self.rope_theta = rope_theta
        self.use_givens = givens
        self.telemetry: Optional[dict] = None
        self.qk_norm = qk_norm
        if qk_norm:
            self.p1_norm = HeadRMSNorm(self.d_head, **fk)
            self.p2_norm = HeadRMSNorm(self.d_head, **fk)
        self.w1 = nn.Linear(d_model, d_model, bias=False, **fk)
        self.w2 = nn.Linear(d_model, d_model, bias=False, **fk)
        self.wi = nn.Linear(d_model, d_model, bias=False, **fk)
        self.wo = nn.Linear(d_model, d_model, bias=False, **fk)
        self.out_gate = out_gate
        if out_gate:
            self.wg = nn.Linear(d_model, d_model, bias=False, **fk)
        self.use_rope = rope
        self.lam = nn.Parameter(torch.tensor(float(lambda_init), dtype=torch.float32, device=device))
        self.lam._no_weight_decay = True
        if givens:
            self.theta = nn.Parameter(torch.zeros(n_heads // 2, dtype=torch.float32, device=device))
            self.theta._no_weight_decay = True
            if layer_idx % 2 == 0:
                a = torch.arange(0, n_heads, 2)
                b = torch.arange(1, n_heads, 2)
            else:
                a = torch.arange(1, n_heads, 2)
                b = (torch.arange(2, n_heads + 1, 2)) % n_heads
            self.register_buffer("pair_a", a, persistent=False)
            self.register_buffer("pair_b", b, persistent=False)
        self.register_buffer("inv_freq", rope_inv_freq(self.d_head, rope_theta, device), persistent=False)

    def _apply(self, fn, recurse=True):
        # `.to(dtype)`, `.half()`, `.bfloat16()` would round the RoPE frequencies (an angle error of
        # radians at positions in the thousands); the reference recomputes them in fp32 on every call
        # (relation.py:39). Keep the buffer fp32 on whatever device the parameters moved to.
        super()._apply(fn, recurse)
        self._buffers["inv_freq"] = rope_inv_freq(self.d_head, self.rope_theta, self.lam.device)
        return self

    def _givens(self, info: torch.Tensor) -> torch.Tensor:
        """Givens mixing of head pairs for callers that rotate rows themselves (relation.py:160-174,
        graph.py:165): info [B, H, T, dh]; pairs (0,1),(2,3),... on even layers, (1,2),...,(H-1,0) on
        odd ones; (a, b) -> (c a - s b, s a + c b) with c, s = cos / sin(theta) in info's dtype. The
        module's forward applies the same rotation inside its HIP prologue kernels."""
        if not self.use_givens:
            return info
        H = info.shape[1]
        c = torch.cos(self.theta).to(info.dtype)[None, :, None, None]
        s = torch.sin(self.theta).to(info.dtype)[None, :, None, None]
        first = torch.arange(self.layer_idx % 2, H, 2, device=info.device)
        second = (first + 1) % H
        ia, ib = info.index_select(1, first), info.index_select(1, second)
        out = torch.empty_like(info)
        out.index_copy_(1, first, c * ia - s * ib)
        out.index_copy_(1, second, s * ia + c * ib)
        return out

    # ------------------------------------------------------------------------------------------
    def heads(self, x: torch.Tensor, S: int):
        """Projections -> (QK-Norm) -> RoPE / Givens: (p1, p2, I~) as [B, H, T, dh] views."""
        B, T, D = x.shape
        H, dh = self.n_heads, self.d_head
        w = torch.cat([self.w1.weight, self.w2.weight, self.wi.weight], dim=0)
        inv = self.inv_freq if self.use_rope else None
        theta = self.theta if self.use_givens else None
        bf16 = x.dtype == torch.bfloat16 or (torch.is_autocast_enabled() and
                                             torch.get_autocast_dtype("cuda") == torch.bfloat16)
        if USE_FUSED_PROLOGUE and bf16 and dh in (64, 96, 128) and (H * dh) % 32 == 0:
            norm = (self.p1_norm.weight, self.p2_norm.weight, self.p1_norm.eps) if self.qk_norm else None
            return qkv_rope(x.to(torch.bfloat16), w.to(torch.bfloat16), H, inv, theta, self.layer_idx, S, norm)
        qkv = F.linear(x, w)
        if self.qk_norm:
            q, k, v = qkv.split(D, dim=-1)
            q = self.p1_norm(q.reshape(B, T, H, dh)).reshape(B, T, D)
            k = self.p2_norm(k.reshape(B, T, H, dh)).reshape(B, T, D)
            qkv = torch.cat([q, k, v], dim=-1)
        return rope_givens(qkv, H, inv, theta, self.layer_idx, S)

    def _out(self, y: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """[B, H, T, dh] -> [B, T, D] -> optional output gate -> wo (relation.py:176-182)."""
        B, H, T, dh = y.shape
        y = y.transpose(1, 2).reshape(B, T, H * dh)
        if self.out_gate:
            bf16 = y.dtype == torch.bfloat16 and (x.dtype == torch.bfloat16 or torch.is_autocast_enabled())
            if USE_FUSED_GATE and bf16 and y.is_cuda and (H * dh) % 128 == 0:
                y = out_gate(x.to(torch.bfloat16), self.wg.weight.to(torch.bfloat16), y)
            else:
                y = y * torch.sigmoid(self.wg(x))
        return linear_wgrad(y, self.wo.weight)

    def forward(self, x: torch.Tensor, cache: Optional[RelationCache] = None, return_cache: bool = False,
                return_gates: bool = False):
        """x: [B, T, D]. With a cache, x holds the new T positions appended after S cached ones.
        Returns out [B, T, D], then (in this order, when asked) the updated cache and the exchange
        mass g [B, H, T] (relation.py:184-268)."""
        if not USE_FLASH:
            raise RuntimeError("mote_amd.relation has only the HIP path (USE_FLASH = False is not supported)")
        if not x.is_cuda:
            raise RuntimeError("FullRelation needs the HIP library and an MI355X (x is on the CPU)")
        B, T, D = x.shape
        arena = isinstance(cache, ArenaLayer)
        S = cache.n if arena else (0 if cache is None else cache[0].shape[2])
        p1, p2, info = self.heads(x, S)
        if arena:
            cache.write(p2, info)
            p2_all, info_all = cache.views(S + T)
        elif cache is not None:
            p2_all = torch.cat([cache[0], p2], dim=2)
            info_all = torch.cat([cache[1], info], dim=2)
        else:
            p2_all, info_all = p2, info
        new_cache = cache if arena else (p2_all, info_all)
        if p2_all.dtype != p1.dtype:  # an arena kept in another dtype than the activations
            p1 = p1.to(p2_all.dtype)
        y, g = flash_relation(p1, p2_all, info_all, self.lam, self.tau_s, q_start=S)
        if y.dtype != x.dtype and not torch.is_autocast_enabled():
            y = y.to(x.dtype)  # an arena in a narrower dtype than an fp32 module
        out = self._out(y, x)
        extras = []
        if return_cache:
            extras.append(new_cache)
        if self.telemetry is not None:
            self.telemetry["exchange_mass"] = float(g[0, :, -1].detach().mean())
        if return_gates:
            extras.append(g)
        return (out, *extras) if extras else out
