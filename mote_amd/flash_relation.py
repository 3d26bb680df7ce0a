"""FlashRelation on MI355X — the fused Relation core behind Mote's call signatures.

Mirrors mote/model/flash_relation.py: the same public function `flash_relation`, the same
`torch.library` custom ops `mote::relation_fwd` / `mote::relation_bwd` (schemas of
flash_relation.py:620-641, with fake implementations and autograd, so `torch.compile(fullgraph=True)`
traces through them), the same `DETERMINISTIC` switch (MOTE_DETERMINISTIC_RELATION,
flash_relation.py:51). The kernels are the hand-written HIP ones in libmote_relation.so; there is no
other implementation behind these names, and calling them without the library or without a GPU
raises.

Additions with no counterpart in the reference:
* `flash_relation_varlen` / `mote::relation_fwd_varlen`: packed sequences with `cu_seqlens` (the
  reference pads to a bucket instead, mote/model/dc.py:192-218).
* Output layout: Y is allocated token-major ([B, T, H, D] memory, returned as the [B, H, T, D]
  view), so `FullRelation._out`'s transpose to [B, T, H*D] is free.
"""

from __future__ import annotations

import math
import os
from typing import Tuple

import torch
import torch.nn.functional as F

from . import _lib as L

DETERMINISTIC = os.environ.get("MOTE_DETERMINISTIC_RELATION", "0") == "1"  # atomic-free backward


def _hip_ready() -> bool:
    return L.available() and torch.cuda.is_available()


HAS_HIP = _hip_ready()
HAS_TRITON = HAS_HIP  # the name the reference's callers test (relation.py:29, 228); no Triton here


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """The kernels read 16-byte chunks: unit stride on the last axis, strides a multiple of the
    chunk and a 16-byte aligned base. Anything else is copied to a contiguous tensor."""
    epc = 16 // t.element_size()
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % epc for s in t.stride()[:-1]):
        return t.contiguous()
    return t


def _check_device(*ts):
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("flash_relation needs the HIP library and an MI355X: tensors are on the CPU")


def _token_major(B, H, T, D, like: torch.Tensor, dtype) -> torch.Tensor:
    """Empty [B, H, T, D] view over [B, T, H, D] memory."""
    return torch.empty(B, T, H, D, device=like.device, dtype=dtype).transpose(1, 2)


def _fwd_workspace(a, device):
    """Scratch for the split of the longest query blocks (partial softmax states); the caller keeps
    the returned tensor alive until the launch is queued (the caching allocator orders reuse)."""
    n = int(L.lib().mote_relation_fwd_workspace(a))
    if n == 0:
        a.workspace, a.workspace_bytes = None, 0
        return None
    ws = torch.empty(n, device=device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), n
    return ws


def _launch_fwd(p1, p2, info, lam, tau_s: float, q_start: int):
    B, H, TQ, D = p1.shape
    TK = p2.shape[2]
    if TK != q_start + TQ:
        raise ValueError("keys must cover exactly the cached prefix plus the new positions")
    if p2.dtype != p1.dtype or info.dtype != p1.dtype:
        raise TypeError("p1, p2 and info must share a dtype")
    _check_device(p1, p2, info, lam)
    p1, p2, info = _aligned(p1), _aligned(p2), _aligned(info)
    lam32 = lam.detach().to(torch.float32).reshape(1).contiguous()
    y = _token_major(B, H, TQ, D, p1, info.dtype)
    ibar = torch.empty(B, H, TQ, D, device=p1.device, dtype=torch.float32)
    lse = torch.empty(B, H, TQ, device=p1.device, dtype=torch.float32)
    g = torch.empty(B, H, TQ, device=p1.device, dtype=torch.float32)
    a = L.FwdArgs()
    a.dtype = L.dtype_code(p1)
    a.B, a.H, a.TQ, a.TK, a.D, a.q_start = B, H, TQ, TK, D, q_start
    a.tau_s = float(tau_s)
    a.p1, a.p2, a.info, a.y = L.view(p1), L.view(p2), L.view(info), L.view(y)
    a.ibar, a.lse, a.g, a.lam = ibar.data_ptr(), lse.data_ptr(), g.data_ptr(), lam32.data_ptr()
    a.cu_seqlens, a.total_rows = None, 0
    ws = _fwd_workspace(a, p1.device)
    L.check(L.lib().mote_relation_fwd(a, L.stream_of(p1)), "mote_relation_fwd")
    return y, g, ibar, lse


def _launch_bwd(p1, p2, info, ibar, lse, g, dy, tau_s: float, q_start: int, deterministic: bool):
    B, H, TQ, D = p1.shape
    TK = p2.shape[2]
    _check_device(p1, p2, info, dy)
    p1, p2, info = _aligned(p1), _aligned(p2), _aligned(info)
    dy = _aligned(dy.to(p1.dtype))
    ibar, lse, g = ibar.contiguous(), lse.contiguous(), g.contiguous()
    dp1 = _token_major(B, H, TQ, D, p1, p1.dtype)
    dp2 = _token_major(B, H, TK, D, p1, p2.dtype)
    dinfo = _token_major(B, H, TK, D, p1, info.dtype)
    dlam = torch.empty((), device=p1.device, dtype=torch.float32)
    a = L.BwdArgs()
    a.dtype = L.dtype_code(p1)
    a.B, a.H, a.TQ, a.TK, a.D, a.q_start = B, H, TQ, TK, D, q_start
    a.tau_s = float(tau_s)
    a.deterministic = int(bool(deterministic))
    a.p1, a.p2, a.info, a.dy = L.view(p1), L.view(p2), L.view(info), L.view(dy)
    a.ibar, a.lse, a.g = ibar.data_ptr(), lse.data_ptr(), g.data_ptr()
    a.dp1, a.dp2, a.dinfo = L.view(dp1), L.view(dp2), L.view(dinfo)
    a.dlam = dlam.data_ptr()
    nbytes = L.lib().mote_relation_bwd_workspace(a)
    ws = torch.empty(max(int(nbytes), 16), device=p1.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    L.check(L.lib().mote_relation_bwd(a, L.stream_of(p1)), "mote_relation_bwd")
    return dp1, dp2, dinfo, dlam


@torch.library.custom_op("mote::relation_fwd", mutates_args=())
def _relation_fwd(p1: torch.Tensor, p2: torch.Tensor, info: torch.Tensor, lam: torch.Tensor, tau_s: float,
                  q_start: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    return _launch_fwd(p1, p2, info, lam, tau_s, q_start)


@_relation_fwd.register_fake
def _relation_fwd_fake(p1, p2, info, lam, tau_s, q_start):
    B, H, TQ, D = p1.shape
    return (
        p1.new_empty((B, TQ, H, D), dtype=info.dtype).transpose(1, 2),
        p1.new_empty((B, H, TQ), dtype=torch.float32),
        p1.new_empty((B, H, TQ, D), dtype=torch.float32),
        p1.new_empty((B, H, TQ), dtype=torch.float32),
    )


@torch.library.custom_op("mote::relation_bwd", mutates_args=())
def _relation_bwd(p1: torch.Tensor, p2: torch.Tensor, info: torch.Tensor, ibar: torch.Tensor, lse: torch.Tensor,
                  g: torch.Tensor, dy: torch.Tensor, tau_s: float,
                  q_start: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    return _launch_bwd(p1, p2, info, ibar, lse, g, dy, tau_s, q_start, DETERMINISTIC)


@_relation_bwd.register_fake
def _relation_bwd_fake(p1, p2, info, ibar, lse, g, dy, tau_s, q_start):
    B, H, TQ, D = p1.shape
    TK = p2.shape[2]
    return (
        p1.new_empty((B, TQ, H, D)).transpose(1, 2),
        p1.new_empty((B, TK, H, D), dtype=p2.dtype).transpose(1, 2),
        p1.new_empty((B, TK, H, D), dtype=info.dtype).transpose(1, 2),
        p1.new_empty((), dtype=torch.float32),
    )


def _setup_context(ctx, inputs, output):
    p1, p2, info, lam, tau_s, q_start = inputs
    y, g, ibar, lse = output
    ctx.save_for_backward(p1, p2, info, ibar, lse, g)
    ctx.tau_s, ctx.q_start = tau_s, q_start


def _backward(ctx, dy, _dg, _dibar, _dlse):
    p1, p2, info, ibar, lse, g = ctx.saved_tensors
    dp1, dp2, dinfo, dlam = _relation_bwd(p1, p2, info, ibar, lse, g, dy, ctx.tau_s, ctx.q_start)
    return dp1, dp2, dinfo, dlam, None, None


_relation_fwd.register_autograd(_backward, setup_context=_setup_context)


def flash_relation(p1: torch.Tensor, p2: torch.Tensor, info: torch.Tensor, lam: torch.Tensor, tau_s: float = 2.0,
                   q_start: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused Full Relation (mote/model/flash_relation.py:657-663).

    p1 [B,H,T,D] (RoPE applied); p2/info [B,H,q_start+T,D] (RoPE / Givens applied; any row/head
    strides, e.g. decode-arena views). Returns (Y [B,H,T,D] in info's dtype, g [B,H,T] fp32 exchange
    mass; no gradient flows through g)."""
    if not HAS_HIP or not p1.is_cuda:
        raise RuntimeError("flash_relation needs the HIP library (libmote_relation.so) and an MI355X")
    y, g, _ibar, _lse = _relation_fwd(p1, p2, info, lam, float(tau_s), int(q_start))
    return y, g.detach()


def relation_reference(p1: torch.Tensor, p2: torch.Tensor, info: torch.Tensor, lam: torch.Tensor, tau_s: float = 2.0,
                       q_start: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """The same function materialized in fp32, for callers' tests (flash_relation.py:666-682):
    scores U = p1 P2^T / sqrt(D) over every (query, key) pair, Self sigmoid(U_ii / tau_s) on the
    diagonal, SiLU(U_ij) - lam ln(i + 1) over the strict past, softmax, Y = F I~, g = the past's
    share of F. O(TQ * TK) memory; nothing in this package calls it."""
    TQ, D = p1.shape[-2], p1.shape[-1]
    TK = p2.shape[-2]
    q, k, v = p1.float(), p2.float(), info.float()
    u = torch.matmul(q, k.transpose(-1, -2)) / math.sqrt(D)
    pos = torch.arange(q_start, q_start + TQ, device=q.device).unsqueeze(-1)  # absolute query index
    key = torch.arange(TK, device=q.device).unsqueeze(0)
    count = torch.log((pos + 1).float())
    scores = torch.where(key == pos, torch.sigmoid(u / tau_s), F.silu(u) - lam.float() * count)
    scores = scores.masked_fill(key > pos, float("-inf"))
    flow = torch.softmax(scores, dim=-1)
    return torch.matmul(flow, v), (flow * (key < pos)).sum(-1)


# ---- varlen prefill (forward only) -------------------------------------------------------------
@torch.library.custom_op("mote::relation_fwd_varlen", mutates_args=())
def _relation_fwd_varlen(p1: torch.Tensor, p2: torch.Tensor, info: torch.Tensor, lam: torch.Tensor,
                         cu_seqlens: torch.Tensor, max_seqlen: int,
                         tau_s: float) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    H, total, D = p1.shape
    _check_device(p1, p2, info, lam, cu_seqlens)
    p1, p2, info = (_aligned(t.unsqueeze(0)) for t in (p1, p2, info))
    cu = cu_seqlens.to(torch.int32).contiguous()
    nseq = cu.numel() - 1
    lam32 = lam.detach().to(torch.float32).reshape(1).contiguous()
    y = torch.empty(total, H, D, device=p1.device, dtype=info.dtype).permute(1, 0, 2)
    ibar = torch.empty(H, total, D, device=p1.device, dtype=torch.float32)
    lse = torch.empty(H, total, device=p1.device, dtype=torch.float32)
    g = torch.empty(H, total, device=p1.device, dtype=torch.float32)
    a = L.FwdArgs()
    a.dtype = L.dtype_code(p1)
    a.B, a.H, a.TQ, a.TK, a.D, a.q_start = nseq, H, int(max_seqlen), int(max_seqlen), D, 0
    a.tau_s = float(tau_s)
    a.p1, a.p2, a.info = L.view(p1), L.view(p2), L.view(info)
    a.y = L.view(y.unsqueeze(0))
    a.ibar, a.lse, a.g, a.lam = ibar.data_ptr(), lse.data_ptr(), g.data_ptr(), lam32.data_ptr()
    a.cu_seqlens, a.total_rows = cu.data_ptr(), total
    ws = _fwd_workspace(a, p1.device)
    L.check(L.lib().mote_relation_fwd(a, L.stream_of(p1)), "mote_relation_fwd (varlen)")
    return y, g, ibar, lse


@_relation_fwd_varlen.register_fake
def _relation_fwd_varlen_fake(p1, p2, info, lam, cu_seqlens, max_seqlen, tau_s):
    H, total, D = p1.shape
    return (
        p1.new_empty((total, H, D), dtype=info.dtype).permute(1, 0, 2),
        p1.new_empty((H, total), dtype=torch.float32),
        p1.new_empty((H, total, D), dtype=torch.float32),
        p1.new_empty((H, total), dtype=torch.float32),
    )


def flash_relation_varlen(p1: torch.Tensor, p2: torch.Tensor, info: torch.Tensor, lam: torch.Tensor,
                          cu_seqlens: torch.Tensor, max_seqlen: int, tau_s: float = 2.0):
    """Relation prefill over packed sequences: p1/p2/info are [H, total, D] views (any row/head
    strides, e.g. a [total, H, D] projection output permuted); sequence b owns rows
    [cu_seqlens[b], cu_seqlens[b+1]) and starts at position 0. Returns (Y [H, total, D], g [H, total]).
    Equals `flash_relation` applied to each sequence alone."""
    if not HAS_HIP or not p1.is_cuda:
        raise RuntimeError("flash_relation_varlen needs the HIP library (libmote_relation.so) and an MI355X")
    y, g, _ibar, _lse = _relation_fwd_varlen(p1, p2, info, lam, cu_seqlens, int(max_seqlen), float(tau_s))
    return y, g
