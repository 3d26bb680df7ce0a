"""The one-chunk Relation decode step on MI355X.

`relation_decode` is the core of GraphDecoder._relation_step (mote/infer/graph.py:158-186) as one
HIP launch: RoPE at the device position S, Givens, the cast to the cache dtype, the append of the
new P2 / I~ row at S, and the softmax read of rows [0, S]. `RelationDecodeStep` wraps a FullRelation
layer and its arena rows the way the graph decoder does (projections before, `_out` after) with
static buffers, so a whole step can be captured in a HIP graph (torch.cuda.CUDAGraph) and replayed:
S stays on the device and, with `advance=True`, the kernel itself moves it forward.

Batch B > 1 runs B independent sequences in one launch (the reference decodes batch 1).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from . import _lib as L
from .arena import RelationArena


def decode_workspace(B: int, H: int, D: int, capacity: int, device, dtype=torch.bfloat16) -> torch.Tensor:
    """A workspace for `relation_decode`: per-split partials and the completion counters, zeroed
    here once; every call leaves the counters at zero again. Calls that share one must not overlap."""
    a = L.DecodeArgs()
    a.dtype, a.B, a.H, a.D, a.capacity = L.dtype_code(torch.empty(0, dtype=dtype)), B, H, D, capacity
    n = int(L.lib().mote_relation_decode_workspace(a))
    return torch.zeros(max(n, 16), device=device, dtype=torch.uint8)


def _check_run(run: Optional[torch.Tensor], dev) -> None:
    if run is not None and (run.dtype not in (torch.bool, torch.uint8) or run.numel() != 1 or run.device != dev):
        raise ValueError("run must be a one-element bool or uint8 tensor on the inputs' device")


def _f32_param(t: torch.Tensor, n: int, name: str, dev) -> torch.Tensor:
    if not torch.is_tensor(t) or t.numel() != n or t.device != dev:
        raise ValueError(f"{name} must be a tensor of {n} element(s) on the inputs' device")
    return t.detach().to(torch.float32).reshape(n).contiguous()


def relation_decode(p1: torch.Tensor, p2: torch.Tensor, info: torch.Tensor, S: torch.Tensor, cache_p2: torch.Tensor,
                    cache_info: torch.Tensor, lam: torch.Tensor, tau_s: float = 2.0,
                    inv_freq: Optional[torch.Tensor] = None, theta: Optional[torch.Tensor] = None, layer_idx: int = 0,
                    advance: bool = False, workspace: Optional[torch.Tensor] = None, y: Optional[torch.Tensor] = None,
                    g: Optional[torch.Tensor] = None, xm: Optional[torch.Tensor] = None,
                    run: Optional[torch.Tensor] = None, rope_f32: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """One decode step for B sequences.

    p1, p2, info: raw projections of the new chunk, [B, H, dh] (head stride dh, any batch stride),
        in the cache dtype; RoPE (inv_freq) and Givens (theta, pairing by layer_idx parity) are
        applied on the device.
    S: int64 [B] device positions; row S[b] of the caches receives the new P2 / I~ row.
    cache_p2, cache_info: [B, H, capacity, dh] views (RelationArena.p2(layer) / .info(layer)).
    xm: optional fp32 [B] that receives the mean of g over the heads (graph.py:186), worked out by
        the kernel's last head of each sequence.
    run: optional one-element bool / uint8 device tensor (e.g. the router's boundary bit): when it
        holds 0 the launch writes nothing at all (no append, no advance, no y / g / xm), so one
        captured graph serves both branches of the graph decoder's conditional main step.
    rope_f32: RoPE with fp32 tables and arithmetic, rounded once into the cache dtype (the graph
        decoder's rows when its x is fp32 under serving autocast, graph.py:158-172); otherwise the
        tables and every operation of the rotation round to the cache dtype (x in that dtype).
    Returns (y [B, H, dh] in the cache dtype, g [B, H] fp32 exchange mass = 1 - F_SS).
    """
    if p1.dim() != 3:
        raise ValueError("p1/p2/info must be [B, H, dh]")
    B, H, D = p1.shape
    dev = p1.device
    for t in (p1, p2, info):
        if t.shape != p1.shape or t.stride(-1) != 1 or t.stride(1) != D or t.stride(0) != p1.stride(0):
            raise ValueError("p1/p2/info must be [B, H, dh] with head stride dh and one batch stride")
        if t.dtype != cache_p2.dtype or t.device != dev:
            raise TypeError("decode inputs must be in the cache dtype, on the cache's device")
    if cache_p2.dim() != 4 or tuple(cache_p2.shape[:2]) != (B, H) or cache_p2.shape[3] != D:
        raise ValueError(f"cache_p2 must be [B, H, capacity, dh] = [{B}, {H}, *, {D}], got {tuple(cache_p2.shape)}")
    if cache_info.shape != cache_p2.shape or cache_info.dtype != cache_p2.dtype:
        raise ValueError("cache_info must have cache_p2's shape and dtype")
    for t in (cache_p2, cache_info):
        if t.device != dev or t.stride(-1) != 1:
            raise ValueError("the caches must be on the inputs' device with unit stride on dh")
    cap = cache_p2.shape[2]
    # S is read as int64 and, with advance, written back by the kernel: no conversion is possible
    if S.dtype != torch.int64 or S.device != dev or S.numel() != B or not S.is_contiguous():
        raise ValueError(f"S must be a contiguous int64 device tensor of B = {B} positions")
    # fp32 device copies of the small parameters (no copy when they already are; the temporaries
    # stay referenced until the launch is queued, and the caching allocator orders their reuse)
    lam32 = _f32_param(lam, 1, "lam", dev)
    inv32 = None if inv_freq is None else _f32_param(inv_freq, D // 2, "inv_freq", dev)
    th32 = None if theta is None else _f32_param(theta, H // 2, "theta", dev)
    if xm is not None and (xm.dtype != torch.float32 or xm.numel() != B or not xm.is_contiguous() or xm.device != dev):
        raise ValueError("xm must be a contiguous fp32 tensor of B elements")
    _check_run(run, dev)
    if workspace is not None and (workspace.device != dev or not workspace.is_contiguous()):
        raise ValueError("workspace must be a contiguous tensor on the inputs' device")
    if y is not None and (y.shape != (B, H, D) or y.dtype != p1.dtype or y.device != dev or y.stride(-1) != 1
                          or y.stride(1) != D):
        raise ValueError("y must be [B, H, dh] in the cache dtype with head stride dh")
    if g is not None and (g.shape != (B, H) or g.dtype != torch.float32 or g.device != dev or not g.is_contiguous()):
        raise ValueError("g must be a contiguous fp32 [B, H] tensor")
    if not p1.is_cuda:
        raise RuntimeError("relation_decode needs the HIP library and an MI355X")
    if workspace is None:
        workspace = decode_workspace(B, H, D, cap, dev, p1.dtype)
    if y is None:
        y = torch.empty(B, H, D, device=dev, dtype=p1.dtype)
    if g is None:
        g = torch.empty(B, H, device=dev, dtype=torch.float32)
    a = L.DecodeArgs()
    a.dtype = L.dtype_code(p1)
    a.B, a.H, a.D, a.capacity = B, H, D, cap
    flags = (L.MOTE_DECODE_ADVANCE if advance else 0) | (L.MOTE_DECODE_ROPE_F32 if rope_f32 else 0)
    a.layer_parity, a.flags, a.tau_s = int(layer_idx) % 2, flags, float(tau_s)
    a.lam = lam32.data_ptr()
    a.inv_freq, a.theta = L.ptr(inv32), L.ptr(th32)
    a.S = S.data_ptr()
    a.p1, a.p2, a.info, a.in_sb = p1.data_ptr(), p2.data_ptr(), info.data_ptr(), p1.stride(0)
    a.cache_p2, a.cache_info = L.view(cache_p2), L.view(cache_info)
    a.y, a.y_sb, a.g = y.data_ptr(), y.stride(0), g.data_ptr()
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    if xm is not None:
        a.xm = xm.data_ptr()
    a.run = L.ptr(run)
    L.check(L.lib().mote_relation_decode(a, L.stream_of(p1)), "mote_relation_decode")
    return y, g


def skinny_linear(x: torch.Tensor, w: torch.Tensor, out: Optional[torch.Tensor] = None,
                  run: Optional[torch.Tensor] = None, g: Optional[torch.Tensor] = None,
                  xm: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y [B, N] = x [B, K] w[N, K]^T for the decode engine's per-token projections (bf16, B <= 16,
    N % 16 == 0, K % 128 == 0, K <= 1024): one launch of mote_skinny_gemm. With `run` (a device
    flag) the launch leaves `out` untouched when the flag is 0. With g (fp32 [B, H], contiguous) and
    xm (fp32 [B]) the same launch writes xm[b] = mean of g[b] in head order (graph.py:186)."""
    B, K = x.shape
    N = w.shape[0]
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise TypeError("skinny_linear: bf16 x and w")
    if x.stride(-1) != 1 or w.stride(-1) != 1 or w.shape[1] != K:
        raise ValueError("skinny_linear: x [B, K] and w [N, K] with unit element stride")
    _check_run(run, x.device)
    if out is None:
        out = torch.empty(B, N, device=x.device, dtype=x.dtype)
    a = L.SkinnyGemmArgs()
    a.dtype, a.B, a.N, a.K = L.dtype_code(x), B, N, K
    a.x, a.x_sr = x.data_ptr(), x.stride(0)
    a.w, a.w_sr = w.data_ptr(), w.stride(0)
    a.y, a.y_sr = out.data_ptr(), out.stride(0)
    a.run = L.ptr(run)
    if xm is not None:
        if (g is None or g.dtype != torch.float32 or xm.dtype != torch.float32 or not g.is_contiguous()
                or not xm.is_contiguous() or g.dim() != 2 or g.shape[0] != B or xm.numel() != B
                or g.device != x.device or xm.device != x.device):
            raise ValueError("skinny_linear: xm needs fp32 contiguous g [B, H] and xm [B] on x's device")
        a.g, a.xm, a.heads = g.data_ptr(), xm.data_ptr(), g.shape[1]
    L.check(L.lib().mote_skinny_gemm(a, L.stream_of(x)), "mote_skinny_gemm")
    return out


def _skinny_ok(B: int, x: torch.Tensor, *ws: torch.Tensor) -> bool:
    return (x.is_cuda and x.dtype == torch.bfloat16 and 1 <= B <= 16 and
            all(w.dtype == torch.bfloat16 and w.shape[0] % 16 == 0 and w.shape[1] % 128 == 0 and w.shape[1] <= 1024
                for w in ws))


class RelationDecodeStep:
    """GraphDecoder._relation_step (graph.py:151-187) for one FullRelation layer over its arena rows.

    Holds the static tensors a captured graph needs (fp32 lam/theta/inv_freq copies and the stacked
    projection weight [w1; w2; wi], refreshed by `sync_params()`, the workspace, outputs).
    `__call__(x [B,1,D], S)` returns (out [B,1,D], xm [B] = mean over heads of the exchange mass,
    graph.py:186)."""

    def __init__(self, mixer, arena: RelationArena, layer: int):
        self.mixer, self.arena, self.layer = mixer, arena, layer
        dev = arena.device
        B, H, D = arena.batch, mixer.n_heads, mixer.d_head
        self.B = B
        self.workspace = decode_workspace(B, H, D, arena.capacity, dev, arena.dtype)
        self.y = torch.empty(B, H, D, device=dev, dtype=arena.dtype)
        self.g = torch.empty(B, H, device=dev, dtype=torch.float32)
        self.xm = torch.empty(B, device=dev, dtype=torch.float32)
        self.lam = torch.empty((), device=dev, dtype=torch.float32)
        self.theta = torch.empty(max(H // 2, 1), device=dev, dtype=torch.float32) if mixer.use_givens else None
        self.inv_freq = mixer.inv_freq.to(device=dev, dtype=torch.float32).clone() if mixer.use_rope else None
        self.w_qkv = None
        self._bufs: dict = {}
        self.sync_params()

    @torch.no_grad()
    def sync_params(self) -> None:
        """Refresh the step's copies of the layer's parameters (after an optimiser step; a captured
        graph keeps reading these same tensors)."""
        m = self.mixer
        w = torch.cat([m.w1.weight, m.w2.weight, m.wi.weight], dim=0)
        if self.w_qkv is None or self.w_qkv.shape != w.shape or self.w_qkv.dtype != w.dtype:
            self.w_qkv = w.detach().clone()
        else:
            self.w_qkv.copy_(w)
        self.lam.copy_(self.mixer.lam.detach().float())
        if self.theta is not None:
            self.theta.copy_(self.mixer.theta.detach().float())

    def _static(self, name: str, shape, dtype) -> torch.Tensor:
        """A persistent output buffer (a predicated launch that does not run leaves it as it was)."""
        t = self._bufs.get(name)
        if t is None or tuple(t.shape) != tuple(shape) or t.dtype != dtype:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("run the predicated decode step once outside the capture first (its "
                                   "persistent outputs are allocated then)")
            t = torch.zeros(shape, device=self.arena.device, dtype=dtype)
            self._bufs[name] = t
        return t

    @torch.no_grad()
    def __call__(self, x: torch.Tensor, S: torch.Tensor, advance: bool = False, run: Optional[torch.Tensor] = None,
                 xm: Optional[torch.Tensor] = None):
        """One new chunk per sequence: x [B, 1, D] -> (out [B, 1, D], xm [B]).

        run: optional device flag; with it every write of the step (arena append, S advance, the
        outputs, xm) happens only when the flag is nonzero, and the outputs live in persistent
        buffers that keep their last values otherwise (the bf16 skinny path: B <= 16, T = 1).
        xm: optional fp32 [B] buffer for the exchange mass (default: the step's own)."""
        m = self.mixer
        B, T, Dm = x.shape
        H, dh = m.n_heads, m.d_head
        skinny = T == 1 and _skinny_ok(B, x, self.w_qkv, m.wo.weight, *([m.wg.weight] if m.out_gate else []))
        if run is not None and not skinny:
            raise ValueError("a predicated decode step needs the bf16 skinny path (B <= 16, one chunk)")
        xm = self.xm if xm is None else xm
        if skinny:  # bf16 decode shapes: the skinny product instead of the general GEMM library
            qbuf = self._static("qkv", (B, 3 * H * dh), x.dtype) if run is not None else None
            qkv = skinny_linear(x.reshape(B, Dm), self.w_qkv, qbuf, run).view(B, 3, H, dh)
        else:
            qkv = F.linear(x, self.w_qkv).view(B, 3, H, dh)
        qkv = qkv.to(self.arena.dtype)
        if m.qk_norm:
            q = m.p1_norm(qkv[:, 0])
            k = m.p2_norm(qkv[:, 1])
            qkv = torch.stack([q, k, qkv[:, 2]], dim=1)
        # on the skinny path the wo launch writes xm (its mean of g needs no count of finished heads
        # in the decode launch)
        # RoPE tables at x's dtype (graph.py:161): an fp32 x (serving autocast) rotates in fp32
        rope_f32 = x.dtype == torch.float32 and self.arena.dtype != torch.float32
        relation_decode(qkv[:, 0], qkv[:, 1], qkv[:, 2], S, self.arena.p2(self.layer), self.arena.info(self.layer),
                        self.lam, m.tau_s, self.inv_freq, self.theta, m.layer_idx, advance, self.workspace,
                        self.y, self.g, None if skinny else xm, run, rope_f32)
        if skinny:  # _out (relation.py:176-182) on the skinny product
            y = self.y.to(x.dtype).reshape(B, H * dh)
            if m.out_gate:
                gbuf = self._static("gate", (B, Dm), x.dtype) if run is not None else None
                y = y * torch.sigmoid(skinny_linear(x.reshape(B, Dm), m.wg.weight, gbuf, run))
            obuf = self._static("out", (B, Dm), x.dtype) if run is not None else None
            return skinny_linear(y, m.wo.weight, obuf, run, g=self.g, xm=xm).view(B, 1, Dm), xm
        y = self.y.to(x.dtype).view(B, H, 1, dh)
        return m._out(y, x), xm
