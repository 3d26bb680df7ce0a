"""CPU restatement of Mote's chunk gather and EMA dechunk (test infrastructure only).

Follows mote/model/dc.py of the reference: `chunk_layer_ref` is ChunkLayer.forward (:192-218),
`ema_chunked_ref` the block closed form DeChunkLayer._ema_chunked (:236-282), `dechunk_ref`
DeChunkLayer.forward (:312-337) and `dechunk_step_ref` DeChunkLayer.step (:339-349). Gradients are
autograd of these functions (the reference has no hand-written backward for them).

Pins (tests/test_dc_oracle.py): the closed form against the plain sequential recurrence and against
the block loop it replaced (the reference's own tests/test_dechunk_static.py and
tests/test_mote_model.py:75-92, restated), brute-force loops over bytes for the routing, the gather
and the expansion to bytes, the closed form of a constant p, central finite differences for the
gradients, and the bit-level rounding order of the decode step. Planted mistakes (plug without the
-1, the EMA reading p of the previous chunk, p not clamped, the exclusive prefix replaced by
s_incl - logd) are injected through `_plant` and each must fail one of the pins. Nothing in the product
imports this module.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn.functional as F


def route_ref(mask: torch.Tensor):
    """cum (inclusive boundary count), perm (boundaries in order, then the rest in order) and num per
    row: the index work of dc.py:209-214 and :320-327 (argsort of t + L * !mask has unique keys)."""
    B, L = mask.shape
    token_idx = torch.arange(L)[None, :] + (~mask.bool()).long() * L
    perm = torch.argsort(token_idx, dim=1)
    cum = torch.cumsum(mask.long(), dim=1)
    return cum, perm, mask.long().sum(-1)


def chunk_layer_ref(hidden: torch.Tensor, mask: torch.Tensor, bucket: int = 1, exact: bool = False):
    """ChunkLayer.forward (dc.py:205-216): boundary rows compacted to the front, M = max count rounded
    up to `bucket` (capped at L) unless exact; returns (out [B, M, D], next_mask [B, M])."""
    B, L, D = hidden.shape
    _, perm, num = route_ref(mask)
    M = int(num.max()) if B > 0 else 0
    if bucket > 1 and not exact:
        M = min(L, -(-M // bucket) * bucket)
    order = perm[:, :M].to(hidden.device)
    out = torch.gather(hidden, 1, order[:, :, None].expand(-1, -1, D))
    next_mask = torch.arange(M)[None, :] < num[:, None]
    return out, next_mask.to(hidden.device)


def ema_sequential_ref(x: torch.Tensor, p: torch.Tensor, init: Optional[torch.Tensor] = None) -> torch.Tensor:
    """z_t = p_t x_t + (1 - p_t) z_{t-1}, one step at a time (the definition the reference's tests hold
    the closed form to)."""
    B, M, D = x.shape
    z = torch.zeros(B, D, dtype=x.dtype) if init is None else init.to(x.dtype)
    outs = []
    for t in range(M):
        z = p[:, t, None] * x[:, t] + (1 - p[:, t, None]) * z
        outs.append(z)
    return torch.stack(outs, dim=1) if outs else x[:, :0]


def ema_block_loop_ref(x, p, C=64, init=None):
    """Within-block closed form with a loop across blocks (the form dc.py:268-276 replaced; kept by the
    reference's tests/test_dechunk_static.py:11-37 as a second definition)."""
    B, M, D = x.shape
    wdt = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf, pf = x.to(wdt), p.to(wdt)
    pad = (-M) % C
    if pad:
        xf = F.pad(xf, (0, 0, 0, pad))
        pf = F.pad(pf, (0, pad))
    nb = xf.shape[1] // C
    xf, pf = xf.view(B, nb, C, D), pf.view(B, nb, C)
    L = torch.cumsum(torch.log1p(-pf), dim=-1)
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))
    A = torch.exp((L[..., :, None] - L[..., None, :]).masked_fill(~mask, float("-inf")))
    local = torch.matmul(A, pf[..., None] * xf)
    carry = torch.zeros(B, D, dtype=wdt) if init is None else init.to(wdt)
    decay = torch.exp(L)
    blocks = []
    for b in range(nb):
        blk = local[:, b] + decay[:, b, :, None] * carry[:, None, :]
        blocks.append(blk)
        carry = blk[:, -1]
    return torch.stack(blocks, dim=1).reshape(B, nb * C, D)[:, :M].to(x.dtype)


def ema_chunked_ref(x: torch.Tensor, p: torch.Tensor, C: int = 64, init: Optional[torch.Tensor] = None,
                    _plant: Optional[str] = None) -> torch.Tensor:
    """DeChunkLayer._ema_chunked (dc.py:236-282): within a block of C steps
    z_t = sum_{s<=t} exp(L_t - L_s) p_s x_s + exp(L_t) z_in with L_t = sum_{u<=t} log(1 - p_u); the
    carry into block b in closed form from the blocks' end values and an exclusive prefix of the
    block decays. Works in float64 for float64 input, else float32, and returns x's dtype."""
    B, M, D = x.shape
    wdt = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf, pf = x.to(wdt), p.to(wdt)
    if _plant == "p_prev":
        pf = torch.cat([pf[:, :1], pf[:, :-1]], dim=1)
    pad = (-M) % C
    if pad:
        xf = F.pad(xf, (0, 0, 0, pad))
        pf = F.pad(pf, (0, pad))                                    # p = 0: state carried unchanged
    nb = xf.shape[1] // C
    xf, pf = xf.view(B, nb, C, D), pf.view(B, nb, C)
    L = torch.cumsum(torch.log1p(-pf), dim=-1)                      # [B, nb, C]
    tri = torch.tril(torch.ones(C, C, dtype=torch.bool, device=x.device))
    A = torch.exp((L[..., :, None] - L[..., None, :]).masked_fill(~tri, float("-inf")))
    local = torch.matmul(A, pf[..., None] * xf)                     # [B, nb, C, D]
    decay_t = torch.exp(L)
    e = local[:, :, -1]
    logd = L[:, :, -1]
    s_incl = torch.cumsum(logd, dim=-1)
    if _plant == "s_incl_minus":
        s_excl = s_incl - logd
    else:
        s_excl = torch.cat([torch.zeros_like(s_incl[..., :1]), s_incl[..., :-1]], dim=-1)
    w = s_excl[:, :, None] - s_incl[:, None, :]
    lower = torch.tril(torch.ones(nb, nb, dtype=torch.bool, device=x.device), diagonal=-1)
    w = torch.exp(w.masked_fill(~lower, float("-inf")))
    carry_in = torch.matmul(w, e)
    if init is not None:
        carry_in = carry_in + torch.exp(s_excl)[..., None] * init.to(wdt)[:, None, :]
    out = local + decay_t[..., None] * carry_in[:, :, None, :]
    return out.reshape(B, nb * C, D)[:, :M].to(x.dtype)


def dechunk_ref(hidden: torch.Tensor, mask: torch.Tensor, prob: torch.Tensor, eps: float = 1e-4,
                init: Optional[torch.Tensor] = None, _plant: Optional[str] = None) -> torch.Tensor:
    """DeChunkLayer.forward (dc.py:312-335): p of the selected positions, clamped; the EMA over the
    chunk rows; every byte reads the value of the last boundary at or before it (with `init`, the
    decode-state form: bytes before the first boundary read init). Returns [B, L, D] in hidden's dtype."""
    B, L = mask.shape
    p = prob[..., 1].float()
    if _plant != "no_clamp":
        p = torch.clamp(p, min=eps, max=1 - eps)
    token_idx = torch.arange(L, device=hidden.device)[None, :] + (~mask.bool()).long() * L
    order = torch.argsort(token_idx, dim=1)[:, : hidden.shape[1]]
    p = torch.gather(p, 1, order)
    if init is None:
        sm = ema_chunked_ref(hidden, p, _plant=_plant)
        plug = torch.cumsum(mask.long(), dim=1)
        if _plant != "plug_no_minus":
            plug = plug - 1
        plug = plug.clamp(min=0)
    else:
        sm = ema_chunked_ref(hidden, p, init=init.float()) if hidden.shape[1] > 0 else hidden.float()[:, :0]
        sm = torch.cat([init.float()[:, None, :], sm.float()], dim=1)
        plug = torch.cumsum(mask.long(), dim=1)
    out = torch.gather(sm, 1, plug[:, :, None].expand(-1, -1, sm.shape[-1]))
    return out.to(hidden.dtype)


def dechunk_brute(hidden: torch.Tensor, mask: torch.Tensor, prob: torch.Tensor, eps: float = 1e-4,
                  init: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The same map as loops in float64: run z over the row's boundaries in order (chunk row m takes
    the m-th boundary's p), then byte t reads the value after the last boundary at or before it. A row
    with no boundary and no carried value reads chunk row 0 at byte 0's p everywhere."""
    B, L = mask.shape
    D = hidden.shape[-1]
    out = torch.zeros(B, L, D, dtype=torch.float64)
    for b in range(B):
        bpos = [t for t in range(L) if bool(mask[b, t])]
        z = init[b].double() if init is not None else torch.zeros(D, dtype=torch.float64)
        zs = [z]
        for m, t in enumerate(bpos):
            pv = min(max(float(prob[b, t, 1]), eps), 1 - eps)
            z = pv * hidden[b, m].double() + (1 - pv) * z
            zs.append(z)
        if init is None and not bpos:
            pv = min(max(float(prob[b, 0, 1]), eps), 1 - eps)
            zs.append(pv * hidden[b, 0].double())
        k = 0
        for t in range(L):
            k += int(bool(mask[b, t]))
            out[b, t] = zs[k] if init is not None else zs[max(k, 1)]
    return out


def dechunk_step_ref(hidden: torch.Tensor, mask: torch.Tensor, prob: torch.Tensor, last: torch.Tensor,
                     eps: float = 1e-4) -> torch.Tensor:
    """DeChunkLayer.step (dc.py:339-349): the same eager ops in the state's dtype; `last` is updated in
    place and returned."""
    B = mask.shape[0]
    D = last.shape[-1]
    p = torch.zeros(B, dtype=last.dtype)
    p[mask] = prob[mask, 1].clamp(min=eps, max=1 - eps).to(p.dtype)
    cur = torch.zeros(B, D, dtype=last.dtype)
    if hidden.shape[0] > 0:
        cur[mask] = hidden.squeeze(1).to(cur.dtype)
    result = p[:, None] * cur + (1 - p[:, None]) * last
    last.copy_(result)
    return result.unsqueeze(1)
