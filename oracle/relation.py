"""CPU restatement of the Relation mixer — TEST INFRASTRUCTURE (see the package header).

Every function restates the reference (noahsabaj/mote) in plain PyTorch on the CPU; the cited
file:line is the code it follows. The HIP library is checked against these functions; nothing in
the product imports them.

How each function is pinned (tests/test_oracle.py holds the checks):

* `relation_reference` — against `oracle.brute.relation_brute` (float64 scalar loops), a T = 2 case
  worked by hand (hard-coded numbers), the T = 1 closed form (Y = I~_0, g = 0), and invariants:
  causality, cache split == one shot, g in (0, 1), F_ii = 1 - g.
* `relation_online` — against `relation_reference` in float64 with scores large enough to force the
  conditional rescale; lambda cancels inside the past (I-bar does not depend on lambda).
* `relation_backward` (analytic) — against autograd of `relation_reference` and against central
  finite differences in float64.
* `rope_*` — table == direct, position 0 is the identity, norms of (k, k + d/2) pairs are preserved,
  scores depend only on the position difference.
* `givens` — against an explicit 2x2 rotation per head pair, theta = 0 is the identity, rotating by
  -theta undoes it, odd layers pair (H-1, 0).
* `FullRelationRef` / `decode_step_ref` — module == composition of the pinned parts; decode at
  position S == the last row of a full forward over S + 1 positions.
* `decode_rows_ref` — bit for bit (bf16 and fp32) the pinned `rope_tables` + `apply_rope` and
  `givens` applied at position S in the operand dtype; the rows `decode_step_ref` writes into the
  cache; in float64 the last row of `FullRelationRef.heads` over S + 1 positions.
* `HeadRMSNormRef` — `torch.nn.functional.rms_norm` in float64 (rows below and above eps), the
  closed form of a constant row, bf16 within one rounding of the float64 value.
* Planted mistakes (log i for log(i+1), the self term counted in g, a missing 1/tau, a Givens sign
  flip, a RoPE sign flip, RoPE tables not rounded to the operand dtype, one rounding instead of the
  reference's one per op, odd layers paired like even ones, eps outside the root of QK-Norm) are
  injected through `_plant` and each must fail one of the pins above.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

NEG_INF = float("-inf")


# ---------------------------------------------------------------------------------------------
# Relation core
# ---------------------------------------------------------------------------------------------
def relation_reference(p1, p2, info, lam, tau_s: float = 2.0, q_start: int = 0,
                       dtype=torch.float32, _plant: Optional[str] = None):
    """Materialized Relation: mote/model/flash_relation.py:666-682 (== relation.py:240-268 with the
    inputs upcast first).

    p1 [B,H,TQ,D] (RoPE applied), p2/info [B,H,q_start+TQ,D]; lam a scalar tensor.
    R_ij = sigmoid(U_ii / tau_s) on the diagonal, SiLU(U_ij) - lam*ln(i+1) strictly in the past,
    -inf in the future (i is the absolute 0-based query index); F = softmax_j(R); Y = F I~;
    g_i = sum_{j<i} F_ij. Returns (Y [B,H,TQ,D], g [B,H,TQ]) in `dtype`.
    """
    TQ, D = p1.shape[2], p1.shape[3]
    TK = p2.shape[2]
    assert TK == q_start + TQ, "keys must be the cached prefix plus the new rows"
    q, k, v = p1.to(dtype), p2.to(dtype), info.to(dtype)
    u = torch.matmul(q, k.transpose(-1, -2)) / math.sqrt(D)
    qpos = torch.arange(q_start, q_start + TQ, device=p1.device)
    kpos = torch.arange(TK, device=p1.device)
    diag = qpos[:, None] == kpos[None, :]
    past = kpos[None, :] < qpos[:, None]
    if _plant == "log_i":  # planted mistake: count term ln(i) instead of ln(i+1)
        count = torch.log(qpos.clamp(min=1).to(dtype))[:, None]
    else:
        count = torch.log((qpos + 1).to(dtype))[:, None]
    tau = 1.0 if _plant == "no_tau" else tau_s
    lam_ = lam.to(dtype) if torch.is_tensor(lam) else torch.tensor(lam, dtype=dtype)
    scores = torch.where(diag, torch.sigmoid(u / tau), F.silu(u) - lam_ * count)
    scores = scores.masked_fill(~(diag | past), NEG_INF)
    flow = torch.softmax(scores, dim=-1)
    y = torch.matmul(flow, v)
    gmask = (past | diag) if _plant == "g_with_self" else past
    g = flow.masked_fill(~gmask, 0.0).sum(-1)
    return y, g


def relation_online(p1, p2, info, lam, tau_s: float = 2.0, q_start: int = 0, block: int = 16,
                    thresh: float = 8.0, dtype=torch.float64):
    """The fused (online-softmax) form: mote/model/flash_relation.py:3-8 (algebra) and :100-183.

    The strictly-past exchange scores are scanned in key blocks with a running max m (log2 units),
    sum l and weighted sum z; m is only raised when a block exceeds it by more than `thresh`
    (flash_relation.py:57, 124-134). The row is completed with
    L = m ln2 + ln l, I-bar = z / l, S = sigmoid(U_ii / tau), A = L - lam ln(i+1),
    g = sigmoid(A - S) (0 without a past), Y = (1 - g) I~_i + g I-bar.
    Returns (Y, g, ibar, lse) with lse in natural units (-inf without a past).
    """
    B, H, TQ, D = p1.shape
    TK = p2.shape[2]
    assert TK == q_start + TQ
    log2e = 1.0 / math.log(2.0)
    q, k, v = p1.to(dtype), p2.to(dtype), info.to(dtype)
    scale = 1.0 / math.sqrt(D)
    qpos = torch.arange(q_start, q_start + TQ)
    m = torch.full((B, H, TQ), NEG_INF, dtype=dtype)
    l = torch.zeros((B, H, TQ), dtype=dtype)
    z = torch.zeros((B, H, TQ, D), dtype=dtype)
    for j0 in range(0, TK, block):
        j1 = min(TK, j0 + block)
        u = torch.einsum("bhid,bhjd->bhij", q, k[:, :, j0:j1]) * scale
        e2 = u * torch.sigmoid(u) * log2e
        valid = torch.arange(j0, j1)[None, :] < qpos[:, None]
        e2 = e2.masked_fill(~valid, NEG_INF)
        bmax = e2.amax(-1)
        grow = bmax > m + thresh
        m_new = torch.where(grow, bmax, m)
        alpha = torch.where(grow, torch.exp2(m - torch.where(torch.isinf(m_new), 0.0, m_new)), torch.ones_like(m))
        alpha = torch.where(torch.isinf(m) & grow, torch.zeros_like(m), alpha)
        z = z * alpha[..., None]
        l = l * alpha
        m = m_new
        msafe = torch.where(torch.isinf(m), torch.zeros_like(m), m)
        p = torch.exp2(e2 - msafe[..., None])
        l = l + p.sum(-1)
        z = z + torch.einsum("bhij,bhjd->bhid", p, v[:, :, j0:j1])
    has = l > 0
    lsafe = torch.where(has, l, torch.ones_like(l))
    lse = torch.where(has, (m + torch.log2(lsafe)) * math.log(2.0), torch.full_like(l, NEG_INF))
    ibar = z / lsafe[..., None]
    idx = qpos.view(1, 1, TQ, 1).expand(B, H, TQ, D)
    kself = torch.gather(k, 2, idx)
    iself = torch.gather(v, 2, idx)
    uii = (q * kself).sum(-1) * scale
    s = torch.sigmoid(uii / tau_s)
    lam_ = lam.to(dtype) if torch.is_tensor(lam) else torch.tensor(lam, dtype=dtype)
    a = lse - lam_ * torch.log((qpos + 1).to(dtype))
    g = torch.where(has, torch.sigmoid(a - s), torch.zeros_like(a))
    y = (1.0 - g)[..., None] * iself + g[..., None] * ibar
    return y, g, ibar, lse


def relation_backward(p1, p2, info, lam, dy, tau_s: float = 2.0, q_start: int = 0, dtype=torch.float64):
    """Analytic gradients of Y w.r.t. (p1, p2, info, lam): mote/model/flash_relation.py:10-15.

    dI-bar = g dY, dg = dY.(I-bar - I~_i), dA = dg g (1-g), dS = -dA, dlam = -sum dA ln(i+1),
    dU_ii = dS S (1-S) / tau, w_ij = exp(E_ij - L_i), Delta = dI-bar.I-bar,
    dE_ij = w_ij (dI-bar_i.I~_j - Delta_i + dA_i), dU_ij = dE_ij SiLU'(U_ij),
    dP1 = dU P2 / sqrt(D), dP2 = dU^T P1 / sqrt(D), dI~_j = sum_i w_ij dI-bar_i + (1 - g_j) dY_j.
    """
    B, H, TQ, D = p1.shape
    TK = p2.shape[2]
    q, k, v, dyf = p1.to(dtype), p2.to(dtype), info.to(dtype), dy.to(dtype)
    scale = 1.0 / math.sqrt(D)
    y, g, ibar, lse = relation_online(q, k, v, lam, tau_s, q_start, dtype=dtype)
    qpos = torch.arange(q_start, q_start + TQ)
    kpos = torch.arange(TK)
    past = kpos[None, :] < qpos[:, None]
    idx = qpos.view(1, 1, TQ, 1).expand(B, H, TQ, D)
    kself = torch.gather(k, 2, idx)
    iself = torch.gather(v, 2, idx)
    u = torch.matmul(q, k.transpose(-1, -2)) * scale
    sig = torch.sigmoid(u)
    e = u * sig
    lse_safe = torch.where(torch.isinf(lse), torch.zeros_like(lse), lse)
    w = torch.exp(e - lse_safe[..., None]).masked_fill(~past, 0.0)
    dibar = g[..., None] * dyf
    dgate = (dyf * (ibar - iself)).sum(-1)
    da = dgate * g * (1.0 - g)
    lam_dlam = -(da * torch.log((qpos + 1).to(dtype))).sum()
    uii = (q * kself).sum(-1) * scale
    s = torch.sigmoid(uii / tau_s)
    duii = (-da) * s * (1.0 - s) / tau_s
    delta = (dibar * ibar).sum(-1)
    dw = torch.matmul(dibar, v.transpose(-1, -2))
    de = w * (dw - delta[..., None] + da[..., None])
    du = de * (sig * (1.0 + u * (1.0 - sig)))
    dp1 = torch.matmul(du, k) * scale + duii[..., None] * kself * scale
    dp2 = torch.matmul(du.transpose(-1, -2), q) * scale
    dinfo = torch.matmul(w.transpose(-1, -2), dibar)
    dp2[:, :, q_start:] += duii[..., None] * q * scale
    dinfo[:, :, q_start:] += (1.0 - g)[..., None] * dyf
    return dp1, dp2, dinfo, lam_dlam


def relation_dlam_terms(p1, p2, info, lam, dy, tau_s: float = 2.0, q_start: int = 0, dtype=torch.float64):
    """The summands of dlam = -sum_i dA_i ln(i+1) (flash_relation.py:12), [B,H,TQ]. Their absolute
    sum is the natural scale of dlam, which cancels heavily across rows."""
    TQ = p1.shape[2]
    q, k, v, dyf = p1.to(dtype), p2.to(dtype), info.to(dtype), dy.to(dtype)
    _, g, ibar, _ = relation_online(q, k, v, lam, tau_s, q_start, dtype=dtype)
    qpos = torch.arange(q_start, q_start + TQ)
    iself = v[:, :, q_start:]
    da = (dyf * (ibar - iself)).sum(-1) * g * (1.0 - g)
    return -da * torch.log((qpos + 1).to(dtype))


def relation_grads_autograd(p1, p2, info, lam, dy, tau_s: float = 2.0, q_start: int = 0, dtype=torch.float32):
    """Gradients of sum(Y * dy) through `relation_reference` by autograd (the way the reference's
    kernel tests obtain their ground truth, tests/test_flash_relation.py:28-39)."""
    leaves = [t.detach().to(dtype).requires_grad_(True) for t in (p1, p2, info)]
    lam_leaf = (lam.detach() if torch.is_tensor(lam) else torch.tensor(lam)).to(dtype).requires_grad_(True)
    y, _ = relation_reference(*leaves, lam_leaf, tau_s, q_start, dtype=dtype)
    grads = torch.autograd.grad((y * dy.to(dtype)).sum(), [*leaves, lam_leaf])
    return grads


# ---------------------------------------------------------------------------------------------
# RoPE and Givens
# ---------------------------------------------------------------------------------------------
def rope_inv_freq(dim: int, theta: float) -> torch.Tensor:
    """fp32 inverse frequencies 1 / theta^(2k/dim), k < dim/2: mote/model/relation.py:39."""
    k2 = torch.arange(0, dim, 2, dtype=torch.float32)
    return 1.0 / (theta ** (k2 / dim))


def rope_cos_sin(positions: torch.Tensor, dim: int, theta: float, dtype):
    """cos/sin tables [T, dim] for the rotate-half convention: mote/model/relation.py:37-42."""
    ang = positions.to(torch.float32)[:, None] * rope_inv_freq(dim, theta)[None, :]
    full = torch.cat([ang, ang], dim=-1)
    return full.cos().to(dtype), full.sin().to(dtype)


def rotate_half(x: torch.Tensor, _plant: Optional[str] = None) -> torch.Tensor:
    """(x1, x2) -> (-x2, x1) over the two halves of the last axis: mote/model/relation.py:61-63."""
    h = x.shape[-1] // 2
    lo, hi = x[..., :h], x[..., h:]
    if _plant == "rope_sign":  # planted mistake: rotation in the wrong direction
        return torch.cat([hi, -lo], dim=-1)
    return torch.cat([-hi, lo], dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, _plant: Optional[str] = None):
    """x [B,H,T,d] * cos + rotate_half(x) * sin, tables [T,d]: mote/model/relation.py:66-68."""
    return x * cos[None, None] + rotate_half(x, _plant) * sin[None, None]


def givens_pairs(n_heads: int, layer_idx: int):
    """Head pairs (a, b): (0,1),(2,3),... on even layers, (1,2),...,(H-1,0) on odd layers:
    mote/model/relation.py:150-157, 167-174."""
    if layer_idx % 2 == 0:
        a = list(range(0, n_heads, 2))
        b = list(range(1, n_heads, 2))
    else:
        a = list(range(1, n_heads, 2))
        b = [(x + 1) % n_heads for x in a]
    return a, b


def givens(info: torch.Tensor, theta: torch.Tensor, layer_idx: int, _plant: Optional[str] = None):
    """Rotate the information states of each head pair by theta_p: mote/model/relation.py:160-174.

    (a, b) -> (c a - s b, s a + c b) with c, s = cos/sin(theta) cast to info's dtype (:165-166)."""
    H = info.shape[1]
    c = torch.cos(theta).to(info.dtype)[None, :, None, None]
    s = torch.sin(theta).to(info.dtype)[None, :, None, None]
    if _plant == "givens_sign":
        s = -s
    a, b = givens_pairs(H, layer_idx)
    ia, ib = info[:, a], info[:, b]
    out = info.clone()
    out[:, a] = c * ia - s * ib
    out[:, b] = s * ia + c * ib
    return out


def rope_tables(S: int, T: int, dim: int, theta: float, dtype):
    """cos/sin for absolute positions S..S+T-1 (relation.py:48-58, without the memo)."""
    return rope_cos_sin(torch.arange(S, S + T), dim, theta, dtype)


# ---------------------------------------------------------------------------------------------
# Module and decode step
# ---------------------------------------------------------------------------------------------
class HeadRMSNormRef(nn.Module):
    """QK-Norm over the head dim with a learnable gain, fp32 math: mote/model/relation.py:71-94."""

    def __init__(self, dim: int, eps: float = 1e-5, dtype=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype))

    def forward(self, x, _plant: Optional[str] = None):
        xf = x.float()
        if _plant == "eps_outside":  # planted mistake: eps added after the root
            yf = xf / (xf.pow(2).mean(-1, keepdim=True).sqrt() + self.eps)
        else:
            yf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (yf * self.weight.float()).to(x.dtype)


class FullRelationRef(nn.Module):
    """The materialized FullRelation: parameters as mote/model/relation.py:97-157 (same names, same
    construction order, so a seed gives the same weights), forward as :184-268 taking the
    materialized branch (:240-268). `cache` is None or a (P2, I~) tuple of [B,H,S,dh] tensors."""

    def __init__(self, d_model, n_heads, layer_idx, tau_s=2.0, lambda_init=0.5, rope_theta=10000.0,
                 givens=True, qk_norm=False, out_gate=False, rope=True, dtype=None):
        super().__init__()
        self.d_model, self.n_heads, self.d_head = d_model, n_heads, d_model // n_heads
        self.layer_idx, self.tau_s, self.rope_theta = layer_idx, tau_s, rope_theta
        self.use_givens, self.qk_norm, self.out_gate, self.use_rope = givens, qk_norm, out_gate, rope
        if qk_norm:
            self.p1_norm = HeadRMSNormRef(self.d_head, dtype=dtype)
            self.p2_norm = HeadRMSNormRef(self.d_head, dtype=dtype)
        self.w1 = nn.Linear(d_model, d_model, bias=False, dtype=dtype)
        self.w2 = nn.Linear(d_model, d_model, bias=False, dtype=dtype)
        self.wi = nn.Linear(d_model, d_model, bias=False, dtype=dtype)
        self.wo = nn.Linear(d_model, d_model, bias=False, dtype=dtype)
        if out_gate:
            self.wg = nn.Linear(d_model, d_model, bias=False, dtype=dtype)
        self.lam = nn.Parameter(torch.tensor(float(lambda_init), dtype=torch.float32))
        if givens:
            self.theta = nn.Parameter(torch.zeros(n_heads // 2, dtype=torch.float32))

    def heads(self, x, S: int):
        """Projections -> QK-Norm -> RoPE(S..) on p1/p2 -> Givens on I~ (relation.py:204-215)."""
        B, T, D = x.shape
        H, dh = self.n_heads, self.d_head
        p1 = self.w1(x).view(B, T, H, dh).transpose(1, 2)
        p2 = self.w2(x).view(B, T, H, dh).transpose(1, 2)
        info = self.wi(x).view(B, T, H, dh).transpose(1, 2)
        if self.qk_norm:
            p1, p2 = self.p1_norm(p1), self.p2_norm(p2)
        if self.use_rope:
            cos, sin = rope_tables(S, T, dh, self.rope_theta, x.dtype)
            p1, p2 = apply_rope(p1, cos, sin), apply_rope(p2, cos, sin)
        if self.use_givens:
            info = givens(info, self.theta, self.layer_idx)
        return p1, p2, info

    def out(self, y, x):
        """[B,H,T,dh] -> [B,T,D] -> optional sigmoid gate -> wo (relation.py:176-182)."""
        B, H, T, dh = y.shape
        y = y.transpose(1, 2).reshape(B, T, H * dh)
        if self.out_gate:
            y = y * torch.sigmoid(self.wg(x))
        return self.wo(y)

    def forward(self, x, cache=None, return_cache=False, return_gates=False):
        B, T, D = x.shape
        S = 0 if cache is None else cache[0].shape[2]
        p1, p2, info = self.heads(x, S)
        if cache is not None:
            p2_all, info_all = torch.cat([cache[0], p2], 2), torch.cat([cache[1], info], 2)
        else:
            p2_all, info_all = p2, info
        u = torch.matmul(p1, p2_all.transpose(-1, -2)).float() / math.sqrt(self.d_head)
        qpos = torch.arange(S, S + T)
        kpos = torch.arange(S + T)
        diag = qpos[:, None] == kpos[None, :]
        past = kpos[None, :] < qpos[:, None]
        count = torch.log((qpos + 1).float())[:, None]
        r = torch.where(diag, torch.sigmoid(u / self.tau_s), F.silu(u) - self.lam.float() * count)
        r = r.masked_fill(~(diag | past), NEG_INF)
        flow = torch.softmax(r, dim=-1)
        y = torch.matmul(flow.to(info_all.dtype), info_all)
        out = self.out(y, x)
        extras = []
        if return_cache:
            extras.append((p2_all, info_all))
        if return_gates:
            extras.append(flow.masked_fill(~past, 0.0).sum(-1))
        return (out, *extras) if extras else out


@torch.no_grad()
def decode_step_ref(mod: FullRelationRef, x: torch.Tensor, p2buf: torch.Tensor, infobuf: torch.Tensor,
                    S: int, Cb: Optional[int] = None):
    """One new chunk at position S through the graph decoder's Relation step:
    mote/infer/graph.py:151-187. x [1,1,D]; p2buf/infobuf [1,H,capacity,dh] are written at row S
    (index_copy_, :173-175) and read over rows [0, Cb) with rows past S masked (:176-184).
    Returns (out [1,1,D], y [1,H,1,dh], xm = mean_h(1 - F_ii) (:186))."""
    H, dh = mod.n_heads, mod.d_head
    if Cb is None:
        Cb = S + 1
    p1 = mod.w1(x).view(1, 1, H, dh).transpose(1, 2)
    p2 = mod.w2(x).view(1, 1, H, dh).transpose(1, 2)
    info = mod.wi(x).view(1, 1, H, dh).transpose(1, 2)
    if mod.qk_norm:
        p1, p2 = mod.p1_norm(p1), mod.p2_norm(p2)
    ang = torch.tensor(float(S), dtype=torch.float32) * rope_inv_freq(dh, mod.rope_theta)
    full = torch.cat([ang, ang], dim=-1)
    cos, sin = full.cos().to(x.dtype)[None, None, None], full.sin().to(x.dtype)[None, None, None]
    if mod.use_rope:
        p1 = p1 * cos + rotate_half(p1) * sin
        p2 = p2 * cos + rotate_half(p2) * sin
    if mod.use_givens:
        info = givens(info, mod.theta, mod.layer_idx)
    at = p2buf.dtype
    p1, p2, info = p1.to(at), p2.to(at), info.to(at)
    p2buf[:, :, S] = p2[:, :, 0]
    infobuf[:, :, S] = info[:, :, 0]
    k_all, v_all = p2buf[:, :, :Cb], infobuf[:, :, :Cb]
    u = torch.matmul(p1, k_all.transpose(-1, -2)).float() / math.sqrt(dh)
    kpos = torch.arange(Cb)
    diag, past = kpos == S, kpos < S
    r = torch.where(diag, torch.sigmoid(u / mod.tau_s), F.silu(u) - mod.lam.float() * math.log(S + 1.0))
    r = r.masked_fill(~(diag | past), NEG_INF)
    flow = torch.softmax(r, dim=-1)
    y = torch.matmul(flow.to(v_all.dtype), v_all)
    xm = (1.0 - flow[..., S]).mean()
    return mod.out(y, x), y, xm


def relation_decode_ref(p1, p2buf, infobuf, S, lam, tau_s: float = 2.0, dtype=torch.float32):
    """The decode core alone: p1 [B,H,dh] queries at positions S[b] (RoPE applied), caches
    [B,H,>=S+1,dh] whose row S[b] already holds the new P2 / I~ row. Returns (y [B,H,dh], g [B,H]).
    Row b is `relation_reference` restricted to its last query (graph.py:177-186)."""
    B, H, dh = p1.shape
    ys, gs = [], []
    for b in range(B):
        s = int(S[b])
        qb = p1[b : b + 1, :, None, :]
        kb = p2buf[b : b + 1, :, : s + 1]
        vb = infobuf[b : b + 1, :, : s + 1]
        full_q = torch.zeros(1, H, s + 1, dh, dtype=qb.dtype)
        full_q[:, :, s] = qb[:, :, 0]
        y, g = relation_reference(full_q[:, :, s:], kb, vb, lam, tau_s, q_start=s, dtype=dtype)
        ys.append(y[0, :, 0])
        gs.append(g[0, :, 0])
    return torch.stack(ys), torch.stack(gs)


def decode_rows_ref(p1, p2, info, S, inv_freq, theta, layer_idx: int, dtype, _plant: Optional[str] = None,
                    rope_dtype=None):
    """The new chunk's rows as the graph decoder prepares them (mote/infer/graph.py:158-172).

    Inputs are the raw projections [B, H, dh]; the arithmetic runs in `dtype` (the model dtype of
    the projections, which is also the cache dtype here), one torch op at a time, so every product
    and every sum is rounded to `dtype` exactly where the reference rounds it:
    * RoPE at position S[b]: fp32 angles float(S) * inv_freq (graph.py:159), emb = cat(f, f),
      cos / sin cast to `dtype` (:161), then p * cos + rotate_half(p) * sin (:163-164);
    * Givens on I~ with c, s = cos / sin(theta) cast to `dtype`, pairs by layer parity
      (relation.py:160-174): (a, b) -> (c a - s b, s a + c b);
    * the cast to the cache dtype (graph.py:171-172), a no-op here.
    `rope_dtype` (default `dtype`) is x's dtype, the dtype of the RoPE tables (graph.py:161): with
    float32 (the graph decoder under serving autocast, x fp32 and bf16 projections) the rotation runs
    in fp32 and the cast of graph.py:171-172 rounds it once into `dtype`; Givens stays in `dtype`.
    `inv_freq` / `theta` None skip RoPE / Givens. Returns three [B, H, dh] tensors in `dtype`.
    `_plant` injects a mistake for the pins: "cos_unrounded" (tables kept in fp32),
    "single_rounding" (the rotation in float64, rounded once), "odd_pairs_shifted" (odd layers
    pair (0,1),(2,3)... like even ones)."""
    B, H, dh = p1.shape
    outs = []
    for b in range(B):
        s = int(S[b])
        q, k, v = (t[b : b + 1, :, None, :].to(dtype) for t in (p1, p2, info))
        if inv_freq is not None:
            freqs = torch.tensor(float(s), dtype=torch.float32) * inv_freq.float().cpu()
            emb = torch.cat([freqs, freqs])
            cos, sin = emb.cos(), emb.sin()
            if _plant == "single_rounding":
                c64, s64 = cos.to(dtype).double(), sin.to(dtype).double()
                q = (q.double() * c64 + rotate_half(q.double()) * s64).to(dtype)
                k = (k.double() * c64 + rotate_half(k.double()) * s64).to(dtype)
            else:
                rd = dtype if rope_dtype is None else rope_dtype
                if _plant != "cos_unrounded":
                    cos, sin = cos.to(rd), sin.to(rd)
                q = (q.to(rd) * cos + rotate_half(q.to(rd)) * sin).to(dtype)
                k = (k.to(rd) * cos + rotate_half(k.to(rd)) * sin).to(dtype)
        if theta is not None:
            c = torch.cos(theta.float().cpu()).to(dtype)[None, :, None, None]
            sn = torch.sin(theta.float().cpu()).to(dtype)[None, :, None, None]
            odd = layer_idx % 2 == 1 and _plant != "odd_pairs_shifted"
            first = list(range(1, H, 2)) if odd else list(range(0, H, 2))
            second = [(h + 1) % H for h in first]
            ia, ib = v[:, first], v[:, second]
            v = v.clone()
            v[:, first] = c * ia - sn * ib
            v[:, second] = sn * ia + c * ib
        outs.append([t[0, :, 0].to(dtype) for t in (q, k, v)])
    return tuple(torch.stack([o[i] for o in outs]) for i in range(3))
