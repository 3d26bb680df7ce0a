"""Pins for the CPU oracle (oracle/), run on the CPU.

Each check is written so that a plausible transcription mistake fails it; the last group plants
such mistakes in the oracle (through its `_plant` hook) and asserts that a pin catches each one.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import relation as O
from oracle.brute import relation_brute


def _inputs(B, H, TQ, S, D, seed=0, scale=0.7, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    mk = lambda T: (torch.randn(B, H, T, D, generator=g, dtype=torch.float64) * scale).to(dtype)
    return mk(TQ), mk(S + TQ), mk(S + TQ)


# ------------------------------------------------------------------------------------------------
# pin functions (return True when the implementation passes)
# ------------------------------------------------------------------------------------------------
def pin_brute(_plant=None) -> bool:
    ok = True
    for (B, H, TQ, S, D, seed) in [(1, 2, 9, 0, 8, 0), (2, 1, 5, 4, 6, 1), (1, 1, 12, 0, 4, 2)]:
        p1, p2, info = _inputs(B, H, TQ, S, D, seed)
        lam = torch.tensor(0.4, dtype=torch.float64)
        y, g = O.relation_reference(p1, p2, info, lam, 2.0, S, dtype=torch.float64, _plant=_plant)
        yb, gb = relation_brute(p1.numpy(), p2.numpy(), info.numpy(), 0.4, 2.0, S)
        ok &= np.allclose(y.numpy(), yb, atol=1e-12, rtol=1e-12)
        ok &= np.allclose(g.numpy(), gb, atol=1e-12, rtol=1e-12)
    return bool(ok)


def pin_two_positions_by_hand(_plant=None) -> bool:
    """T = 2, D = 4, lambda = 0.5, tau = 2 with U_10 = 1 and U_11 = 0, worked in 40-digit decimal
    arithmetic: R_10 = SiLU(1) - 0.5 ln 2, R_11 = sigmoid(0 / 2) = 0.5, F_10 = 1/(1 + e^(R_11 - R_10))."""
    p1 = torch.tensor([[[[0.0, 0, 0, 0], [2.0, 0, 0, 0]]]], dtype=torch.float64)
    p2 = torch.tensor([[[[1.0, 0, 0, 0], [0.0, 2.0, 0, 0]]]], dtype=torch.float64)
    info = torch.tensor([[[[1.0, 2.0, 0, 0], [0.0, 1.0, 3.0, 0]]]], dtype=torch.float64)
    y, g = O.relation_reference(p1, p2, info, torch.tensor(0.5, dtype=torch.float64), 2.0, 0,
                                dtype=torch.float64, _plant=_plant)
    F10 = 0.4711533167896688377484793684435742815708
    want_y1 = [0.4711533167896688377, 1.471153316789668838, 1.586540049630993487, 0.0]
    ok = torch.allclose(y[0, 0, 0], torch.tensor([1.0, 2.0, 0, 0], dtype=torch.float64), atol=1e-15)
    ok &= abs(float(g[0, 0, 0])) == 0.0
    ok &= torch.allclose(y[0, 0, 1], torch.tensor(want_y1, dtype=torch.float64), atol=1e-14)
    ok &= abs(float(g[0, 0, 1]) - F10) < 1e-14
    return bool(ok)


def pin_identities(_plant=None) -> bool:
    """F_ii = 1 - g_i; g_i = sigmoid(L_i - lam ln(i+1) - S_i) with L_i the past log-sum-exp; g in
    (0, 1) past row 0 and g_0 = 0."""
    B, H, T, D = 1, 2, 11, 8
    p1, p2, info = _inputs(B, H, T, 0, D, seed=5)
    lam = 0.3
    y, g = O.relation_reference(p1, p2, info, torch.tensor(lam, dtype=torch.float64), 2.0, 0,
                                dtype=torch.float64, _plant=_plant)
    u = p1 @ p2.transpose(-1, -2) / math.sqrt(D)
    ok = True
    for i in range(T):
        S_i = 1.0 / (1.0 + torch.exp(-u[..., i, i] / 2.0))
        if i == 0:
            ok &= bool((g[..., 0] == 0).all())
            continue
        e = u[..., i, :i] * torch.sigmoid(u[..., i, :i])
        L = torch.logsumexp(e, -1)
        want = torch.sigmoid(L - lam * math.log(i + 1.0) - S_i)
        ok &= torch.allclose(g[..., i], want, atol=1e-12)
        ok &= bool(((g[..., i] > 0) & (g[..., i] < 1)).all())
    return bool(ok)


# ------------------------------------------------------------------------------------------------
# the pins themselves
# ------------------------------------------------------------------------------------------------
def test_materialized_matches_float64_loops():
    assert pin_brute()


def test_two_positions_worked_by_hand():
    assert pin_two_positions_by_hand()


def test_gate_identities_and_range():
    assert pin_identities()


def test_single_position_is_pure_self():
    p1, p2, info = _inputs(2, 3, 1, 0, 16)
    y, g = O.relation_reference(p1, p2, info, torch.tensor(0.5), 2.0, 0, dtype=torch.float64)
    assert torch.equal(y, info)
    assert float(g.abs().max()) == 0.0


def test_causality_and_cache_split():
    """Rows before a change are unaffected by it; a split at s (q_start = s) reproduces rows s.."""
    p1, p2, info = _inputs(2, 2, 20, 0, 8, seed=3)
    lam = torch.tensor(0.45, dtype=torch.float64)
    y, g = O.relation_reference(p1, p2, info, lam, 2.0, 0, dtype=torch.float64)
    p1b, p2b, infob = p1.clone(), p2.clone(), info.clone()
    p1b[:, :, 13:] += 1.0
    p2b[:, :, 13:] -= 0.5
    infob[:, :, 13:] *= 3.0
    y2, _ = O.relation_reference(p1b, p2b, infob, lam, 2.0, 0, dtype=torch.float64)
    assert torch.allclose(y[:, :, :13], y2[:, :, :13], atol=1e-14)
    for s in (1, 7, 19):
        ys, gs = O.relation_reference(p1[:, :, s:], p2, info, lam, 2.0, s, dtype=torch.float64)
        assert torch.allclose(ys, y[:, :, s:], atol=1e-13)
        assert torch.allclose(gs, g[:, :, s:], atol=1e-13)


@pytest.mark.parametrize("scale", [0.7, 3.0])
@pytest.mark.parametrize("S", [0, 13])
def test_online_form_matches_materialized(scale, S):
    """The fused scan (conditional rescale included; scale 3 forces it) is the same function."""
    p1, p2, info = _inputs(2, 2, 41, S, 12, seed=4, scale=scale)
    lam = torch.tensor(0.5, dtype=torch.float64)
    y, g = O.relation_reference(p1, p2, info, lam, 2.0, S, dtype=torch.float64)
    yo, go, ibar, lse = O.relation_online(p1, p2, info, lam, 2.0, S, block=8)
    assert torch.allclose(yo, y, atol=1e-12, rtol=1e-12)
    assert torch.allclose(go, g, atol=1e-12)
    if S == 0:
        assert torch.isinf(lse[..., 0]).all() and (lse[..., 0] < 0).all()


def test_lambda_only_moves_the_gate():
    """The -lam ln(i+1) term is constant across a row's past, so it cancels inside I-bar."""
    p1, p2, info = _inputs(1, 2, 17, 3, 8, seed=6)
    a = O.relation_online(p1, p2, info, torch.tensor(0.1, dtype=torch.float64), 2.0, 3)
    b = O.relation_online(p1, p2, info, torch.tensor(1.7, dtype=torch.float64), 2.0, 3)
    assert torch.allclose(a[2], b[2], atol=1e-13)  # I-bar
    assert torch.allclose(a[3], b[3], atol=1e-13)  # past LSE
    assert not torch.allclose(a[1], b[1], atol=1e-3)  # the gate moves


@pytest.mark.parametrize("S", [0, 5])
def test_analytic_backward_matches_autograd(S):
    p1, p2, info = _inputs(2, 2, 19, S, 8, seed=7)
    lam = torch.tensor(0.4, dtype=torch.float64)
    dy = torch.randn(2, 2, 19, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(8))
    ga = O.relation_backward(p1, p2, info, lam, dy, 2.0, S)
    gb = O.relation_grads_autograd(p1, p2, info, lam, dy, 2.0, S, dtype=torch.float64)
    for a, b in zip(ga, gb):
        assert torch.allclose(a, b, atol=1e-11, rtol=1e-10)


def test_backward_matches_finite_differences():
    p1, p2, info = _inputs(1, 1, 6, 2, 4, seed=9)
    lam = torch.tensor(0.4, dtype=torch.float64)
    dy = torch.randn(1, 1, 6, 4, dtype=torch.float64, generator=torch.Generator().manual_seed(10))
    grads = O.relation_backward(p1, p2, info, lam, dy, 2.0, 2)

    def f(a, b, c, l):
        return float((O.relation_reference(a, b, c, l, 2.0, 2, dtype=torch.float64)[0] * dy).sum())

    eps = 1e-6
    args = [p1, p2, info, lam]
    for which in range(4):
        base = args[which]
        flat = base.reshape(-1)
        for idx in range(0, flat.numel(), max(1, flat.numel() // 9)):
            plus = [a.clone() for a in args]
            minus = [a.clone() for a in args]
            plus[which].reshape(-1)[idx] += eps
            minus[which].reshape(-1)[idx] -= eps
            fd = (f(*plus) - f(*minus)) / (2 * eps)
            an = float(grads[which].reshape(-1)[idx])
            assert abs(fd - an) < 1e-7 * max(1.0, abs(fd)), (which, idx, fd, an)


# ------------------------------------------------------------------------------------------------
# RoPE and Givens
# ------------------------------------------------------------------------------------------------
def test_rope_tables_and_identities():
    cos, sin = O.rope_tables(5, 17, 16, 10000.0, torch.float32)
    c2, s2 = O.rope_cos_sin(torch.arange(5, 22), 16, 10000.0, torch.float32)
    assert torch.equal(cos, c2) and torch.equal(sin, s2)
    x = torch.randn(2, 3, 17, 16, dtype=torch.float64)
    c0, s0 = O.rope_cos_sin(torch.zeros(17, dtype=torch.long), 16, 10000.0, torch.float64)
    assert torch.allclose(O.apply_rope(x, c0, s0), x)  # position 0: identity
    c, s = O.rope_cos_sin(torch.arange(100, 117), 16, 10000.0, torch.float64)
    r = O.apply_rope(x, c, s)
    # a rotation of each (k, k + d/2) pair by angle pos * inv_freq[k]
    n0 = x[..., :8] ** 2 + x[..., 8:] ** 2
    n1 = r[..., :8] ** 2 + r[..., 8:] ** 2
    assert torch.allclose(n0, n1, atol=1e-12)
    inv = O.rope_inv_freq(16, 10000.0).double()
    ang = 100.0 * inv[3]
    want_lo = x[0, 0, 0, 3] * math.cos(ang) - x[0, 0, 0, 11] * math.sin(ang)
    want_hi = x[0, 0, 0, 11] * math.cos(ang) + x[0, 0, 0, 3] * math.sin(ang)
    assert abs(float(r[0, 0, 0, 3]) - float(want_lo)) < 1e-6
    assert abs(float(r[0, 0, 0, 11]) - float(want_hi)) < 1e-6


def pin_rope_relative(_plant=None) -> bool:
    """<RoPE(q, m), RoPE(k, n)> depends on m - n only, and the (k, k+d/2) pair rotates
    counter-clockwise by m * inv_freq[k] (first coordinate gets -sin * second)."""
    q = torch.randn(1, 1, 1, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    k = torch.randn(1, 1, 1, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    dots = []
    for m, n in [(7, 3), (27, 23), (1004, 1000)]:
        cm, sm = O.rope_cos_sin(torch.tensor([m]), 8, 10000.0, torch.float64)
        cn, sn = O.rope_cos_sin(torch.tensor([n]), 8, 10000.0, torch.float64)
        dots.append(float((O.apply_rope(q, cm, sm, _plant) * O.apply_rope(k, cn, sn, _plant)).sum()))
    # the tables are fp32 (as the reference's), so the angle carries ~pos * 6e-8 rad of rounding
    ok = abs(dots[0] - dots[1]) < 1e-5 and abs(dots[0] - dots[2]) < 5e-4
    e0 = torch.zeros(1, 1, 1, 8, dtype=torch.float64)
    e0[..., 0] = 1.0
    c, s = O.rope_cos_sin(torch.tensor([1]), 8, 10000.0, torch.float64)
    r = O.apply_rope(e0, c, s, _plant)
    ok &= abs(float(r[..., 4]) - math.sin(1.0)) < 1e-6  # e_0 -> cos e_0 + sin e_{d/2} (fp32 table)
    return bool(ok)


def test_rope_relative_position():
    assert pin_rope_relative()


def pin_givens(_plant=None) -> bool:
    ok = True
    for layer in (0, 1):
        H = 8
        theta = torch.linspace(-1.0, 1.0, H // 2, dtype=torch.float32)
        info = torch.randn(2, H, 5, 6, dtype=torch.float64)
        out = O.givens(info, theta.double(), layer, _plant)
        a_idx, b_idx = O.givens_pairs(H, layer)
        for p, (a, b) in enumerate(zip(a_idx, b_idx)):
            c, s = math.cos(float(theta[p])), math.sin(float(theta[p]))
            rot = torch.tensor([[c, -s], [s, c]], dtype=torch.float64)
            pair = torch.stack([info[:, a], info[:, b]], -1)  # [..., 2]
            want = pair @ rot.T
            ok &= torch.allclose(out[:, a], want[..., 0], atol=1e-12)
            ok &= torch.allclose(out[:, b], want[..., 1], atol=1e-12)
        back = O.givens(out, -theta.double(), layer, _plant)
        ok &= torch.allclose(back, info, atol=1e-12)
    return bool(ok)


def test_givens_rotations():
    assert pin_givens()
    assert O.givens_pairs(8, 0) == ([0, 2, 4, 6], [1, 3, 5, 7])
    assert O.givens_pairs(8, 1) == ([1, 3, 5, 7], [2, 4, 6, 0])
    info = torch.randn(1, 4, 3, 8)
    assert torch.equal(O.givens(info, torch.zeros(2), 1), info)


# ------------------------------------------------------------------------------------------------
# module and decode step
# ------------------------------------------------------------------------------------------------
def _module(d_model=64, n_heads=4, layer_idx=1, seed=0):
    torch.manual_seed(seed)
    m = O.FullRelationRef(d_model, n_heads, layer_idx, dtype=torch.float64)
    with torch.no_grad():
        m.theta.uniform_(-0.3, 0.3)
        m.lam.fill_(0.4)
    return m


def test_module_is_the_composition_of_its_parts():
    m = _module()
    x = torch.randn(2, 10, 64, dtype=torch.float64)
    out, g = m(x, return_gates=True)
    p1, p2, info = m.heads(x, 0)
    y, g2 = O.relation_reference(p1, p2, info, m.lam.double(), m.tau_s, 0, dtype=torch.float64)
    # the module path upcasts the scores with .float() (relation.py:241): fp32-level agreement
    assert torch.allclose(out, m.out(y, x), atol=1e-5)
    assert torch.allclose(g, g2.to(g.dtype), atol=1e-5)


def test_module_causal_and_cache_split():
    """tests/test_mote_model.py:22-36 restated on the oracle module."""
    m = _module()
    x = torch.randn(2, 10, 64, dtype=torch.float64)
    y = m(x)
    x2 = x.clone()
    x2[:, 7:] += 1.0
    assert torch.allclose(m(x2)[:, :7], y[:, :7], atol=1e-6)
    y_pre, cache = m(x[:, :6], return_cache=True)
    y_rest = m(x[:, 6:], cache=cache)
    assert torch.allclose(torch.cat([y_pre, y_rest], 1), y, atol=1e-5)
    _, g = m(x, return_gates=True)
    assert torch.all(g[:, :, 0] == 0) and torch.all(g[:, :, 1:] > 0) and torch.all(g < 1)


def test_decode_step_is_the_last_row_of_a_full_forward():
    m = _module(layer_idx=0, seed=2)
    S = 9
    x = torch.randn(1, S + 1, 64, dtype=torch.float64)
    full, g = m(x, return_gates=True)
    _, (p2c, ic) = m(x[:, :S], return_cache=True)
    cap = 16
    p2buf = torch.zeros(1, 4, cap, 16, dtype=torch.float64)
    ibuf = torch.zeros_like(p2buf)
    p2buf[:, :, :S], ibuf[:, :, :S] = p2c, ic
    out, y, xm = O.decode_step_ref(m, x[:, S:], p2buf, ibuf, S, Cb=cap)
    assert torch.allclose(out[0, 0], full[0, S], atol=1e-5)
    assert abs(float(xm) - float(g[0, :, S].mean())) < 1e-5
    yd, gd = O.relation_decode_ref(m.heads(x, 0)[0][:, :, S], p2buf, ibuf, torch.tensor([S]),
                                   m.lam.double(), m.tau_s, dtype=torch.float64)
    assert torch.allclose(yd[0], y[0, :, 0], atol=1e-5)


# ------------------------------------------------------------------------------------------------
# planted mistakes: each one must fail at least one pin
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("plant,pins", [
    ("log_i", [pin_brute, pin_two_positions_by_hand, pin_identities]),
    ("no_tau", [pin_brute, pin_two_positions_by_hand, pin_identities]),
    ("g_with_self", [pin_brute, pin_two_positions_by_hand, pin_identities]),
])
def test_planted_core_mistakes_are_caught(plant, pins):
    failed = [p.__name__ for p in pins if not p(_plant=plant)]
    assert failed, f"planted mistake {plant!r} passed every pin"


def test_planted_rope_and_givens_mistakes_are_caught():
    assert not pin_rope_relative(_plant="rope_sign")
    assert not pin_givens(_plant="givens_sign")


def test_dlam_terms_sum_to_dlam():
    p1, p2, info = _inputs(2, 2, 23, 4, 8, seed=13)
    lam = torch.tensor(0.4, dtype=torch.float64)
    dy = torch.randn(2, 2, 23, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(14))
    terms = O.relation_dlam_terms(p1, p2, info, lam, dy, 2.0, 4)
    dlam = O.relation_grads_autograd(p1, p2, info, lam, dy, 2.0, 4, dtype=torch.float64)[3]
    assert abs(float(terms.sum()) - float(dlam)) < 1e-12


# ------------------------------------------------------------------------------------------------
# the decode step's new rows and QK-Norm
# ------------------------------------------------------------------------------------------------
def _decode_raw(B, H, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    raw = [(torch.randn(B, H, D, generator=g) * 0.8).to(dtype) for _ in range(3)]
    theta = torch.rand(H // 2, generator=g) * 0.6 - 0.3
    return raw, theta


def pin_decode_rows(_plant=None) -> bool:
    """decode_rows_ref at positions S equals the separately pinned pieces applied one position at a
    time in the same dtype: rope_tables(S, 1) + apply_rope on p1 / p2 and givens on I~ (torch
    rounds every product and sum to the operand dtype, which is where the reference rounds).
    bf16 must agree bit for bit; so must fp32. Both parities, with and without RoPE / Givens."""
    ok = True
    for dtype in (torch.bfloat16, torch.float32):
        for layer in (0, 1):
            B, H, D = 3, 8, 96
            raw, theta = _decode_raw(B, H, D, 11 + layer, dtype)
            S = torch.tensor([0, 517, 4351])
            inv = O.rope_inv_freq(D, 10000.0)
            got = O.decode_rows_ref(*raw, S, inv, theta, layer, dtype, _plant=_plant)
            for b in range(B):
                cos, sin = O.rope_tables(int(S[b]), 1, D, 10000.0, dtype)
                q = O.apply_rope(raw[0][b][None, :, None, :], cos, sin)[0, :, 0]
                k = O.apply_rope(raw[1][b][None, :, None, :], cos, sin)[0, :, 0]
                v = O.givens(raw[2][b][None, :, None, :], theta, layer)[0, :, 0]
                ok &= torch.equal(got[0][b], q) and torch.equal(got[1][b], k) and torch.equal(got[2][b], v)
            # the switches: no RoPE leaves p1 / p2 as they are, no Givens leaves I~
            off = O.decode_rows_ref(*raw, S, None, None, layer, dtype, _plant=_plant)
            ok &= all(torch.equal(o, r) for o, r in zip(off, raw))
    return bool(ok)


def test_decode_rows_match_rope_and_givens_at_position_s():
    assert pin_decode_rows()


def test_decode_rows_are_the_rows_decode_step_writes():
    """The rows decode_step_ref (the graph decoder's step, restated op by op) writes at S are
    decode_rows_ref of the layer's raw projections, in bf16 and fp32."""
    for dtype in (torch.bfloat16, torch.float32):
        for layer in (0, 1):
            torch.manual_seed(20 + layer)
            m = O.FullRelationRef(64, 4, layer, dtype=dtype)
            with torch.no_grad():
                m.theta.uniform_(-0.3, 0.3)
            S, cap = 23, 32
            x = torch.randn(1, 1, 64).to(dtype)
            p2buf = torch.zeros(1, 4, cap, 16, dtype=dtype)
            ibuf = torch.zeros_like(p2buf)
            O.decode_step_ref(m, x, p2buf, ibuf, S, Cb=cap)
            with torch.no_grad():
                raw = [lin(x).view(1, 4, 16) for lin in (m.w1, m.w2, m.wi)]
            q, k, v = O.decode_rows_ref(*raw, torch.tensor([S]), O.rope_inv_freq(16, 10000.0), m.theta.detach(),
                                        layer, dtype)
            assert torch.equal(p2buf[0, :, S], k[0]) and torch.equal(ibuf[0, :, S], v[0])
            assert float(p2buf[0, :, S + 1:].abs().sum()) == 0.0


def test_decode_rows_match_the_module_heads_at_the_last_position():
    """In float64 the rows at S are the last row of FullRelationRef.heads over S + 1 positions."""
    torch.manual_seed(5)
    m = O.FullRelationRef(64, 4, 1, dtype=torch.float64)
    with torch.no_grad():
        m.theta.uniform_(-0.3, 0.3)
    S = 40
    x = torch.randn(1, S + 1, 64, dtype=torch.float64)
    p1, p2, info = m.heads(x, 0)
    with torch.no_grad():
        raw = [lin(x[:, S:]).view(1, 4, 16) for lin in (m.w1, m.w2, m.wi)]
    q, k, v = O.decode_rows_ref(*raw, torch.tensor([S]), O.rope_inv_freq(16, 10000.0), m.theta.detach(), 1,
                                torch.float64)
    for got, want in ((q, p1), (k, p2), (v, info)):
        assert torch.allclose(got[0], want[0, :, S], atol=1e-12)


@pytest.mark.parametrize("plant", ["cos_unrounded", "single_rounding", "odd_pairs_shifted"])
def test_planted_decode_row_mistakes_are_caught(plant):
    assert not pin_decode_rows(_plant=plant), f"planted mistake {plant!r} passed"


def pin_decode_rows_rope_f32(_plant=None) -> bool:
    """The graph decoder under serving autocast (graph.py:158-172 with x fp32): bf16 projections
    rotated with fp32 tables in fp32 and rounded once into the bf16 arena. Pinned by what one
    rounding means: fp32 arithmetic reproduces the exact rotation of the same bf16 inputs and fp32
    table values to within a few fp32 ulps, so nearly every element is the bf16 rounding of the
    float64 rotation (the rest sit on a rounding tie) and none is off by more than one bf16 ulp.
    The per-op bf16 convention (`_plant="per_op"`: tables and every operation rounded to bf16)
    misses the first count by far; Givens on I~ is the same in both conventions."""
    B, H, D = 4, 8, 96
    raw, theta = _decode_raw(B, H, D, 31, torch.bfloat16)
    S = torch.tensor([0, 9, 1234, 4351])
    inv = O.rope_inv_freq(D, 10000.0)
    rd = None if _plant == "per_op" else torch.float32
    got = O.decode_rows_ref(*raw, S, inv, theta, 1, torch.bfloat16, rope_dtype=rd)
    plain = O.decode_rows_ref(*raw, S, inv, theta, 1, torch.bfloat16)
    ok = torch.equal(got[2], plain[2])
    same = total = 0
    for b in range(B):
        cos, sin = O.rope_tables(int(S[b]), 1, D, 10000.0, torch.float32)  # fp32 tables: angles in fp32
        for t in range(2):
            x = raw[t][b][None, :, None, :].double()
            exact = (x * cos.double() + O.rotate_half(x) * sin.double())[0, :, 0]
            want = exact.to(torch.bfloat16)
            same += int((got[t][b] == want).sum())
            total += want.numel()
            ulp = (exact.abs().clamp(min=1e-30).log2().floor() - 7).exp2()
            ok &= bool(((got[t][b].double() - exact).abs() <= ulp * 1.0001).all())
    return bool(ok and same >= 0.995 * total)


def test_decode_rows_rope_f32_is_one_rounding_of_the_exact_rotation():
    assert pin_decode_rows_rope_f32()


def test_planted_per_op_rounding_fails_the_rope_f32_pin():
    assert not pin_decode_rows_rope_f32(_plant="per_op")


def pin_head_rms_norm(_plant=None) -> bool:
    """QK-Norm (relation.py:71-94): float64 against torch.nn.functional.rms_norm with the gain, on
    rows of very different scales (eps matters for the small ones); the closed form of a constant
    row, c w / sqrt(c^2 + eps); bf16 within one bf16 rounding of the float64 value."""
    g = torch.Generator().manual_seed(3)
    dh = 96
    norm = O.HeadRMSNormRef(dh, dtype=torch.float64)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(dh, generator=g, dtype=torch.float64) + 0.5)
    x = torch.randn(2, 4, 7, dh, generator=g, dtype=torch.float64)
    x[:, :, :3] *= 1e-3  # mean square ~1e-6, below eps
    ok = True
    got = norm(x, _plant=_plant)
    want = F.rms_norm(x, (dh,), norm.weight.detach(), eps=1e-5)
    ok &= torch.allclose(got, want, rtol=1e-6, atol=1e-9)
    c = 0.003
    row = torch.full((1, 1, 1, dh), c, dtype=torch.float64)
    closed = c * norm.weight.detach() / math.sqrt(c * c + 1e-5)
    ok &= torch.allclose(norm(row, _plant=_plant)[0, 0, 0], closed, rtol=1e-6)
    nb = O.HeadRMSNormRef(dh, dtype=torch.bfloat16)
    with torch.no_grad():
        nb.weight.copy_(norm.weight.detach().to(torch.bfloat16))
    xb = x.to(torch.bfloat16)
    gb = nb(xb, _plant=_plant)
    wb = F.rms_norm(xb.double(), (dh,), nb.weight.detach().double(), eps=1e-5)
    ok &= gb.dtype == torch.bfloat16 and bool(((gb.double() - wb).abs() <= wb.abs() * 2 ** -8 + 1e-30).all())
    return bool(ok)


def test_head_rms_norm():
    assert pin_head_rms_norm()


def test_planted_head_rms_norm_mistake_is_caught():
    assert not pin_head_rms_norm(_plant="eps_outside")
