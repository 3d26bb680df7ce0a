"""CPU pins of the add+RMSNorm oracle (oracle/norm.py) and the host logic of mote_amd.norm.

The oracle restates mote/model/norm.py:36-59; these tests tie it to what fixes it independently:
torch's own rms_norm, a closed form, autograd and finite differences, and the reference's dtype
rules for the returned residual stream. Each planted mistake must fail one of them.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import norm as O


def _inputs(rows=6, D=40, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, D, generator=g, dtype=dtype)
    res = torch.randn(rows, D, generator=g, dtype=dtype)
    w = (torch.randn(D, generator=g, dtype=dtype) * 0.2 + 1.0)
    return x, res, w


def test_forward_matches_torch_rms_norm():
    x, res, w = _inputs()
    for eps in (1e-5, 0.3):
        want = F.rms_norm(x + res, (x.shape[-1],), w, eps)
        got = O.rms_norm_ref(x, w, res, eps=eps, compute_dtype=torch.float64)
        assert torch.allclose(got, want, atol=1e-12, rtol=1e-12)


def test_forward_closed_form_constant_row():
    # a row of constant c: mean(s^2) = c^2, so y = c w / sqrt(c^2 + eps)
    D, eps = 12, 0.25
    w = torch.linspace(0.5, 2.0, D, dtype=torch.float64)
    for c in (-3.0, 0.5, 2.0):
        x = torch.full((1, D), c, dtype=torch.float64)
        got = O.rms_norm_ref(x, w, eps=eps, compute_dtype=torch.float64)
        assert torch.allclose(got[0], c * w / (c * c + eps) ** 0.5, atol=1e-14)


@pytest.mark.parametrize("plant", ["eps_outside", "sum_not_mean", "no_weight"])
def test_forward_plants_fail(plant):
    x, res, w = _inputs()
    want = F.rms_norm(x + res, (x.shape[-1],), w, 0.3)
    got = O.rms_norm_ref(x, w, res, eps=0.3, compute_dtype=torch.float64, _plant=plant)
    assert not torch.allclose(got, want, atol=1e-6)


def _autograd_grads(x, res, w, eps, dy, dro):
    x, res, w = (t.clone().requires_grad_(True) for t in (x, res, w))
    y, s = O.rms_norm_ref(x, w, res, prenorm=True, eps=eps, compute_dtype=torch.float64)
    ((y * dy).sum() + (s * dro).sum()).backward()
    return x.grad, res.grad, w.grad


@pytest.mark.parametrize("with_dro", [False, True])
def test_backward_matches_autograd(with_dro):
    x, res, w = _inputs(seed=1)
    g = torch.Generator().manual_seed(9)
    dy = torch.randn(x.shape, generator=g, dtype=torch.float64)
    dro = torch.randn(x.shape, generator=g, dtype=torch.float64) if with_dro else torch.zeros_like(x)
    gx, gres, gw = _autograd_grads(x, res, w, 0.1, dy, dro)
    ds, dw = O.rms_norm_backward_ref(dy, x + res, w, eps=0.1, dres_out=dro if with_dro else None)
    assert torch.allclose(ds, gx, atol=1e-12) and torch.allclose(ds, gres, atol=1e-12)
    assert torch.allclose(dw, gw, atol=1e-12)


@pytest.mark.parametrize("plant", ["no_proj", "r_squared"])
def test_backward_plants_fail(plant):
    x, res, w = _inputs(seed=1)
    dy = torch.randn(x.shape, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    gx, _, _ = _autograd_grads(x, res, w, 0.1, dy, torch.zeros_like(x))
    ds, _ = O.rms_norm_backward_ref(dy, x + res, w, eps=0.1, _plant=plant)
    assert not torch.allclose(ds, gx, atol=1e-6)


def test_backward_finite_differences():
    # central differences of sum(y * dy) in float64 pin the closed form without autograd
    x, _, w = _inputs(rows=2, D=8, seed=3)
    dy = torch.randn(x.shape, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    ds, dw = O.rms_norm_backward_ref(dy, x, w, eps=0.05)
    h = 1e-6

    def f(xx, ww):
        return float((O.rms_norm_ref(xx, ww, eps=0.05, compute_dtype=torch.float64) * dy).sum())

    for idx in [(0, 0), (0, 5), (1, 3), (1, 7)]:
        xp, xm = x.clone(), x.clone()
        xp[idx] += h
        xm[idx] -= h
        assert abs((f(xp, w) - f(xm, w)) / (2 * h) - float(ds[idx])) < 1e-7
    for d in (0, 4, 7):
        wp, wm = w.clone(), w.clone()
        wp[d] += h
        wm[d] -= h
        assert abs((f(x, wp) - f(x, wm)) / (2 * h) - float(dw[d])) < 1e-7


def test_prenorm_stream_dtypes():
    # norm.py:50-55: the stream is fp32 when residual_in_fp32 and a residual or prenorm; the dtype
    # of x + residual otherwise; x itself without a residual when not residual_in_fp32
    x = torch.randn(3, 16).bfloat16()
    res = torch.randn(3, 16)
    w = torch.ones(16)
    y, s = O.rms_norm_ref(x, w, res, prenorm=True)
    assert y.dtype == torch.bfloat16 and s.dtype == torch.float32
    assert torch.equal(s, x.float() + res)
    y, s = O.rms_norm_ref(x, w, None, prenorm=True)
    assert s.dtype == torch.float32 and torch.equal(s, x.float())
    y, s = O.rms_norm_ref(x, w, None, prenorm=True, residual_in_fp32=False)
    assert s is x
    y, s = O.rms_norm_ref(x, w, res.bfloat16(), prenorm=True, residual_in_fp32=False)
    assert s.dtype == torch.bfloat16 and torch.equal(s, x + res.bfloat16())


def test_sum_dtype_rules_match_oracle():
    from mote_amd.norm import _sum_dtype

    x = torch.randn(2, 8).bfloat16()
    w = torch.ones(8)
    for res in (None, torch.randn(2, 8), torch.randn(2, 8).bfloat16()):
        for prenorm in (False, True):
            for fp32 in (False, True):
                out = O.rms_norm_ref(x, w, res, prenorm=True, residual_in_fp32=fp32)
                want = out[1].dtype if (prenorm or res is not None) else x.dtype
                assert _sum_dtype(x, res, prenorm, fp32) == want


def test_rmsnorm_module_signature_and_cpu_error():
    from mote_amd.norm import RMSNorm

    m = RMSNorm(16, eps=1e-6)
    assert m.eps == 1e-6 and m.weight.shape == (16,) and torch.equal(m.weight.detach(), torch.ones(16))
    with pytest.raises(RuntimeError, match="HIP"):
        m(torch.randn(2, 16), residual=torch.randn(2, 16), prenorm=True)
