"""Parity of the fused add+RMSNorm (mote_amd.norm, HIP) with the pure-PyTorch RMSNorm of
mote/model/norm.py:46-59, restated in oracle/norm.py.

The first two tests mirror the reference's tests/test_fused_norm.py:25-86 (its Triton kernel against
the pure path, with the same inputs, loss and tolerances); the rest cover the shapes and dtypes the
kernel's boundary admits: every row width class, ragged and strided rows, the bf16 stream, empty
inputs, the multi-pass backward and the argument errors.
"""

from __future__ import annotations

import pytest
import torch

from oracle import norm as O

pytestmark = pytest.mark.gpu


def _weight(D, seed, dev):
    torch.manual_seed(seed)
    return torch.randn(D, device=dev) * 0.2 + 1.0


def _run(fn, x, res, prenorm):
    """loss = mean(y^2) (+ mean(sin(new_res)) with prenorm), as tests/test_fused_norm.py:36-45."""
    x = x.clone().requires_grad_(True)
    res_in = res.clone().requires_grad_(True) if res is not None else None
    out = fn(x, res_in)
    if prenorm:
        y, new_res = out
        loss = y.float().pow(2).mean() + new_res.float().sin().mean()
    else:
        y, new_res = out, None
        loss = y.float().pow(2).mean()
    loss.backward()
    return y, new_res, x.grad, (res_in.grad if res_in is not None else None)


def _pair(D, seed, dev, prenorm, residual_in_fp32=True, eps=1e-5):
    from mote_amd.norm import RMSNorm

    w = _weight(D, seed, dev)
    mod = RMSNorm(D, eps=eps, device=dev, dtype=torch.float32)
    with torch.no_grad():
        mod.weight.copy_(w)
    wref = w.clone().requires_grad_(True)

    def ours(x, res):
        return mod(x, residual=res, prenorm=prenorm, residual_in_fp32=residual_in_fp32)

    def ref(x, res):
        return O.rms_norm_ref(x, wref, res, prenorm=prenorm, residual_in_fp32=residual_in_fp32, eps=eps)

    return ours, ref, mod, wref


@pytest.mark.parametrize("with_residual", [True, False])
def test_prenorm_matches_reference(cuda, with_residual):
    # tests/test_fused_norm.py:49-67
    ours, ref, mod, wref = _pair(384, 0, cuda, prenorm=True)
    torch.manual_seed(0)
    x = torch.randn(2, 96, 384, device=cuda, dtype=torch.bfloat16)
    res = torch.randn(2, 96, 384, device=cuda, dtype=torch.float32) if with_residual else None
    y_r, res_r, gx_r, gres_r = _run(ref, x, res, True)
    y_f, res_f, gx_f, gres_f = _run(ours, x, res, True)
    assert y_f.dtype == y_r.dtype == torch.bfloat16
    assert res_f.dtype == res_r.dtype == torch.float32
    assert torch.allclose(y_f.float(), y_r.float(), atol=2e-2, rtol=2e-2)
    assert torch.allclose(res_f, res_r, atol=1e-5, rtol=1e-5)
    assert torch.allclose(gx_f.float(), gx_r.float(), atol=2e-2, rtol=2e-2)
    if with_residual:
        assert torch.allclose(gres_f, gres_r, atol=1e-3, rtol=1e-3)
    assert torch.allclose(mod.weight.grad, wref.grad, atol=1e-2, rtol=1e-2)


def test_final_norm_matches_reference(cuda):
    # tests/test_fused_norm.py:70-78
    ours, ref, mod, wref = _pair(384, 1, cuda, prenorm=False)
    torch.manual_seed(1)
    x = torch.randn(3, 64, 384, device=cuda, dtype=torch.float32)
    y_r, _, gx_r, _ = _run(ref, x, None, False)
    y_f, _, gx_f, _ = _run(ours, x, None, False)
    assert torch.allclose(y_f, y_r, atol=1e-4, rtol=1e-4)
    assert torch.allclose(gx_f, gx_r, atol=1e-4, rtol=1e-4)
    assert torch.allclose(mod.weight.grad, wref.grad, atol=1e-3, rtol=1e-3)


def _check_f64(cuda, rows, D, xdt, rdt, prenorm, fp32, strided=False, seed=3):
    """Forward and every gradient against the float64 oracle (closed-form backward)."""
    from mote_amd.norm import add_rms_norm

    g = torch.Generator(device="cpu").manual_seed(seed)
    pad = 8 if strided else 0
    xs = torch.randn(rows, D + pad, generator=g).to(xdt).to(cuda)
    x = xs[:, :D]
    res = torch.randn(rows, D + pad, generator=g).to(rdt).to(cuda)[:, :D] if rdt is not None else None
    w = (torch.randn(D, generator=g) * 0.2 + 1.0).to(cuda)
    dy = torch.randn(rows, D, generator=g).to(xdt).to(cuda)
    xg = x.detach().clone().requires_grad_(True) if not strided else x.detach().requires_grad_(True)
    rg = res.detach().requires_grad_(True) if res is not None else None
    wg = w.clone().requires_grad_(True)
    out = add_rms_norm(xg, wg, rg, 1e-5, prenorm, fp32)
    y, s = out if prenorm else (out, None)
    sdt = O.rms_norm_ref(x, w, res, prenorm=True, residual_in_fp32=fp32)[1].dtype if prenorm else None
    dro = torch.randn(rows, D, generator=g).to(sdt).to(cuda) if prenorm else None
    loss = (y.float() * dy.float()).sum() + ((s.float() * dro.float()).sum() if prenorm else 0.0)
    loss.backward()
    # the stream s the kernel normalises is the one the reference forms in its own dtypes
    s_ref = O.rms_norm_ref(x, w, res, prenorm=True, residual_in_fp32=fp32)[1] if (prenorm or res is not None) else x
    y64 = O.rms_norm_ref(s_ref.double(), w.double(), eps=1e-5, compute_dtype=torch.float64)
    tol_y = 1e-5 if xdt == torch.float32 else 8e-3
    assert torch.allclose(y.double(), y64, atol=tol_y, rtol=tol_y), float((y.double() - y64).abs().max())
    if prenorm:
        assert s.dtype == s_ref.dtype and torch.equal(s, s_ref)
    ds, dw = O.rms_norm_backward_ref(dy.float(), s_ref.float(), w, eps=1e-5,
                                     dres_out=dro.float() if prenorm else None)
    tol_x = 1e-4 if xdt == torch.float32 else 1e-2
    scale = ds.abs().max().item()
    assert (xg.grad.double() - ds).abs().max().item() <= tol_x * scale
    if rg is not None:
        tol_r = 1e-4 if rdt == torch.float32 else 1e-2
        assert rg.grad.dtype == rdt and (rg.grad.double() - ds).abs().max().item() <= tol_r * scale
    assert (wg.grad.double() - dw).abs().max().item() <= 1e-4 * dw.abs().max().item() + 1e-4


@pytest.mark.parametrize("D", [4, 64, 200, 256, 384, 516, 768, 1024, 1500, 2048])
def test_widths_prenorm_bf16_fp32_stream(cuda, D):
    _check_f64(cuda, 37, D, torch.bfloat16, torch.float32, True, True)


@pytest.mark.parametrize("rows", [1, 3, 4, 5, 4095, 10003])
def test_ragged_rows_and_multipass_backward(cuda, rows):
    # 10003 rows: more than the backward's 1024 workgroups x 4 waves, so waves take several rows
    _check_f64(cuda, rows, 768, torch.bfloat16, torch.float32, True, True, seed=rows)


@pytest.mark.parametrize("case", [
    ("f32_f32_final", torch.float32, None, False, True),
    ("bf16_final", torch.bfloat16, None, False, True),
    ("bf16_no_res_prenorm", torch.bfloat16, None, True, True),
    ("bf16_bf16_stream", torch.bfloat16, torch.bfloat16, True, False),
    ("f32_bf16_fp32stream", torch.float32, torch.bfloat16, True, True),
    ("bf16_res_not_prenorm", torch.bfloat16, torch.float32, False, True),
])
def test_dtype_combinations(cuda, case):
    _, xdt, rdt, prenorm, fp32 = case
    _check_f64(cuda, 67, 384, xdt, rdt, prenorm, fp32)


def test_strided_rows(cuda):
    _check_f64(cuda, 50, 512, torch.bfloat16, torch.float32, True, True, strided=True)


def test_no_residual_no_fp32_returns_x(cuda):
    from mote_amd.norm import add_rms_norm

    x = torch.randn(5, 64, device=cuda, dtype=torch.bfloat16)
    w = torch.ones(64, device=cuda)
    y, s = add_rms_norm(x, w, None, 1e-5, True, False)
    assert s is x


def test_empty_rows(cuda):
    from mote_amd.norm import RMSNorm

    m = RMSNorm(128, device=cuda)
    x = torch.randn(0, 128, device=cuda, dtype=torch.bfloat16, requires_grad=True)
    res = torch.randn(0, 128, device=cuda, requires_grad=True)
    y, s = m(x, residual=res, prenorm=True)
    assert y.shape == (0, 128) and s.shape == (0, 128)
    (y.float().sum() + s.sum()).backward()
    assert x.grad.shape == (0, 128) and torch.equal(m.weight.grad, torch.zeros(128, device=cuda))


def test_weight_gradient_is_deterministic(cuda):
    from mote_amd.norm import RMSNorm

    m = RMSNorm(768, device=cuda)
    g = torch.Generator(device="cpu").manual_seed(7)
    x = torch.randn(6000, 768, generator=g).bfloat16().to(cuda)
    res = torch.randn(6000, 768, generator=g).to(cuda)
    grads = []
    for _ in range(3):
        m.zero_grad(set_to_none=True)
        xx, rr = x.clone().requires_grad_(True), res.clone().requires_grad_(True)
        y, s = m(xx, residual=rr, prenorm=True)
        (y.float().pow(2).mean() + s.sin().mean()).backward()
        grads.append((m.weight.grad.clone(), xx.grad.clone(), rr.grad.clone()))
    for a, b in zip(grads[0], grads[1]):
        assert torch.equal(a, b)
    for a, b in zip(grads[0], grads[2]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("D", [6, 2052])
def test_unsupported_width_raises(cuda, D):
    from mote_amd.norm import add_rms_norm

    x = torch.randn(4, D, device=cuda)
    with pytest.raises(RuntimeError, match="D = "):
        add_rms_norm(x, torch.ones(D, device=cuda))
