"""mote_wgrad: the projections' weight gradient dW = A^T X (bf16, fp32 sums over the token rows),
through the C ABI and through mote::wgrad, against the float64 product of the same bf16 inputs.

The inputs are bf16, so the float64 product is the exact sum; the kernel's only roundings are its
fp32 accumulation and the one bf16 rounding of each output (2^-9 of the element), so 4e-3 of the
largest element bounds it. A transposed operand, a dropped or doubled stage, or the rows past M of
a ragged last stage counted would each miss by far more.
"""

from __future__ import annotations

import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _abi_wgrad(a: torch.Tensor, x: torch.Tensor, dw: torch.Tensor) -> None:
    from mote_amd import _lib as Lb

    args = Lb.WgradArgs()
    args.dtype, args.M, args.N, args.K = Lb.MOTE_BF16, a.shape[0], a.shape[1], x.shape[1]
    args.a, args.a_sr = a.data_ptr(), a.stride(0)
    args.x, args.x_sr = x.data_ptr(), x.stride(0)
    args.dw, args.dw_sr = dw.data_ptr(), dw.stride(0)
    n = int(Lb.lib().mote_wgrad_workspace(args))
    ws = torch.full((max(n, 16),), 0x7F, device=a.device, dtype=torch.uint8)  # NaN-patterned partials
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    Lb.check(Lb.lib().mote_wgrad(args, Lb.stream_of(a)), "mote_wgrad")
    torch.cuda.synchronize()


# (M, N, K): one stage, ragged last stages (1, 63, 65 rows past a stage), one tile and many splits,
# the Mote-96M prologue (2304 x 768, four splits) and gate (768 x 768) shapes
CASES = [(1, 128, 128), (63, 256, 128), (64, 128, 256), (65, 384, 128), (300, 1536, 512), (2000, 128, 128),
         (4964, 2304, 768), (4964, 768, 768), (9001, 256, 384)]


@pytest.mark.parametrize("M,N,K", CASES)
def test_wgrad_matches_float64(cuda, M, N, K):
    print(f"case wgrad M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, N, generator=g).bfloat16()
    x = torch.randn(M, K, generator=g).bfloat16()
    ref = a.double().t() @ x.double()
    ac, xc = a.to(cuda), x.to(cuda)
    dw = torch.full((N, K), float("nan"), device=cuda, dtype=torch.bfloat16)
    _abi_wgrad(ac, xc, dw)
    assert rel_err(dw, ref) < 4e-3, rel_err(dw, ref)
    again = torch.full_like(dw, float("nan"))
    _abi_wgrad(ac, xc, again)
    assert torch.equal(dw, again), "bitwise reproducible"


def test_wgrad_strided_rows(cuda):
    """Operands and output as column windows of wider row-major tensors (row strides above the
    widths): only the window is read and written."""
    print("case wgrad strided", flush=True)
    g = torch.Generator().manual_seed(3)
    A = torch.randn(777, 640, generator=g).bfloat16().to(cuda)
    X = torch.randn(777, 512, generator=g).bfloat16().to(cuda)
    a, x = A[:, 128:384], X[:, 256:384]
    out = torch.full((256, 384), 7.0, device=cuda, dtype=torch.bfloat16)
    dw = out[:, 128:256]
    _abi_wgrad(a, x, dw)
    ref = a.cpu().double().t() @ x.cpu().double()
    assert rel_err(dw, ref) < 4e-3
    assert bool((out[:, :128] == 7).all()) and bool((out[:, 256:] == 7).all())


def test_wgrad_empty_reduction_writes_zeros(cuda):
    print("case wgrad M=0", flush=True)
    a = torch.empty(0, 128, device=cuda, dtype=torch.bfloat16)
    x = torch.empty(0, 256, device=cuda, dtype=torch.bfloat16)
    dw = torch.full((128, 256), float("nan"), device=cuda, dtype=torch.bfloat16)
    _abi_wgrad(a, x, dw)
    assert bool((dw == 0).all())


def test_weight_grad_op_and_dispatch(cuda):
    """mote::wgrad through weight_grad (batched rows, a non-contiguous x) against torch's product,
    the op's registration checked by opcheck, and the library product for widths off 128."""
    from mote_amd.relation import _wgrad, weight_grad

    print("case wgrad op", flush=True)
    g = torch.Generator().manual_seed(5)
    a = torch.randn(2, 301, 384, generator=g).bfloat16().to(cuda)
    xw = torch.randn(2, 301, 512, generator=g).bfloat16().to(cuda)
    x = xw[..., :256]
    got = weight_grad(a, x)
    ref = a.reshape(-1, 384).double().t() @ x.reshape(-1, 256).double()
    assert got.shape == (384, 256) and got.dtype == torch.bfloat16
    assert rel_err(got, ref) < 4e-3
    torch.library.opcheck(_wgrad, (a.reshape(-1, 384), x.reshape(-1, 256).contiguous()))
    odd = weight_grad(a[..., :200], x)  # N = 200: the library product
    assert rel_err(odd, a[..., :200].reshape(-1, 200).double().t() @ x.reshape(-1, 256).double()) < 1e-2


@pytest.mark.parametrize("autocast", [False, True])
def test_module_weight_gradients_on_wgrad(cuda, monkeypatch, autocast):
    """FullRelation's backward with the weight gradients of the prologue, the gate and wo on
    mote_wgrad against the same step with them on the GEMM library: bf16 weights, or fp32 weights
    under bf16 autocast (the weights' bf16 casts carry the gradients back to fp32)."""
    from mote_amd import relation as R

    print(f"case wgrad module autocast={autocast}", flush=True)
    torch.manual_seed(12)
    dtype = torch.float32 if autocast else torch.bfloat16
    m = R.FullRelation(256, 4, 1, out_gate=True, dtype=dtype).to(cuda)
    x = (torch.randn(2, 300, 256, device=cuda) * 0.5).to(dtype)
    dy = torch.randn(2, 300, 256, device=cuda).to(dtype)

    def grads(use):
        monkeypatch.setattr(R, "USE_WGRAD", use)
        m.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            out = m(xi)
        (out.float() * dy.float()).sum().backward()
        return {n: p.grad.clone() for n, p in m.named_parameters() if p.grad is not None}, xi.grad.clone()

    got, gx = grads(True)
    ref, rx = grads(False)
    assert set(got) == set(ref) and {"w1.weight", "wo.weight", "wg.weight"} <= set(got)
    for n in ref:
        assert got[n].dtype == ref[n].dtype, n
        assert rel_err(got[n], ref[n]) < 1e-2, (n, rel_err(got[n], ref[n]))
    assert rel_err(gx, rx) < 1e-2
