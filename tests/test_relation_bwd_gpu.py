"""Fused backward through the HIP library against autograd of the CPU oracle (float64).

Follows the reference's gradient tests (tests/test_flash_relation.py:28-100) with the BASELINE
tolerances: 1e-5 relative in fp32, 2e-2 relative in bf16 (relative = max|a-b| / max|ref|).
"""

from __future__ import annotations

import pytest
import torch

from conftest import rel_err
from oracle import relation as O

pytestmark = pytest.mark.gpu


def _inputs(B, H, TQ, S, D, dtype, seed=0, scale=0.7):
    g = torch.Generator().manual_seed(seed)
    mk = lambda T: (torch.randn(B, H, T, D, generator=g) * scale).to(dtype).cuda().requires_grad_(True)
    p1, p2, info = mk(TQ), mk(S + TQ), mk(S + TQ)
    lam = torch.tensor(0.5, device="cuda", requires_grad=True)
    dy = (torch.randn(B, H, TQ, D, generator=g)).to(dtype).cuda()
    return p1, p2, info, lam, dy


def _grads(p1, p2, info, lam, dy, S, deterministic=False):
    import mote_amd.flash_relation as fr

    old = fr.DETERMINISTIC
    fr.DETERMINISTIC = deterministic
    try:
        y, g = fr.flash_relation(p1, p2, info, lam, 2.0, q_start=S)
        grads = torch.autograd.grad((y.float() * dy.float()).sum(), [p1, p2, info, lam])
    finally:
        fr.DETERMINISTIC = old
    torch.cuda.synchronize()
    return grads


def _oracle_grads(p1, p2, info, lam, dy, S):
    return O.relation_grads_autograd(p1.detach().cpu(), p2.detach().cpu(), info.detach().cpu(), lam.detach().cpu(),
                                     dy.cpu(), 2.0, S, dtype=torch.float64)


NAMES = ["dp1", "dp2", "dinfo", "dlam"]


def _check(got, ref, tol, p1, p2, info, lam, dy, S):
    """Tensors: max|a-b| / max|ref| < tol. dlam is one scalar that cancels across rows, so its error
    is measured against the sum of the magnitudes of its summands instead of |dlam| itself."""
    for a, b, n in zip(got, ref, NAMES):
        assert a.shape == b.shape, n
        if n == "dlam":
            terms = O.relation_dlam_terms(p1.detach().cpu(), p2.detach().cpu(), info.detach().cpu(),
                                          lam.detach().cpu(), dy.cpu(), 2.0, S)
            err = abs(float(a) - float(b)) / max(float(terms.abs().sum()), 1e-3)
        else:
            err = rel_err(a, b)
        assert err < tol, (n, err)


@pytest.mark.parametrize("det", [False, True])
@pytest.mark.parametrize("D", [48, 64, 96])
@pytest.mark.parametrize("TQ,S", [(16, 0), (50, 0), (130, 0), (300, 0), (20, 37), (64, 64)])
def test_fp32_grads_match_oracle(cuda, D, TQ, S, det):
    print(f"case fp32 grads D={D} TQ={TQ} S={S} det={det}", flush=True)
    p1, p2, info, lam, dy = _inputs(2, 3, TQ, S, D, torch.float32)
    got = _grads(p1, p2, info, lam, dy, S, det)
    ref = _oracle_grads(p1, p2, info, lam, dy, S)
    _check(got, ref, 1e-5, p1, p2, info, lam, dy, S)
    for a, b, n in zip(got, ref, NAMES):  # the reference's own bounds (test_flash_relation.py:35-38)
        assert torch.allclose(a.cpu().double(), b, atol=3e-4, rtol=2e-3), n


@pytest.mark.parametrize("D", [96, 112, 24])
def test_odd_head_dim_grads(cuda, D):
    p1, p2, info, lam, dy = _inputs(1, 2, 90, 0, D, torch.float32)
    got = _grads(p1, p2, info, lam, dy, 0)
    ref = _oracle_grads(p1, p2, info, lam, dy, 0)
    _check(got, ref, 1e-5, p1, p2, info, lam, dy, 0)


def test_rescale_branch_grads(cuda):
    p1, p2, info, lam, dy = _inputs(1, 2, 200, 0, 64, torch.float32, seed=3, scale=3.0)
    got = _grads(p1, p2, info, lam, dy, 0)
    ref = _oracle_grads(p1, p2, info, lam, dy, 0)
    _check(got, ref, 1e-5, p1, p2, info, lam, dy, 0)


@pytest.mark.parametrize("D", [64, 96, 128])
def test_bf16_scale3_stress_grads(cuda, D):
    """Scores of scale 3 (|U| up to ~30, the reference's rescale stress, tests/test_flash_relation.py:54-57)
    in bf16 through the tile kernels: outputs and gradients within 2e-2 of the float64 oracle."""
    import mote_amd.flash_relation as fr

    print(f"case bf16 scale-3 grads D={D}", flush=True)
    p1, p2, info, lam, dy = _inputs(1, 4, 333, 0, D, torch.bfloat16, seed=11, scale=3.0)
    y, g = fr.flash_relation(p1, p2, info, lam, 2.0)
    yr, gr = O.relation_reference(p1.detach().cpu(), p2.detach().cpu(), info.detach().cpu(), lam.detach().cpu(), 2.0, 0,
                                  dtype=torch.float64)
    assert rel_err(y, yr) < 2e-2 and rel_err(g, gr) < 2e-2
    got = _grads(p1, p2, info, lam, dy, 0)
    ref = _oracle_grads(p1, p2, info, lam, dy, 0)
    _check(got, ref, 2e-2, p1, p2, info, lam, dy, 0)


@pytest.mark.parametrize("det", [False, True])
@pytest.mark.parametrize("D", [32, 48, 64, 96, 128])
@pytest.mark.parametrize("TQ", [33, 257])
def test_bf16_grads(cuda, D, TQ, det):
    print(f"case bf16 grads D={D} TQ={TQ} det={det}", flush=True)
    p1, p2, info, lam, dy = _inputs(2, 4, TQ, 0, D, torch.bfloat16)
    got = _grads(p1, p2, info, lam, dy, 0, det)
    ref = _oracle_grads(p1, p2, info, lam, dy, 0)
    for a, n in zip(got, NAMES):
        assert a.dtype == (torch.float32 if n == "dlam" else torch.bfloat16), n
    _check(got, ref, 2e-2, p1, p2, info, lam, dy, 0)


def test_bf16_flagship_prefix_grads(cuda):
    p1, p2, info, lam, dy = _inputs(1, 8, 700, 64, 96, torch.bfloat16, seed=2)
    got = _grads(p1, p2, info, lam, dy, 64)
    ref = _oracle_grads(p1, p2, info, lam, dy, 64)
    _check(got, ref, 2e-2, p1, p2, info, lam, dy, 64)


@pytest.mark.parametrize("D,TQ,S", [(64, 100, 37), (96, 129, 200), (128, 65, 63), (32, 1, 5)])
def test_bf16_prefix_grads(cuda, D, TQ, S):
    """Cached prefixes that do not align with the 64-row blocks of the tile kernels."""
    print(f"case bf16 prefix grads D={D} TQ={TQ} S={S}", flush=True)
    p1, p2, info, lam, dy = _inputs(2, 2, TQ, S, D, torch.bfloat16, seed=7)
    got = _grads(p1, p2, info, lam, dy, S)
    ref = _oracle_grads(p1, p2, info, lam, dy, S)
    _check(got, ref, 2e-2, p1, p2, info, lam, dy, S)


def test_bf16_tile_path_is_bitwise_reproducible(cuda):
    """The bf16 kernels use no atomics: both settings of the switch give identical bits."""
    p1, p2, info, lam, dy = _inputs(1, 8, 777, 0, 64, torch.bfloat16, seed=6)
    a = _grads(p1, p2, info, lam, dy, 0, False)
    b = _grads(p1, p2, info, lam, dy, 0, False)
    c = _grads(p1, p2, info, lam, dy, 0, True)
    for x, y, z, n in zip(a, b, c, NAMES):
        assert torch.equal(x, y) and torch.equal(x, z), n


def test_one_pass_and_two_pass_agree(cuda):
    """tests/test_flash_relation.py:60-68: the atomic and the deterministic backward agree."""
    p1, p2, info, lam, dy = _inputs(2, 2, 150, 10, 96, torch.float32, seed=1)
    fast = _grads(p1, p2, info, lam, dy, 10, False)
    slow = _grads(p1, p2, info, lam, dy, 10, True)
    for a, b, n in zip(fast, slow, NAMES):
        assert torch.allclose(a, b, atol=3e-5, rtol=1e-5), n


def test_deterministic_mode_is_bitwise_reproducible(cuda):
    p1, p2, info, lam, dy = _inputs(1, 8, 1000, 0, 96, torch.bfloat16, seed=5)
    a = _grads(p1, p2, info, lam, dy, 0, True)
    b = _grads(p1, p2, info, lam, dy, 0, True)
    for x, y, n in zip(a, b, NAMES):
        assert torch.equal(x, y), n


def test_empty_query_rows_give_zero_prefix_grads(cuda):
    p1, p2, info, lam, dy = _inputs(1, 2, 0, 6, 32, torch.float32)
    got = _grads(p1, p2, info, lam, dy, 6)
    assert got[0].shape == (1, 2, 0, 32)
    assert float(got[1].abs().max()) == 0.0 and float(got[2].abs().max()) == 0.0
    assert float(got[3]) == 0.0


def test_c3_full_size_bf16_against_fp32_kernels(cuda):
    """Config C3 at its real size (T = 4964 chunks, H = 8, dh = 96): the bf16 tile kernels against
    the fp32 kernels (pinned to the float64 oracle at 1e-5 by the tests above) on the same inputs,
    upcast. Y, g and every gradient within 2e-2; dlam against the summed magnitude of its terms
    -dA_i ln(i+1) (it cancels across rows), worked out on the device from the fp32 forward."""
    print("case C3 full size T=4964 H=8 D=96 bf16 vs fp32 kernels", flush=True)
    import mote_amd.flash_relation as fr

    T = 4964
    p1, p2, info, lam, dy = _inputs(1, 8, T, 0, 96, torch.bfloat16, seed=2)
    up = lambda t: t.detach().float().requires_grad_(True)
    p1f, p2f, infof, lamf = up(p1), up(p2), up(info), up(lam)
    y, g = fr.flash_relation(p1, p2, info, lam, 2.0, q_start=0)
    yf, gf = fr.flash_relation(p1f, p2f, infof, lamf, 2.0, q_start=0)
    assert rel_err(y, yf) < 2e-2
    assert float((g - gf).abs().max()) < 2e-2
    got = torch.autograd.grad((y.float() * dy.float()).sum(), [p1, p2, info, lam])
    ref = torch.autograd.grad((yf * dy.float()).sum(), [p1f, p2f, infof, lamf])
    for a, b, n in zip(got[:3], ref[:3], NAMES):
        assert a.shape == b.shape and a.dtype == torch.bfloat16, n
        assert rel_err(a, b) < 2e-2, (n, rel_err(a, b))
    with torch.no_grad():
        _, gg, ibar, _ = torch.ops.mote.relation_fwd(p1f, p2f, infof, lamf, 2.0, 0)
        dA = (dy.float() * (ibar - infof)).sum(-1) * gg * (1 - gg)
        scale = float((dA * torch.log(torch.arange(1, T + 1, device=cuda, dtype=torch.float32))).abs().sum())
    assert abs(float(got[3]) - float(ref[3])) / max(scale, 1e-3) < 2e-2
    assert torch.isfinite(got[3])
