"""FullRelation and its RoPE / Givens prologue through the HIP library against the CPU oracle
module (oracle.relation.FullRelationRef), following tests/test_relation_paths.py:19-48,
tests/test_givens_and_rope.py and tests/test_mote_model.py:22-36 of the reference."""

from __future__ import annotations

import pytest
import torch

from conftest import rel_err
from oracle import relation as O

pytestmark = pytest.mark.gpu


def _pair(d_model, n_heads, layer_idx, seed=0, **kw):
    from mote_amd.relation import FullRelation

    torch.manual_seed(seed)
    mine = FullRelation(d_model, n_heads, layer_idx, device="cuda", dtype=torch.float32, **kw)
    with torch.no_grad():
        mine.theta.uniform_(-0.3, 0.3)
        mine.lam.fill_(0.4)
    ref = O.FullRelationRef(d_model, n_heads, layer_idx, dtype=torch.float32, **kw)
    missing, unexpected = ref.load_state_dict({k: v.detach().cpu() for k, v in mine.state_dict().items()}, strict=False)
    assert not unexpected and not missing, (missing, unexpected)
    return mine, ref


# (H, D, T): the row-staged kernels at several row widths and partial last blocks, and D = 40
# (D/2 not a multiple of the 16-byte chunk in bf16), which takes the per-row kernels
@pytest.mark.parametrize("H,D,T", [(8, 64, 37), (8, 96, 301), (2, 48, 53), (4, 32, 9), (2, 40, 23)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layer_idx", [0, 1])
def test_rope_givens_forward_and_grads(cuda, dtype, layer_idx, H, D, T):
    from mote_amd.relation import rope_givens, rope_inv_freq

    print(f"case rope_givens {dtype} layer={layer_idx} H={H} D={D} T={T}", flush=True)
    B, S = 2, 11
    g = torch.Generator().manual_seed(layer_idx)
    qkv = (torch.randn(B, T, 3 * H * D, generator=g) * 0.8).to(dtype)
    theta = torch.rand(H // 2, generator=g) * 0.6 - 0.3
    inv = rope_inv_freq(D, 10000.0)
    qd = qkv.cuda().requires_grad_(True)
    td = theta.cuda().requires_grad_(True)
    p1, p2, info = rope_givens(qd, H, inv.cuda(), td, layer_idx, S)
    # oracle: the reference's table semantics with tables in the operand dtype
    cos, sin = O.rope_tables(S, T, D, 10000.0, dtype)
    qr = qkv.double().requires_grad_(True)
    tr = theta.double().requires_grad_(True)
    q, k, v = (qr[..., i * H * D:(i + 1) * H * D].view(B, T, H, D).transpose(1, 2) for i in range(3))
    c, s = cos.double(), sin.double()
    r1, r2 = O.apply_rope(q, c, s), O.apply_rope(k, c, s)
    # the dtype-rounded value with the gradient of the unrounded function (autograd passes through
    # the reference's `.to(dtype)` cast unchanged)
    cg = torch.cos(tr).detach().to(dtype).double() + (torch.cos(tr) - torch.cos(tr).detach())
    sg = torch.sin(tr).detach().to(dtype).double() + (torch.sin(tr) - torch.sin(tr).detach())
    a_idx, b_idx = O.givens_pairs(H, layer_idx)
    ia, ib = v[:, a_idx], v[:, b_idx]
    rv = v.clone()
    rv[:, a_idx] = cg[None, :, None, None] * ia - sg[None, :, None, None] * ib
    rv[:, b_idx] = sg[None, :, None, None] * ia + cg[None, :, None, None] * ib
    tol = 1e-6 if dtype == torch.float32 else 8e-3
    for got, want in zip((p1, p2, info), (r1, r2, rv)):
        assert rel_err(got, want) < tol, rel_err(got, want)
    w = [torch.randn(B, H, T, D, generator=g) for _ in range(3)]
    loss = sum((t.float() * wi.cuda()).sum() for t, wi in zip((p1, p2, info), w))
    dq, dt = torch.autograd.grad(loss, [qd, td])
    lr = sum((t * wi.double()).sum() for t, wi in zip((r1, r2, rv), w))
    dqr, dtr = torch.autograd.grad(lr, [qr, tr])
    gtol = 1e-5 if dtype == torch.float32 else 2e-2
    assert rel_err(dq, dqr) < gtol, rel_err(dq, dqr)
    assert rel_err(dt, dtr) < gtol, rel_err(dt, dtr)


@pytest.mark.parametrize("d_model,n_heads,T", [(192, 2, 130), (128, 2, 70), (96, 2, 40), (768, 8, 300)])
@pytest.mark.parametrize("layer_idx", [0, 1])
def test_module_matches_oracle_fp32(cuda, d_model, n_heads, T, layer_idx):
    print(f"case module d={d_model} H={n_heads} T={T} layer={layer_idx}", flush=True)
    mine, ref = _pair(d_model, n_heads, layer_idx)
    x = torch.randn(2, T, d_model, generator=torch.Generator().manual_seed(1)) * 0.8
    wgt = torch.linspace(-1, 1, 2 * T * d_model).view(2, T, d_model)
    xd = x.cuda().requires_grad_(True)
    out, g = mine(xd, return_gates=True)
    (out * wgt.cuda()).sum().backward()
    xr = x.clone().requires_grad_(True)
    outr, gr = ref(xr, return_gates=True)
    (outr * wgt).sum().backward()
    assert rel_err(out, outr) < 1e-5, rel_err(out, outr)
    assert float((g.cpu() - gr).abs().max()) < 1e-5
    assert rel_err(xd.grad, xr.grad) < 1e-5, rel_err(xd.grad, xr.grad)
    grads_r = dict(ref.named_parameters())
    for n, p in mine.named_parameters():
        assert rel_err(p.grad, grads_r[n].grad) < 1e-5, (n, rel_err(p.grad, grads_r[n].grad))


@pytest.mark.parametrize("layer_idx", [0, 1])
def test_c1_mote1m_layer_matches_oracle(cuda, layer_idx):
    """the Mote-1M Relation layer (d_model 192, 4 heads, dh 48), fp32, B = 2,
    T = 256, hidden N(0,1) then RMSNorm (eps 1e-5, unit weight), weights from seed 0, theta ~
    U(-0.3, 0.3) and lam = 0.4; the forward output and the gates against the oracle module."""
    print(f"case C1 layer={layer_idx}", flush=True)
    mine, ref = _pair(192, 4, layer_idx, seed=0)
    x = torch.randn(2, 256, 192, generator=torch.Generator().manual_seed(0))
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)
    out, g = mine(x.cuda(), return_gates=True)
    outr, gr = ref(x, return_gates=True)
    assert rel_err(out, outr) < 1e-5, rel_err(out, outr)
    assert float((g.cpu() - gr).abs().max()) < 1e-5


def test_module_bf16_autocast(cuda):
    mine, ref = _pair(768, 8, 1, seed=3)
    x = torch.randn(1, 500, 768, generator=torch.Generator().manual_seed(2))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out, g = mine(x.cuda(), return_gates=True)
    outr, gr = ref(x, return_gates=True)
    assert rel_err(out.float(), outr) < 2e-2, rel_err(out.float(), outr)
    assert float((g.cpu() - gr).abs().max()) < 2e-2


def test_module_causal_cache_split_and_gates(cuda):
    """tests/test_mote_model.py:22-36 on the HIP module."""
    from mote_amd.relation import FullRelation

    torch.manual_seed(0)
    m = FullRelation(64, 4, layer_idx=1, device="cuda")
    x = torch.randn(2, 10, 64, device="cuda")
    y = m(x)
    x2 = x.clone()
    x2[:, 7:] += 1.0
    assert torch.allclose(m(x2)[:, :7], y[:, :7], atol=1e-5)
    y_pre, cache = m(x[:, :6], return_cache=True)
    y_rest = m(x[:, 6:], cache=cache)
    assert torch.allclose(torch.cat([y_pre, y_rest], 1), y, atol=1e-4)
    _, g = m(x, return_gates=True)
    assert torch.all(g[:, :, 0] == 0) and torch.all(g[:, :, 1:] > 0) and torch.all(g < 1)


def test_module_arena_prefill_and_steps(cuda):
    """Prefill through the arena, then one-chunk continuations, equal the one-shot forward."""
    from mote_amd.arena import ArenaState, RelationArena
    from mote_amd.relation import FullRelation

    torch.manual_seed(1)
    m = FullRelation(128, 4, layer_idx=0, device="cuda")
    with torch.no_grad():
        m.theta.uniform_(-0.3, 0.3)
    x = torch.randn(1, 40, 128, device="cuda")
    full = m(x)
    arena = RelationArena(1, 4, 64, 32, "cuda", torch.float32)
    st = ArenaState(arena)
    outs = [m(x[:, :30], cache=st[0])]
    st.advance(30)
    for t in range(30, 40):
        outs.append(m(x[:, t:t + 1], cache=st[0]))
        st.advance(1)
    assert torch.allclose(torch.cat(outs, 1), full, atol=1e-5)
    assert torch.isfinite(arena.buf).all()


def test_decode_step_module_matches_oracle(cuda):
    from mote_amd.arena import RelationArena
    from mote_amd.decode import RelationDecodeStep

    mine, ref = _pair(768, 8, 1, seed=4)
    S, cap = 900, 1024
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, S + 1, 768, generator=g)
    _, (p2c, ic) = ref(x[:, :S], return_cache=True)
    arena = RelationArena(1, 8, cap, 96, "cuda", torch.float32)
    arena.buf[0, 0, :, :S] = p2c[0].detach().cuda()
    arena.buf[0, 1, :, :S] = ic[0].detach().cuda()
    step = RelationDecodeStep(mine, arena, 0)
    Sd = torch.tensor([S], device="cuda")
    out, xm = step(x[:, S:].cuda(), Sd, advance=True)
    p2buf = torch.zeros(1, 8, cap, 96)
    ibuf = torch.zeros(1, 8, cap, 96)
    p2buf[:, :, :S], ibuf[:, :, :S] = p2c.detach(), ic.detach()
    outr, yr, xmr = O.decode_step_ref(ref, x[:, S:], p2buf, ibuf, S, Cb=cap)
    assert rel_err(out, outr) < 1e-5, rel_err(out, outr)
    assert abs(float(xm) - float(xmr)) < 1e-5
    assert int(Sd) == S + 1
    assert rel_err(arena.buf[0, 0, :, S], p2buf[0, :, S]) < 1e-5
    assert rel_err(arena.buf[0, 1, :, S], ibuf[0, :, S]) < 1e-5
    # a parameter update reaches the step through sync_params() (the step keeps its own stacked
    # projection weight and fp32 copies, which a captured graph reads)
    with torch.no_grad():
        for m in (mine, ref):
            m.w2.weight.mul_(0.5)
            m.lam.add_(0.25)
    step.sync_params()
    x2 = torch.randn(1, 1, 768, generator=g)
    out2, xm2 = step(x2.cuda(), Sd, advance=True)
    outr2, _, xmr2 = O.decode_step_ref(ref, x2, p2buf, ibuf, S + 1, Cb=cap)
    assert rel_err(out2, outr2) < 1e-5, rel_err(out2, outr2)
    assert abs(float(xm2) - float(xmr2)) < 1e-5
    assert int(Sd) == S + 2
