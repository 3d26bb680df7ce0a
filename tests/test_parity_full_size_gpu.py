"""Parity at the benchmark shapes and on the module options, through the HIP library, against the
float64 CPU oracle: config C2 at its full size, the bf16 tile backward at the C3 length, FullRelation
with QK-Norm / output gate / no RoPE / no Givens, the reference's rounding points of the RoPE /
Givens kernels, and the custom ops under torch.library.opcheck and torch.compile(fullgraph=True)
(tests/test_relation_paths.py:51-78 of the reference)."""

from __future__ import annotations

import pytest
import torch

from conftest import rel_err
from oracle import relation as O

pytestmark = pytest.mark.gpu


def _rms(x, eps=1e-5):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def _rotated_ref(qkv, H, inv, theta, parity, pos0=0):
    """float64 RoPE / Givens of a [B, T, 3 H dh] projection with the operand-dtype tables, leaves
    (qkv, theta) for autograd."""
    B, T, D3 = qkv.shape
    D = D3 // (3 * H)
    q, k, v = (qkv[..., i * H * D:(i + 1) * H * D].reshape(B, T, H, D).transpose(1, 2) for i in range(3))
    cos, sin = O.rope_tables(pos0, T, D, 10000.0, torch.bfloat16)
    q, k = O.apply_rope(q, cos.double(), sin.double()), O.apply_rope(k, cos.double(), sin.double())
    return q, k, O.givens(v, theta, parity)


def test_c2_mote32m_layer_full_size_against_oracle(cuda):
    """BASELINE config C2 at its full size: the seed-1 byte mask gives chunk counts [622, 657, 604,
    658] for B = 4, padded to 658; a Mote-32M layer (d_model 512, 8 heads, dh 64) in bf16 through
    mote::rope_givens -> relation_fwd -> relation_bwd -> rope_givens_bwd. Each sequence's real rows
    against the float64 oracle on that sequence alone (pad rows get no upstream gradient, as a
    masked loss gives them): Y, g, d(qkv) within 2e-2; d(theta) within 2e-2 of its scale; dlam
    against the sum of |terms|."""
    from mote_amd.relation import FullRelation

    g = torch.Generator().manual_seed(1)
    mask = torch.rand(4, 2048, generator=g) < (1.0 / 3.3)
    mask[:, 0] = True
    M = mask.sum(-1).tolist()
    assert M == [622, 657, 604, 658]
    T, H, D, Dm = max(M), 8, 64, 512
    print(f"case C2 full size M={M}", flush=True)
    torch.manual_seed(1)
    x = _rms(torch.randn(4, T, Dm))
    m = FullRelation(Dm, H, 0)
    with torch.no_grad():
        m.theta.uniform_(-0.3, 0.3)
        m.lam.fill_(0.4)
    w = torch.cat([m.w1.weight, m.w2.weight, m.wi.weight], 0).detach()
    qkv = (x @ w.t()).to(torch.bfloat16)
    dy = torch.randn(4, H, T, D, generator=g).to(torch.bfloat16)
    for b, mb in enumerate(M):
        dy[b, :, mb:] = 0
    ops = torch.ops.mote
    qd, thd, lamd, invd = qkv.cuda(), m.theta.detach().cuda(), m.lam.detach().cuda(), m.inv_freq.cuda()
    p1, p2, info = ops.rope_givens(qd, invd, thd, H, 0, 0)
    y, gg, ibar, lse = ops.relation_fwd(p1, p2, info, lamd, 2.0, 0)
    dp1, dp2, dinfo, dlam = ops.relation_bwd(p1, p2, info, ibar, lse, gg, dy.cuda(), 2.0, 0)
    dqkv, dth = ops.rope_givens_bwd(dp1, dp2, dinfo, qd, invd, thd, H, 0, 0)
    torch.cuda.synchronize()
    dth_ref = torch.zeros(H // 2, dtype=torch.float64)
    dlam_ref, dlam_scale = 0.0, 0.0
    for b, mb in enumerate(M):
        qr = qkv[b:b + 1, :mb].double().requires_grad_(True)
        tr = m.theta.detach().double().requires_grad_(True)
        lr = m.lam.detach().double().requires_grad_(True)
        q, k, v = _rotated_ref(qr, H, m.inv_freq, tr, 0)
        yr, gr = O.relation_reference(q, k, v, lr, 2.0, 0, dtype=torch.float64)
        (yr * dy[b:b + 1, :, :mb].double()).sum().backward()
        assert rel_err(y[b:b + 1, :, :mb], yr) < 2e-2, (b, rel_err(y[b:b + 1, :, :mb], yr))
        assert float((gg[b, :, :mb].cpu().double() - gr[0].detach()).abs().max()) < 2e-2
        assert rel_err(dqkv[b, :mb], qr.grad[0]) < 2e-2, (b, rel_err(dqkv[b, :mb], qr.grad[0]))
        dth_ref += tr.grad
        dlam_ref += float(lr.grad)
        terms = O.relation_dlam_terms(q.detach(), k.detach(), v.detach(), lr.detach(), dy[b:b + 1, :, :mb], 2.0, 0)
        dlam_scale += float(terms.abs().sum())
    assert rel_err(dth, dth_ref) < 2e-2, rel_err(dth, dth_ref)
    assert abs(float(dlam) - dlam_ref) / max(dlam_scale, 1e-3) < 2e-2


def test_bf16_tile_backward_at_c3_length_against_oracle(cuda):
    """The bf16 tile kernels (forward, key kernel, dQ kernel with the dU^T pair table of 78 query
    blocks) at the C3 length T = 4964 with 2 heads of dh 96 (seed 2), against the float64 oracle:
    Y, g and dP1 / dP2 / dI~ within 2e-2, dlam against the sum of |terms|."""
    from mote_amd.flash_relation import flash_relation

    T, H, D = 4964, 2, 96
    print(f"case bf16 tiles T={T} H={H} D={D}", flush=True)
    g = torch.Generator().manual_seed(2)
    p1, p2, info, dy = ((torch.randn(1, H, T, D, generator=g) * 0.9).to(torch.bfloat16) for _ in range(4))
    lam = torch.tensor(0.4)
    xs = [t.cuda().requires_grad_(True) for t in (p1, p2, info, lam)]
    y, gg = flash_relation(*xs, 2.0, 0)
    grads = torch.autograd.grad((y.float() * dy.cuda().float()).sum(), xs)
    torch.cuda.synchronize()
    yr, gr = O.relation_reference(p1, p2, info, lam, 2.0, 0, dtype=torch.float64)
    dr = O.relation_backward(p1, p2, info, lam.double(), dy, 2.0, 0)
    assert rel_err(y, yr) < 2e-2, rel_err(y, yr)
    assert float((gg.cpu().double() - gr).abs().max()) < 2e-2
    for name, a, b in zip(("dp1", "dp2", "dinfo"), grads[:3], dr[:3]):
        assert rel_err(a, b) < 2e-2, (name, rel_err(a, b))
    terms = O.relation_dlam_terms(p1, p2, info, lam, dy, 2.0, 0)
    assert abs(float(grads[3]) - float(dr[3])) / float(terms.abs().sum()) < 2e-2


def _option_pair(seed, **kw):
    from mote_amd.relation import FullRelation

    torch.manual_seed(seed)
    mine = FullRelation(192, 2, 1, device="cuda", dtype=torch.float32, **kw)
    with torch.no_grad():
        if mine.use_givens:
            mine.theta.uniform_(-0.3, 0.3)
        mine.lam.fill_(0.4)
        if mine.qk_norm:
            mine.p1_norm.weight.uniform_(0.5, 1.5)
            mine.p2_norm.weight.uniform_(0.5, 1.5)
    ref = O.FullRelationRef(192, 2, 1, dtype=torch.float32, **kw)
    missing, unexpected = ref.load_state_dict({k: v.detach().cpu() for k, v in mine.state_dict().items()}, strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    return mine, ref


OPTIONS = [dict(qk_norm=True), dict(out_gate=True), dict(rope=False), dict(givens=False),
           dict(qk_norm=True, out_gate=True, rope=False, givens=False)]


@pytest.mark.parametrize("kw", OPTIONS, ids=lambda kw: "+".join(kw))
def test_module_options_fp32(cuda, kw):
    """FullRelation's switches (relation.py:128-147, 204-215), fp32, outputs and every parameter's
    gradient against the oracle module within 1e-5."""
    print(f"case module options fp32 {kw}", flush=True)
    mine, ref = _option_pair(11, **kw)
    x = torch.randn(2, 150, 192, generator=torch.Generator().manual_seed(12))
    wgt = torch.randn(2, 150, 192, generator=torch.Generator().manual_seed(13))
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


@pytest.mark.parametrize("kw", OPTIONS, ids=lambda kw: "+".join(kw))
def test_module_options_bf16_autocast(cuda, kw):
    print(f"case module options autocast {kw}", flush=True)
    mine, ref = _option_pair(14, **kw)
    x = torch.randn(1, 300, 192, generator=torch.Generator().manual_seed(15))
    wgt = torch.randn(1, 300, 192, generator=torch.Generator().manual_seed(16))
    xd = x.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out, g = mine(xd, return_gates=True)
    (out.float() * wgt.cuda()).sum().backward()
    xr = x.clone().requires_grad_(True)
    outr, gr = ref(xr, return_gates=True)
    (outr * wgt).sum().backward()
    assert rel_err(out.float(), outr) < 2e-2, rel_err(out.float(), outr)
    assert float((g.cpu() - gr).abs().max()) < 2e-2
    assert rel_err(xd.grad, xr.grad) < 2e-2, rel_err(xd.grad, xr.grad)
    grads_r = dict(ref.named_parameters())
    for n, p in mine.named_parameters():
        if n in ("lam", "theta"):  # sums over every row with heavy cancellation: covered in fp32 above
            continue
        assert rel_err(p.grad, grads_r[n].grad) < 2e-2, (n, rel_err(p.grad, grads_r[n].grad))


def test_bf16_module_keeps_exact_rope_angles(cuda):
    """A module cast with .to(torch.bfloat16) at positions up to 4100 against the oracle module
    with the same (bf16-valued) weights: bf16 RoPE frequencies would be radians off there."""
    from mote_amd.relation import FullRelation

    print("case bf16 module angles", flush=True)
    torch.manual_seed(21)
    mine = FullRelation(192, 2, 0).to(torch.bfloat16).cuda()
    with torch.no_grad():
        mine.theta.uniform_(-0.3, 0.3)
    ref = O.FullRelationRef(192, 2, 0, dtype=torch.float64)
    ref.load_state_dict({k: v.detach().double().cpu() for k, v in mine.state_dict().items()})
    x = torch.randn(1, 4100, 192, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16)
    out = mine(x.cuda())
    outr = ref(x.double())
    assert mine.inv_freq.dtype == torch.float32
    assert rel_err(out[:, -64:].float(), outr[:, -64:]) < 2e-2, rel_err(out[:, -64:].float(), outr[:, -64:])


@pytest.mark.parametrize("layer_idx", [0, 1])
def test_rope_givens_kernel_rounds_like_the_reference(cuda, layer_idx):
    """In bf16 the RoPE / Givens kernel rounds each product and each sum to bf16, as the reference's
    eager ops do (p cos + rotate_half(p) sin, c a - s b): its rows equal the oracle's bf16 ops bit
    for bit (a handful of table entries may differ by one ulp of fp32 cos / sin at a bf16 rounding
    boundary; one rounding instead of three would differ in about a third of the elements), and
    FullRelation._givens on the device equals the kernel's I~ exactly."""
    from mote_amd.relation import FullRelation, rope_givens

    print(f"case rounding points layer={layer_idx}", flush=True)
    B, T, H, D = 2, 777, 8, 96
    g = torch.Generator().manual_seed(30 + layer_idx)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(torch.bfloat16)
    m = FullRelation(H * D, H, layer_idx, device="cuda")
    with torch.no_grad():
        m.theta.uniform_(-0.5, 0.5)
    p1, p2, info = rope_givens(qkv.cuda(), H, m.inv_freq, m.theta.detach(), layer_idx, 123)
    q, k, v = (qkv[..., i * H * D:(i + 1) * H * D].reshape(B, T, H, D).transpose(1, 2) for i in range(3))
    cos, sin = O.rope_tables(123, T, D, 10000.0, torch.bfloat16)
    for got, want in ((p1, O.apply_rope(q, cos, sin)), (p2, O.apply_rope(k, cos, sin)),
                      (info, O.givens(v, m.theta.detach().cpu(), layer_idx))):
        got = got.cpu()
        diff = (got.float() - want.float()).abs()
        ulp = want.float().abs() * 2.0 ** -7 + 1e-30
        assert bool((diff <= ulp).all())
        assert float((got != want).float().mean()) < 1e-4
    assert torch.equal(m._givens(v.cuda()).cpu(), info.cpu())


def _op_samples(dev):
    g = torch.Generator().manual_seed(40)
    B, H, T, D, S = 1, 2, 70, 64, 9
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).to(dev)
    p1, p2, info = mk(B, H, T, D), mk(B, H, S + T, D), mk(B, H, S + T, D)
    lam = torch.tensor(0.4, device=dev)
    y, gg, ibar, lse = torch.ops.mote.relation_fwd(p1, p2, info, lam, 2.0, S)
    qkv = mk(B, T, 3 * H * D)
    x = mk(B, T, H * D)
    w = (torch.randn(3 * H * D, H * D, generator=g) / (H * D) ** 0.5).to(torch.bfloat16).to(dev)
    inv = O.rope_inv_freq(D, 10000.0).to(dev)
    theta = torch.rand(H // 2, generator=g).to(dev)
    cu = torch.tensor([0, 30, 70], dtype=torch.int32, device=dev)
    pv = [mk(H, 70, D) for _ in range(3)]
    return {
        "relation_fwd": (p1, p2, info, lam, 2.0, S),
        "relation_bwd": (p1, p2, info, ibar, lse, gg, mk(B, H, T, D), 2.0, S),
        "rope_givens": (qkv, inv, theta, H, 1, 5),
        "qkv_rope": (x, w, inv, theta, H, 0, 3, True),
        "relation_fwd_varlen": (*pv, lam, cu, 40, 2.0),
    }


@pytest.mark.parametrize("name", ["relation_fwd", "relation_bwd", "rope_givens", "qkv_rope", "relation_fwd_varlen"])
def test_custom_ops_pass_opcheck(cuda, name):
    """torch.library.opcheck: schema, fake kernel (shapes, dtypes and strides of the real outputs),
    autograd registration and AOT dispatch agree with the real op."""
    import mote_amd.relation  # noqa: F401  (registers the prologue ops)

    print(f"case opcheck {name}", flush=True)
    args = _op_samples(cuda)[name]
    grad_args = []
    for a in args:
        if torch.is_tensor(a) and a.is_floating_point() and name in ("relation_fwd", "rope_givens", "qkv_rope"):
            a = a.detach().requires_grad_(True)
        grad_args.append(a)
    torch.library.opcheck(getattr(torch.ops.mote, name).default, tuple(grad_args))


@pytest.mark.parametrize("autocast", [False, True])
def test_torch_compile_fullgraph_matches_eager(cuda, autocast):
    """FullRelation under torch.compile(fullgraph=True, backend="aot_eager"): the custom ops trace
    without a graph break and the compiled forward and backward match eager, with the reference's
    tolerances (tests/test_relation_paths.py:51-78); under bf16 autocast (the fused prologue op)
    within 1e-2 of each tensor's scale."""
    from mote_amd.relation import FullRelation

    print(f"case torch.compile fullgraph autocast={autocast}", flush=True)
    torch._dynamo.reset()
    torch.manual_seed(0)
    mod = FullRelation(128, 2, layer_idx=1, device="cuda", dtype=torch.float32)
    with torch.no_grad():
        mod.theta.uniform_(-0.3, 0.3)
    x = torch.randn(2, 48, 128, device="cuda") * 0.8
    res = []
    for fn in (mod, torch.compile(mod, fullgraph=True, backend="aot_eager")):
        mod.zero_grad()
        xi = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            y = fn(xi)
        y.float().sum().backward()
        res.append((y.detach().float(), xi.grad.clone(), {n: p.grad.clone() for n, p in mod.named_parameters()}))
    (ye, dxe, ge), (yc, dxc, gc) = res
    if autocast:
        assert rel_err(yc, ye) < 1e-2 and rel_err(dxc, dxe) < 1e-2
        for n in ge:
            assert rel_err(gc[n], ge[n]) < 1e-2, n
        return
    assert torch.allclose(ye, yc, atol=1e-4, rtol=1e-4), (ye - yc).abs().max()
    assert torch.allclose(dxe, dxc, atol=2e-4, rtol=1e-3), (dxe - dxc).abs().max()
    for n in ge:
        assert torch.allclose(ge[n], gc[n], atol=2e-4, rtol=1e-3), (n, (ge[n] - gc[n]).abs().max().item())
