"""The decode step (one HIP launch per layer) against the CPU oracle: the core, the append, the
device-side position advance, batch 16, edge positions, and replay inside a HIP graph."""

from __future__ import annotations

import pytest
import torch

from conftest import rel_err
from oracle import relation as O

pytestmark = pytest.mark.gpu


def _setup(B, H, D, cap, S, dtype, seed=0, theta=True, rope=True):
    g = torch.Generator().manual_seed(seed)
    kc = (torch.randn(B, H, cap, D, generator=g) * 0.7).to(dtype)
    vc = (torch.randn(B, H, cap, D, generator=g) * 0.7).to(dtype)
    raw = [(torch.randn(B, H, D, generator=g) * 0.7).to(dtype) for _ in range(3)]
    th = (torch.rand(H // 2, generator=g) * 0.6 - 0.3) if theta else None
    inv = O.rope_inv_freq(D, 10000.0) if rope else None
    Sv = torch.tensor(S, dtype=torch.int64)
    return kc, vc, raw, th, inv, Sv


def _oracle(kc, vc, raw, th, inv, Sv, layer_idx, lam, dtype):
    q, k, v = O.decode_rows_ref(*raw, Sv, inv, th, layer_idx, dtype)
    kc2, vc2 = kc.clone(), vc.clone()
    for b in range(kc.shape[0]):
        kc2[b, :, int(Sv[b])] = k[b]
        vc2[b, :, int(Sv[b])] = v[b]
    y, gg = O.relation_decode_ref(q, kc2, vc2, Sv, torch.tensor(lam), 2.0, dtype=torch.float64)
    return y, gg, kc2, vc2


def _check_append(kd, vd, kc2, vc2, dtype):
    if dtype == torch.bfloat16:
        assert torch.equal(kd.cpu(), kc2) and torch.equal(vd.cpu(), vc2)
    else:
        assert rel_err(kd, kc2) < 1e-5 and rel_err(vd, vc2) < 1e-5


def _run(kc, vc, raw, th, inv, Sv, layer_idx, lam, advance=False):
    from mote_amd.decode import relation_decode

    kd, vd = kc.cuda(), vc.cuda()
    Sd = Sv.cuda()
    y, gg = relation_decode(*(t.cuda() for t in raw), Sd, kd, vd, torch.tensor(lam, device="cuda"), 2.0,
                            None if inv is None else inv.cuda(), None if th is None else th.cuda(), layer_idx,
                            advance=advance)
    torch.cuda.synchronize()
    return y, gg, kd, vd, Sd


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("S", [1, 37, 700, 4096])
@pytest.mark.parametrize("layer_idx", [0, 1])
def test_decode_batch1_matches_oracle(cuda, dtype, tol, S, layer_idx):
    print(f"case decode b1 {dtype} S={S} layer={layer_idx}", flush=True)
    kc, vc, raw, th, inv, Sv = _setup(1, 8, 96, 4352, [S], dtype, seed=S)
    y, gg, kd, vd, _ = _run(kc, vc, raw, th, inv, Sv, layer_idx, 0.4)
    yr, gr, kc2, vc2 = _oracle(kc, vc, raw, th, inv, Sv, layer_idx, 0.4, dtype)
    assert rel_err(y, yr) < tol, rel_err(y, yr)
    assert float((gg.cpu().double() - gr).abs().max()) < tol
    # the append wrote row S and nothing else: bit-exact in bf16 (one rounding of the same value);
    # in fp32 the kernel's single-precision rotation is within the fp32 bar of the float64 one
    _check_append(kd, vd, kc2, vc2, dtype)


def test_decode_batch16_mixed_positions(cuda):
    S = [4096, 1, 17, 2049, 300, 4351, 64, 65, 1000, 3000, 5, 4095, 128, 129, 2500, 4000]
    kc, vc, raw, th, inv, Sv = _setup(16, 8, 96, 4352, S, torch.bfloat16, seed=3)
    y, gg, kd, vd, _ = _run(kc, vc, raw, th, inv, Sv, 1, 0.5)
    yr, gr, kc2, vc2 = _oracle(kc, vc, raw, th, inv, Sv, 1, 0.5, torch.bfloat16)
    assert rel_err(y, yr) < 2e-2
    assert float((gg.cpu().double() - gr).abs().max()) < 2e-2
    assert torch.equal(kd.cpu(), kc2) and torch.equal(vd.cpu(), vc2)


@pytest.mark.parametrize("layer_idx", [0, 1])
def test_decode_rope_f32_convention(cuda, layer_idx):
    """MOTE_DECODE_ROPE_F32 (the graph decoder with fp32 x under serving autocast, graph.py:158-172):
    the appended rows against decode_rows_ref with fp32 tables and one rounding: bit for bit except
    where the kernel's fp32 sincos and the host's differ across a rounding tie (at most 0.5 % of the
    elements, never more than one bf16 ulp); y and g within 2e-2 of the oracle step on those rows."""
    from mote_amd.decode import relation_decode

    print(f"case decode rope_f32 layer={layer_idx}", flush=True)
    S = [4096, 3, 777, 4351]
    kc, vc, raw, th, inv, Sv = _setup(4, 8, 96, 4352, S, torch.bfloat16, seed=41 + layer_idx)
    kd, vd, Sd = kc.cuda(), vc.cuda(), Sv.cuda()
    y, gg = relation_decode(*(t.cuda() for t in raw), Sd, kd, vd, torch.tensor(0.4, device="cuda"), 2.0, inv.cuda(),
                            th.cuda(), layer_idx, rope_f32=True)
    torch.cuda.synchronize()
    q, k, v = O.decode_rows_ref(*raw, Sv, inv, th, layer_idx, torch.bfloat16, rope_dtype=torch.float32)
    kc2, vc2 = kc.clone(), vc.clone()
    for b in range(4):
        kc2[b, :, S[b]] = k[b]
        vc2[b, :, S[b]] = v[b]
    assert torch.equal(vd.cpu(), vc2)  # Givens: the same convention either way
    kg = kd.cpu()
    assert torch.equal(kg[:, :, :4096][:, :, [s for s in range(4096) if s not in S]],
                       kc[:, :, [s for s in range(4096) if s not in S]])
    rows_got = torch.stack([kg[b, :, S[b]] for b in range(4)]).double()
    rows_want = k.double()
    diff = (rows_got - rows_want).abs()
    ulp = (rows_want.abs().clamp(min=1e-30).log2().floor() - 7).exp2()
    assert bool((diff <= ulp * 1.0001).all()) and float((diff == 0).double().mean()) >= 0.995
    yr, gr = O.relation_decode_ref(q, kc2, vc2, Sv, torch.tensor(0.4), 2.0, dtype=torch.float64)
    assert rel_err(y, yr) < 2e-2 and float((gg.cpu().double() - gr).abs().max()) < 2e-2


def test_decode_position_zero_is_pure_self(cuda):
    kc, vc, raw, th, inv, Sv = _setup(2, 4, 64, 512, [0, 0], torch.float32)
    y, gg, kd, vd, _ = _run(kc, vc, raw, th, inv, Sv, 0, 0.5)
    q, k, v = O.decode_rows_ref(*raw, Sv, inv, th, 0, torch.float32)
    assert torch.allclose(y.cpu(), v, atol=1e-6)
    assert float(gg.abs().max()) == 0.0


def test_decode_advance_and_no_rope_no_givens(cuda):
    kc, vc, raw, th, inv, Sv = _setup(2, 4, 48, 256, [10, 200], torch.float32, theta=False, rope=False)
    y, gg, kd, vd, Sd = _run(kc, vc, raw, th, inv, Sv, 0, 0.3, advance=True)
    yr, gr, _, _ = _oracle(kc, vc, raw, th, inv, Sv, 0, 0.3, torch.float32)
    assert rel_err(y, yr) < 1e-5
    assert Sd.cpu().tolist() == [11, 201]


def test_decode_out_of_range_position_is_flagged(cuda):
    kc, vc, raw, th, inv, Sv = _setup(2, 4, 64, 128, [5, 128], torch.float32)
    y, gg, kd, vd, _ = _run(kc, vc, raw, th, inv, Sv, 0, 0.5)
    assert torch.isnan(y[1]).all() and torch.isnan(gg[1]).all()
    assert torch.isfinite(y[0]).all()
    assert torch.equal(kd[1].cpu(), kc[1])  # nothing appended for the bad sequence


def test_decode_replays_in_a_hip_graph(cuda):
    """A captured step with the device-side advance, replayed with eager work in between, equals
    the same steps run eagerly (every replay checked)."""
    from mote_amd.decode import decode_workspace, relation_decode

    B, H, D, cap = 2, 8, 96, 1024
    kc, vc, raw, th, inv, Sv = _setup(B, H, D, cap, [300, 301], torch.bfloat16, seed=9)
    steps = 5
    g = torch.Generator().manual_seed(10)
    xs = [[(torch.randn(B, H, D, generator=g) * 0.7).to(torch.bfloat16) for _ in range(3)] for _ in range(steps)]
    # eager
    ke, ve, Se = kc.cuda(), vc.cuda(), Sv.cuda()
    lam = torch.tensor(0.4, device="cuda")
    eager = []
    for s in range(steps):
        y, gg = relation_decode(*(t.cuda() for t in xs[s]), Se, ke, ve, lam, 2.0, inv.cuda(), th.cuda(), 1, advance=True)
        eager.append((y.clone(), gg.clone()))
    # graph
    kg, vg, Sg = kc.cuda(), vc.cuda(), Sv.cuda()
    ins = [torch.empty(B, H, D, device="cuda", dtype=torch.bfloat16) for _ in range(3)]
    ws = decode_workspace(B, H, D, cap, "cuda", torch.bfloat16)
    yb = torch.empty(B, H, D, device="cuda", dtype=torch.bfloat16)
    gb = torch.empty(B, H, device="cuda")
    invd, thd = inv.cuda(), th.cuda()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            relation_decode(*ins, Sg, kg, vg, lam, 2.0, invd, thd, 1, advance=True, workspace=ws, y=yb, g=gb)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for s in range(steps):
        for dst, src in zip(ins, xs[s]):
            dst.copy_(src.cuda())
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yb, eager[s][0]), s
        assert torch.equal(gb, eager[s][1]), s
        _ = (yb.float() * 2).sum()  # eager work between replays
    assert torch.equal(kg, ke) and torch.equal(vg, ve) and torch.equal(Sg, Se)


def test_decode_exchange_mass_mean_over_heads(cuda):
    """xm (graph.py:186): the kernel's last head of every sequence writes the mean of g over the heads
    (fixed head order); checked against the kernel's own g and the oracle's, over two calls in a row
    (the completion counts return to zero) with the position advancing."""
    from mote_amd.decode import decode_workspace, relation_decode

    print("case decode xm b16", flush=True)
    S = [4096, 1, 17, 2049, 300, 4351 - 1, 64, 65, 1000, 3000, 5, 4095, 128, 129, 2500, 4000]
    kc, vc, raw, th, inv, Sv = _setup(16, 8, 96, 4352, S, torch.bfloat16, seed=8)
    kd, vd, Sd = kc.cuda(), vc.cuda(), Sv.cuda()
    ws = decode_workspace(16, 8, 96, 4352, "cuda")
    xm = torch.full((16,), float("nan"), device="cuda")
    for call in range(2):
        y, gg = relation_decode(*(t.cuda() for t in raw), Sd, kd, vd, torch.tensor(0.5, device="cuda"), 2.0,
                                inv.cuda(), th.cuda(), 1, advance=True, workspace=ws, xm=xm)
        torch.cuda.synchronize()
        assert float((xm - gg.mean(-1)).abs().max()) < 1e-6, call
        if call == 0:
            _, gr, _, _ = _oracle(kc, vc, raw, th, inv, Sv, 1, 0.5, torch.bfloat16)
            assert float((xm.cpu().double() - gr.mean(-1)).abs().max()) < 2e-2
        assert torch.equal(Sd.cpu(), Sv + call + 1)


def test_decode_counts_across_mixed_calls(cuda):
    """Calls that neither advance S nor ask for xm skip the per-sequence count; interleaved with calls
    that do, on one workspace, every call still sees zeroed counters: S moves exactly on the advancing
    calls, xm equals the mean of that call's g, and y / g match the oracle at the position in hand."""
    from mote_amd.decode import decode_workspace, relation_decode

    print("case decode mixed counts b4", flush=True)
    S = [100, 4000, 1, 2049]
    kc, vc, raw, th, inv, Sv = _setup(4, 8, 96, 4352, S, torch.bfloat16, seed=11)
    kd, vd, Sd = kc.cuda(), vc.cuda(), Sv.cuda()
    ws = decode_workspace(4, 8, 96, 4352, "cuda")
    kref, vref, Sref = kc.clone(), vc.clone(), Sv.clone()
    for call, (adv, want_xm) in enumerate([(False, False), (True, False), (False, True), (False, False),
                                           (True, True), (False, False)]):
        xm = torch.full((4,), float("nan"), device="cuda") if want_xm else None
        y, gg = relation_decode(*(t.cuda() for t in raw), Sd, kd, vd, torch.tensor(0.4, device="cuda"), 2.0,
                                inv.cuda(), th.cuda(), 0, advance=adv, workspace=ws, xm=xm)
        torch.cuda.synchronize()
        yr, gr, kref, vref = _oracle(kref, vref, raw, th, inv, Sref, 0, 0.4, torch.bfloat16)
        assert rel_err(y, yr) < 2e-2 and float((gg.cpu().double() - gr).abs().max()) < 2e-2, call
        if want_xm:
            assert float((xm - gg.mean(-1)).abs().max()) < 1e-6, call
        Sref = Sref + int(adv)
        assert torch.equal(Sd.cpu(), Sref), call
    _check_append(kd, vd, kref, vref, torch.bfloat16)


@pytest.mark.parametrize("B,N,K,xpad", [(1, 2304, 768, 0), (16, 2304, 768, 0), (5, 768, 768, 64), (3, 48, 128, 0),
                                        (16, 64, 1024, 8)])
def test_skinny_linear_matches_float64(cuda, B, N, K, xpad):
    """The decode engine's skinny product against float64 x W^T rounded to bf16 (one rounding; the
    fp32 accumulation order may move a result by one bf16 step)."""
    from mote_amd.decode import skinny_linear

    print(f"case skinny B={B} N={N} K={K} xpad={xpad}", flush=True)
    g = torch.Generator().manual_seed(B * 7 + N + K)
    xs = torch.randn(B, K + xpad, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) / K ** 0.5).bfloat16()
    y = skinny_linear(xs.cuda()[:, :K], w.cuda())
    ref = (xs[:, :K].double() @ w.double().t())
    assert y.shape == (B, N) and y.dtype == torch.bfloat16
    assert rel_err(y, ref) < 1e-2, rel_err(y, ref)


def test_decode_step_skinny_path_matches_library_path(cuda):
    """RelationDecodeStep in bf16 at batch 16: the skinny-product projections give the same step
    (out, xm, the appended rows and the advanced position) as the hipBLASLt path."""
    import mote_amd.decode as Dm
    from mote_amd.arena import RelationArena
    from mote_amd.relation import FullRelation

    print("case decode step skinny vs library", flush=True)
    torch.manual_seed(13)
    m = FullRelation(768, 8, 1).cuda()
    with torch.no_grad():
        m.theta.uniform_(-0.3, 0.3)
    for lin in (m.w1, m.w2, m.wi, m.wo):
        lin.to(torch.bfloat16)
    outs = []
    for skinny in (True, False):
        arena = RelationArena(1, 8, 512, 96, "cuda", torch.bfloat16, batch=16)
        g = torch.Generator().manual_seed(14)
        arena.buf.copy_(torch.randn(arena.buf.shape, generator=g).bfloat16())
        step = Dm.RelationDecodeStep(m, arena, 0)
        S = torch.tensor([300 + 7 * b for b in range(16)], device="cuda")
        x = torch.randn(16, 1, 768, generator=g).bfloat16().cuda()
        orig = Dm._skinny_ok
        if not skinny:
            Dm._skinny_ok = lambda *a: False
        try:
            out, xm = step(x, S, advance=True)
        finally:
            Dm._skinny_ok = orig
        torch.cuda.synchronize()
        outs.append((out.clone(), xm.clone(), arena.buf.clone(), S.clone()))
    (o1, x1, b1, s1), (o2, x2, b2, s2) = outs
    assert rel_err(o1, o2) < 2e-2, rel_err(o1, o2)
    assert float((x1 - x2).abs().max()) < 2e-2
    assert rel_err(b1, b2) < 2e-2 and torch.equal(s1, s2)


def test_skinny_linear_writes_the_exchange_mass(cuda):
    """The skinny product's side job: xm[b] = mean of g[b] over the heads in head order, the same
    arithmetic as the decode launch's own xm; nothing written when the predicate is 0."""
    from mote_amd.decode import skinny_linear

    print("case skinny xm", flush=True)
    g0 = torch.Generator().manual_seed(3)
    x = torch.randn(5, 768, generator=g0).bfloat16().cuda()
    w = torch.randn(768, 768, generator=g0).bfloat16().cuda()
    g = torch.rand(5, 8, generator=g0).cuda()
    xm = torch.full((5,), float("nan"), device="cuda")
    y = skinny_linear(x, w, g=g, xm=xm)
    torch.cuda.synchronize()
    want = torch.zeros(5)
    for h in range(8):
        want = want + g.cpu()[:, h]
    assert torch.equal(xm.cpu(), want / 8.0)
    assert torch.equal(y, skinny_linear(x, w))
    run = torch.zeros(1, dtype=torch.uint8, device="cuda")
    xm2 = torch.full((5,), 7.0, device="cuda")
    skinny_linear(x, w, torch.empty_like(y), run, g=g, xm=xm2)
    torch.cuda.synchronize()
    assert bool((xm2 == 7.0).all())
    with pytest.raises(ValueError):
        skinny_linear(x, w, g=None, xm=xm)
