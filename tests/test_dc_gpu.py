"""Parity of the chunk gather and EMA dechunk (mote_amd.dc, HIP) with the reference's dc.py:192-352,
restated in oracle/dc.py.

Integer work (routing, gather, its backward) is compared bit for bit; the EMA in fp32 against the
float64 oracle within 2e-5 of the largest magnitude (5e-5 for the backward, whose sums run over bytes
and chunks), bf16 within 2e-2; the decode step bit for bit. Cases: the Mote-96M shape (16384 bytes,
Bernoulli(1/3.3) boundaries, D0 = 512, bucket 64), rows without boundaries, bytes before the first
boundary, bucket padding, the carried decode state, strided inputs, byte-level causality.
"""

from __future__ import annotations

import pytest
import torch

from oracle import dc as O

pytestmark = pytest.mark.gpu


def _mask(B, L, seed, rate=1 / 3.3, first=True):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, L, generator=g) < rate
    if first:
        m[:, 0] = True
    return m


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-3))


@pytest.mark.parametrize("L", [1, 7, 1000, 8192, 8193, 16384, 20000])
def test_route_matches_oracle(cuda, L):
    from mote_amd.dc import chunk_route

    m = _mask(4, L, L, first=False)
    m[1] = False
    m[2] = True
    cum, perm, num, cu = chunk_route(m.to(cuda))
    cr, pr, nr = O.route_ref(m)
    assert torch.equal(cum.cpu().long(), cr) and torch.equal(perm.cpu().long(), pr)
    assert torch.equal(num.cpu().long(), nr)
    assert cu.cpu().tolist() == [0] + torch.cumsum(nr, 0).tolist()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bucket,exact", [(1, False), (64, False), (64, True)])
def test_chunk_layer_matches_oracle(cuda, dtype, bucket, exact):
    from mote_amd.dc import ChunkLayer

    B, L, D = 3, 3000, 512
    m = _mask(B, L, 1)
    m[2, 1:] = False                               # a row with one boundary
    hs = torch.randn(B, L, D + 64, generator=torch.Generator().manual_seed(2)).to(dtype)
    h = hs[..., :D]
    out_r, nm_r = O.chunk_layer_ref(h, m, bucket, exact)
    hg = hs.to(cuda)[..., :D].detach().requires_grad_(True)     # strided rows on the device
    assert hg.stride(1) == D + 64
    out, nm = ChunkLayer(bucket)(hg, m.to(cuda), exact=exact)
    assert out.shape == out_r.shape and torch.equal(out.cpu(), out_r)
    assert torch.equal(nm.cpu(), nm_r.cpu())
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(3)).to(dtype)
    out.backward(dout.to(cuda))
    hr = h.clone().requires_grad_(True)
    O.chunk_layer_ref(hr, m, bucket, exact)[0].backward(dout)
    assert torch.equal(hg.grad.cpu(), hr.grad)


def test_chunk_pack_layout(cuda):
    from mote_amd.dc import chunk_pack

    B, L, D = 4, 2048, 256
    m = _mask(B, L, 4)
    h = torch.randn(B, L, D, generator=torch.Generator().manual_seed(5)).bfloat16()
    packed, cu, mx = chunk_pack(h.to(cuda), m.to(cuda))
    num = m.sum(-1)
    assert cu.cpu().tolist() == [0] + torch.cumsum(num, 0).tolist() and mx == int(num.max())
    want = torch.cat([h[b][m[b]] for b in range(B)])
    assert torch.equal(packed.cpu(), want)


def _strided(h, dev, pad=32):
    """h on the device as the first D columns of wider rows (the zc_full[..., :D0] view, hnet.py:239)."""
    buf = torch.zeros(*h.shape[:-1], h.shape[-1] + pad, device=dev, dtype=h.dtype)
    buf[..., : h.shape[-1]] = h.to(dev)
    return buf[..., : h.shape[-1]]


def _dechunk_case(B, L, D, seed, dtype, with_init=False, pad=0):
    g = torch.Generator().manual_seed(seed)
    m = _mask(B, L, seed, first=not with_init)
    if B > 2:
        m[2] = False                               # no boundary in this row
    if B > 1:
        m[1, :3] = False                           # bytes before the first boundary
    num = m.sum(-1)
    M = max(int(num.max()), 1) + pad
    h = torch.randn(B, M, D, generator=g).to(dtype)
    prob = torch.rand(B, L, 2, generator=g)
    prob[:, ::11, 1] = 1.0                         # clamped from above
    prob[:, 5::13, 1] = 0.0                        # clamped from below
    init = torch.randn(B, D, generator=g) if with_init else None
    return m, h, prob, init


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_init", [False, True])
@pytest.mark.parametrize("pad", [32, 34])
def test_dechunk_forward_matches_oracle(cuda, dtype, with_init, pad):
    """Rows of D + 32 elements: the 16-byte vector path; D + 34 (rows off 16-byte boundaries): the
    two-channel path."""
    from mote_amd.dc import DeChunkLayer, DeChunkState

    D = 384
    print(f"case dechunk fwd {dtype} init={with_init} row pad={pad}", flush=True)
    m, h, prob, init = _dechunk_case(3, 1500, D, 6, dtype, with_init, pad=40)
    want = O.dechunk_brute(h.double(), m, prob.double(), 1e-4, init.double() if init is not None else None)
    layer = DeChunkLayer(D)
    st = DeChunkState(last_value=init.to(cuda).clone()) if with_init else None
    out = layer(_strided(h, cuda, pad), m.to(cuda), prob.to(cuda), st)
    assert out.dtype == dtype and out.shape == (3, 1500, D)
    tol = 2e-5 if dtype == torch.float32 else 2e-2
    assert _rel(out, want) < tol
    if with_init:
        assert torch.equal(st.last_value.cpu(), out[:, -1].cpu().float())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [256, 202])
def test_dechunk_backward_matches_autograd(cuda, dtype, D):
    """D = 256: the 16-byte vector path; D = 202 (not a multiple of 8, heads of 2): the two-channel path."""
    from mote_amd.dc import DeChunkLayer

    print(f"case dechunk bwd {dtype} D={D}", flush=True)
    m, h, prob, _ = _dechunk_case(3, 1500, D, 7, dtype, pad=40)
    dy = torch.randn(3, 1500, D, generator=torch.Generator().manual_seed(8)).to(dtype)
    hr = h.double().requires_grad_(True)
    prr = prob.double().requires_grad_(True)
    (O.dechunk_ref(hr, m, prr, 1e-4) * dy.double()).sum().backward()
    hg = _strided(h, cuda).detach().requires_grad_(True)
    pg = prob.to(cuda).requires_grad_(True)
    out = DeChunkLayer(D, headdim=32 if D % 32 == 0 else 2)(hg, m.to(cuda), pg)
    out.backward(dy.to(cuda))
    tol = 5e-5 if dtype == torch.float32 else 2e-2
    assert hg.grad.dtype == dtype and pg.grad.dtype == torch.float32
    assert _rel(hg.grad, hr.grad) < tol
    assert _rel(pg.grad, prr.grad) < tol
    assert float(pg.grad[..., 0].abs().max()) == 0.0


def test_dechunk_full_size_fwd_bwd(cuda):
    # the Mote-96M shape: 16384 bytes, ~4965 boundaries (seed 2), D0 = 512, bucket 64, fp32
    from mote_amd.dc import ChunkLayer, DeChunkLayer

    L, D = 16384, 512
    m = _mask(1, L, 2)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, L, D, generator=g)
    prob = torch.rand(1, L, 2, generator=g)
    dy = torch.randn(1, L, D, generator=g)
    xg = x.to(cuda).requires_grad_(True)
    pg = prob.to(cuda).requires_grad_(True)
    hc, _ = ChunkLayer(64)(xg, m.to(cuda))
    out = DeChunkLayer(D)(hc, m.to(cuda), pg)
    out.backward(dy.to(cuda))
    xr = x.double().requires_grad_(True)
    prr = prob.double().requires_grad_(True)
    hr, _ = O.chunk_layer_ref(xr, m, 64)
    (O.dechunk_ref(hr, m, prr, 1e-4) * dy.double()).sum().backward()
    assert hc.shape[1] % 64 == 0
    want = O.dechunk_ref(hr.detach(), m, prob.double(), 1e-4)
    assert _rel(out, want) < 2e-5
    assert _rel(xg.grad, xr.grad) < 5e-5
    assert _rel(pg.grad, prr.grad) < 5e-5


def test_dechunk_causal_bit_for_bit(cuda):
    # changing bytes after t (boundaries and probabilities) leaves every output at or before t unchanged
    from mote_amd.dc import ChunkLayer, DeChunkLayer

    L, D, t = 6000, 256, 3700
    m = _mask(1, L, 10)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, L, D, generator=g)
    prob = torch.rand(1, L, 2, generator=g)
    m2, p2 = m.clone(), prob.clone()
    m2[0, t + 1:] = torch.rand(L - t - 1, generator=g) < 0.9
    p2[0, t + 1:] = torch.rand(L - t - 1, 2, generator=g)

    def run(mm, pp):
        hc, _ = ChunkLayer(64)(x.to(cuda), mm.to(cuda))
        return DeChunkLayer(D)(hc, mm.to(cuda), pp.to(cuda))

    a, b = run(m, prob), run(m2, p2)
    assert torch.equal(a[:, : t + 1], b[:, : t + 1])


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_dechunk_step_bit_exact(cuda, state_dtype):
    from mote_amd.dc import DeChunkLayer, DeChunkState

    g = torch.Generator().manual_seed(12)
    B, D = 7, 320
    mask = torch.tensor([True, False, True, True, False, False, True])
    prob = torch.rand(B, 2, generator=g)
    prob[2, 1] = 1.0
    hidden = torch.randn(int(mask.sum()), 1, D, generator=g).bfloat16()
    last = torch.randn(B, D, generator=g).to(state_dtype)
    want_last = last.clone()
    want = O.dechunk_step_ref(hidden, mask, prob, want_last, 1e-4)
    st = DeChunkState(last_value=last.to(cuda))
    got = DeChunkLayer(D).step(hidden.to(cuda), mask.to(cuda), prob.to(cuda), st)
    assert torch.equal(got.cpu(), want) and torch.equal(st.last_value.cpu(), want_last)
    # no boundary in the batch: the state is carried unchanged
    mask0 = torch.zeros(B, dtype=torch.bool)
    got0 = DeChunkLayer(D).step(hidden[:0].to(cuda), mask0.to(cuda), prob.to(cuda), st)
    assert torch.equal(got0[:, 0].cpu(), want_last)


def test_dechunk_prefill_then_steps_match_one_pass(cuda):
    # a prefill with a carried state, then decode steps, equals the forward over the whole row
    from mote_amd.dc import ChunkLayer, DeChunkLayer, DeChunkState

    L, D, L0 = 400, 128, 300
    m = _mask(1, L, 13)
    g = torch.Generator().manual_seed(14)
    x = torch.randn(1, L, D, generator=g)
    prob = torch.rand(1, L, 2, generator=g)
    layer = DeChunkLayer(D)
    hc, _ = ChunkLayer()(x.to(cuda), m.to(cuda), exact=True)
    full = layer(hc, m.to(cuda), prob.to(cuda))
    st = DeChunkState(last_value=torch.zeros(1, D, device=cuda))
    hc0, _ = ChunkLayer()(x[:, :L0].to(cuda), m[:, :L0].to(cuda), exact=True)
    part = layer(hc0, m[:, :L0].to(cuda), prob[:, :L0].to(cuda), st)
    outs = [part]
    for t in range(L0, L):
        mk = m[:, t].to(cuda)
        h = x[:, t:t + 1].to(cuda)[mk]
        outs.append(layer.step(h, mk, prob[:, t].to(cuda), st))
    got = torch.cat(outs, 1)
    assert _rel(got, full) < 2e-5


def test_errors(cuda):
    from mote_amd.dc import DeChunkLayer, chunk_route

    with pytest.raises(RuntimeError, match="no chunk rows"):
        DeChunkLayer(64)(torch.zeros(1, 0, 64, device=cuda), torch.zeros(1, 8, dtype=torch.bool, device=cuda),
                         torch.rand(1, 8, 2, device=cuda))
    cum, perm, num, cu = chunk_route(torch.zeros(0, 5, dtype=torch.bool, device=cuda))
    assert cum.shape == (0, 5) and cu.cpu().tolist() == [0]
