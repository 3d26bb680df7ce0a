"""CPU pins of the chunk / dechunk oracle (oracle/dc.py) and the host logic of mote_amd.dc.

The closed-form EMA is held to the plain recurrence and to the block loop it replaced, with the cases
of the reference's tests/test_dechunk_static.py and tests/test_mote_model.py:75-92; routing, gather
and the expansion to bytes to brute-force loops; gradients to finite differences. Each planted
mistake must fail one of them.
"""

from __future__ import annotations

import pytest
import torch

from oracle import dc as O


@torch.no_grad()
@pytest.mark.parametrize("M,C,with_init", [(300, 64, False), (300, 64, True), (64, 64, True), (5, 64, False),
                                           (257, 32, True)])
def test_ema_closed_form_matches_loop_and_sequential(M, C, with_init):
    # tests/test_dechunk_static.py:50-61 of the reference
    torch.manual_seed(0)
    x = torch.randn(2, M, 8, dtype=torch.float64)
    p = torch.rand(2, M, dtype=torch.float64).clamp(1e-4, 1 - 1e-4)
    init = torch.randn(2, 8, dtype=torch.float64) if with_init else None
    a = O.ema_chunked_ref(x, p, C=C, init=init)
    assert torch.allclose(a, O.ema_block_loop_ref(x, p, C=C, init=init), atol=1e-10, rtol=1e-10)
    assert torch.allclose(a, O.ema_sequential_ref(x, p, init=init), atol=1e-9, rtol=1e-9)


def test_ema_gradients_match_loop():
    # tests/test_dechunk_static.py:64-77 of the reference
    torch.manual_seed(1)
    x = torch.randn(2, 200, 8, dtype=torch.float64)
    p = torch.rand(2, 200, dtype=torch.float64).clamp(1e-4, 1 - 1e-4)
    init = torch.randn(2, 8, dtype=torch.float64)
    dy = torch.randn(2, 200, 8, dtype=torch.float64)
    grads = []
    for fn in (O.ema_chunked_ref, O.ema_block_loop_ref):
        xa, pa, ia = x.clone().requires_grad_(True), p.clone().requires_grad_(True), init.clone().requires_grad_(True)
        (fn(xa, pa, C=64, init=ia) * dy).sum().backward()
        grads.append((xa.grad, pa.grad, ia.grad))
    for a, b in zip(*grads):
        assert torch.allclose(a, b, atol=1e-9, rtol=1e-9)


def test_ema_constant_p_closed_form():
    # x = 1, p = c, z_-1 = 0: z_t = 1 - (1 - c)^(t + 1)
    c, M = 0.3, 150
    x = torch.ones(1, M, 1, dtype=torch.float64)
    p = torch.full((1, M), c, dtype=torch.float64)
    t = torch.arange(M, dtype=torch.float64)
    assert torch.allclose(O.ema_chunked_ref(x, p)[0, :, 0], 1 - (1 - c) ** (t + 1), atol=1e-12)


@pytest.mark.parametrize("plant", ["p_prev", "s_incl_minus"])
def test_ema_plants_fail(plant):
    torch.manual_seed(2)
    x = torch.randn(1, 300, 4, dtype=torch.float64)
    p = torch.rand(1, 300, dtype=torch.float64).clamp(1e-4, 1 - 1e-4)
    if plant == "s_incl_minus":
        # a rounding-level slip: the pin is causality bit for bit (tests/test_prefix_invariance.py of the
        # reference). Changing p of the last chunk (row 299, block 256..319) must leave rows 256..298 alone.
        got = O.ema_chunked_ref(x.float(), p.float(), _plant=plant)
        want = O.ema_chunked_ref(x.float(), p.float())
        p2 = p.clone()
        p2[:, -1] = 0.9
        bad = O.ema_chunked_ref(x.float(), p2.float(), _plant=plant)
        good = O.ema_chunked_ref(x.float(), p2.float())
        assert torch.equal(good[:, 256:299], want[:, 256:299])
        assert not torch.equal(bad[:, 256:299], got[:, 256:299])
        return
    got = O.ema_chunked_ref(x, p, _plant=plant)
    assert not torch.allclose(got, O.ema_sequential_ref(x, p), atol=1e-6)


def _mask(B, L, seed, rate=1 / 3.3, first=True):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, L, generator=g) < rate
    if first:
        m[:, 0] = True
    return m


def test_route_brute():
    m = _mask(3, 97, 0, first=False)
    m[1] = False
    m[2] = True
    cum, perm, num = O.route_ref(m)
    for b in range(3):
        bp = [t for t in range(97) if m[b, t]]
        other = [t for t in range(97) if not m[b, t]]
        assert perm[b].tolist() == bp + other
        assert num[b] == len(bp)
        assert cum[b].tolist() == [sum(int(v) for v in m[b, : t + 1]) for t in range(97)]


@pytest.mark.parametrize("bucket,exact", [(1, False), (16, False), (16, True)])
def test_chunk_layer_brute(bucket, exact):
    m = _mask(2, 60, 1)
    h = torch.randn(2, 60, 4, dtype=torch.float64)
    out, nm = O.chunk_layer_ref(h, m, bucket, exact)
    num = m.sum(-1)
    M = int(num.max())
    if bucket > 1 and not exact:
        M = min(60, -(-M // bucket) * bucket)
    assert out.shape == (2, M, 4)
    for b in range(2):
        order = [t for t in range(60) if m[b, t]] + [t for t in range(60) if not m[b, t]]
        for i in range(M):
            assert torch.equal(out[b, i], h[b, order[i]])
        assert nm[b].tolist() == [i < int(num[b]) for i in range(M)]


@pytest.mark.parametrize("with_init", [False, True])
def test_dechunk_matches_brute(with_init):
    torch.manual_seed(3)
    B, L, D = 3, 120, 6
    m = _mask(B, L, 3, first=not with_init)
    m[2] = False                    # a row with no boundary
    m[1, 0] = False                 # bytes before the first boundary
    num = m.sum(-1)
    M = int(num.max()) + 5          # padded rows, as bucketing leaves them
    h = torch.randn(B, M, D, dtype=torch.float64)
    prob = torch.rand(B, L, 2, dtype=torch.float64)
    prob[0, 3, 1], prob[0, 5, 1] = 0.0, 1.0   # clamped ends
    init = torch.randn(B, D, dtype=torch.float64) if with_init else None
    got = O.dechunk_ref(h, m, prob, 1e-4, init)
    want = O.dechunk_brute(h, m, prob, 1e-4, init)
    assert torch.allclose(got, want, atol=1e-10)


@pytest.mark.parametrize("plant", ["plug_no_minus", "no_clamp"])
def test_dechunk_plants_fail(plant):
    torch.manual_seed(4)
    B, L, D = 2, 80, 4
    m = _mask(B, L, 4)
    M = int(m.sum(-1).max()) + 3
    h = torch.randn(B, M, D, dtype=torch.float64)
    prob = torch.rand(B, L, 2, dtype=torch.float64)
    prob[:, ::7, 1] = 1.0
    got = O.dechunk_ref(h, m, prob, 1e-2, None, _plant=plant)
    assert not torch.allclose(got, O.dechunk_brute(h, m, prob, 1e-2), atol=1e-6)


def test_dechunk_gradients_finite_differences():
    torch.manual_seed(5)
    B, L, D = 1, 24, 3
    m = _mask(B, L, 5)
    m[0, 1] = True
    M = int(m.sum())
    h = torch.randn(B, M, D, dtype=torch.float64, requires_grad=True)
    prob = torch.rand(B, L, 2, dtype=torch.float64)
    prob[0, 1, 1] = 0.0                                   # clamped: no gradient there
    prob.requires_grad_(True)
    dy = torch.randn(B, L, D, dtype=torch.float64)
    (O.dechunk_ref(h, m, prob, 1e-4) * dy).sum().backward()
    f = lambda hh, pp: float((O.dechunk_ref(hh, m, pp, 1e-4) * dy).sum())  # noqa: E731
    eps = 1e-6
    for idx in [(0, 0, 0), (0, M // 2, 1), (0, M - 1, 2)]:
        hp, hm = h.detach().clone(), h.detach().clone()
        hp[idx] += eps
        hm[idx] -= eps
        assert abs((f(hp, prob.detach()) - f(hm, prob.detach())) / (2 * eps) - float(h.grad[idx])) < 1e-7
    # p passes through .float() (dc.py:319), so its steps are taken at 1e-4 and held to 1e-3 relative
    bpos = [t for t in range(L) if m[0, t] and t != 1]
    hp_ = 1e-4
    for t in bpos[:4] + [1]:
        pp, pm = prob.detach().clone(), prob.detach().clone()
        pp[0, t, 1] += hp_
        pm[0, t, 1] -= hp_
        fd = (f(h.detach(), pp) - f(h.detach(), pm)) / (2 * hp_)
        if t == 1:
            assert float(prob.grad[0, t, 1]) == 0.0
        else:
            assert abs(float(prob.grad[0, t, 1]) - fd) < 1e-3 * max(1.0, abs(fd))
    assert float(prob.grad[..., 0].abs().max()) == 0.0


def test_dechunk_step_rounding_order():
    # bf16 state: every eager op rounds to bf16 (p * cur, 1 - p, (1 - p) * last, the sum)
    g = torch.Generator().manual_seed(6)
    B, D = 5, 16
    mask = torch.tensor([True, False, True, True, False])
    prob = torch.rand(B, 2, generator=g)
    prob[3, 1] = 1.0
    hidden = torch.randn(3, 1, D, generator=g)
    last = torch.randn(B, D, generator=g).bfloat16()
    want = last.clone()
    res = O.dechunk_step_ref(hidden, mask, prob, want, 1e-4)
    r = 0
    for b in range(B):
        for d in range(D):
            if mask[b]:
                p = torch.tensor(min(max(float(prob[b, 1]), 1e-4), 1 - 1e-4)).bfloat16()
                cur = hidden[r, 0, d].bfloat16()
            else:
                p, cur = torch.tensor(0.0).bfloat16(), torch.tensor(0.0).bfloat16()
            v = (p * cur) + ((1 - p) * last[b, d])
            assert torch.equal(v, res[b, 0, d]), (b, d)
        r += int(mask[b])


def test_dc_module_signatures_and_cpu_error():
    from mote_amd.dc import ChunkLayer, DeChunkLayer

    cl = ChunkLayer(bucket=64)
    assert cl.bucket == 64 and ChunkLayer(0).bucket == 1
    dl = DeChunkLayer(512, prob_clamp=1e-3)
    assert (dl.d_model, dl.headdim, dl.block_size, dl.eps, dl.nheads) == (512, 32, 256, 1e-3, 16)
    st = dl.allocate_inference_cache(2, "cpu", torch.float32)
    assert st.last_value.shape == (2, 512)
    with pytest.raises(RuntimeError, match="HIP"):
        cl(torch.randn(1, 8, 16), torch.ones(1, 8, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="HIP"):
        dl(torch.randn(1, 8, 512), torch.ones(1, 8, dtype=torch.bool), torch.rand(1, 8, 2))
