"""The EMA dechunk's vector path (64-channel strips, rows on 16-byte boundaries) against its
two-channel path (the same values in rows off 16-byte boundaries) and the float64 oracle (oracle/dc.py,
restating dc.py:236-335).

The two paths compose the chunks' fp32 maps in different groupings, so they agree to rounding (2e-6 of
the largest magnitude in fp32, bf16 outputs within one rounding; the chunk sums of dout are the same
bits), and each is deterministic: repeated calls, calls that alternate shapes and replays of a captured
graph are compared bit for bit. Cases: rows without boundaries, bytes before the first boundary, every
byte a boundary, a single chunk, one segment, many groups (M above 4096), B > 1, a carried value, fp32
and bf16, widths 8 to 768 including last strips of 8 channels (the backward's vector path stops at 512).
"""

from __future__ import annotations

import pytest
import torch

from oracle import dc as O

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp(min=1e-3))


def _case(B, L, D, seed, dtype, rate=1 / 3.3, first=True, init=False):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, L, generator=g) < rate
    if first:
        m[:, 0] = True
    if B > 2:
        m[2] = False
    if B > 1 and L > 3:
        m[1, :3] = False
    num = m.sum(-1)
    M = max(int(num.max()), 1)
    h = torch.randn(B, M, D, generator=g).to(dtype)
    prob = torch.rand(B, L, 2, generator=g)
    prob[:, ::11, 1] = 1.0
    prob[:, 5::13, 1] = 0.0
    ini = torch.randn(B, D, generator=g) if init else None
    dy = torch.randn(B, L, D, generator=g).to(dtype)
    return m, h, prob, ini, dy


def _dev(t, dev, offset):
    """t on the device, in rows of D + 2 elements when offset (off 16-byte boundaries: the two-channel
    path), else contiguous (the vector path)."""
    if not offset:
        return t.to(dev)
    buf = torch.zeros(*t.shape[:-1], t.shape[-1] + 2, device=dev, dtype=t.dtype)
    buf[..., : t.shape[-1]] = t.to(dev)
    return buf[..., : t.shape[-1]]


def _run(dev, m, h, prob, ini, dy, vector, backward=True):
    from mote_amd import dc

    mask = m.to(dev)
    cum, perm, num, _ = dc.chunk_route(mask)
    hd, pd = _dev(h, dev, not vector), prob.to(dev)
    out, w = dc.dechunk(hd, pd, perm, num, mask, cum, 1e-4, ini.to(dev) if ini is not None else None)
    grads = None
    if backward and ini is None:
        grads = dc.dechunk_bwd(_dev(dy, dev, not vector), hd, pd, perm, num, mask, cum, w, 1e-4)
    torch.cuda.synchronize()
    return out, w, grads


CASES = [
    # B, L, D, rate, first, init
    (1, 1, 8, 0.3, True, False),          # one byte
    (1, 5, 64, 0.3, True, False),
    (3, 100, 64, 0.3, True, False),       # one segment; rows without boundaries / late first boundary
    (2, 700, 128, 1.0, True, False),      # every byte a boundary
    (2, 700, 128, 0.0, False, True),      # no boundary at all, carried value
    (1, 1500, 256, 1 / 3.3, True, False),
    (3, 1500, 384, 1 / 3.3, False, True),
    (1, 16384, 512, 1 / 3.3, True, False),  # the Mote-96M window
    (2, 20000, 512, 0.9, True, False),      # 288 segments, 72 groups: several waits per quarter
    (1, 3000, 768, 1 / 3.3, True, False),   # forward: twelve strips; backward: the two-channel path
    (2, 2000, 72, 1 / 3.3, True, False),    # a last strip of 8 channels
    (1, 2500, 200, 1 / 3.3, False, True),   # a last strip of 8 channels, carried value
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}L{c[1]}D{c[2]}r{c[3]:.2f}i{int(c[5])}" for c in CASES])
def test_vector_path_matches_two_channel_path_and_oracle(cuda, dtype, case):
    B, L, D, rate, first, init = case
    print(f"case dechunk vector path {dtype} B={B} L={L} D={D} rate={rate} init={init}", flush=True)
    m, h, prob, ini, dy = _case(B, L, D, 20 + L % 97, dtype, rate, first, init)
    if int(m.sum(-1).max()) == 0 and not init:
        pytest.skip("no chunk and no carried value")
    o1, w1, g1 = _run(cuda, m, h, prob, ini, dy, True)
    o2, w2, g2 = _run(cuda, m, h, prob, ini, dy, False)
    f32 = dtype == torch.float32
    assert _rel(o1, o2) < (2e-6 if f32 else 8e-3)
    for bb, nb in enumerate(m.sum(-1).tolist()):  # w is written for the row's chunks only
        if nb:
            assert _rel(w1[bb, :nb], w2[bb, :nb]) < (2e-6 if f32 else 8e-3)
    want = O.dechunk_brute(h.double(), m, prob.double(), 1e-4, ini.double() if ini is not None else None)
    assert _rel(o1, want) < (2e-5 if f32 else 2e-2)
    if g1 is not None:
        assert _rel(g1[0], g2[0]) < (2e-6 if f32 else 8e-3)
        assert _rel(g1[1], g2[1]) < (2e-5 if f32 else 2e-2)
        assert float(g1[1][..., 0].abs().max()) == 0.0


def test_vector_path_repeats_bit_for_bit_across_shapes(cuda):
    """Calls of alternating shapes and both directions: every repeat of a call returns the same bits."""
    a = _case(1, 16384, 512, 3, torch.bfloat16)
    b = _case(2, 5000, 256, 4, torch.float32)
    ra = _run(cuda, *a, True)
    rb = _run(cuda, *b, True)
    for _ in range(3):
        for ref, args in ((ra, a), (rb, b)):
            o, w, gr = _run(cuda, *args, True)
            n = int(args[0].sum(-1).min())
            assert torch.equal(o, ref[0]) and torch.equal(w[:, :n], ref[1][:, :n])
            assert torch.equal(gr[0], ref[2][0]) and torch.equal(gr[1], ref[2][1])


def test_vector_path_graph_replays(cuda):
    """A captured forward + backward replayed several times, with eager calls of another shape on the
    same stream between the replays: every replay equals the eager result."""
    from mote_amd import dc

    m, h, prob, _, dy = _case(1, 8192, 512, 5, torch.bfloat16)
    m2, h2, prob2, _, dy2 = _case(1, 3000, 512, 6, torch.bfloat16)
    mask, hd, pd, gd = m.to(cuda), h.to(cuda), prob.to(cuda), dy.to(cuda)
    cum, perm, num, _ = dc.chunk_route(mask)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ref_o, ref_w = dc.dechunk(hd, pd, perm, num, mask, cum, 1e-4, None)
        ref_g = dc.dechunk_bwd(gd, hd, pd, perm, num, mask, cum, ref_w, 1e-4)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            o, w = dc.dechunk(hd, pd, perm, num, mask, cum, 1e-4, None)
            gh, gp = dc.dechunk_bwd(gd, hd, pd, perm, num, mask, cum, w, 1e-4)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for _ in range(4):
        with torch.cuda.stream(side):
            graph.replay()
            _run(cuda, m2, h2, prob2, None, dy2, True)  # another shape on the same stream in between
        torch.cuda.synchronize()
        n = int(m.sum())
        assert torch.equal(o, ref_o) and torch.equal(w[:, :n], ref_w[:, :n])
        assert torch.equal(gh, ref_g[0]) and torch.equal(gp, ref_g[1])
