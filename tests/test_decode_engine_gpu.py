"""The decode-engine pieces on the GPU: prefix-store pages moved by the HIP DMA path, and the graph
decoder's Relation step (RelationMainStep, the drop-in for mote/infer/graph.py:151-187) captured once
as a HIP graph with the boundary bit as a device predicate (in place of graph.py:44-57's conditional
node), replayed over a run of bits against eager steps."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_arena_growth_allocates_inside_the_serving_pool(cuda):
    """engine.py:327 hands the arena its MemPool; growth (arena.py:101) allocates the new store there."""
    from mote_amd.arena import RelationArena

    print("case arena pool growth", flush=True)
    arena = RelationArena(2, 4, 256, 64, "cuda", torch.bfloat16, batch=2)
    arena.store[:, :, 1, :, :10] = 3.0
    pool = torch.cuda.MemPool()
    arena.pool = pool
    assert arena.ensure(300) and arena.capacity == 512
    ptr = arena.store.data_ptr()
    segs = pool.snapshot()
    assert any(s["address"] <= ptr < s["address"] + s["total_size"] for s in segs)
    assert bool((arena.store[:, :, 1, :, :10] == 3.0).all())  # the other slot's rows travelled
    assert float(arena.store[:, :, :, :, 256:].float().abs().sum()) == 0.0
    torch.cuda.synchronize()


@pytest.mark.parametrize("batch,dtype", [(1, torch.bfloat16), (3, torch.bfloat16), (1, torch.float32)])
def test_pages_round_trip_through_dma(cuda, batch, dtype):
    from mote_amd.arena import RelationArena
    from mote_amd.prefix import PAGE, ArenaPages, Branch

    print(f"case pages dma batch={batch} {dtype}", flush=True)
    g = torch.Generator().manual_seed(batch)
    src = RelationArena(12, 8, 1024, 96, "cuda", dtype, batch=batch)
    src.store.copy_(torch.randn(src.store.shape, generator=g).to(dtype))
    pages = ArenaPages()
    b = Branch()
    seq = batch - 1
    for c0, c1 in ((0, 100), (100, 600), (600, 700)):
        pages.store_rows(b, src, c0, c1, seq=seq)
    assert all(p.is_pinned() for p in b.pages) and [p.shape[3] for p in b.pages] == [PAGE, PAGE, 256]
    want = src.store[:, :, seq].cpu()
    got = torch.cat([p for p in b.pages], dim=3)[:, :, :, :700]
    assert torch.equal(got, want[:, :, :, :700])
    dst = RelationArena(12, 8, 256, 96, "cuda", dtype, batch=batch)
    pages.hydrate(b, 700, dst, seq=0)
    torch.cuda.synchronize()
    assert dst.capacity >= 700
    assert torch.equal(dst.store[:, :, 0, :, :700].cpu(), want[:, :, :, :700])
    assert float(dst.store[:, :, 0, :, 700:].abs().sum()) == 0.0
    child = pages.fork(b, 650)
    dst2 = RelationArena(12, 8, 1024, 96, "cuda", dtype, batch=batch)
    pages.hydrate(child, 650, dst2, seq=seq)
    torch.cuda.synchronize()
    assert torch.equal(dst2.store[:, :, seq, :, :650].cpu(), want[:, :, :, :650])


def _stack(n_layers, seed):
    from mote_amd.relation import FullRelation

    torch.manual_seed(seed)
    mods = []
    for li in range(n_layers):
        m = FullRelation(768, 8, li, device="cuda", dtype=torch.bfloat16)
        with torch.no_grad():
            m.theta.uniform_(-0.3, 0.3)
            m.lam.fill_(0.4)
        mods.append(m)
    return mods


def test_predicated_main_step_graph_matches_eager_steps(cuda):
    """Three Mote-96M Relation layers, bf16, batch 1, a 300-row cache: one captured graph of the
    RelationMainStep chain, replayed for bits 1, 0, 1, 1, 0, 0, 1 with a new chunk each time. Every
    replay equals the eager chain run only on the 1 bits: the layer outputs, the arena rows, S and
    the per-layer exchange mass, bit for bit; on a 0 bit nothing changes at all."""
    from mote_amd.arena import RelationArena
    from mote_amd.graph import RelationMainStep

    L, S0, cap = 3, 300, 512
    mods = _stack(L, 5)
    g = torch.Generator().manual_seed(6)
    init = (torch.randn(L, 2, 1, 8, cap, 96, generator=g) * 0.7).to(torch.bfloat16)
    init[..., S0:, :] = 0

    def fresh():
        a = RelationArena(L, 8, cap, 96, "cuda", torch.bfloat16)
        a.store.copy_(init)
        S = torch.tensor([S0], dtype=torch.int64, device="cuda")
        xm = torch.zeros(L, 1, device="cuda")
        return a, S, xm

    bits = [1, 0, 1, 1, 0, 0, 1]
    xs = [(torch.randn(1, 1, 768, generator=g)).to(torch.bfloat16).cuda() for _ in bits]

    # eager: the chain runs only on the 1 bits
    ae, Se, xme = fresh()
    eager = RelationMainStep(ae, Se, xme)
    ref = []
    out = torch.zeros(1, 1, 768, device="cuda", dtype=torch.bfloat16)
    for bit, x in zip(bits, xs):
        if bit:
            h = x
            for li, m in enumerate(mods):
                h = eager(m, h, None, None, li)
            out = h.clone()
        torch.cuda.synchronize()
        ref.append((out.clone(), ae.store.clone(), Se.clone(), xme.clone()))

    # one graph, predicated on a device flag
    ag, Sg, xmg = fresh()
    run = torch.zeros(1, dtype=torch.bool, device="cuda")
    x_in = torch.zeros(1, 1, 768, device="cuda", dtype=torch.bfloat16)
    step = RelationMainStep(ag, Sg, xmg, run=run)

    def chain():
        h = x_in
        for li, m in enumerate(mods):
            h = step(m, h, None, None, li)
        return h

    before = ag.store.clone()
    chain()  # warm-up with the flag at 0: allocates the persistent outputs, writes nothing
    torch.cuda.synchronize()
    assert torch.equal(ag.store, before) and int(Sg) == S0
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(gr, stream=side):
            h_out = chain()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for i, (bit, x) in enumerate(zip(bits, xs)):
        print(f"case predicated replay {i} bit={bit}", flush=True)
        x_in.copy_(x)
        run.fill_(bool(bit))
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        o, st, S, xm = ref[i]
        assert int(Sg) == int(S)
        assert torch.equal(ag.store, st), i
        assert torch.equal(xmg, xm), i
        if any(bits[: i + 1]):
            assert torch.equal(h_out, o), i
