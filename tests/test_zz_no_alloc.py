"""The no-allocation decode entry point, mote_relation_decode_static, through the C ABI against
mote_relation_decode with a caller workspace: on calls in a row (the second with a smaller
batch, capacity and fill) the outputs y, g, xm, the appended cache rows and the advanced positions
are identical bit for bit (same kernel, same split count, deterministic merge order). A third call
goes back to a larger batch with another head dim: the shared array's counters stay valid. Two
slots driven from two unordered streams at once give each stream the workspace entry point's
results."""

from __future__ import annotations

import pytest
import torch

from oracle import relation as O

pytestmark = pytest.mark.gpu


def _inputs(B, H, D, cap, S, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return dict(
        kc=(torch.randn(B, H, cap, D, generator=g) * 0.7).to(dtype),
        vc=(torch.randn(B, H, cap, D, generator=g) * 0.7).to(dtype),
        raw=[(torch.randn(B, H, D, generator=g) * 0.7).to(dtype) for _ in range(3)],
        theta=torch.rand(H // 2, generator=g) * 0.6 - 0.3,
        inv=O.rope_inv_freq(D, 10000.0),
        S=torch.tensor(S, dtype=torch.int64),
        lam=torch.tensor(0.45),
    )


def _call(entry: str, inp, layer_parity: int, slot: int = 0):
    """One decode step through the named C entry point on fresh device copies of `inp` (the static
    entry point on scratch slot `slot`)."""
    from mote_amd import _lib as L

    dev = torch.device("cuda")
    kc, vc = inp["kc"].to(dev), inp["vc"].to(dev)
    raw = [t.to(dev) for t in inp["raw"]]
    S = inp["S"].to(dev)
    lam, inv, theta = inp["lam"].to(dev), inp["inv"].to(dev), inp["theta"].to(dev)
    B, H, cap, D = kc.shape
    y = torch.full((B, H, D), float("nan"), device=dev, dtype=kc.dtype)
    g = torch.full((B, H), float("nan"), device=dev)
    xm = torch.full((B,), float("nan"), device=dev)
    a = L.DecodeArgs()
    a.dtype = L.dtype_code(kc)
    a.B, a.H, a.D, a.capacity = B, H, D, cap
    a.layer_parity, a.flags, a.tau_s = layer_parity, L.MOTE_DECODE_ADVANCE, 2.0
    a.lam, a.inv_freq, a.theta, a.S = lam.data_ptr(), inv.data_ptr(), theta.data_ptr(), S.data_ptr()
    a.p1, a.p2, a.info, a.in_sb = raw[0].data_ptr(), raw[1].data_ptr(), raw[2].data_ptr(), raw[0].stride(0)
    a.cache_p2, a.cache_info = L.view(kc), L.view(vc)
    a.y, a.y_sb, a.g, a.xm = y.data_ptr(), y.stride(0), g.data_ptr(), xm.data_ptr()
    ws = None
    if entry == "mote_relation_decode":
        ws = torch.zeros(int(L.lib().mote_relation_decode_workspace(a)), device=dev, dtype=torch.uint8)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    else:
        a.workspace, a.workspace_bytes, a.static_slot = None, 0, slot
    L.check(getattr(L.lib(), entry)(a, L.stream_of(kc)), entry)
    torch.cuda.synchronize()
    return [t.cpu() for t in (y, g, xm, kc, vc, S)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_static_scratch_entry_point_matches_the_workspace_one(cuda, dtype):
    cases = [  # (B, H, D, capacity, positions, layer parity): the second call is smaller
        (16, 8, 96, 4352, [4096, 1, 17, 2049, 300, 4351, 64, 65, 1000, 3000, 5, 4095, 128, 129, 2500, 4000], 1),
        (1, 8, 96, 1024, [700], 0),
        (4, 8, 64, 2048, [2047, 0, 900, 33], 1),
    ]
    for i, (B, H, D, cap, S, parity) in enumerate(cases):
        print(f"case no-alloc decode {dtype} call {i}: B={B} H={H} D={D} cap={cap}", flush=True)
        inp = _inputs(B, H, D, cap, S, seed=60 + i, dtype=dtype)
        want = _call("mote_relation_decode", inp, parity)
        got = _call("mote_relation_decode_static", inp, parity)
        for name, a, b in zip(("y", "g", "xm", "cache_p2", "cache_info", "S"), got, want):
            assert torch.equal(a, b), (i, name)
        assert torch.equal(got[5], inp["S"] + 1)
        assert bool(torch.isfinite(got[0]).all())


def test_static_slots_on_two_streams_at_once(cuda):
    """Slots 1 and 2 driven from two unordered streams, each with a queue of steps launched before
    either is waited for, so the two streams' decode kernels overlap on the GPU: every step's
    outputs equal the workspace entry point's bit for bit. Sharing one slot here would race."""
    from mote_amd import _lib as L

    dev = torch.device("cuda")
    shapes = [(16, 8, 96, 2048, 1), (8, 16, 128, 2048, 0)]
    inps = [_inputs(B, H, D, cap, [(37 * i + 5 * s) % (cap - 1) for i in range(B)], seed=90 + s, dtype=torch.bfloat16)
            for s, (B, H, D, cap, _) in enumerate(shapes)]
    want = [_call("mote_relation_decode", inp, shp[4]) for inp, shp in zip(inps, shapes)]
    for slot in (1, 2):  # first calls clear the slots, outside the concurrent part
        _call("mote_relation_decode_static", inps[0], shapes[0][4], slot=slot)
    steps = 6
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    state = []
    for s, (inp, (B, H, D, cap, parity)) in enumerate(zip(inps, shapes)):
        kc, vc = inp["kc"].to(dev), inp["vc"].to(dev)
        raw = [t.to(dev) for t in inp["raw"]]
        outs = []
        for _ in range(steps):  # one fresh copy of the mutated state per step
            outs.append(dict(kc=kc.clone(), vc=vc.clone(), S=inp["S"].to(dev),
                             y=torch.full((B, H, D), float("nan"), device=dev, dtype=kc.dtype),
                             g=torch.full((B, H), float("nan"), device=dev),
                             xm=torch.full((B,), float("nan"), device=dev)))
        state.append((raw, inp["lam"].to(dev), inp["inv"].to(dev), inp["theta"].to(dev), outs))
    torch.cuda.synchronize()
    print("case no-alloc decode: slots 1 and 2 on two streams", flush=True)
    keep = []
    for k in range(steps):  # interleave the two streams' launches
        for s, (B, H, D, cap, parity) in enumerate(shapes):
            raw, lam, inv, theta, outs = state[s]
            o = outs[k]
            a = L.DecodeArgs()
            a.dtype, a.B, a.H, a.D, a.capacity = L.MOTE_BF16, B, H, D, cap
            a.layer_parity, a.flags, a.tau_s = parity, L.MOTE_DECODE_ADVANCE, 2.0
            a.lam, a.inv_freq, a.theta, a.S = lam.data_ptr(), inv.data_ptr(), theta.data_ptr(), o["S"].data_ptr()
            a.p1, a.p2, a.info, a.in_sb = raw[0].data_ptr(), raw[1].data_ptr(), raw[2].data_ptr(), raw[0].stride(0)
            a.cache_p2, a.cache_info = L.view(o["kc"]), L.view(o["vc"])
            a.y, a.y_sb, a.g, a.xm = o["y"].data_ptr(), o["y"].stride(0), o["g"].data_ptr(), o["xm"].data_ptr()
            a.static_slot = 1 + s
            keep.append(a)
            L.check(L.lib().mote_relation_decode_static(a, streams[s].cuda_stream), "mote_relation_decode_static")
    torch.cuda.synchronize()
    for s in range(2):
        for k, o in enumerate(state[s][4]):
            got = [o[n].cpu() for n in ("y", "g", "xm", "kc", "vc", "S")]
            for name, a, b in zip(("y", "g", "xm", "cache_p2", "cache_info", "S"), got, want[s]):
                assert torch.equal(a, b), (s, k, name)


def test_static_entry_point_under_graph_capture(cuda):
    """The use the entry point exists for: a first call on a fresh slot under capture is refused on
    the host (its clear would be captured and rerun on every replay); after one eager call on the
    slot, one captured step replayed on new inputs (copied into the captured buffers, with eager work
    and synchronisation between the replays) equals the workspace entry point on each."""
    from mote_amd import _lib as L

    dev = torch.device("cuda")
    B, H, D, cap, parity = 4, 8, 96, 1024, 1
    S0 = [1000, 3, 511, 64]
    inps = [_inputs(B, H, D, cap, S0, seed=70 + i, dtype=torch.bfloat16) for i in range(4)]
    buf = {k: (v.to(dev) if k != "raw" else [t.to(dev) for t in v]) for k, v in inps[0].items()}
    y = torch.full((B, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    g = torch.full((B, H), float("nan"), device=dev)
    xm = torch.full((B,), float("nan"), device=dev)
    a = L.DecodeArgs()
    a.dtype, a.B, a.H, a.D, a.capacity = L.MOTE_BF16, B, H, D, cap
    a.layer_parity, a.flags, a.tau_s = parity, L.MOTE_DECODE_ADVANCE, 2.0
    a.lam, a.inv_freq, a.theta, a.S = (buf[k].data_ptr() for k in ("lam", "inv", "theta", "S"))
    raw = buf["raw"]
    a.p1, a.p2, a.info, a.in_sb = raw[0].data_ptr(), raw[1].data_ptr(), raw[2].data_ptr(), raw[0].stride(0)
    a.cache_p2, a.cache_info = L.view(buf["kc"]), L.view(buf["vc"])
    a.y, a.y_sb, a.g, a.xm = y.data_ptr(), y.stride(0), g.data_ptr(), xm.data_ptr()
    a.static_slot = 3  # no other test uses slot 3, so it is fresh here
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    print("case no-alloc decode: first call on a fresh slot under capture", flush=True)
    refused = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(refused, stream=side):
            y.zero_()  # keeps the refused capture's graph non-empty; it is never replayed
            rc = L.lib().mote_relation_decode_static(a, side.cuda_stream)
    assert rc == 1 and b"must not be captured" in L.lib().mote_last_error()
    torch.cuda.synchronize()
    L.check(L.lib().mote_relation_decode_static(a, L.stream_of(y)), "mote_relation_decode_static")  # clears slot 3
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(gr, stream=side):
            L.check(L.lib().mote_relation_decode_static(a, side.cuda_stream), "mote_relation_decode_static")
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for i, inp in enumerate(inps):
        print(f"case no-alloc decode: replay {i}", flush=True)
        want = _call("mote_relation_decode", inp, parity)
        for k, v in inp.items():
            if k == "raw":
                for dst, src in zip(raw, v):
                    dst.copy_(src)
            else:
                buf[k].copy_(v)
        for t in (y, g, xm):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        got = [t.cpu() for t in (y, g, xm, buf["kc"], buf["vc"], buf["S"])]
        for name, u, w in zip(("y", "g", "xm", "cache_p2", "cache_info", "S"), got, want):
            assert torch.equal(u, w), (i, name)
