"""The no-allocation decode entry point, mote_relation_decode_static, through the C ABI against
mote_relation_decode with a caller workspace: on calls in a row (the second with a smaller
batch, capacity and fill) the outputs y, g, xm, the appended cache rows and the advanced positions
are identical bit for bit (same kernel, same split count, deterministic merge order). A third call
goes back to a larger batch with another head dim: the shared array's counters stay valid."""

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


def _call(entry: str, inp, layer_parity: int):
    """One decode step through the named C entry point on fresh device copies of `inp`."""
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
        a.workspace, a.workspace_bytes = None, 0
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
