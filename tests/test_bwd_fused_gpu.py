"""The bf16 tile backward's key and query work in one launch against the same work in two launches,
both through the C ABI. The library takes the one-launch form by default for head dims up to 96
(MOTE_BWD_FUSED=0 selects the two launches); these tests set MOTE_BWD_FUSED=1 around their one-launch
calls so that the comparison holds whatever the environment says, and get the two-launch form by
calling the key and query stages separately.

The one-launch form walks each key block's query blocks from the last down and reads the dU
quadrants through agent-scope loads once their counts are complete; the two-launch form walks up.
dP1 has the same products in the same order in both (bit-identical); dP2 and dI~ add the same terms
in the opposite order (fp32 accumulation, one bf16 rounding: elements differ by at most an ulp or
so); both are also checked
against the float64 oracle at the bf16 tolerance of the other backward tests (2e-2).
"""

from __future__ import annotations

import contextlib
import os

import pytest
import torch

from conftest import rel_err
from oracle import relation as O

pytestmark = pytest.mark.gpu


def _inputs(B, H, TQ, S, D, seed, scale=0.7):
    g = torch.Generator().manual_seed(seed)
    mk = lambda T: (torch.randn(B, H, T, D, generator=g) * scale).to(torch.bfloat16).cuda()
    p1, p2, info = mk(TQ), mk(S + TQ), mk(S + TQ)
    lam = torch.tensor(0.4, device="cuda")
    dy = torch.randn(B, H, TQ, D, generator=g).to(torch.bfloat16).cuda()
    return p1, p2, info, lam, dy


@contextlib.contextmanager
def _one_launch():
    """MOTE_BWD_FUSED=1 for the duration (the library reads it on every call)."""
    old = os.environ.get("MOTE_BWD_FUSED")
    os.environ["MOTE_BWD_FUSED"] = "1"
    try:
        yield
    finally:
        if old is None:
            del os.environ["MOTE_BWD_FUSED"]
        else:
            os.environ["MOTE_BWD_FUSED"] = old


def _bwd(p1, p2, info, lam, dy, S, split: bool):
    """(dp1, dp2, dinfo, dlam) of mote_relation_bwd: one call with every stage, or the rows and key
    stages in one call and the query and finish stages in a second (the two-launch form)."""
    from mote_amd import _lib as Lb
    from mote_amd.flash_relation import _token_major

    y, g, ibar, lse = torch.ops.mote.relation_fwd(p1, p2, info, lam, 2.0, S)
    B, H, TQ, D = p1.shape
    dp1 = _token_major(B, H, TQ, D, p1, p1.dtype)
    dp2 = _token_major(B, H, S + TQ, D, p1, p1.dtype)
    dinfo = _token_major(B, H, S + TQ, D, p1, p1.dtype)
    dlam = torch.empty((), device=p1.device, dtype=torch.float32)
    a = Lb.BwdArgs()
    a.dtype, a.B, a.H, a.TQ, a.TK, a.D, a.q_start = Lb.dtype_code(p1), B, H, TQ, S + TQ, D, S
    a.tau_s, a.deterministic = 2.0, 0
    a.p1, a.p2, a.info, a.dy = Lb.view(p1), Lb.view(p2), Lb.view(info), Lb.view(dy)
    a.ibar, a.lse, a.g = ibar.data_ptr(), lse.data_ptr(), g.data_ptr()
    a.dp1, a.dp2, a.dinfo, a.dlam = Lb.view(dp1), Lb.view(dp2), Lb.view(dinfo), dlam.data_ptr()
    ws = torch.full((int(Lb.lib().mote_relation_bwd_workspace(a)),), 0xA5, device=p1.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    st = Lb.stream_of(p1)
    if split:
        for stages in (Lb.MOTE_BWD_ROWS | Lb.MOTE_BWD_KEYS, Lb.MOTE_BWD_QUERIES | Lb.MOTE_BWD_FINISH):
            a.stages = stages
            Lb.check(Lb.lib().mote_relation_bwd(a, st), "mote_relation_bwd")
    else:
        a.stages = 0
        with _one_launch():
            Lb.check(Lb.lib().mote_relation_bwd(a, st), "mote_relation_bwd")
    torch.cuda.synchronize()
    return dp1, dp2, dinfo, dlam


# (B, H, TQ, S, D): one and several key blocks, ragged last blocks, cached prefixes (q_start > 0,
# aligned or not), 1, 2, 4 and 8 queues of the launch with one to three heads each, every head dim
# of the launch, the C3 length at full width and longer ones (where the library picks the one-launch
# form itself)
CASES = [
    (1, 2, 40, 0, 64),
    (2, 3, 333, 0, 64),
    (1, 1, 190, 0, 32),
    (1, 4, 700, 0, 96),
    (2, 2, 257, 100, 96),
    (1, 1, 64, 64, 96),
    (2, 3, 2001, 0, 64),
    (2, 2, 2000, 100, 96),
    (1, 8, 4964, 0, 96),
    (2, 8, 3000, 0, 64),
    (1, 8, 8192, 0, 96),
]


@pytest.mark.parametrize("B,H,TQ,S,D", CASES)
def test_one_launch_matches_two_launches(cuda, B, H, TQ, S, D):
    print(f"case fused bwd B={B} H={H} TQ={TQ} S={S} D={D}", flush=True)
    p1, p2, info, lam, dy = _inputs(B, H, TQ, S, D, seed=TQ + S)
    one = _bwd(p1, p2, info, lam, dy, S, split=False)
    two = _bwd(p1, p2, info, lam, dy, S, split=True)
    assert torch.equal(one[0], two[0]), "dP1"
    for a, b, n in zip(one[1:3], two[1:3], ("dP2", "dI~")):
        # one bf16 ulp of the largest element is up to 2^-7 of it (a rounding flip of the fp32 sums)
        assert rel_err(a.float(), b.float()) < 1e-2, n
    assert abs(float(one[3]) - float(two[3])) <= 1e-5 * max(abs(float(two[3])), 1.0), "dlam"
    # repeat: bitwise reproducible
    again = _bwd(p1, p2, info, lam, dy, S, split=False)
    for a, b in zip(one, again):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,H,TQ,S,D", [(1, 2, 300, 0, 96), (2, 2, 150, 40, 64)])
def test_one_launch_matches_oracle(cuda, B, H, TQ, S, D):
    print(f"case fused bwd oracle B={B} H={H} TQ={TQ} S={S} D={D}", flush=True)
    p1, p2, info, lam, dy = _inputs(B, H, TQ, S, D, seed=7)
    got = _bwd(p1, p2, info, lam, dy, S, split=False)
    ref = O.relation_grads_autograd(p1.cpu(), p2.cpu(), info.cpu(), lam.cpu(), dy.cpu(), 2.0, S, dtype=torch.float64)
    for a, b, n in zip(got[:3], ref[:3], ("dP1", "dP2", "dI~")):
        assert rel_err(a.cpu().double(), b) < 2e-2, n
    terms = O.relation_dlam_terms(p1.cpu(), p2.cpu(), info.cpu(), lam.cpu(), dy.cpu(), 2.0, S)
    assert abs(float(got[3]) - float(ref[3])) / max(float(terms.abs().sum()), 1e-3) < 2e-2


def test_one_launch_graph_replays(cuda):
    """Captured once, replayed with eager work and synchronisations between the replays: the rows
    stage clears the launch's counters in every replay, and every replay equals the eager call."""
    print("case fused bwd graph replays", flush=True)
    p1, p2, info, lam, dy = _inputs(1, 2, 600, 0, 96, seed=11)
    ref = _bwd(p1, p2, info, lam, dy, 0, split=False)
    y, g, ibar, lse = torch.ops.mote.relation_fwd(p1, p2, info, lam, 2.0, 0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side), _one_launch():
        torch.ops.mote.relation_bwd(p1, p2, info, ibar, lse, g, dy, 2.0, 0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), _one_launch():
        with torch.cuda.graph(gr, stream=side):
            outs = torch.ops.mote.relation_bwd(p1, p2, info, ibar, lse, g, dy, 2.0, 0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for r in range(3):
        for t in outs:
            t.fill_(float("nan"))
        _ = (p1.float() * 2).sum()  # eager work between replays
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, ref):
            assert torch.equal(a, b), f"replay {r}"


def test_wait_that_gives_up_writes_nan_rows(cuda):
    """The query jobs' bounded wait: forced from the host to give up (MOTE_BWD_UNREACHABLE_WAIT=1 puts
    every count's target out of reach and allows four polls), each query job writes its dP1 rows as
    NaN and ends, so the launch finishes; the key work's outputs are unaffected."""
    print("case fused bwd wait gives up", flush=True)
    p1, p2, info, lam, dy = _inputs(1, 2, 300, 0, 96, seed=5)
    ref = _bwd(p1, p2, info, lam, dy, 0, split=True)
    os.environ["MOTE_BWD_UNREACHABLE_WAIT"] = "1"
    try:
        got = _bwd(p1, p2, info, lam, dy, 0, split=False)
    finally:
        del os.environ["MOTE_BWD_UNREACHABLE_WAIT"]
    assert torch.isnan(got[0].float()).all(), "dP1"
    for a, b, n in zip(got[1:3], ref[1:3], ("dP2", "dI~")):
        assert rel_err(a.float(), b.float()) < 1e-2, n
    again = _bwd(p1, p2, info, lam, dy, 0, split=False)  # the switch is read per call
    assert torch.equal(again[0], ref[0])
