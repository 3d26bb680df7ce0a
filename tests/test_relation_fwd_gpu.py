"""Fused forward through the HIP library against the CPU oracle (oracle/relation.py).

Cases follow the reference's kernel tests (tests/test_flash_relation.py:42-107) plus the BASELINE
tolerances: 1e-5 relative in fp32 and 2e-2 relative in bf16, relative = max|a-b| / max|ref|.
"""

from __future__ import annotations

import pytest
import torch

from conftest import rel_err
from oracle import relation as O

pytestmark = pytest.mark.gpu


def _inputs(B, H, TQ, S, D, dtype, seed=0, scale=0.7, dev="cuda"):
    g = torch.Generator(device="cpu").manual_seed(seed)
    mk = lambda T: (torch.randn(B, H, T, D, generator=g) * scale).to(dtype).to(dev)
    return mk(TQ), mk(S + TQ), mk(S + TQ)


def _oracle(p1, p2, info, lam, S, dtype=torch.float64):
    return O.relation_reference(p1.cpu(), p2.cpu(), info.cpu(), torch.tensor(lam), 2.0, S, dtype=dtype)


@pytest.mark.parametrize("D", [48, 64, 96])
@pytest.mark.parametrize("TQ,S", [(16, 0), (50, 0), (130, 0), (300, 0), (20, 37), (64, 64), (1, 0), (1, 9)])
def test_fp32_forward_matches_oracle(cuda, D, TQ, S):
    from mote_amd.flash_relation import flash_relation

    print(f"case fp32 D={D} TQ={TQ} S={S}", flush=True)
    p1, p2, info = _inputs(2, 3, TQ, S, D, torch.float32)
    lam = torch.tensor(0.5, device=cuda)
    y, g = flash_relation(p1, p2, info, lam, 2.0, q_start=S)
    torch.cuda.synchronize()
    yr, gr = _oracle(p1, p2, info, 0.5, S)
    assert y.shape == (2, 3, TQ, D) and y.dtype == torch.float32
    assert rel_err(y, yr) < 1e-5, rel_err(y, yr)
    assert float((g.cpu().double() - gr).abs().max()) < 1e-5
    # the reference's own bounds (tests/test_flash_relation.py:31-32)
    assert torch.allclose(y.cpu().double(), yr, atol=2e-4, rtol=1e-3)


@pytest.mark.parametrize("D", [96, 112, 24])
def test_odd_head_dims(cuda, D):
    from mote_amd.flash_relation import flash_relation

    print(f"case odd D={D}", flush=True)
    p1, p2, info = _inputs(1, 2, 90, 0, D, torch.float32)
    y, g = flash_relation(p1, p2, info, torch.tensor(0.5, device=cuda), 2.0)
    yr, gr = _oracle(p1, p2, info, 0.5, 0)
    assert rel_err(y, yr) < 1e-5
    assert float((g.cpu().double() - gr).abs().max()) < 1e-5


def test_rescale_branch_large_scores(cuda):
    """Scores spanning far more than 2^8 across key blocks force the conditional rescale."""
    from mote_amd.flash_relation import flash_relation

    p1, p2, info = _inputs(1, 2, 200, 0, 64, torch.float32, seed=3, scale=3.0)
    y, g = flash_relation(p1, p2, info, torch.tensor(0.5, device=cuda), 2.0)
    yr, gr = _oracle(p1, p2, info, 0.5, 0)
    assert rel_err(y, yr) < 1e-5
    assert float((g.cpu().double() - gr).abs().max()) < 1e-5


@pytest.mark.parametrize("D", [32, 48, 64, 96, 128])
@pytest.mark.parametrize("TQ", [33, 257])
def test_bf16_forward(cuda, D, TQ):
    from mote_amd.flash_relation import flash_relation

    print(f"case bf16 D={D} TQ={TQ}", flush=True)
    p1, p2, info = _inputs(2, 4, TQ, 0, D, torch.bfloat16)
    y, g = flash_relation(p1, p2, info, torch.tensor(0.5, device=cuda), 2.0)
    yr, gr = _oracle(p1, p2, info, 0.5, 0)
    assert y.dtype == torch.bfloat16
    assert rel_err(y, yr) < 2e-2, rel_err(y, yr)
    assert float((y.cpu().double() - yr).abs().max()) < 4e-2
    assert float((g.cpu().double() - gr).abs().max()) < 2e-2


def test_bf16_prefix_flagship_shape(cuda):
    """D = 96 with a cached prefix at a chunk count past the bucket (test_flash_relation.py:88-100)."""
    from mote_amd.flash_relation import flash_relation

    p1, p2, info = _inputs(1, 8, 700, 64, 96, torch.bfloat16, seed=2)
    y, g = flash_relation(p1, p2, info, torch.tensor(0.5, device=cuda), 2.0, q_start=64)
    yr, gr = _oracle(p1, p2, info, 0.5, 64)
    assert rel_err(y, yr) < 2e-2
    assert float((g.cpu().double() - gr).abs().max()) < 2e-2


@pytest.mark.parametrize("D,TQ,S", [(96, 6300, 0), (64, 1200, 5100), (128, 6200, 37)])
def test_bf16_long_rows_split(cuda, D, TQ, S):
    """Rows long enough that the longest query blocks run as two workgroups whose partial softmax
    states merge in a second launch."""
    from mote_amd.flash_relation import flash_relation

    print(f"case bf16 split D={D} TQ={TQ} S={S}", flush=True)
    p1, p2, info = _inputs(1, 2, TQ, S, D, torch.bfloat16, seed=13)
    y, g = flash_relation(p1, p2, info, torch.tensor(0.4, device=cuda), 2.0, q_start=S)
    yr, gr = _oracle(p1, p2, info, 0.4, S)
    assert rel_err(y, yr) < 2e-2, rel_err(y, yr)
    assert float((g.cpu().double() - gr).abs().max()) < 2e-2


def test_split_and_whole_rows_agree(cuda):
    """The same launch with and without the workspace (split halves merged vs one workgroup per
    query block) gives the same statistics to float rounding."""
    from mote_amd import _lib as L

    B, H, T, D = 1, 2, 6400, 96
    p1, p2, info = _inputs(B, H, T, 0, D, torch.bfloat16, seed=14)
    lam = torch.tensor([0.5], device=cuda)
    outs = []
    for use_ws in (False, True):
        y = torch.empty(B, H, T, D, device=cuda, dtype=torch.bfloat16)
        ibar = torch.empty(B, H, T, D, device=cuda)
        lse = torch.empty(B, H, T, device=cuda)
        g = torch.empty(B, H, T, device=cuda)
        a = L.FwdArgs()
        a.dtype, a.B, a.H, a.TQ, a.TK, a.D, a.q_start, a.tau_s = L.MOTE_BF16, B, H, T, T, D, 0, 2.0
        a.p1, a.p2, a.info, a.y = L.view(p1), L.view(p2), L.view(info), L.view(y)
        a.ibar, a.lse, a.g, a.lam = ibar.data_ptr(), lse.data_ptr(), g.data_ptr(), lam.data_ptr()
        n = int(L.lib().mote_relation_fwd_workspace(a))
        assert n > 0
        ws = torch.empty(n, device=cuda, dtype=torch.uint8)
        if use_ws:
            a.workspace, a.workspace_bytes = ws.data_ptr(), n
        L.check(L.lib().mote_relation_fwd(a, L.stream_of(p1)), "fwd")
        torch.cuda.synchronize()
        outs.append((ibar, lse, g, y))
    (ib0, l0, g0, y0), (ib1, l1, g1, y1) = outs
    assert rel_err(ib1, ib0) < 1e-5
    assert torch.equal(torch.isinf(l1), torch.isinf(l0))  # rows without a past: LSE = -inf in both
    fin = torch.isfinite(l0)
    assert float((l1[fin] - l0[fin]).abs().max()) < 1e-4
    assert float((g1 - g0).abs().max()) < 1e-5
    assert float((y1.float() - y0.float()).abs().max()) <= 2 ** -6 * float(y0.float().abs().max())


def test_first_position_is_pure_self(cuda):
    from mote_amd.flash_relation import flash_relation

    p1, p2, info = _inputs(1, 2, 16, 0, 64, torch.float32)
    y, g = flash_relation(p1, p2, info, torch.tensor(0.5, device=cuda), 2.0)
    assert torch.allclose(y[:, :, 0], info[:, :, 0], atol=1e-6)
    assert float(g[:, :, 0].abs().max()) == 0.0


def test_strided_arena_views(cuda):
    """P2 / I~ read in place from a [1, H, capacity, D] buffer (head stride capacity * D), the way
    the decode arena hands them over (flash_relation.py:513-525)."""
    from mote_amd.flash_relation import flash_relation

    H, D, cap, S, T = 4, 64, 512, 100, 77
    g = torch.Generator().manual_seed(11)
    buf = (torch.randn(2, H, cap, D, generator=g) * 0.7).to(cuda)
    p1 = (torch.randn(1, H, T, D, generator=g) * 0.7).to(cuda)
    p2v, iv = buf[0:1, :, : S + T], buf[1:2, :, : S + T]
    y, gg = flash_relation(p1, p2v, iv, torch.tensor(0.3, device=cuda), 2.0, q_start=S)
    yr, gr = _oracle(p1, p2v.contiguous(), iv.contiguous(), 0.3, S)
    assert rel_err(y, yr) < 1e-5


def test_varlen_equals_per_sequence(cuda):
    from mote_amd.flash_relation import flash_relation_varlen

    H, D = 4, 96
    lens = [37, 200, 1, 129, 64, 6300]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    total = int(cu[-1])
    g = torch.Generator().manual_seed(12)
    x = [(torch.randn(total, H, D, generator=g) * 0.7) for _ in range(3)]
    p1, p2, info = (t.to(torch.bfloat16).to(cuda).permute(1, 0, 2) for t in x)  # [H, total, D] views
    y, gg = flash_relation_varlen(p1, p2, info, torch.tensor(0.5, device=cuda), cu.to(cuda), max(lens), 2.0)
    for b, n in enumerate(lens):
        r0 = int(cu[b])
        sl = slice(r0, r0 + n)
        yr, gr = _oracle(p1[None, :, sl], p2[None, :, sl], info[None, :, sl], 0.5, 0)
        assert rel_err(y[:, sl], yr[0]) < 2e-2, (b, rel_err(y[:, sl], yr[0]))
        assert float((gg[:, sl].cpu().double() - gr[0]).abs().max()) < 2e-2


def test_c5_varlen_full_size_equals_dense(cuda):
    """BASELINE config C5 at full size: 8 packed sequences of U[1000, 5000] chunks (seed 4), H = 8,
    dh = 96, bf16. The oracle cannot run at this size; the packed path must equal the dense path run
    on each sequence alone (the small varlen test above pins both against the oracle)."""
    from mote_amd.flash_relation import flash_relation, flash_relation_varlen

    H, D = 8, 96
    lens = torch.randint(1000, 5001, (8,), generator=torch.Generator().manual_seed(4)).tolist()
    print(f"case C5 lens={lens}", flush=True)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    total = int(cu[-1])
    g = torch.Generator().manual_seed(14)
    x = [torch.randn(total, H, D, generator=g).to(torch.bfloat16).to(cuda) for _ in range(3)]
    p1, p2, info = (t.permute(1, 0, 2) for t in x)  # [H, total, D] views of [total, H, D] memory
    lam = torch.tensor(0.5, device=cuda)
    y, gg = flash_relation_varlen(p1, p2, info, lam, cu.to(cuda), max(lens), 2.0)
    assert torch.isfinite(y.float()).all() and torch.isfinite(gg).all()
    for b, n in enumerate(lens):
        sl = slice(int(cu[b]), int(cu[b]) + n)
        yd, gd = flash_relation(p1[None, :, sl], p2[None, :, sl], info[None, :, sl], lam, 2.0, 0)
        assert rel_err(y[:, sl], yd[0]) < 1e-3, (b, rel_err(y[:, sl], yd[0]))
        assert float((gg[:, sl] - gd[0]).abs().max()) < 1e-3


def test_empty_query_block_and_shapes(cuda):
    from mote_amd.flash_relation import flash_relation

    p1, p2, info = _inputs(1, 2, 0, 5, 32, torch.float32)
    y, g = flash_relation(p1, p2, info, torch.tensor(0.5, device=cuda), 2.0, q_start=5)
    assert y.shape == (1, 2, 0, 32) and g.shape == (1, 2, 0)
    with pytest.raises(ValueError):
        flash_relation(p1, p2[:, :, :3], info[:, :, :3], torch.tensor(0.5, device=cuda), 2.0, q_start=5)


@pytest.mark.parametrize("B,H,T,S,D,varlen", [
    (1, 8, 700, 0, 96, True), (4, 8, 1000, 0, 96, False), (2, 4, 333, 50, 64, False), (1, 2, 2000, 0, 128, False),
    (3, 3, 129, 0, 32, False), (1, 6, 64, 64, 96, False),
])
def test_persistent_equals_one_job_per_workgroup(cuda, monkeypatch, B, H, T, S, D, varlen):
    """The tile forward's persistent form (jobs from per-queue counters, MOTE_FWD_PERSIST=1) runs the
    same per-job code as one workgroup per job (MOTE_FWD_PERSIST=0): every output bit for bit, with
    1 / 2 / 4 / 8 queues, cached prefixes, ragged packed sequences and every tile head dim."""
    from mote_amd.flash_relation import flash_relation  # noqa: F401  (registers the ops)

    print(f"case fwd persistent B={B} H={H} T={T} S={S} D={D} varlen={varlen}", flush=True)
    lam = torch.tensor(0.45, device=cuda)
    if varlen:
        lens = [T, T // 3, T // 2 + 7]
        cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
        total = int(cu[-1])
        g = torch.Generator().manual_seed(21)
        x = [torch.randn(total, H, D, generator=g).to(torch.bfloat16).to(cuda) for _ in range(3)]
        args = tuple(t.permute(1, 0, 2) for t in x) + (lam, cu.to(cuda), max(lens), 2.0)
        op = torch.ops.mote.relation_fwd_varlen
    else:
        p1, p2, info = _inputs(B, H, T, S, D, torch.bfloat16, seed=22)
        args = (p1, p2, info, lam, 2.0, S)
        op = torch.ops.mote.relation_fwd
    outs = []
    for flag in ("0", "1"):
        monkeypatch.setenv("MOTE_FWD_PERSIST", flag)
        outs.append([t.clone() for t in op(*args)])
        torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
