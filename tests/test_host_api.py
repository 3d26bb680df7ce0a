"""The host-side surface on the CPU: every name the reference's callers import, the torch-level RoPE /
Givens helpers against the oracle, the fp32 RoPE frequencies of a cast module, the decode entry
point's argument checks, the arena's sizing / growth / residency, and the determinism switch.
No GPU and no compute call into the HIP library."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import relation as O


def test_reference_callers_find_their_names():
    """The imports of mote/infer/graph.py:39, mote/model/relation.py:28-33, the kernel tests
    (tests/test_flash_relation.py:11, tests/test_givens_and_rope.py:6) and the train loop's
    determinism switch (mote/determinism.py:41-62) resolve against this package."""
    from mote_amd.flash_relation import DETERMINISTIC, HAS_TRITON, flash_relation, relation_reference  # noqa: F401
    from mote_amd.relation import (FLASH_MIN_T, USE_FLASH, FullRelation, HeadRMSNorm, RelationCache,  # noqa: F401
                                   _apply_rope, _rope_cos_sin, _rotate_half, rope_tables)
    from mote_amd.arena import ArenaLayer, ArenaState, RelationArena  # noqa: F401
    from mote_amd import determinism

    assert callable(FullRelation._givens) and callable(determinism.apply) and callable(determinism.state)


def test_relation_reference_matches_the_oracle():
    from mote_amd.flash_relation import relation_reference

    g = torch.Generator().manual_seed(4)
    for S in (0, 9):
        p1 = torch.randn(2, 3, 17, 24, generator=g)
        p2 = torch.randn(2, 3, S + 17, 24, generator=g)
        info = torch.randn(2, 3, S + 17, 24, generator=g)
        lam = torch.tensor(0.4)
        y, gg = relation_reference(p1, p2, info, lam, 2.0, S)
        yr, gr = O.relation_reference(p1, p2, info, lam, 2.0, S, dtype=torch.float64)
        assert y.dtype == torch.float32 and gg.dtype == torch.float32
        assert torch.allclose(y.double(), yr, atol=1e-5) and torch.allclose(gg.double(), gr, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_helpers_match_the_oracle(dtype):
    from mote_amd.relation import _apply_rope, _rope_cos_sin, _rotate_half, rope_tables

    x = torch.randn(2, 4, 19, 96).to(dtype)
    c, s = rope_tables(300, 19, 96, 10000.0, dtype, "cpu")
    co, so = O.rope_tables(300, 19, 96, 10000.0, dtype)
    assert torch.equal(c, co) and torch.equal(s, so)
    assert rope_tables(300, 19, 96, 10000.0, dtype, "cpu")[0] is c  # memoised
    c2, s2 = _rope_cos_sin(torch.arange(300, 319), 96, 10000.0, dtype)
    assert torch.equal(c2, co) and torch.equal(s2, so)
    assert torch.equal(_rotate_half(x), O.rotate_half(x))
    assert torch.equal(_apply_rope(x, c, s), O.apply_rope(x, co, so))


@pytest.mark.parametrize("layer_idx", [0, 1])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_givens_method_matches_the_oracle(layer_idx, dtype):
    from mote_amd.relation import FullRelation

    m = FullRelation(64, 8, layer_idx)
    with torch.no_grad():
        m.theta.uniform_(-0.5, 0.5)
    info = torch.randn(3, 8, 5, 8).to(dtype)
    assert torch.equal(m._givens(info), O.givens(info, m.theta.detach(), layer_idx))
    m2 = FullRelation(64, 8, layer_idx, givens=False)
    assert m2._givens(info) is info


def test_cast_module_keeps_exact_rope_frequencies():
    """`.to(torch.bfloat16)` / `.half()` leave the frequencies fp32 and bit-identical to the
    reference's fp32 table (relation.py:39); rounded to bf16 they would be off by radians at
    positions in the thousands."""
    from mote_amd.relation import FullRelation

    want = O.rope_inv_freq(96, 10000.0)
    for cast in (lambda m: m.to(torch.bfloat16), lambda m: m.half(), lambda m: m.to(dtype=torch.float64)):
        m = cast(FullRelation(768, 8, 0))
        assert m.inv_freq.dtype == torch.float32 and torch.equal(m.inv_freq, want)
        assert m.w1.weight.dtype != torch.float32
    ang_err = float((4000 * want - 4000 * want.bfloat16().float()).abs().max())
    assert ang_err > 1.0  # what the cast used to do


def test_module_without_a_gpu_raises():
    from mote_amd.relation import FullRelation

    m = FullRelation(64, 4, 0)
    with pytest.raises(RuntimeError):
        m(torch.randn(1, 5, 64))


# ---- relation_decode argument checks (all raised before any launch) ------------------------------
def _decode_args(B=2, H=4, D=32, cap=64, dtype=torch.bfloat16):
    mk = lambda *s: torch.zeros(*s, dtype=dtype)
    return dict(p1=mk(B, H, D), p2=mk(B, H, D), info=mk(B, H, D), S=torch.zeros(B, dtype=torch.int64),
                cache_p2=mk(B, H, cap, D), cache_info=mk(B, H, cap, D), lam=torch.tensor(0.5),
                inv_freq=O.rope_inv_freq(D, 10000.0), theta=torch.zeros(H // 2))


@pytest.mark.parametrize("bad,exc", [
    (dict(S=torch.zeros(2, dtype=torch.int32)), ValueError),
    (dict(S=torch.zeros(3, dtype=torch.int64)), ValueError),
    (dict(S=torch.zeros(4, dtype=torch.int64)[::2]), ValueError),
    (dict(cache_info=torch.zeros(2, 4, 32, 32, dtype=torch.bfloat16)), ValueError),
    (dict(cache_info=torch.zeros(2, 4, 64, 32, dtype=torch.float32)), ValueError),
    (dict(cache_p2=torch.zeros(2, 4, 64, 16, dtype=torch.bfloat16)), ValueError),
    (dict(p2=torch.zeros(2, 4, 32, dtype=torch.float32)), TypeError),
    (dict(inv_freq=torch.ones(8)), ValueError),
    (dict(theta=torch.ones(3)), ValueError),
    (dict(lam=torch.ones(2)), ValueError),
    (dict(p1=torch.zeros(2, 4, 64, dtype=torch.bfloat16)[..., ::2]), ValueError),
])
def test_decode_rejects_bad_arguments(bad, exc):
    from mote_amd.decode import relation_decode

    args = _decode_args()
    args.update(bad)
    with pytest.raises(exc):
        relation_decode(**args)


def test_decode_rejects_bad_outputs_and_needs_a_gpu():
    from mote_amd.decode import relation_decode

    with pytest.raises(ValueError):
        relation_decode(**_decode_args(), xm=torch.zeros(3))
    with pytest.raises(ValueError):
        relation_decode(**_decode_args(), g=torch.zeros(2, 4, dtype=torch.float64))
    with pytest.raises(ValueError):
        relation_decode(**_decode_args(), y=torch.zeros(2, 4, 32))
    with pytest.raises(RuntimeError):  # valid arguments, but on the CPU
        relation_decode(**_decode_args())
    # a bf16 parameter is converted, not misread: the checks pass and only the device is refused
    args = _decode_args()
    args.update(lam=torch.tensor(0.5, dtype=torch.bfloat16), theta=torch.zeros(2, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        relation_decode(**args)


# ---- arena -----------------------------------------------------------------------------------------
def test_arena_layout_views_and_sizing():
    from mote_amd.arena import ArenaState, RelationArena

    a = RelationArena(3, 4, 256, 16, "cpu", torch.float32)
    assert a.buf.shape == (3, 2, 4, 256, 16) and a.p2(1).shape == (1, 4, 256, 16)
    assert a.buf.data_ptr() == a.store.data_ptr() and a.p2(1).stride(1) == 256 * 16
    assert a.bytes_per_chunk == 3 * 2 * 4 * 16 * 4 and a.nbytes() == a.bytes_per_chunk * 256
    b = RelationArena(2, 4, 128, 16, "cpu", torch.bfloat16, batch=5)
    assert b.buf.shape == (2, 2, 5, 4, 128, 16) and b.info(1).shape == (5, 4, 128, 16)
    # the reference's sizing rule: ceil((int(seq / bpic * margin) + 1) / bucket) buckets, at least one
    assert RelationArena.capacity_for(16384, 3.3) == 6400
    assert RelationArena.capacity_for(0, 3.3) == 256
    assert RelationArena.capacity_for(1023, 1.0, bucket=256, margin=1.0) == 1024
    assert RelationArena.capacity_for(1024, 1.0, bucket=256, margin=1.0) == 1280
    st = ArenaState(a)
    assert len(st) == 3 and [layer.layer for layer in st] == [0, 1, 2]
    for layer in st:
        layer.write(torch.ones(1, 4, 7, 16) * (layer.layer + 1), torch.full((1, 4, 7, 16), -1.0))
    st.advance(7)
    c = st.copy()
    c.advance(3)
    assert st.n == 7 and c.n == 10 and c.arena is a
    p2, info = st[2].views(7)
    assert torch.equal(p2, torch.full((1, 4, 7, 16), 3.0)) and float(info.sum()) == -7 * 4 * 16
    assert float(a.buf[:, :, :, 7:].abs().sum()) == 0.0
    with pytest.raises(RuntimeError):
        ArenaState(a, 250)[0].write(torch.zeros(1, 4, 7, 16), torch.zeros(1, 4, 7, 16))


def test_arena_growth_keeps_claimed_rows_only():
    from mote_amd.arena import RelationArena

    a = RelationArena(2, 2, 256, 8, "cpu", torch.float32)
    a.buf[..., :100, :] = 2.0
    assert not a.ensure(256) and a.generation == 0
    a.claim(owner=7, rows=100)
    assert a.ensure(257) and a.capacity == 512 and a.generation == 1
    assert a.owner == 7 and a.n_valid == 100
    assert bool((a.buf[..., :100, :] == 2.0).all()) and float(a.buf[..., 100:, :].abs().sum()) == 0.0
    assert a.ensure(1600) and a.capacity == 2048  # next power-of-two multiple
    a.invalidate()
    assert a.ensure(2049) and a.capacity == 4096 and a.owner is None and a.n_valid == 0
    assert float(a.buf.abs().sum()) == 0.0  # nothing live: nothing carried over, zeroed
    with pytest.raises(ValueError):
        a.claim(1, 5000)


def test_determinism_switch_round_trip():
    from mote_amd import determinism, flash_relation

    before = (flash_relation.DETERMINISTIC, torch.are_deterministic_algorithms_enabled())
    try:
        determinism.apply(True)
        st = determinism.state()
        assert st["reproducible"] and st["relation_backward"] == "two-pass" and flash_relation.DETERMINISTIC
        determinism.apply(False)
        st = determinism.state()
        assert not st["reproducible"] and st["relation_backward"] == "atomics"
    finally:
        flash_relation.DETERMINISTIC = before[0]
        torch.use_deterministic_algorithms(before[1])


def test_head_rms_norm_module_matches_the_oracle():
    from mote_amd.relation import HeadRMSNorm

    n, r = HeadRMSNorm(96), O.HeadRMSNormRef(96)
    with torch.no_grad():
        n.weight.uniform_(0.5, 1.5)
        r.weight.copy_(n.weight)
    x = torch.randn(2, 8, 11, 96).bfloat16()
    assert torch.equal(n(x), r(x))
    assert math.isfinite(float(n(x).float().sum()))


@pytest.mark.parametrize("T,qk_norm,dtype,fused", [(64, False, torch.bfloat16, True),
                                                     (80000, False, torch.bfloat16, True),
                                                     (80000, True, torch.bfloat16, True),
                                                     (64, False, torch.float32, False)])
def test_fused_prologue_dispatch(monkeypatch, T, qk_norm, dtype, fused):
    """FullRelation.heads takes the fused prologue for bf16 activations at every row count, with and
    without QK-Norm, and the product + RoPE kernel path for fp32. The launches are replaced by
    recorders, so this runs on the CPU."""
    from mote_amd import relation as R

    calls = []
    monkeypatch.setattr(R, "qkv_rope", lambda *a, **k: calls.append("fused") or ("p1", "p2", "info"))
    monkeypatch.setattr(R, "rope_givens", lambda *a, **k: calls.append("unfused") or ("p1", "p2", "info"))
    m = R.FullRelation(128, 2, 1, qk_norm=qk_norm, dtype=dtype)
    x = torch.zeros(1, T, 128, dtype=dtype)
    m.heads(x, 0)
    assert calls == ["fused" if fused else "unfused"]
