"""Prefix-store pages of the decode arena (mote/infer/prefix_cache.py:122-186) on the CPU: row
round trips through pages, page sizes and tail growth, forks sharing full pages, the hot-arena case
that copies nothing, and a batched arena's sequence slots. (The HIP DMA path of the same copies is
tested on the GPU in tests/test_decode_engine_gpu.py.)"""

from __future__ import annotations

import pytest
import torch

from mote_amd.arena import RelationArena
from mote_amd.prefix import PAGE, ArenaPages


def _filled(n_layers=2, H=4, cap=1024, dh=8, batch=1, seed=0):
    a = RelationArena(n_layers, H, cap, dh, "cpu", torch.float32, batch=batch)
    a.store.copy_(torch.randn(a.store.shape, generator=torch.Generator().manual_seed(seed)))
    return a


def test_store_and_hydrate_round_trip_in_pieces():
    from mote_amd.prefix import Branch

    src = _filled()
    pages = ArenaPages(pin=False)
    b = Branch()
    for c0, c1 in ((0, 5), (5, 300), (300, 700)):  # crosses two page boundaries, grows the tail
        pages.store_rows(b, src, c0, c1)
    assert b.n_chunks == 700 and [p.shape[3] for p in b.pages] == [PAGE, PAGE, 256]
    assert pages.rows_copied_out == 700
    dst = RelationArena(2, 4, 256, 8, "cpu", torch.float32)
    pages.hydrate(b, 700, dst)
    assert dst.capacity >= 700 and dst.owner == b.id and dst.n_valid == 700
    assert torch.equal(dst.buf[..., :700, :], src.buf[..., :700, :])
    with pytest.raises(ValueError):
        pages.store_rows(b, src, 600, 800)  # not an append


def test_tail_pages_grow_by_doubling():
    from mote_amd.prefix import Branch

    src = _filled()
    pages = ArenaPages(pin=False)
    b = Branch()
    pages.store_rows(b, src, 0, 3)
    assert b.pages[0].shape[3] == 16
    pages.store_rows(b, src, 3, 40)
    assert b.pages[0].shape[3] == 64
    pages.store_rows(b, src, 40, 200)
    assert b.pages[0].shape[3] == PAGE
    assert torch.equal(b.pages[0][:, :, :, :200], src.buf[..., :200, :])


def test_fork_shares_full_pages_and_copies_the_partial_one():
    from mote_amd.prefix import Branch

    src = _filled()
    pages = ArenaPages(pin=False)
    parent = Branch()
    pages.store_rows(parent, src, 0, 600)
    child = pages.fork(parent, 530)
    assert child.n_chunks == 530 and child.id != parent.id
    assert child.pages[0] is parent.pages[0] and child.pages[1] is parent.pages[1]
    assert child.pages[2] is not parent.pages[2] and child.pages[2].shape[3] == 530 - 2 * PAGE
    assert ArenaPages.nbytes([parent, child]) == sum(p.numel() * 4 for p in parent.pages) + child.pages[2].numel() * 4
    # the child continues with rows of its own; the parent's pages are untouched
    other = _filled(seed=1)
    pages.store_rows(child, other, 530, 560)
    assert torch.equal(child.pages[2][:, :, :, 530 - 512:560 - 512], other.buf[..., 530:560, :])
    assert torch.equal(parent.pages[2][:, :, :, :88], src.buf[..., 512:600, :])
    dst = RelationArena(2, 4, 1024, 8, "cpu", torch.float32)
    pages.hydrate(child, 560, dst)
    assert torch.equal(dst.buf[..., :530, :], src.buf[..., :530, :])
    assert torch.equal(dst.buf[..., 530:560, :], other.buf[..., 530:560, :])
    with pytest.raises(ValueError):
        pages.fork(parent, 601)


def test_hydrating_the_resident_branch_copies_nothing():
    from mote_amd.prefix import Branch

    src = _filled()
    pages = ArenaPages(pin=False)
    b = Branch()
    pages.store_rows(b, src, 0, 300)
    dst = RelationArena(2, 4, 512, 8, "cpu", torch.float32)
    pages.hydrate(b, 300, dst)
    assert pages.rows_copied_in == 300
    dst.buf[..., :300, :] += 1.0  # had it copied again, these would be overwritten
    pages.hydrate(b, 200, dst)
    assert pages.rows_copied_in == 300 and dst.n_valid == 200
    assert torch.equal(dst.buf[..., :200, :], src.buf[..., :200, :] + 1.0)
    other = Branch()
    pages.store_rows(other, _filled(seed=3), 0, 50)
    pages.hydrate(other, 50, dst)  # another branch: copied, residency moves
    assert pages.rows_copied_in == 350 and dst.owner == other.id


def test_batched_arena_slots():
    from mote_amd.prefix import Branch

    src = _filled(batch=3, cap=512, seed=4)
    pages = ArenaPages(pin=False)
    b = Branch()
    pages.store_rows(b, src, 0, 270, seq=2)
    dst = RelationArena(2, 4, 512, 8, "cpu", torch.float32, batch=3)
    pages.hydrate(b, 270, dst, seq=1)
    assert torch.equal(dst.store[:, :, 1, :, :270], src.store[:, :, 2, :, :270])
    assert float(dst.store[:, :, 0].abs().sum()) == 0.0 and float(dst.store[:, :, 2].abs().sum()) == 0.0
