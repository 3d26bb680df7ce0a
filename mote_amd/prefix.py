"""Prefix-store pages of the decode arena: a conversation's {P2, I~} rows kept on the host.

The arena half of the reference's prefix store (mote/infer/prefix_cache.py:53-70, 122-186): a branch
(one linear conversation history) owns the arena rows of the chunks it has read, stored in pinned host
pages of PAGE rows; full pages never change, so a fork shares them by reference and copies only its
partial tail page; `hydrate` makes the arena hold a branch's rows again, and does nothing when the
arena already holds them (the arena's residency record, `owner` / `n_valid`). The anchors, byte
lookup and budget of the reference's store belong to its serving engine, not to this path.

Layout of a page: [n_layers, 2, H, rows, dh], the arena's own layout for a row range, so each
(layer, kind) plane of a page segment is one 2-D copy of H head runs: `mote_arena_page_copy` issues
them as DMA (hipMemcpy2DAsync between the arena's head pitch and the page's), with no staging copy
and no kernel. Pages of a batched arena store one sequence slot (`seq`).

Tail pages grow by doubling up to PAGE rows: a branch of a few chunks does not hold a whole page, and
a growing branch reallocates its tail O(log PAGE) times.
"""

from __future__ import annotations

import itertools
from typing import List

import torch

from . import _lib as L
from .arena import RelationArena

PAGE = 256  # rows per full page: the decode bucket width


class Branch:
    """One conversation history's arena rows on the host (prefix_cache.py:53-70)."""

    _ids = itertools.count(1)

    def __init__(self):
        self.id = next(Branch._ids)
        self.pages: List[torch.Tensor] = []  # [n_layers, 2, H, rows, dh]; all but the last hold PAGE rows
        self.n_chunks = 0


def _copy_rows(arena: RelationArena, seq: int, arena_row0: int, page: torch.Tensor, page_row0: int, rows: int,
               to_page: bool) -> None:
    """Rows [arena_row0, +rows) of sequence `seq` <-> page rows [page_row0, +rows)."""
    if rows <= 0:
        return
    st = arena.store  # [n_layers, 2, batch, H, capacity, dh]
    if arena.device.type == "cuda":
        a = L.PageCopyArgs()
        a.to_page, a.planes, a.H, a.D = int(bool(to_page)), arena.n_layers * 2, arena.n_heads, arena.d_head
        a.elem_bytes, a.rows = st.element_size(), int(rows)
        a.arena, a.a_plane, a.a_head, a.arena_row0 = st[0, 0, seq].data_ptr(), st.stride(1), st.stride(3), int(arena_row0)
        a.page, a.p_plane, a.p_head, a.page_row0 = page.data_ptr(), page.stride(1), page.stride(2), int(page_row0)
        L.check(L.lib().mote_arena_page_copy(a, L.stream_of(st)), "mote_arena_page_copy")
        return
    # an arena on the host (bookkeeping tests): plain tensor copies
    view = st[:, :, seq, :, arena_row0:arena_row0 + rows]
    pv = page[:, :, :, page_row0:page_row0 + rows]
    (pv.copy_(view) if to_page else view.copy_(pv))


class ArenaPages:
    def __init__(self, pin: bool = True):
        self.pin = pin
        self.rows_copied_out = 0
        self.rows_copied_in = 0

    def new_page(self, arena: RelationArena, rows: int = PAGE) -> torch.Tensor:
        shape = (arena.n_layers, 2, arena.n_heads, int(rows), arena.d_head)
        pin = self.pin and arena.device.type == "cuda"
        return torch.empty(shape, dtype=arena.dtype, device="cpu", pin_memory=pin)

    def store_rows(self, branch: Branch, arena: RelationArena, c0: int, c1: int, seq: int = 0) -> None:
        """Append arena rows [c0, c1) of sequence `seq` to the branch (c0 == branch.n_chunks);
        returns once the rows are on the host."""
        if c0 != branch.n_chunks:
            raise ValueError(f"store_rows appends at row {branch.n_chunks}, not {c0}")
        c = c0
        while c < c1:
            pi, off = divmod(c, PAGE)
            take = min(PAGE - off, c1 - c)
            need = off + take
            if pi == len(branch.pages):
                branch.pages.append(self.new_page(arena, self._tail_rows(need)))
            elif branch.pages[pi].shape[3] < need:  # the tail outgrew its rows: double it (at most PAGE)
                grown = self.new_page(arena, self._tail_rows(need, branch.pages[pi].shape[3]))
                grown[:, :, :, :off].copy_(branch.pages[pi][:, :, :, :off])
                branch.pages[pi] = grown
            _copy_rows(arena, seq, c, branch.pages[pi], off, take, to_page=True)
            c += take
        if arena.device.type == "cuda" and c1 > c0:
            torch.cuda.current_stream(arena.device).synchronize()  # the pages are complete on return
        self.rows_copied_out += max(c1 - c0, 0)
        branch.n_chunks = max(branch.n_chunks, c1)

    @staticmethod
    def _tail_rows(need: int, have: int = 0) -> int:
        rows = max(have, 16)
        while rows < need:
            rows *= 2
        return min(rows, PAGE)

    def hydrate(self, branch: Branch, n_chunks: int, arena: RelationArena, seq: int = 0) -> None:
        """Make arena rows [0, n_chunks) of sequence `seq` hold the branch's chunks; returns once
        the rows are in the arena, so the branch's pages may be freed or reused right after. A
        batch-1 arena that already holds the branch is left alone (the hot case: no copy). Growing
        a batched arena keeps every other slot's rows (the arena carries them across growth)."""
        if n_chunks > branch.n_chunks:
            raise ValueError(f"the branch holds {branch.n_chunks} rows, not {n_chunks}")
        if arena.batch == 1 and arena.owner == branch.id and arena.n_valid >= n_chunks:
            arena.claim(branch.id, n_chunks)
            return
        if arena.batch == 1:
            arena.invalidate()  # nothing of the old owner is worth carrying across a growth
        arena.ensure(n_chunks)
        c = 0
        while c < n_chunks:
            pi, off = divmod(c, PAGE)
            take = min(PAGE - off, n_chunks - c)
            _copy_rows(arena, seq, c, branch.pages[pi], off, take, to_page=False)
            c += take
        if arena.device.type == "cuda" and n_chunks > 0:
            # the DMA reads pinned pages that torch's caching host allocator does not know are in
            # use: wait for it, so a page freed after return cannot be handed out while still read
            torch.cuda.current_stream(arena.device).synchronize()
        if arena.batch == 1:
            arena.claim(branch.id, n_chunks)
        self.rows_copied_in += n_chunks

    def fork(self, parent: Branch, at_chunks: int) -> Branch:
        """A new branch holding the parent's first `at_chunks` rows: its full pages shared, the
        partial page copied (prefix_cache.py:169-176)."""
        if at_chunks > parent.n_chunks:
            raise ValueError(f"fork at {at_chunks} rows of a branch holding {parent.n_chunks}")
        nb = Branch()
        full, rem = divmod(at_chunks, PAGE)
        nb.pages = list(parent.pages[:full])
        if rem:
            src = parent.pages[full]
            tail = torch.empty((*src.shape[:3], rem, src.shape[4]), dtype=src.dtype, pin_memory=src.is_pinned())
            tail.copy_(src[:, :, :, :rem])
            nb.pages.append(tail)
        nb.n_chunks = at_chunks
        return nb

    @staticmethod
    def nbytes(branches: List[Branch]) -> int:
        """Host bytes of the branches' pages, shared pages counted once."""
        seen = {}
        for b in branches:
            for p in b.pages:
                seen[id(p)] = p.numel() * p.element_size()
        return sum(seen.values())
