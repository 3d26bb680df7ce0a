"""The decode arena driven through the call sequences of the reference's callers, on the CPU.

Each test replays what one caller does with `mote/model/arena.py`'s objects:
* the inference state of a hybrid main network (mote/model/hnet.py:286-301 allocate + prefill,
  :366-368 moving / cloning a state, :419-424 one decode step);
* the prefix store's hydrate and commit (mote/infer/prefix_cache.py:155-167, 216), which assign the
  arena's residency record;
* the serving engine handing its MemPool to the arena (mote/infer/engine.py:327).
The "recurrent layer" below is a stand-in state (a named tuple of tensors) for the non-Relation
layers of a hybrid main network; the arena only stores it.
"""

from __future__ import annotations

import dataclasses
from typing import NamedTuple

import pytest
import torch

from mote_amd.arena import ArenaLayer, ArenaState, RelationArena
from mote_amd.prefix import ArenaPages, Branch


class RecState(NamedTuple):  # what a recurrent layer's allocate_inference_cache would return
    conv: torch.Tensor
    ssm: torch.Tensor


N_LAYERS, H, DH = 4, 2, 8
RECURRENT = (1, 3)  # layer pattern of a hybrid main network: 0, 2 Relation; 1, 3 recurrent


def _alloc_state(arena):
    """hnet.py:286-293: one recurrent state per non-Relation layer, handed to ArenaState."""
    mamba_main = {i: RecState(torch.zeros(1, 4), torch.zeros(1, 2, 3)) for i in RECURRENT}
    return ArenaState(arena, 0, mamba_main)


def _main_network(x, caches):
    """A stand-in main network over T new chunks: Relation layers append their rows to the arena
    (ArenaLayer.write), recurrent layers return an updated state (what return_caches gives)."""
    T = x.shape[1]
    new = []
    for i in range(len(caches)):
        c = caches[i]
        if isinstance(c, ArenaLayer):
            rows = torch.full((1, H, T, DH), float(10 * i + 1)) + torch.arange(T).view(1, 1, T, 1)
            c.write(rows, -rows)
            new.append(c)
        else:
            assert isinstance(c, RecState)
            new.append(RecState(c.conv + T, c.ssm + 1))
    return x, new


def _run_main(state, T):
    """hnet.py:295-301 (prefill) and :419-424 (one step): ensure, run, set recurrent states, advance."""
    state.main.arena.ensure(state.main.n + T)
    _, new_caches = _main_network(torch.zeros(1, T, 1), state.main)
    for i in state.main.mamba:
        state.main.set(i, new_caches[i])
    state.main.advance(T)


@dataclasses.dataclass
class InferenceState:  # the fields of hnet's state that matter here
    main: ArenaState
    decoder: torch.Tensor


def _map_state(state, fn):
    """hnet.py:366-368: rebuild the state with fn applied to every tensor; the arena is shared and
    only the ArenaState's count and recurrent tensors travel (o.map(fn))."""
    return InferenceState(main=state.main.map(fn), decoder=fn(state.decoder))


def test_hybrid_state_prefill_step_and_move():
    arena = RelationArena(N_LAYERS, H, 16, DH, "cpu", torch.float32)
    state = InferenceState(main=_alloc_state(arena), decoder=torch.zeros(3))
    assert set(state.main.mamba) == set(RECURRENT)
    assert isinstance(state.main[0], ArenaLayer) and isinstance(state.main[1], RecState)
    assert [type(x).__name__ for x in state.main] == ["ArenaLayer", "RecState", "ArenaLayer", "RecState"]

    _run_main(state, 5)  # prefill of 5 chunks
    assert state.main.n == 5
    assert float(state.main[1].conv[0, 0]) == 5.0 and float(state.main[3].ssm.sum()) == 6.0
    assert torch.equal(arena.buf[2, 0, :, :5, 0], (21.0 + torch.arange(5.0)).expand(H, 5))

    snapshot = _map_state(state, lambda t: t.clone())  # clone_state: a rollback point
    for _ in range(3):
        _run_main(state, 1)  # three decode steps
    assert state.main.n == 8 and float(state.main[1].conv[0, 0]) == 8.0
    # the snapshot kept its own recurrent tensors and count; the arena is the same object
    assert snapshot.main.n == 5 and float(snapshot.main[1].conv[0, 0]) == 5.0
    assert snapshot.main.arena is arena and snapshot.main[1] is not state.main[1]
    assert isinstance(snapshot.main[1], RecState)  # named tuples survive the walk

    moved = _map_state(state, lambda t: t.to(torch.float64))  # a dtype / device move
    assert moved.main[3].ssm.dtype == torch.float64 and moved.main.n == 8 and moved.main.arena is arena
    c = state.main.copy()
    c.set(1, RecState(torch.ones(1, 4), torch.ones(1, 2, 3)))
    c.set(0, "ignored")  # a Relation layer keeps its rows in the arena: set leaves it alone
    assert float(state.main[1].conv[0, 0]) == 8.0 and isinstance(c[0], ArenaLayer) and c.mamba.keys() == {1, 3}


def test_pure_relation_state_keeps_the_two_argument_form():
    arena = RelationArena(2, H, 16, DH, "cpu", torch.float32)
    st = ArenaState(arena, 3)
    assert st.mamba == {} and st.copy().n == 3 and st.map(lambda t: t).arena is arena
    with pytest.raises(IndexError):
        st[2]


def test_prefix_store_assigns_the_residency_record():
    """prefix_cache.py:155-167 (hydrate) and :216 (commit) read and assign owner / n_valid."""
    src = RelationArena(N_LAYERS, H, 512, DH, "cpu", torch.float32)
    src.store.copy_(torch.randn(src.store.shape, generator=torch.Generator().manual_seed(0)))
    pages = ArenaPages(pin=False)
    b = Branch()
    pages.store_rows(b, src, 0, 300)

    arena = RelationArena(N_LAYERS, H, 256, DH, "cpu", torch.float32)
    arena.owner, arena.n_valid = b.id, 120  # commit (prefix_cache.py:216)
    assert arena.owner == b.id and arena.n_valid == 120
    # hydrate's hot case (:157-159): the arena already holds the branch; only n_valid moves
    if arena.owner == b.id and arena.n_valid >= 100:
        arena.n_valid = 100
    assert arena.n_valid == 100 and arena.owner == b.id
    # growth keeps the owned rows [0, n_valid) (arena.py:102-109)
    arena.buf[..., :100, :] = 4.0
    assert arena.ensure(300) and arena.capacity == 512
    assert bool((arena.buf[..., :100, :] == 4.0).all()) and float(arena.buf[..., 100:, :].abs().sum()) == 0.0
    # the cold case through this package's pages, which ends in the same assignment
    pages.hydrate(b, 300, arena)
    assert (arena.owner, arena.n_valid) == (b.id, 300)
    assert torch.equal(arena.buf[..., :300, :], src.buf[..., :300, :])
    arena.owner = None  # a new conversation
    assert arena.ensure(513) and float(arena.buf.abs().sum()) == 0.0 and arena.n_valid == 0
    with pytest.raises(ValueError):
        arena.n_valid = arena.capacity + 1


def test_hydrating_one_slot_of_a_batched_arena_that_must_grow_keeps_the_others():
    src = RelationArena(2, H, 512, DH, "cpu", torch.float32)
    src.store.copy_(torch.randn(src.store.shape, generator=torch.Generator().manual_seed(1)))
    pages = ArenaPages(pin=False)
    b = Branch()
    pages.store_rows(b, src, 0, 300)

    arena = RelationArena(2, H, 256, DH, "cpu", torch.float32, batch=2)
    arena.store.copy_(torch.randn(arena.store.shape, generator=torch.Generator().manual_seed(2)))
    before = arena.store.clone()
    pages.hydrate(b, 300, arena, seq=1)  # the arena grows from 256 to 512 rows
    assert arena.capacity == 512 and arena.generation == 1
    assert torch.equal(arena.store[:, :, 0, :, :256], before[:, :, 0])  # slot 0 untouched
    assert float(arena.store[:, :, 0, :, 256:].abs().sum()) == 0.0
    assert torch.equal(arena.store[:, :, 1, :, :300], src.buf[..., :300, :])


def test_pool_is_an_attribute_the_engine_sets():
    """engine.py:327 assigns arena.pool; on a host arena it is ignored, as in the reference
    (arena.py:101). The GPU test of the pool is in tests/test_decode_engine_gpu.py."""
    arena = RelationArena(1, H, 8, DH, "cpu", torch.float32)
    assert arena.pool is None
    arena.pool = object()
    assert arena.ensure(9) and arena.capacity == 16
