"""The {P2, I~} decode arena: every Relation layer's cache rows in one device allocation.

Interface of mote/model/arena.py:30-143 (RelationArena, ArenaLayer, ArenaState and the members
their callers touch); the storage and its management are this package's own.

Storage. One tensor `store` [n_layers, 2, batch, H, capacity, dh]: kind 0 holds P2 rows, kind 1
I~ rows, one slot per independent sequence (batched decode; the reference serves one sequence,
docs/shape.md:255). Within a (layer, kind, sequence) the rows of a head are contiguous and heads
are capacity * dh elements apart, the head stride the HIP forward and decode kernels take as an
argument, so nothing is ever gathered or transposed. `buf` is the store itself, or for batch 1 the
reference's [n_layers, 2, H, capacity, dh] view of it (same memory).

Rows at or past a sequence's fill are never read by the HIP kernels (they stop at S), but callers
that read a whole bucket width and mask (mote/infer/graph.py:176-184) multiply masked weights into
them, so the store is created and grown zeroed: stale values there are finite, never garbage.

Growth. `ensure(rows)` reallocates to the next power-of-two multiple of the current capacity and
bumps `generation` (captured graphs hold the old addresses and must be recaptured). In a batch-1
arena, rows are carried over only when a prefix store has declared them live (`owner` set, rows
[0, n_valid)); otherwise the old store is released before the new one is allocated, so the peak is
the new size alone. A batched arena has no per-slot residency record (decode advances each slot's
fill on the device), so its growth carries every slot's rows up to the old capacity. With `pool`
set (a `torch.cuda.MemPool`), the new store is allocated inside that pool.
"""

from __future__ import annotations

import contextlib
import dataclasses
from typing import Any, Callable, Iterator, Optional, Tuple

import torch


class RelationArena:
    """Cache rows of `n_layers` Relation layers for `batch` sequences (see the module docstring)."""

    def __init__(self, n_layers: int, n_heads: int, capacity: int, d_head: int, device, dtype, batch: int = 1):
        if capacity <= 0 or batch <= 0:
            raise ValueError("an arena needs a positive capacity and batch")
        self.n_layers, self.n_heads, self.d_head = int(n_layers), int(n_heads), int(d_head)
        self.batch = int(batch)
        self.device = torch.device(device)
        self.dtype = dtype
        self.generation = 0
        self._resident: Tuple[Optional[int], int] = (None, 0)  # (prefix-store owner, live rows)
        self.pool = None  # a serving MemPool: growth allocates inside it (engine.py:327)
        self.store = self._zeros(int(capacity))

    # ---- sizing ---------------------------------------------------------------------------------
    @staticmethod
    def capacity_for(seq_len: int, bpic: float, bucket: int = 256, margin: float = 1.25) -> int:
        """Rows for a `seq_len`-byte context at `bpic` bytes per chunk: the expected chunk count
        with `margin` headroom plus one row, in whole decode buckets (at least one). The same
        numbers as arena.py:54-62, so an engine sizing from a checkpoint's bpic gets the same
        capacity."""
        expected = int(seq_len / max(float(bpic), 1e-6) * float(margin))
        buckets = max(1, (expected + bucket) // bucket)  # ceil((expected + 1) / bucket)
        return buckets * bucket

    @property
    def capacity(self) -> int:
        return self.store.shape[4]

    @property
    def bytes_per_chunk(self) -> int:
        """Bytes one more row costs across every layer, kind, sequence and head."""
        return self.n_layers * 2 * self.batch * self.n_heads * self.d_head * self.store.element_size()

    def nbytes(self) -> int:
        return self.store.numel() * self.store.element_size()

    def _zeros(self, capacity: int) -> torch.Tensor:
        shape = (self.n_layers, 2, self.batch, self.n_heads, capacity, self.d_head)
        return torch.zeros(shape, device=self.device, dtype=self.dtype)

    # ---- views ----------------------------------------------------------------------------------
    @property
    def buf(self) -> torch.Tensor:
        """The store; for batch 1 as the reference's [n_layers, 2, H, capacity, dh] view."""
        return self.store[:, :, 0] if self.batch == 1 else self.store

    def p2(self, layer: int) -> torch.Tensor:
        """[batch, H, capacity, dh] view of a layer's P2 rows."""
        return self.store[layer, 0]

    def info(self, layer: int) -> torch.Tensor:
        """[batch, H, capacity, dh] view of a layer's I~ rows."""
        return self.store[layer, 1]

    def rows(self, c0: int, c1: int) -> torch.Tensor:
        """Rows [c0, c1) of every layer, kind, sequence and head, as a view of `buf`'s layout."""
        return self.buf[..., c0:c1, :]

    # ---- residency (which prefix-store branch's rows are live) ----------------------------------
    @property
    def owner(self) -> Optional[int]:
        """The prefix-store branch whose rows [0, n_valid) the arena holds (None: nothing live).
        Assignable, as the prefix store does (prefix_cache.py:158, 167, 216)."""
        return self._resident[0]

    @owner.setter
    def owner(self, owner: Optional[int]) -> None:
        self._resident = (owner, self._resident[1])

    @property
    def n_valid(self) -> int:
        return self._resident[1]

    @n_valid.setter
    def n_valid(self, rows: int) -> None:
        rows = int(rows)
        if not 0 <= rows <= self.capacity:
            raise ValueError(f"n_valid of {rows} rows in an arena of {self.capacity}")
        self._resident = (self._resident[0], rows)

    def claim(self, owner: int, rows: int) -> None:
        """Declare rows [0, rows) live for prefix-store branch `owner` (kept across growth)."""
        if not 0 <= rows <= self.capacity:
            raise ValueError(f"claim of {rows} rows in an arena of {self.capacity}")
        self._resident = (owner, int(rows))

    def invalidate(self) -> None:
        """Nothing in the arena is live any more (a new conversation, a dropped branch)."""
        self._resident = (None, 0)

    # ---- growth ---------------------------------------------------------------------------------
    def ensure(self, n_chunks: int) -> bool:
        """Make room for `n_chunks` rows. Returns True when the store was reallocated."""
        if n_chunks <= self.capacity:
            return False
        factor = 1 << max(0, (int(n_chunks) - 1) // self.capacity).bit_length()
        self._reallocate(self.capacity * factor)
        return True

    def _allocation_scope(self):
        if self.pool is not None and self.device.type == "cuda":
            return torch.cuda.use_mem_pool(self.pool)
        return contextlib.nullcontext()

    def _reallocate(self, capacity: int) -> None:
        owner, live = self._resident
        if self.batch > 1:
            live = self.capacity  # no per-slot record: every slot's rows travel
        elif owner is None:
            live = 0
        if live == 0:
            self.store = None  # drop the old rows before the new allocation: the peak is the new size
            with self._allocation_scope():
                self.store = self._zeros(capacity)
            self._resident = (None, 0)
        else:
            with self._allocation_scope():
                fresh = self._zeros(capacity)
            fresh[..., :live, :].copy_(self.store[..., :live, :])
            self.store = fresh
        self.generation += 1


class ArenaLayer:
    """What one FullRelation layer sees (arena.py:121-143): its rows and the fill `n` shared by
    every layer of the sequence state."""

    __slots__ = ("arena", "layer", "state")

    def __init__(self, arena: RelationArena, layer: int, state: "ArenaState"):
        self.arena, self.layer, self.state = arena, layer, state

    @property
    def n(self) -> int:
        return self.state.n

    def write(self, p2: torch.Tensor, info: torch.Tensor) -> None:
        """Store T new rows [n, n + T) of every sequence; p2 / info are [batch, H, T, dh]. The state
        advances `n` once every layer has written."""
        n, T = self.state.n, p2.shape[2]
        if n + T > self.arena.capacity:
            raise RuntimeError(f"arena overflow: rows up to {n + T} in a capacity of {self.arena.capacity}")
        self.arena.p2(self.layer)[:, :, n : n + T].copy_(p2)
        self.arena.info(self.layer)[:, :, n : n + T].copy_(info)

    def views(self, upto: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """(P2, I~) rows [0, upto) as [batch, H, upto, dh] views (head stride capacity * dh)."""
        return self.arena.p2(self.layer)[:, :, :upto], self.arena.info(self.layer)[:, :, :upto]


def _map_tensors(o: Any, fn: Callable[[torch.Tensor], Any]) -> Any:
    """`o` rebuilt with `fn` applied to every tensor inside it (lists, tuples, named tuples and
    dataclasses are walked; None, numbers and strings kept; anything else deep-copied), the walk a
    recurrent layer's state needs when a whole inference state is moved or cloned
    (mote/model/tree.py:17-32 is the reference's)."""
    if isinstance(o, torch.Tensor):
        return fn(o)
    if isinstance(o, (list, tuple)):
        items = [_map_tensors(x, fn) for x in o]
        if isinstance(o, list):
            return items
        return type(o)(*items) if hasattr(o, "_fields") else tuple(items)
    if o is None or isinstance(o, (bool, int, float, str)):
        return o
    if dataclasses.is_dataclass(o) and not isinstance(o, type):
        return type(o)(**{f.name: _map_tensors(getattr(o, f.name), fn) for f in dataclasses.fields(o)})
    import copy

    return copy.deepcopy(o)


class ArenaState:
    """The main-network part of an inference state (arena.py:146-186): the shared arena, the number
    of rows `n` this state has written, and `mamba`, the recurrent states of a hybrid main network's
    non-Relation layers (layer index -> state; empty for a pure Relation main network). Indexing a
    Relation layer gives its ArenaLayer, a recurrent layer its stored state; `set` writes a recurrent
    layer's new state back. Copies share the arena and copy `n`; `map` / `copy` apply a function to /
    clone every tensor of the recurrent states."""

    __slots__ = ("arena", "n", "mamba")

    def __init__(self, arena: RelationArena, n: int = 0, mamba: Optional[dict] = None):
        self.arena, self.n = arena, int(n)
        self.mamba = dict(mamba) if mamba else {}

    def __len__(self) -> int:
        return self.arena.n_layers

    def __getitem__(self, layer: int):
        if layer in self.mamba:
            return self.mamba[layer]
        if not 0 <= layer < self.arena.n_layers:
            raise IndexError(layer)
        return ArenaLayer(self.arena, layer, self)

    def __iter__(self) -> Iterator[Any]:
        return (self[i] for i in range(self.arena.n_layers))

    def set(self, layer: int, state) -> None:
        """Store a recurrent layer's new state; Relation layers keep theirs in the arena, so a layer
        that is not in `mamba` is left alone."""
        if layer in self.mamba:
            self.mamba[layer] = state

    def map(self, fn: Callable[[torch.Tensor], Any]) -> "ArenaState":
        """A state sharing the arena, with `fn` applied to every tensor of the recurrent states."""
        return ArenaState(self.arena, self.n, {k: _map_tensors(v, fn) for k, v in self.mamba.items()})

    def copy(self) -> "ArenaState":
        return self.map(lambda t: t.clone())

    def advance(self, T: int) -> None:
        self.n += int(T)
