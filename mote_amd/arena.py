"""The Relation decode arena: one preallocated, append-only home for every layer's {P2, I~} rows.

Same contract as mote/model/arena.py:30-186. `buf[layer, 0]` holds P2 rows and `buf[layer, 1]` I~
rows, [H, capacity, dh] each (the reference layout, batch 1), or [batch, H, capacity, dh] when the
arena is built for `batch` independent sequences (batched decode, which the reference defers,
docs/shape.md:255). Per layer the rows of one head are contiguous and heads are capacity*dh apart,
which is the head stride the HIP kernels read in place.

The buffer is allocated zeroed and grows zeroed (arena.py:38-44): rows past the fill are never read
by the HIP decode kernel, but the reference's bucket-width readers multiply masked rows, so they must
stay finite.
"""

from __future__ import annotations

import contextlib
from typing import Iterator, Optional

import torch


class RelationArena:
    def __init__(self, n_layers: int, n_heads: int, capacity: int, d_head: int, device, dtype, batch: int = 1):
        self.n_layers, self.n_heads, self.d_head = n_layers, n_heads, d_head
        self.batch = int(batch)
        self.capacity = int(capacity)
        self.device = torch.device(device)
        self.dtype = dtype
        self.buf = torch.zeros(self._shape(self.capacity), device=self.device, dtype=dtype)
        self.owner: Optional[int] = None
        self.n_valid: int = 0
        self.generation: int = 0
        self.pool = None

    def _shape(self, cap: int):
        if self.batch == 1:
            return (self.n_layers, 2, self.n_heads, cap, self.d_head)
        return (self.n_layers, 2, self.batch, self.n_heads, cap, self.d_head)

    @staticmethod
    def capacity_for(seq_len: int, bpic: float, bucket: int = 256, margin: float = 1.25) -> int:
        """Rows a `seq_len`-byte context needs at `bpic` bytes per chunk, with `margin` headroom,
        rounded up to the decode bucket (arena.py:54-62)."""
        need = int(seq_len / max(float(bpic), 1e-6) * float(margin)) + 1
        return max(-(-need // bucket) * bucket, bucket)

    @property
    def bytes_per_chunk(self) -> int:
        return self.n_layers * 2 * self.batch * self.n_heads * self.d_head * self.buf.element_size()

    def nbytes(self) -> int:
        return self.buf.numel() * self.buf.element_size()

    def p2(self, layer: int) -> torch.Tensor:
        """[batch, H, capacity, dh] view of a layer's P2 rows."""
        t = self.buf[layer, 0]
        return t.unsqueeze(0) if self.batch == 1 else t

    def info(self, layer: int) -> torch.Tensor:
        t = self.buf[layer, 1]
        return t.unsqueeze(0) if self.batch == 1 else t

    def rows(self, c0: int, c1: int) -> torch.Tensor:
        """All layers' rows [c0, c1) as a view."""
        return self.buf[..., c0:c1, :]

    def ensure(self, n_chunks: int) -> bool:
        """Grow (x2, at least n_chunks) when needed, keeping the owned rows (arena.py:81-115).
        Returns True when a reallocation happened (captured graphs must be recaptured)."""
        if n_chunks <= self.capacity:
            return False
        new_cap = self.capacity
        while new_cap < n_chunks:
            new_cap *= 2
        ctx = torch.cuda.use_mem_pool(self.pool) if (self.pool is not None and self.device.type == "cuda") else contextlib.nullcontext()
        keep = self.n_valid if self.owner is not None else 0
        old = self.buf
        if keep == 0:
            self.buf = old = None
        with ctx:
            buf = torch.zeros(self._shape(new_cap), device=self.device, dtype=self.dtype)
        if old is not None:
            buf[..., :keep, :].copy_(old[..., :keep, :])
        else:
            self.owner, self.n_valid = None, 0
        self.buf = buf
        self.capacity = new_cap
        self.generation += 1
        return True

    def invalidate(self) -> None:
        self.owner, self.n_valid = None, 0


class ArenaLayer:
    """One layer's rows and the shared fill `n` (arena.py:121-143)."""

    __slots__ = ("arena", "layer", "state")

    def __init__(self, arena: RelationArena, layer: int, state: "ArenaState"):
        self.arena, self.layer, self.state = arena, layer, state

    @property
    def n(self) -> int:
        return self.state.n

    def write(self, p2: torch.Tensor, info: torch.Tensor) -> None:
        """Append T rows at [n, n+T); the caller advances `n` once every layer has written."""
        T = p2.shape[2]
        n = self.state.n
        assert n + T <= self.arena.capacity, f"arena overflow: {n + T} > {self.arena.capacity}"
        self.arena.p2(self.layer)[:, :, n : n + T].copy_(p2)
        self.arena.info(self.layer)[:, :, n : n + T].copy_(info)

    def views(self, upto: int):
        """(P2, I~) over rows [0, upto) as [batch, H, upto, dh] views."""
        return self.arena.p2(self.layer)[:, :, :upto], self.arena.info(self.layer)[:, :, :upto]


def _map(obj, fn):
    if torch.is_tensor(obj):
        return fn(obj)
    if isinstance(obj, (list, tuple)):
        return type(obj)(_map(o, fn) for o in obj)
    if isinstance(obj, dict):
        return {k: _map(v, fn) for k, v in obj.items()}
    return obj


class ArenaState:
    """The main-network half of an inference state: the shared arena and this sequence's fill `n`
    (arena.py:146-186). Copying it copies `n`, never the arena; recurrent states of non-Relation
    main layers ride along in `mamba` and are copied."""

    __slots__ = ("arena", "n", "mamba")

    def __init__(self, arena: RelationArena, n: int = 0, mamba: Optional[dict] = None):
        self.arena, self.n = arena, int(n)
        self.mamba = dict(mamba) if mamba else {}

    def __len__(self) -> int:
        return self.arena.n_layers

    def __getitem__(self, layer: int):
        if layer in self.mamba:
            return self.mamba[layer]
        return ArenaLayer(self.arena, layer, self)

    def set(self, layer: int, state) -> None:
        if layer in self.mamba:
            self.mamba[layer] = state

    def map(self, fn) -> "ArenaState":
        return ArenaState(self.arena, self.n, {k: _map(v, fn) for k, v in self.mamba.items()})

    def __iter__(self) -> Iterator[ArenaLayer]:
        return (self[i] for i in range(len(self)))

    def copy(self) -> "ArenaState":
        return self.map(lambda t: t.clone()) if self.mamba else ArenaState(self.arena, self.n)

    def advance(self, T: int) -> None:
        self.n += int(T)
