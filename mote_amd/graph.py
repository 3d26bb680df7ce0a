"""The Relation part of the graph decoder's captured step, on the HIP path.

`RelationMainStep` is a drop-in for GraphDecoder._relation_step (mote/infer/graph.py:151-187):
called as `step(mixer, x, al, Cb, li)` for each Relation layer of the main network, with the
decoder's device position `S` and per-layer exchange-mass buffer (graph.py:186), it runs the layer's
projections, the one-launch decode kernel (RoPE / Givens at S, append at row S, the read of rows
[0, S]) and `_out`, and returns the layer's output.

The reference captures the main step under a CUDA-graph conditional node keyed on the router's
boundary bit (graph.py:44-57, 224-226), so bytes that close no chunk skip it on the device. HIP graphs
here have no conditional nodes; instead every launch of the step takes the bit as a predicate (`run`):
each workgroup reads it and leaves before any write when it is 0. The step's persistent effects (the
arena append, S += 1, the per-layer outputs and the exchange mass) all come from those predicated
launches, so one captured graph serves both branches and the bit still never reaches the host. Bytes
that skip the step cost one empty launch per kernel.

S advances inside the last layer's decode launch (under the predicate) instead of in a separate
`S.add_(1)` (graph.py:207), which would run unconditionally in a graph without conditional nodes.
The bucket width `Cb` of the reference (graph.py:430-433) is accepted and not needed: the kernel
reads exactly rows [0, S].
"""

from __future__ import annotations

from typing import Dict, Optional

import torch

from .arena import ArenaLayer, RelationArena
from .decode import RelationDecodeStep


class RelationMainStep:
    def __init__(self, arena: RelationArena, S: torch.Tensor, xm_dev: Optional[torch.Tensor] = None,
                 run: Optional[torch.Tensor] = None, advance: bool = True):
        """arena: the decode arena (one layer per Relation layer). S: the decoder's int64 device
        position (0-d or [batch]). xm_dev: optional fp32 [n_layers] (batch 1) or [n_layers, batch]
        buffer that receives each layer's exchange mass. run: optional device flag (bool / uint8, one
        element), the predicate of every launch. advance: the last layer's launch moves S on."""
        if S.dtype != torch.int64 or S.numel() != arena.batch or not S.is_contiguous():
            raise ValueError("S must be a contiguous int64 device tensor with one position per sequence")
        self.arena, self.S, self.xm_dev, self.run, self.advance = arena, S, xm_dev, run, advance
        self.steps: Dict[int, RelationDecodeStep] = {}

    def _step(self, mixer, li: int) -> RelationDecodeStep:
        st = self.steps.get(li)
        if st is None or st.mixer is not mixer:
            st = RelationDecodeStep(mixer, self.arena, li)
            self.steps[li] = st
        return st

    def sync_params(self) -> None:
        """Refresh every layer's parameter copies (after an optimiser step)."""
        for st in self.steps.values():
            st.sync_params()

    @torch.no_grad()
    def __call__(self, mixer, x: torch.Tensor, al: Optional[ArenaLayer] = None, Cb: Optional[int] = None,
                 li: Optional[int] = None) -> torch.Tensor:
        """FullRelation.forward for one new chunk at device position S (graph.py:151-187): x [B, 1, D]
        -> out [B, 1, D]. `li` is the layer's arena index (the ArenaLayer's, when only `al` is given)."""
        if li is None:
            if al is None:
                raise ValueError("RelationMainStep needs the layer index or its ArenaLayer")
            li = al.layer
        if al is not None and al.arena is not self.arena:
            raise ValueError("the ArenaLayer belongs to another arena")
        xm = None
        if self.xm_dev is not None:
            xm = self.xm_dev[li].reshape(-1)
            if xm.numel() != self.arena.batch or not xm.is_contiguous():
                raise ValueError("xm_dev must hold one contiguous fp32 row of batch elements per layer")
        last = li == self.arena.n_layers - 1
        out, _ = self._step(mixer, li)(x, self.S.reshape(-1), advance=self.advance and last, run=self.run, xm=xm)
        return out
