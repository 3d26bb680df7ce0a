"""mote_amd — Mote's Relation mixer on MI355X (gfx950): hand-written HIP kernels behind Mote's
`mote.model.flash_relation` / `mote.model.relation` call signatures.

Modules: `flash_relation` (fused core, custom ops, `relation_reference`), `relation` (FullRelation,
its RoPE / Givens prologue and the torch-level RoPE helpers), `arena` (the {P2, I~} decode cache),
`decode` (the one-chunk decode step and the per-layer decode module), `determinism` (the
reproducible-backward switch), `norm` (fused add + RMSNorm), `dc` (chunk gather and EMA dechunk).
The kernels live in `lib/libmote_relation.so`, built by `python -m mote_amd.build`.
"""

__version__ = "0.2.0"
