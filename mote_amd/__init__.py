"""mote_amd — Mote's Relation mixer on MI355X (gfx950): hand-written HIP kernels behind Mote's
`mote.model.flash_relation` / `mote.model.relation` call signatures.

Modules: `flash_relation` (fused core, custom ops), `relation` (FullRelation and its RoPE/Givens
prologue), `arena` (the {P2, I~} decode cache), `decode` (the one-chunk decode step),
`determinism`, `config` (preset shapes). The kernels live in `lib/libmote_relation.so`, built by
`python -m mote_amd.build`.
"""

__version__ = "0.1.0"
