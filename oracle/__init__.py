"""CPU oracle for the Relation hot path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import this
package, and only as the checker (or, for `bench.py`, as the timed CPU baseline). Nothing under
`mote_amd/` imports it: the product path is the HIP library and fails loudly without it.

Contents (each function cites the reference file:line it restates; paths are relative to the
noahsabaj/mote source tree):

* `relation.py` — a pure-PyTorch CPU restatement of the Relation mixer:
  materialized core (`mote/model/flash_relation.py:666-682`, `mote/model/relation.py:240-268`),
  the online-softmax form and the analytic backward (`flash_relation.py:1-15, 100-183, 186-358`),
  RoPE (`relation.py:37-68`), Givens (`relation.py:160-174`), the module (`relation.py:97-268`)
  and the graph decode step (`mote/infer/graph.py:151-187`).
* `brute.py` — float64 scalar loops over (b, h, i, j) for tiny shapes, the independent pin for
  the materialized form.

How each function is pinned (closed forms, invariants, brute force, finite differences, planted
mistakes) is listed in the header of `relation.py`; none of them is "parity unpinned".
"""
