"""float64 scalar loops for the Relation core — TEST INFRASTRUCTURE (see the package header).

An independent restatement of the definition in mote/model/relation.py:3-9 (module docstring) and
mote/model/flash_relation.py:666-682: every score, every softmax and every weighted sum is an
explicit Python loop in double precision, so it shares no tensor code with `oracle.relation`.
Use it for shapes with B*H*T*T*D below ~1e6.
"""

from __future__ import annotations

import math

import numpy as np


def _sigmoid(x: float) -> float:
    if x >= 0:
        return 1.0 / (1.0 + math.exp(-x))
    e = math.exp(x)
    return e / (1.0 + e)


def relation_brute(p1, p2, info, lam: float, tau_s: float = 2.0, q_start: int = 0):
    """Y [B,H,TQ,D] and g [B,H,TQ] as float64 numpy arrays.

    For query i (absolute position q_start + i, 0-based) and key j <= i:
      U_ij = <p1_i, p2_j> / sqrt(D)
      R_ij = 1 / (1 + exp(-U_ii / tau_s))               if j == i  (Self)
      R_ij = U_ij / (1 + exp(-U_ij)) - lam * ln(i + 1)  if j <  i  (Exchange, count calibrated)
      F_i  = softmax over j <= i;  Y_i = sum_j F_ij I~_j;  g_i = sum_{j<i} F_ij.
    """
    q = np.asarray(p1, dtype=np.float64)
    k = np.asarray(p2, dtype=np.float64)
    v = np.asarray(info, dtype=np.float64)
    B, H, TQ, D = q.shape
    y = np.zeros((B, H, TQ, D))
    g = np.zeros((B, H, TQ))
    inv = 1.0 / math.sqrt(D)
    for b in range(B):
        for h in range(H):
            for i in range(TQ):
                ia = q_start + i
                r = []
                for j in range(ia + 1):
                    dot = 0.0
                    for d in range(D):
                        dot += q[b, h, i, d] * k[b, h, j, d]
                    u = dot * inv
                    if j == ia:
                        r.append(_sigmoid(u / tau_s))
                    else:
                        r.append(u * _sigmoid(u) - lam * math.log(ia + 1.0))
                top = max(r)
                e = [math.exp(x - top) for x in r]
                z = sum(e)
                for d in range(D):
                    acc = 0.0
                    for j in range(ia + 1):
                        acc += e[j] * v[b, h, j, d]
                    y[b, h, i, d] = acc / z
                g[b, h, i] = sum(e[:ia]) / z
    return y, g
