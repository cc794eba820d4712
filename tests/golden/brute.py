"""Scalar float64 brute force of paged / varlen attention, written with plain
Python loops and math.exp (no torch matmul or softmax), used to pin the
oracle on small inputs.  Same definitions as the oracle's docstrings:
kv head of query head h is h // (Hq / Hkv); masked keys are excluded; a
query with no visible key yields 0."""

from __future__ import annotations

import math


def attend(qrow, keys, values, scale, keep=None):
    """softmax(scale * q . k_j) weighted sum of v_j over kept j (lists of floats)."""
    idx = [j for j in range(len(keys)) if keep is None or keep[j]]
    if not idx:
        return [0.0] * len(qrow)
    scores = {j: scale * sum(a * b for a, b in zip(qrow, keys[j])) for j in idx}
    top = max(scores.values())
    weights = {j: math.exp(s - top) for j, s in scores.items()}
    total = sum(weights.values())
    out = [0.0] * len(values[0])
    for j in idx:
        w = weights[j] / total
        for d, x in enumerate(values[j]):
            out[d] += w * x
    return out


def paged_decode(q, k_pool, v_pool, table, lens, scale, layout="nhd", valid=None):
    """q: nested [B][Hq][D]; pools nested 4-D lists; returns [B][Hq][D]."""
    out = []
    for b, qb in enumerate(q):
        hq = len(qb)
        if layout == "nhd":
            bs, hkv = len(k_pool[0]), len(k_pool[0][0])
        else:
            hkv, bs = len(k_pool[0]), len(k_pool[0][0])
        group = hq // hkv
        rows = []
        for h in range(hq):
            kvh = h // group
            keys, values, keep = [], [], []
            for t in range(int(lens[b])):
                page, off = int(table[b][t // bs]), t % bs
                if layout == "nhd":
                    keys.append(k_pool[page][off][kvh])
                    values.append(v_pool[page][off][kvh])
                else:
                    keys.append(k_pool[page][kvh][off])
                    values.append(v_pool[page][kvh][off])
                keep.append(True if valid is None or t >= len(valid[b]) else bool(valid[b][t]))
            rows.append(attend(qb[h], keys, values, scale, keep))
        out.append(rows)
    return out


def varlen(q, k, v, cu_q, cu_k, scale, causal):
    """Packed varlen without a pool: q [Tq][Hq][D], k/v [Tk][Hkv][D]."""
    out = [None] * len(q)
    for s in range(len(cu_q) - 1):
        q0, q1, k0, k1 = cu_q[s], cu_q[s + 1], cu_k[s], cu_k[s + 1]
        ql, kl = q1 - q0, k1 - k0
        for i in range(ql):
            hq = len(q[q0 + i])
            group = hq // len(k[k0]) if kl else 1
            row = []
            for h in range(hq):
                keys = [k[k0 + j][h // group] for j in range(kl)]
                values = [v[k0 + j][h // group] for j in range(kl)]
                keep = [(not causal) or j <= kl - ql + i for j in range(kl)]
                row.append(attend(q[q0 + i][h], keys, values, scale, keep))
            out[q0 + i] = row
    return out
