"""Per-query numpy brute force (test infrastructure).

Restates the reference tests' independent oracle
``_reference_compressed`` (``tests/pytorch/test_compressed_butterfly_attention.py:20-85``):
for every (batch, head, query) it enumerates the raw window and the eligible
routed summaries explicitly and takes one softmax in float64.  Block-level
cut-off when ``query_positions`` is None (one-shot prefill), token-level
otherwise.  Heads of ``q`` map to kv heads by ``h // (Hq // Hkv)``.
"""
from __future__ import annotations

import math

import numpy as np


def block_summaries(x: np.ndarray, block_size: int) -> np.ndarray:
    b, h, t, d = x.shape
    n = math.ceil(t / block_size)
    out = np.zeros((b, h, n, d), dtype=np.float64)
    for i in range(n):
        out[:, :, i] = x[:, :, i * block_size: min(t, (i + 1) * block_size)].astype(np.float64).mean(axis=2)
    return out


def compressed_reference(q, k, v, neighbors, *, block_size: int, W: int, query_positions=None,
                         k_summary=None, v_summary=None, scale=None):
    """``neighbors`` is the [N, K] block-neighbour table (-1 padded)."""
    b_, hq, tq, d = q.shape
    hkv, tk = k.shape[1], k.shape[2]
    g = hq // hkv
    ks = block_summaries(k, block_size) if k_summary is None else np.asarray(k_summary, np.float64)
    vs = block_summaries(v, block_size) if v_summary is None else np.asarray(v_summary, np.float64)
    sc = (1.0 / math.sqrt(d)) if scale is None else scale
    pos = np.arange(tq) if query_positions is None else np.asarray(query_positions)
    out = np.zeros((b_, hq, tq, d), dtype=np.float64)
    for bi in range(b_):
        for h in range(hq):
            hk = h // g
            for qi, p in enumerate(pos.tolist()):
                blk = p // block_size
                cut = max(0, blk * block_size - W + 1) if query_positions is None else max(0, p - W + 1)
                lo = max(0, p - W + 1)
                keys = [k[bi, hk, t].astype(np.float64) for t in range(lo, min(tk, p + 1))]
                vals = [v[bi, hk, t].astype(np.float64) for t in range(lo, min(tk, p + 1))]
                for nb in neighbors[blk].tolist():
                    if nb < 0 or nb >= blk or (nb + 1) * block_size > cut:
                        continue
                    keys.append(ks[bi, hk, nb])
                    vals.append(vs[bi, hk, nb])
                if not keys:
                    continue
                kk, vv = np.stack(keys), np.stack(vals)
                s = kk @ q[bi, h, qi].astype(np.float64) * sc
                s = np.exp(s - s.max())
                out[bi, h, qi] = (s / max(s.sum(), 1e-9)) @ vv
    return out
