"""CPU restatement of Butterfly compressed attention (test infrastructure).

One-shot prefill and active rows follow the reference Torch path
(``bna/torch/attention_wayfinder_permute.py:912-1197``): routing tables ->
gather raw window + routed summaries -> concatenate -> one
``F.scaled_dot_product_attention`` with a boolean mask.  The from-cache entry and
the stream helpers follow the MLX semantics (``bna/mlx/attention.py:304-548``,
``1601-1876``), restated in torch fp32.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

NEG = -1e30   # empty-stream max sentinel, bna/mlx/attention.py:38
EPS = 1e-9    # merge/normaliser floor, bna/mlx/attention.py:39


# --------------------------------------------------------------------------- routing tables
def prefill_tables(layout, *, T: int, W: int):
    """Block-level routing for one-shot prefill.

    attention_wayfinder_permute.py:912-966.  Returns raw_idx [N, W+BS-1],
    raw_mask [N, BS, W+BS-1], summary_idx [N, K], summary_mask [N, BS, K].
    """
    if T <= 0 or W <= 0:
        raise ValueError("T and W must be positive")
    bs, n = layout.block_size, layout.num_blocks
    slots = W + bs - 1
    k = layout.block_neighbors.shape[-1]
    nbr = layout.block_neighbors[0]
    off = torch.arange(slots)
    qoff = torch.arange(bs)
    raw_idx = torch.zeros((n, slots), dtype=torch.long)
    raw_mask = torch.zeros((n, bs, slots), dtype=torch.bool)
    sidx = torch.zeros((n, k), dtype=torch.long)
    smask = torch.zeros((n, bs, k), dtype=torch.bool)
    for b in range(n):
        qpos = b * bs + qoff
        qok = qpos < T
        start = max(0, b * bs - W + 1)          # block-level cut-off
        rpos = start + off
        raw_idx[b] = rpos.clamp(0, max(0, T - 1))
        raw_mask[b] = (qok[:, None] & (rpos < T)[None, :] & (rpos[None, :] <= qpos[:, None])
                       & (rpos[None, :] >= qpos[:, None] - W + 1))
        c = 0
        for nb in nbr[b].tolist():
            if nb < 0 or nb >= b or (nb + 1) * bs > start:
                continue
            sidx[b, c] = nb
            smask[b, :, c] = qok
            c += 1
            if c >= k:
                break
    return raw_idx, raw_mask, sidx, smask


def active_tables(layout, *, kv_len: int, query_positions, W: int):
    """Token-level routing for active rows.  attention_wayfinder_permute.py:969-1019."""
    if kv_len <= 0 or W <= 0:
        raise ValueError("kv_len and W must be positive")
    qp = torch.as_tensor(query_positions).long().view(-1)
    bs, n = layout.block_size, layout.num_blocks
    k = layout.block_neighbors.shape[-1]
    nbr = layout.block_neighbors[0]
    off = torch.arange(W)
    raw_idx = torch.zeros((qp.numel(), W), dtype=torch.long)
    raw_mask = torch.zeros((qp.numel(), W), dtype=torch.bool)
    sidx = torch.zeros((qp.numel(), k), dtype=torch.long)
    smask = torch.zeros((qp.numel(), k), dtype=torch.bool)
    for r, p in enumerate(qp.tolist()):
        b = min(max(0, p // max(1, bs)), max(0, n - 1))
        start = max(0, p - W + 1)               # token-level cut-off
        rpos = start + off
        raw_idx[r] = rpos.clamp(0, max(0, kv_len - 1))
        raw_mask[r] = (rpos <= p) & (rpos < kv_len)
        c = 0
        for nb in nbr[b].tolist():
            if nb < 0 or nb >= b or (nb + 1) * bs > start:
                continue
            sidx[r, c] = nb
            smask[r, c] = True
            c += 1
            if c >= k:
                break
    return raw_idx, raw_mask, sidx, smask


def active_tables_from_tail(layout, *, kv_len: int, tail_start: int, num_summary_blocks: int, tail_len: int,
                            query_positions, W: int):
    """Tail-relative active routing.  bna/mlx/attention.py:1601-1666.

    Pinned by tests/test_oracle_attention.py: reduces to ``active_tables`` (itself
    pinned by the reference-written golden tables) for a tail holding the whole
    context with every block pooled, and equals a per-query enumeration over all
    tokens and blocks on tiny layouts; planted off-by-one variants fail both.
    """
    if int(kv_len) <= 0:
        raise ValueError("kv_len must be positive")
    if torch.as_tensor(query_positions).dim() != 1:
        raise ValueError("query_positions must be 1D")
    qp = torch.as_tensor(query_positions).long().view(-1)
    bs, n = layout.block_size, layout.num_blocks
    k = layout.block_neighbors.shape[-1]
    nbr = layout.block_neighbors[0]
    off = torch.arange(W)
    tail_end = tail_start + tail_len
    raw_idx = torch.zeros((qp.numel(), W), dtype=torch.long)
    raw_mask = torch.zeros((qp.numel(), W), dtype=torch.bool)
    sidx = torch.zeros((qp.numel(), k), dtype=torch.long)
    smask = torch.zeros((qp.numel(), k), dtype=torch.bool)
    for r, p in enumerate(qp.tolist()):
        b = min(max(0, p // max(1, bs)), max(0, n - 1))
        start = max(0, p - W + 1)
        rpos = start + off
        raw_mask[r] = (rpos <= p) & (rpos < kv_len) & (rpos >= tail_start) & (rpos < tail_end)
        raw_idx[r] = (rpos - tail_start).clamp(0, max(0, tail_len - 1))
        c = 0
        for nb in nbr[b].tolist():
            if nb < 0 or nb >= b or nb >= num_summary_blocks or (nb + 1) * bs > start:
                continue
            sidx[r, c] = nb
            smask[r, c] = True
            c += 1
            if c >= k:
                break
    return raw_idx, raw_mask, sidx, smask


# --------------------------------------------------------------------------- compressor
def block_mean(x: torch.Tensor, *, seq_len: int, block_size: int, num_blocks: int) -> torch.Tensor:
    """Mean of the valid tokens of every block, fp32 accumulate, cast back.

    attention_wayfinder_permute.py:1022-1043.
    """
    b, h, t, d = x.shape
    if t != seq_len:
        raise ValueError("seq_len mismatch")
    pad = num_blocks * block_size - seq_len
    xw = F.pad(x, (0, 0, 0, pad)) if pad > 0 else x
    blocks = xw.view(b, h, num_blocks, block_size, d)
    pos = torch.arange(num_blocks * block_size).view(num_blocks, block_size)
    valid = (pos < seq_len).to(torch.float32)
    denom = valid.sum(dim=1, keepdim=True).clamp_min(1.0)
    total = (blocks.float() * valid.view(1, 1, num_blocks, block_size, 1)).sum(dim=3)
    return (total / denom.view(1, 1, num_blocks, 1)).to(x.dtype)


# --------------------------------------------------------------------------- one-shot prefill
def prefill(q, k, v, *, layout, W: int, block_chunk_size: int = 0, k_summary=None, v_summary=None):
    """One-shot compressed prefill.  attention_wayfinder_permute.py:1046-1122.

    ``k_summary``/``v_summary`` optionally replace the block means computed from k/v (a
    float32 evaluation over bf16 inputs then keeps the bf16 summaries that path pools)."""
    b, hq, t, d = q.shape
    hkv = k.shape[1]
    if k.shape[2] != t or v.shape[2] != t:
        raise ValueError("prefill requires matching q/k/v lengths")
    bs, n = layout.block_size, layout.num_blocks
    raw_idx, raw_mask, sidx, smask = prefill_tables(layout, T=t, W=W)
    slots, ks = raw_idx.shape[-1], sidx.shape[-1]
    ksum = block_mean(k, seq_len=t, block_size=bs, num_blocks=n) if k_summary is None else k_summary
    vsum = block_mean(v, seq_len=t, block_size=bs, num_blocks=n) if v_summary is None else v_summary
    pad = n * bs - t
    qb = (F.pad(q, (0, 0, 0, pad)) if pad > 0 else q).view(b, hq, n, bs, d)
    c = n if block_chunk_size <= 0 else min(block_chunk_size, n)
    pieces = []
    for s0 in range(0, n, c):
        s1 = min(s0 + c, n)
        m = s1 - s0
        qc = qb[:, :, s0:s1].permute(0, 2, 1, 3, 4).reshape(b * m, hq, bs, d)
        ri = raw_idx[s0:s1]
        kr = k[:, :, ri].permute(0, 2, 1, 3, 4).reshape(b * m, hkv, slots, d)
        vr = v[:, :, ri].permute(0, 2, 1, 3, 4).reshape(b * m, hkv, slots, d)
        si = sidx[s0:s1]
        kk = ksum[:, :, si].permute(0, 2, 1, 3, 4).reshape(b * m, hkv, ks, d)
        vv = vsum[:, :, si].permute(0, 2, 1, 3, 4).reshape(b * m, hkv, ks, d)
        mask = torch.cat([raw_mask[s0:s1], smask[s0:s1]], dim=2)
        mask = mask.unsqueeze(0).expand(b, m, bs, slots + ks).reshape(b * m, 1, bs, slots + ks)
        y = F.scaled_dot_product_attention(qc, torch.cat([kr, kk], 2), torch.cat([vr, vv], 2),
                                           attn_mask=mask, enable_gqa=hkv < hq)
        pieces.append(y.view(b, m, hq, bs, d))
    out = torch.cat(pieces, 1).permute(0, 2, 1, 3, 4).reshape(b, hq, n * bs, d)
    return out[:, :, :t] if pad > 0 else out


# --------------------------------------------------------------------------- active rows
def active(q, k, v, *, layout, query_positions, W: int, k_summary=None, v_summary=None):
    """Active (cached) rows, token-level cut-off.  attention_wayfinder_permute.py:1125-1197.

    ``k_summary``/``v_summary`` optionally replace the full-context recompute
    (the MLX active entry's ``precomputed_*_summary``, bna/mlx/attention.py:1531-1541).
    """
    b, hq, tq, d = q.shape
    hkv, tk = k.shape[1], k.shape[2]
    raw_idx, raw_mask, sidx, smask = active_tables(layout, kv_len=tk, query_positions=query_positions, W=W)
    slots, ks = raw_idx.shape[-1], sidx.shape[-1]
    if k_summary is None:
        k_summary = block_mean(k, seq_len=tk, block_size=layout.block_size, num_blocks=layout.num_blocks)
        v_summary = block_mean(v, seq_len=tk, block_size=layout.block_size, num_blocks=layout.num_blocks)
    kr = k[:, :, raw_idx].permute(0, 2, 1, 3, 4).reshape(b * tq, hkv, slots, d)
    vr = v[:, :, raw_idx].permute(0, 2, 1, 3, 4).reshape(b * tq, hkv, slots, d)
    kk = k_summary[:, :, sidx].permute(0, 2, 1, 3, 4).reshape(b * tq, hkv, ks, d)
    vv = v_summary[:, :, sidx].permute(0, 2, 1, 3, 4).reshape(b * tq, hkv, ks, d)
    qr = q.permute(0, 2, 1, 3).reshape(b * tq, hq, 1, d)
    mask = torch.cat([raw_mask, smask], 1).unsqueeze(0).expand(b, tq, slots + ks).reshape(b * tq, 1, 1, slots + ks)
    y = F.scaled_dot_product_attention(qr, torch.cat([kr, kk], 2), torch.cat([vr, vv], 2),
                                       attn_mask=mask, enable_gqa=hkv < hq)
    return y.reshape(b, tq, hq, d).permute(0, 2, 1, 3).contiguous()


# --------------------------------------------------------------------------- streams + merge (MLX semantics)
def _stream(scores: torch.Tensor, mask: torch.Tensor, vals: torch.Tensor):
    """(o, l, m) of one masked stream in fp32; empty rows give (0, 0, NEG)."""
    s = torch.where(mask, scores, torch.full_like(scores, NEG))
    m = s.amax(-1, keepdim=True)
    e = torch.where(mask, torch.exp(s - m), torch.zeros_like(s))
    l = e.sum(-1, keepdim=True)
    if vals.dim() == e.dim() + 1:       # per-row gathered values [..., tq, K, d]
        o = (e.unsqueeze(-1) * vals).sum(-2)
    else:                               # shared values [..., nk, d]
        o = e @ vals
    o = o / torch.clamp(l, min=EPS)
    anyv = mask.any(-1, keepdim=True)
    o = torch.where(anyv, o, torch.zeros_like(o))
    l = torch.where(anyv, l, torch.zeros_like(l))
    m = torch.where(anyv, m, torch.full_like(m, NEG))
    return o, l, m


def merge(a, b):
    """Online log-sum-exp merge of two (o, l, m) streams.  bna/mlx/attention.py:519-548."""
    oa, la, ma = a
    ob, lb, mb = b
    mt = torch.maximum(ma, mb)
    ca, cb = torch.exp(ma - mt), torch.exp(mb - mt)
    lt = ca * la + cb * lb
    return (ca * la * oa + cb * lb * ob) / torch.clamp(lt, min=EPS)


def swa_stream(q, k, v, *, W: int, scale: float):
    """Sliding-window stream over raw keys.  bna/mlx/attention.py:304-369 (fp32, unchunked).

    Returns (o in q's dtype, l fp32 [B,H,T,1], m fp32 [B,H,T,1]); q, k, v share heads.
    """
    t = q.shape[2]
    pos = torch.arange(t)
    mask = (pos[None, :] <= pos[:, None]) & (pos[None, :] > pos[:, None] - max(1, W))
    s = (q.float() @ k.float().transpose(-1, -2)) * scale
    o, l, m = _stream(s, mask.view(1, 1, t, t), v.float())
    return o.to(q.dtype), l, m


def compressed_stream(q, k_summary, v_summary, *, block_size: int, scale: float, routed_indices=None):
    """Compressed-block stream.  bna/mlx/attention.py:372-516.

    HCA mode (``routed_indices is None``, :411-439): the query at position t of
    block b = t // block_size attends to every summary n < b.  Routed mode
    (:441-516): it attends to ``routed_indices[h, b, j]`` for the entries with
    0 <= idx < b (idx >= num_summaries is treated as invalid; the reference
    gathers such an index out of range).  Rows with nothing to attend give
    (0, 0, -1e30).  Returns (o in q's dtype, l fp32, m fp32); q and the summaries
    share heads.
    """
    b, h, t, d = q.shape
    nb = k_summary.shape[2]
    qblk = torch.arange(t) // int(block_size)
    if routed_indices is None:
        s = (q.float() @ k_summary.float().transpose(-1, -2)) * scale          # [B, H, T, nb]
        valid = torch.arange(nb)[None, :] < qblk[:, None]                     # [T, nb]
        o, l, m = _stream(s, valid.view(1, 1, t, nb), v_summary.float())
        return o.to(q.dtype), l, m
    ri = torch.as_tensor(routed_indices).long()                               # [H, NQB, K]
    if ri.shape[0] != h or ri.shape[1] < int(qblk[-1]) + 1 if t else False:
        raise ValueError("routed_indices must be [H, >= num query blocks, K]")
    idx = ri[:, qblk, :]                                                       # [H, T, K]
    valid = (idx >= 0) & (idx < qblk.view(1, t, 1)) & (idx < nb)
    safe = torch.where(valid, idx, torch.zeros_like(idx))
    heads = torch.arange(h).view(h, 1, 1)
    kg = k_summary.float()[:, heads, safe]                                     # [B, H, T, K, d]
    vg = v_summary.float()[:, heads, safe]
    s = (q.float().unsqueeze(-2) * kg).sum(-1) * scale                         # [B, H, T, K]
    o, l, m = _stream(s, valid.unsqueeze(0), vg)
    return o.to(q.dtype), l, m


def from_cache(q, tail_k, tail_v, k_summary, v_summary, *, layout, query_positions, W: int,
               tail_start: int, kv_len: int, scale: float | None = None):
    """Cache-aware two-stream entry.  bna/mlx/attention.py:1669-1876, in torch fp32.

    ``q`` and the cache tensors share heads (the caller GQA-broadcasts, as
    bna/integrations/qwen_mlx.py:1520-1523 does).
    """
    b, h, tq, d = q.shape
    sc = float(scale if scale is not None else d ** -0.5)
    qp = torch.as_tensor(query_positions).long().view(-1)
    ntail = tail_k.shape[2]
    kabs = tail_start + torch.arange(ntail)
    mask = (kabs[None, :] <= qp[:, None]) & (kabs[None, :] > qp[:, None] - W)
    s = (q.float() @ tail_k.float().transpose(-1, -2)) * sc
    swa = _stream(s, mask.view(1, 1, tq, ntail), tail_v.float())
    # compressed stream: per query, routed summaries older than the window and already pooled
    bs = layout.block_size
    k_slots = layout.block_neighbors.shape[-1]
    nsum = k_summary.shape[2]
    nbr = layout.block_neighbors[0]
    idx = torch.full((tq, k_slots), -1, dtype=torch.long)
    for r, p in enumerate(qp.tolist()):
        blk = p // bs
        if blk < 0 or blk >= nbr.shape[0]:
            continue
        start = max(0, p - W + 1)
        c = 0
        for nb in nbr[blk].tolist():
            if nb < 0 or nb >= blk or (nb + 1) * bs > start or nb >= nsum:
                continue
            idx[r, c] = nb
            c += 1
            if c >= k_slots:
                break
    valid = idx >= 0
    safe = torch.where(valid, idx, torch.zeros_like(idx))
    if nsum == 0:
        kg = torch.zeros((b, h, tq, k_slots, d))
        vg = torch.zeros((b, h, tq, k_slots, d))
    else:
        kg = k_summary.float()[:, :, safe]      # [b, h, tq, K, d]
        vg = v_summary.float()[:, :, safe]
    s2 = (q.float().unsqueeze(-2) * kg).sum(-1) * sc
    cmp = _stream(s2, valid.view(1, 1, tq, k_slots), vg)
    return merge(swa, cmp).to(tail_v.dtype)


def dense_union_attention(q, keys, vals, *, scale: float):
    """Plain softmax over an explicit key list (fp64), used to pin the merge."""
    s = (keys.double() @ q.double()) * scale
    w = torch.softmax(s, 0)
    return w @ vals.double()


def default_scale(d: int) -> float:
    return 1.0 / math.sqrt(d)
