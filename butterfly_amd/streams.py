"""Stream-level compressed attention: the two streams and their online-softmax merge.

The reference builds its one-shot entry from three helpers
(bna/mlx/attention.py:1455-1467): a sliding-window stream over raw keys
(``_swa_stream_attention``, :304-369), a compressed-block stream over block
summaries (``_compressed_stream_attention``, :372-516) and the merge of the two
(``_online_softmax_merge``, :519-548).  This module exposes the same three
operations on HIP kernels (``bfly_swa_stream``, ``bfly_compressed_stream``,
``bfly_softmax_merge``), including the compressed stream's HCA mode
(``routed_indices=None``: every query attends densely to all earlier block
summaries), which no fused entry point takes.

Each stream returns ``(o, l, m)``: ``o`` in the query dtype, ``l`` (sum of
``exp(score - m)``) and ``m`` (row max) in fp32 with shape ``[B, H, T, 1]``.  A
row with nothing to attend returns ``(0, 0, -1e30)``, which merges as a no-op.
Query heads may be a multiple of the key heads (head ``h`` reads key head
``h // (Hq / Hkv)``); the reference requires equal heads, which is the special
case ``Hq == Hkv``.  The underscore names are aliases for drop-in use.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native
from .attention import _c, _check_heads, _dtype_code, _on, _require_cuda, _stream

Stream = Tuple[torch.Tensor, torch.Tensor, torch.Tensor]
NEG = -1e30


def _outputs(q: torch.Tensor):
    b, h, t, d = q.shape
    o = torch.empty_like(q)
    l = torch.empty((b, h, t, 1), dtype=torch.float32, device=q.device)
    m = torch.empty((b, h, t, 1), dtype=torch.float32, device=q.device)
    return o, l, m


def _empty(q: torch.Tensor) -> Stream:
    b, h, t, _ = q.shape
    return (torch.zeros_like(q), torch.zeros((b, h, t, 1), dtype=torch.float32, device=q.device),
            torch.full((b, h, t, 1), NEG, dtype=torch.float32, device=q.device))


def swa_stream_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, n_win: int, scale: float,
                         q_chunk: int = 256) -> Stream:
    """Sliding-window stream: query ``t`` attends to keys ``[max(0, t - n_win + 1), t]``.

    bna/mlx/attention.py:304-369.  ``q_chunk`` is accepted for signature
    compatibility (the kernel needs no chunking).
    """
    del q_chunk
    _require_cuda(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or tuple(k.shape) != tuple(v.shape):
        raise ValueError("q, k, v must be [B, H, T, d] with k and v of equal shape")
    b, hq, t, d = q.shape
    bk, hk, tk, dk = k.shape
    if bk != b or tk != t or dk != d:
        raise ValueError("q, k, v batch/length/head_dim mismatch")
    _check_heads(hq, hk)
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v dtype mismatch")
    if t == 0:
        return _empty(q)
    q, k, v = _c(q), _c(k), _c(v)
    o, l, m = _outputs(q)
    with _on(q.device):
        _native.call("bfly_swa_stream", q.data_ptr(), k.data_ptr(), v.data_ptr(), _dtype_code(q), b, hq, hk, t, d,
                     max(1, int(n_win)), float(scale), o.data_ptr(), l.data_ptr(), m.data_ptr(), _stream(q))
    return o, l, m


def compressed_stream_attention(q: torch.Tensor, k_summary: torch.Tensor, v_summary: torch.Tensor, *,
                                block_size: int, scale: float,
                                routed_indices: Optional[torch.Tensor] = None) -> Stream:
    """Compressed-block stream.  bna/mlx/attention.py:372-516.

    ``routed_indices is None`` (HCA mode): query ``t`` in block ``b = t // block_size``
    attends to every summary ``n < b``.  Otherwise ``routed_indices`` is int
    ``[H, num_query_blocks, K]`` (``-1`` = no entry) and the query attends to the
    entries ``0 <= idx < b``; an index past the last summary counts as no entry.
    """
    _require_cuda(q, k_summary, v_summary)
    if q.dim() != 4 or k_summary.dim() != 4 or tuple(k_summary.shape) != tuple(v_summary.shape):
        raise ValueError("q and the summaries must be [B, H, T|N, d] with equal summary shapes")
    b, hq, t, d = q.shape
    bk, hk, nsum, dk = k_summary.shape
    if bk != b or dk != d:
        raise ValueError("q and summary batch/head_dim mismatch")
    _check_heads(hq, hk)
    if not (q.dtype == k_summary.dtype == v_summary.dtype):
        raise ValueError("q and summary dtype mismatch")
    if int(block_size) <= 0:
        raise ValueError("block_size must be positive")
    if t == 0:
        return _empty(q)
    q, ks, vs = _c(q), _c(k_summary), _c(v_summary)
    routed, rblocks, kcap = None, 0, 0
    if routed_indices is not None:
        ri = torch.as_tensor(routed_indices)
        if ri.dim() != 3 or ri.shape[0] != hq:
            raise ValueError(f"routed_indices must be [H={hq}, num_blocks, K], got {tuple(ri.shape)}")
        nqb = (t + int(block_size) - 1) // int(block_size)
        if ri.shape[1] < nqb:
            raise ValueError(f"routed_indices cover {ri.shape[1]} query blocks, the queries span {nqb}")
        if ri.shape[2] == 0:
            return _empty(q)
        routed = ri.to(device=q.device, dtype=torch.int32).contiguous()
        rblocks, kcap = int(ri.shape[1]), int(ri.shape[2])
    o, l, m = _outputs(q)
    with _on(q.device):
        _native.call("bfly_compressed_stream", q.data_ptr(), ks.data_ptr(), vs.data_ptr(), _dtype_code(q), b, hq, hk,
                     t, d, nsum, int(block_size), routed.data_ptr() if routed is not None else None, rblocks, kcap,
                     float(scale), o.data_ptr(), l.data_ptr(), m.data_ptr(), _stream(q))
    return o, l, m


def online_softmax_merge(a: Stream, b: Stream) -> torch.Tensor:
    """Softmax over the union of two streams' keys from their ``(o, l, m)``.

    bna/mlx/attention.py:519-548; the result is fp32 ``[B, H, Tq, d]``.
    """
    oa, la, ma = a
    ob, lb, mb = b
    _require_cuda(oa, ob)
    if tuple(oa.shape) != tuple(ob.shape) or oa.dim() != 4:
        raise ValueError("stream outputs must share one [B, H, Tq, d] shape")
    bsz, h, t, d = oa.shape
    rows = bsz * h * t
    stats = [_c(x.to(device=oa.device, dtype=torch.float32)).reshape(-1) for x in (la, ma, lb, mb)]
    if any(x.numel() != rows for x in stats):
        raise ValueError("l and m must hold one value per row [B, H, Tq, 1]")
    oa_c, ob_c = _c(oa), _c(ob)
    out = torch.empty((bsz, h, t, d), dtype=torch.float32, device=oa.device)
    if rows == 0:
        return out
    with _on(oa.device):
        _native.call("bfly_softmax_merge", oa_c.data_ptr(), _dtype_code(oa_c), stats[0].data_ptr(),
                     stats[1].data_ptr(), ob_c.data_ptr(), _dtype_code(ob_c), stats[2].data_ptr(),
                     stats[3].data_ptr(), rows, d, out.data_ptr(), _stream(oa))
    return out


_swa_stream_attention = swa_stream_attention
_compressed_stream_attention = compressed_stream_attention
_online_softmax_merge = online_softmax_merge
