"""Compressed Butterfly attention operators (PyTorch-ROCm host, HIP kernels).

Same names, arguments and error behaviour as the reference's operator surface:

* MLX names (return ``(out, None)``): ``compressed_butterfly_attention``
  (bna/mlx/attention.py:1401-1468), ``compressed_butterfly_attention_active``
  (:1471-1598), ``compressed_butterfly_attention_from_cache`` (:1816-1876).
* Torch names (return ``out``): ``butterfly_compressed_attention``
  (bna/torch/attention_wayfinder_permute.py:1046-1122),
  ``butterfly_compressed_attention_active`` (:1125-1197).

Inputs are CUDA (HIP) tensors in [B, H, T, d] layout, float32 or bfloat16.
Query heads may outnumber kv heads (GQA: head h reads kv head h // (Hq/Hkv));
the MLX entries' callers broadcast kv heads first, which is also accepted.
Every call runs on the current torch stream; nothing here falls back to CPU.
"""
from __future__ import annotations

import math
import os
import time
from typing import Any, Dict, Optional

import torch

from . import _native
from ._device import on, stream_of


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _native.DTYPE_F32
    if t.dtype == torch.bfloat16:
        return _native.DTYPE_BF16
    raise ValueError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16")


def _stream(t: torch.Tensor) -> int:
    """Handle of the current stream of t's device (the launch stream of every call)."""
    return stream_of(t)


_on = on


def _require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError("butterfly_amd operators take GPU tensors (device 'cuda')")


def _c(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned base (the C ABI's requirement)."""
    if t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


def _check_heads(hq: int, hkv: int) -> None:
    if hkv <= 0 or hq % hkv != 0:
        raise ValueError(f"query heads {hq} must be a multiple of kv heads {hkv}")


def _scale(scale: Optional[float], d: int) -> float:
    return float(scale) if scale is not None else 1.0 / math.sqrt(d)


# --------------------------------------------------------------------------- profile counters
# With BNA_COMPRESS_PROFILE=1 in the environment (read at import), every compressor call and
# every active-row attention waits for its stream and adds its wall time here, and the
# compressor records the shapes it pooled.  Reference: bna/mlx/attention.py:45-79 (counters,
# reset, dump) and 1561-1595 (attention time of the active entry).
_COMPRESS_PROFILE = os.environ.get("BNA_COMPRESS_PROFILE", "0") == "1"
_compress_stats: Dict[str, Any] = {"calls": 0, "summary_ms": 0.0, "attn_ms": 0.0, "shapes": []}


def _compress_profile_reset() -> None:
    _compress_stats["calls"] = 0
    _compress_stats["summary_ms"] = 0.0
    _compress_stats["attn_ms"] = 0.0
    _compress_stats["shapes"] = []


def _compress_profile_dump() -> Dict[str, Any]:
    return dict(_compress_stats)


# --------------------------------------------------------------------------- compressor
def block_mean_summaries(x: torch.Tensor, *, seq_len: int, block_size: int, num_blocks: int,
                         x2: Optional[torch.Tensor] = None):
    """Mean-pool every block of ``block_size`` tokens (fp32 accumulate, cast back).

    Reference: _block_mean_summaries_torch (attention_wayfinder_permute.py:1022-1043).
    With ``x2`` both tensors are pooled in one launch and a pair is returned.
    """
    _require_cuda(x)
    b, h, t, d = x.shape
    if int(t) != int(seq_len):
        raise ValueError(f"summary seq_len mismatch: x has T={t}, expected {seq_len}")
    x = _c(x)
    out = torch.empty((b, h, int(num_blocks), d), dtype=x.dtype, device=x.device)
    out2 = None
    if x2 is not None:
        if x2.shape != x.shape or x2.dtype != x.dtype:
            raise ValueError("x2 must match x in shape and dtype")
        x2 = _c(x2)
        out2 = torch.empty_like(out)
    t0 = time.perf_counter() if _COMPRESS_PROFILE else 0.0
    with _on(x.device):
        _native.call("bfly_block_mean", x.data_ptr(), out.data_ptr(),
                     x2.data_ptr() if x2 is not None else None, out2.data_ptr() if out2 is not None else None,
                     _dtype_code(x), b * h, int(t), d, int(block_size), int(num_blocks), _stream(x))
        if _COMPRESS_PROFILE:
            # one launch pools both tensors; each counts as a call, as the reference pools them in two
            torch.cuda.current_stream(x.device).synchronize()
            _compress_stats["summary_ms"] += (time.perf_counter() - t0) * 1000.0
            for xx in (x, x2) if x2 is not None else (x,):
                _compress_stats["calls"] += 1
                _compress_stats["shapes"].append({"seq_len": int(seq_len), "block_size": int(block_size),
                                                  "num_blocks": int(num_blocks), "x_shape": list(xx.shape),
                                                  "x_dtype": str(xx.dtype)})
    return (out, out2) if x2 is not None else out


# --------------------------------------------------------------------------- routing tables
def compressed_butterfly_block_index_tensors(layout, *, T: int, local_window_tokens: int):
    """One-shot routing tables (raw_idx, raw_mask, summary_idx, summary_mask) on the GPU.

    Reference: _compressed_butterfly_block_index_tensors
    (attention_wayfinder_permute.py:912-966).  Index tensors are int32, masks bool.
    """
    if int(T) <= 0:
        raise ValueError("T must be positive")
    if int(local_window_tokens) <= 0:
        raise ValueError("local_window_tokens must be positive")
    nb, bs = layout.table.exact(), layout.block_size      # the reference's [N, K] width
    n, k = nb.shape
    slots = int(local_window_tokens) + bs - 1
    dev = nb.device
    raw_idx = torch.empty((n, slots), dtype=torch.int32, device=dev)
    raw_mask = torch.empty((n, bs, slots), dtype=torch.uint8, device=dev)
    sidx = torch.empty((n, k), dtype=torch.int32, device=dev)
    smask = torch.empty((n, bs, k), dtype=torch.uint8, device=dev)
    with _on(dev):
        _native.call("bfly_prefill_tables", nb.data_ptr(), n, k, bs, int(T), int(local_window_tokens),
                     raw_idx.data_ptr(), raw_mask.data_ptr(), sidx.data_ptr(), smask.data_ptr(), _stream(nb))
    return raw_idx, raw_mask.bool(), sidx, smask.bool()


def compressed_butterfly_active_index_tensors(layout, *, kv_len: int, query_positions, local_window_tokens: int,
                                              tail_start: Optional[int] = None, tail_len: Optional[int] = None,
                                              num_summary_blocks: Optional[int] = None):
    """Active-row routing tables on the GPU.

    Reference: _compressed_butterfly_active_index_tensors
    (attention_wayfinder_permute.py:969-1019); with ``tail_start``/``tail_len``
    given, _compressed_butterfly_active_indices_from_tail (bna/mlx/attention.py:1601-1666).
    """
    nb, bs = layout.table.exact(), layout.block_size      # the reference's [N, K] width
    n, k = nb.shape
    dev = nb.device
    qp = torch.as_tensor(query_positions).to(device=dev, dtype=torch.int32).view(-1).contiguous()
    tq, w = qp.numel(), int(local_window_tokens)
    raw_idx = torch.empty((tq, w), dtype=torch.int32, device=dev)
    raw_mask = torch.empty((tq, w), dtype=torch.uint8, device=dev)
    sidx = torch.empty((tq, k), dtype=torch.int32, device=dev)
    smask = torch.empty((tq, k), dtype=torch.uint8, device=dev)
    tail = tail_len is not None
    with _on(dev):
        _native.call("bfly_active_tables", nb.data_ptr(), n, k, bs, int(kv_len), w, qp.data_ptr(), tq,
                     int(tail_start or 0), int(tail_len) if tail else -1,
                     int(num_summary_blocks) if num_summary_blocks is not None else n,
                     raw_idx.data_ptr(), raw_mask.data_ptr(), sidx.data_ptr(), smask.data_ptr(), _stream(nb))
    return raw_idx, raw_mask.bool(), sidx, smask.bool()


# --------------------------------------------------------------------------- one-shot prefill
def compressed_butterfly_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, layout,
                                   local_window_tokens: int, return_weights: bool = False,
                                   block_chunk_size: int = 0, scale: Optional[float] = None):
    """One-shot compressed Butterfly prefill: SWA stream + routed summaries, one softmax.

    ``block_chunk_size`` is accepted for signature compatibility (the reference
    no longer uses it either).  Returns ``(out, None)``.
    """
    del block_chunk_size
    if return_weights:
        raise NotImplementedError("return_weights is not supported for compressed Butterfly attention")
    _require_cuda(q, k, v)
    b, hq, t, d = q.shape
    bk, hk, tk, dk = k.shape
    if tuple(v.shape) != tuple(k.shape) or bk != b:
        raise ValueError("q, k, v batch/shape mismatch")
    if tk != t:
        raise ValueError("Compressed Butterfly prefill requires k/v length to match q length")
    if dk != d:
        raise ValueError("q, k, v head_dim mismatch")
    _check_heads(hq, hk)
    if int(layout.seq_len) != int(t):
        raise ValueError(f"layout.seq_len={layout.seq_len} must match q length {t}")
    if int(local_window_tokens) <= 0:
        raise ValueError("local_window_tokens must be positive")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v dtype mismatch")
    q, k, v = _c(q), _c(k), _c(v)
    n, bs = layout.num_blocks, layout.block_size
    ksum, vsum = block_mean_summaries(k, seq_len=t, block_size=bs, num_blocks=n, x2=v)
    out = torch.empty_like(q)
    nb = layout.neighbors
    with _on(q.device):
        _native.call("bfly_prefill", q.data_ptr(), k.data_ptr(), v.data_ptr(), ksum.data_ptr(), vsum.data_ptr(),
                     _dtype_code(q), b, hq, hk, t, d, nb.data_ptr(), n, nb.shape[1], bs,
                     int(local_window_tokens), _scale(scale, d), out.data_ptr(), _stream(q))
    return out, None


def butterfly_compressed_attention(q, k, v, *, layout, local_window_tokens: int, block_chunk_size: int = 0):
    """Torch-path name of the one-shot prefill (default scale 1/sqrt(d)); returns ``out``."""
    return compressed_butterfly_attention(q, k, v, layout=layout, local_window_tokens=local_window_tokens,
                                          block_chunk_size=block_chunk_size)[0]


# --------------------------------------------------------------------------- active rows / cache
def _positions(query_positions, tq: int, device):
    """(q_pos0, device_positions): a contiguous ascending range is passed as its
    start (the MFMA path); anything else as a device int32 array."""
    if isinstance(query_positions, torch.Tensor) and query_positions.is_cuda:
        return 0, query_positions.to(torch.int32).view(-1).contiguous()
    if isinstance(query_positions, range):
        qp = torch.tensor(list(query_positions), dtype=torch.int64)
    else:
        qp = torch.as_tensor(query_positions).to(torch.int64).view(-1)
    if qp.numel() != tq:
        raise ValueError(f"query_positions has {qp.numel()} entries, q has {tq} rows")
    if tq > 0 and bool((qp == qp[0] + torch.arange(tq)).all()):
        return int(qp[0]), None
    return 0, qp.to(device=device, dtype=torch.int32)


def _attend(q, tail_k, tail_v, pool_k, pool_v, *, layout, q_pos0, qpos_dev, ring_capacity, tail_start,
            kv_len, summary_count, local_window_tokens, scale):
    b, hq, tq, d = q.shape
    hk = tail_k.shape[1]
    out = torch.empty_like(q)
    nb = layout.neighbors
    if (tq == 1 and qpos_dev is None and int(q_pos0) == int(kv_len) - 1 and int(tail_start) < int(kv_len)
            and int(local_window_tokens) <= 64 and nb.shape[1] <= 16 and pool_k.shape[2] > 0
            and (d in (64, 128) or (d == 256 and q.dtype == torch.bfloat16))):
        # a single row at the newest position: the decode kernel
        with _on(q.device):
            _native.call("bfly_decode", q.data_ptr(), _dtype_code(q), b, hq, hk, d, None, None,
                         tail_k.data_ptr(), tail_v.data_ptr(), int(ring_capacity), int(tail_start), int(kv_len),
                         pool_k.data_ptr(), pool_v.data_ptr(), pool_k.shape[2], int(summary_count),
                         layout.table.topology, nb.shape[0], layout.block_size, int(local_window_tokens),
                         _scale(scale, d), out.data_ptr(), _stream(q))
        return out
    with _on(q.device):
        _native.call("bfly_attend_cache", q.data_ptr(), _dtype_code(q), b, hq, hk, tq, d,
                     qpos_dev.data_ptr() if qpos_dev is not None else None, int(q_pos0),
                     tail_k.data_ptr(), tail_v.data_ptr(), int(ring_capacity), int(tail_start), int(kv_len),
                     pool_k.data_ptr(), pool_v.data_ptr(), pool_k.shape[2], int(summary_count),
                     nb.data_ptr(), nb.shape[0], nb.shape[1], layout.block_size, int(local_window_tokens),
                     _scale(scale, d), out.data_ptr(), _stream(q))
    return out


def compressed_butterfly_attention_active(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, layout,
                                          query_positions, local_window_tokens: int, return_weights: bool = False,
                                          scale: Optional[float] = None,
                                          precomputed_k_summary: Optional[torch.Tensor] = None,
                                          precomputed_v_summary: Optional[torch.Tensor] = None,
                                          query_chunk_size: int = 0):
    """Active rows (token-level cut-off) over full K/V.  Returns ``(out, None)``.

    ``query_chunk_size`` is a memory knob in the reference; results do not depend on it.
    """
    del query_chunk_size
    if return_weights:
        raise NotImplementedError("return_weights is not supported by the HIP active path")
    _require_cuda(q, k, v)
    b, hq, tq, d = q.shape
    bk, hk, tk, dk = k.shape
    if bk != b or v.shape[0] != b:
        raise ValueError("q, k, v batch size mismatch")
    if v.shape[2] != tk:
        raise ValueError("k and v sequence length mismatch")
    if dk != d or v.shape[3] != d:
        raise ValueError("q, k, v head_dim mismatch")
    _check_heads(hq, hk)
    if int(tk) <= 0:
        raise ValueError("kv_len must be positive")
    if int(local_window_tokens) <= 0:
        raise ValueError("local_window_tokens must be positive")
    q, k, v = _c(q), _c(k), _c(v)
    n, bs = layout.num_blocks, layout.block_size
    if precomputed_k_summary is not None and precomputed_v_summary is not None:
        ksum, vsum = _c(precomputed_k_summary), _c(precomputed_v_summary)
        if ksum.shape[2] != n or vsum.shape[2] != n:
            raise ValueError(f"precomputed summary block count mismatch: expected {n}, "
                             f"got k={ksum.shape[2]}, v={vsum.shape[2]}")
    else:
        ksum, vsum = block_mean_summaries(k, seq_len=tk, block_size=bs, num_blocks=n, x2=v)
    q_pos0, qpos_dev = _positions(query_positions, tq, q.device)
    if qpos_dev is None and tq > 0 and (q_pos0 < 0 or q_pos0 + tq > tk):
        raise ValueError("query positions must lie in [0, kv_len)")
    t0 = time.perf_counter() if _COMPRESS_PROFILE else 0.0
    out = _attend(q, k, v, ksum, vsum, layout=layout, q_pos0=q_pos0, qpos_dev=qpos_dev, ring_capacity=0,
                  tail_start=0, kv_len=tk, summary_count=n, local_window_tokens=local_window_tokens, scale=scale)
    if _COMPRESS_PROFILE:
        torch.cuda.current_stream(q.device).synchronize()
        _compress_stats["attn_ms"] += (time.perf_counter() - t0) * 1000.0
    return out, None


def butterfly_compressed_attention_active(q, k, v, *, layout, query_positions, local_window_tokens: int):
    """Torch-path name of the active-row entry (default scale); returns ``out``."""
    return compressed_butterfly_attention_active(q, k, v, layout=layout, query_positions=query_positions,
                                                 local_window_tokens=local_window_tokens)[0]


def compressed_butterfly_attention_from_cache(q: torch.Tensor, tail_k: torch.Tensor, tail_v: torch.Tensor,
                                              k_summary: torch.Tensor, v_summary: torch.Tensor, *, layout,
                                              query_positions, local_window_tokens: int, tail_start: int,
                                              kv_len: int, return_weights: bool = False,
                                              scale: Optional[float] = None, query_chunk_size: int = 0):
    """Two-stream attention over a materialised tail + summary pool.  Returns ``(out, None)``.

    ``tail_k[:, :, i]`` holds absolute position ``tail_start + i``; summaries
    ``[0, k_summary.shape[2])`` are the completed blocks.
    """
    del query_chunk_size
    if return_weights:
        raise NotImplementedError("return_weights is not supported for compressed cache attention")
    _require_cuda(q, tail_k, tail_v, k_summary, v_summary)
    b, hq, tq, d = q.shape
    if tail_k.shape[0] != b or tail_v.shape[0] != b:
        raise ValueError("q and cache batch dimensions must match")
    if tail_k.shape[-1] != d or tail_v.shape[-1] != d:
        raise ValueError("q and cache head_dim mismatch")
    _check_heads(hq, tail_k.shape[1])
    if tail_v.shape != tail_k.shape or k_summary.shape != v_summary.shape:
        raise ValueError("k/v tensors must match")
    if int(tail_start) + tail_k.shape[2] != int(kv_len):
        raise ValueError("tail must end at kv_len")
    q_pos0, qpos_dev = _positions(query_positions, tq, q.device)
    if qpos_dev is None and tq > 0 and (q_pos0 < 0 or q_pos0 + tq > int(kv_len)):
        raise ValueError("query positions must lie in [0, kv_len)")
    tail_k, tail_v, k_summary, v_summary, q = _c(tail_k), _c(tail_v), _c(k_summary), _c(v_summary), _c(q)
    out = _attend(q, tail_k, tail_v, k_summary, v_summary, layout=layout, q_pos0=q_pos0, qpos_dev=qpos_dev,
                  ring_capacity=0, tail_start=int(tail_start), kv_len=int(kv_len),
                  summary_count=k_summary.shape[2], local_window_tokens=local_window_tokens, scale=scale)
    return out, None


def compressed_butterfly_attention_cached(q: torch.Tensor, cache, *, layout, local_window_tokens: int,
                                          scale: Optional[float] = None):
    """Active rows straight from a ``CompressedKVCache``'s device ring and pool.

    The queries are the last ``q.shape[2]`` positions of the cache (the
    integration's ``arange(T - q_len, T)``, bna/integrations/qwen_mlx.py:1515).
    No tail is materialised.
    """
    _require_cuda(q)
    st = cache.ring_state()
    tq = q.shape[2]
    return _attend(_c(q), st.ring_k, st.ring_v, st.pool_k, st.pool_v, layout=layout, q_pos0=st.offset - tq,
                   qpos_dev=None, ring_capacity=st.ring_capacity, tail_start=st.tail_start, kv_len=st.offset,
                   summary_count=st.summary_count, local_window_tokens=local_window_tokens, scale=scale)
