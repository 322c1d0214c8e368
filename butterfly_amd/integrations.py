"""Layer-swap surface for PyTorch decoders: compressed Butterfly attention.

Mirrors the reference's ``bna/integrations`` API for the compressed path:

* ``QwenButterflyConfig`` -- the config dataclass and its validation
  (bna/integrations/qwen_mlx.py:84-165).  Only ``path="block_sparse"`` with
  ``block_compression="mean"`` runs Butterfly kernels; anything else is refused
  with ``NotImplementedError``.
* ``ButterflyAttentionCore`` -- the attention dispatch of
  ``QwenButterflyAttention.__call__`` (qwen_mlx.py:1295-1592) after the
  projections: one-shot prefill when ``q_len == k_len``; the cache path
  (``update`` + from-cache attention over positions ``[T - q_len, T)``) when
  the layer has a ``CompressedKVCache`` and ``q_len < k_len``; the stock
  decode fallback (dense attention over the cached tail) when
  ``butterfly_decode_backend == "dense"`` and ``q_len <= 2``
  (qwen_mlx.py:1332-1338, 1273-1293).  The layout is rebuilt for the live
  ``kv_len`` each call (its stage follows ``ceil(kv_len / block_size)``).
  ``last_profile`` records the path and the fallback reason as the reference does.
* ``install_compressed_kv_caches`` (qwen_mlx.py:1795-1819) and
  ``swap_qwen_attention_with_butterfly`` (qwen_mlx.py:1822-1846).
* ``chunked_prefill`` -- the harness's chunked prefill of one layer
  (scripts/bench_qwen_consumer_mlx.py:567-757): the first chunk one-shot,
  later chunks through the cache.

Every attention call runs a HIP kernel of ``libbutterfly_amd.so``.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence

import torch

from .attention import _attend, _c, _on, compressed_butterfly_attention
from .compressed_cache import CompressedKVCache
from .layout import build_block_butterfly_layout

_RULES = {"xor", "bit_reversal", "benes", "causal_shift", "fixed_stride", "random"}


@dataclass
class QwenButterflyConfig:
    """Reference: bna/integrations/qwen_mlx.py:84-165 (field names and checks)."""

    path: str = "block_sparse"
    block_size: int = 128
    block_local_window_blocks: int = 1
    block_partner_count: int = 1
    block_sink_blocks: int = 1
    block_partner_rule: str = "causal_shift"
    block_compression: str = "mean"
    compressed_local_window_tokens: int = 64
    query_chunk_size: int = 64
    wayfinder_decode_backend: str = "active_permute"

    @property
    def butterfly_decode_backend(self) -> str:
        return self.wayfinder_decode_backend

    @butterfly_decode_backend.setter
    def butterfly_decode_backend(self, value: str) -> None:
        self.wayfinder_decode_backend = value

    def __post_init__(self) -> None:
        if self.path not in {"sparse", "permute", "block_sparse"}:
            raise ValueError(f"Unsupported Butterfly path: {self.path!r}")
        if int(self.block_size) <= 0:
            raise ValueError("block_size must be > 0")
        if int(self.block_local_window_blocks) < 0:
            raise ValueError("block_local_window_blocks must be >= 0")
        if int(self.block_partner_count) < 0:
            raise ValueError("block_partner_count must be >= 0")
        if int(self.block_sink_blocks) < 0:
            raise ValueError("block_sink_blocks must be >= 0")
        if self.block_partner_rule not in _RULES:
            raise ValueError(f"Unsupported block_partner_rule: {self.block_partner_rule!r}")
        if self.block_compression not in {"none", "mean"}:
            raise ValueError(f"Unsupported block_compression: {self.block_compression!r}")
        if int(self.compressed_local_window_tokens) <= 0:
            raise ValueError("compressed_local_window_tokens must be > 0")
        if self.wayfinder_decode_backend not in {"active_permute", "dense"}:
            raise ValueError(f"Unsupported butterfly_decode_backend: {self.wayfinder_decode_backend!r}")


@dataclass
class AttentionProfile:
    """Reference: bna/mlx/attention.py:144-162 (the fields the compressed path fills)."""

    graph_build_ms: float = 0.0
    attention_ms: float = 0.0
    total_ms: float = 0.0
    path: str = ""
    notes: Dict[str, Any] = field(default_factory=dict)


def _now_ms() -> float:
    return time.perf_counter() * 1e3


_DEVICE_STEP_NOTES = {"q_len": 1, "device_counters": True, "block_sparse_active_mode": True}


class ButterflyAttentionCore:
    """Compressed Butterfly attention of one layer, after the q/k/v projections.

    ``__call__(q, k, v, cache=None)``: q ``[B, Hq, q_len, d]``; k, v
    ``[B, Hkv, q_len, d]`` are this call's new keys/values (already
    position-encoded).  With a ``CompressedKVCache`` they are appended to it
    first, exactly as ``cache.update_and_fetch`` does in the reference.
    Returns ``[B, Hq, q_len, d]``.
    """

    def __init__(self, cfg: QwenButterflyConfig, layer_idx: int, *, scale: Optional[float] = None) -> None:
        if cfg.path != "block_sparse" or cfg.block_compression != "mean":
            raise NotImplementedError(
                "butterfly_amd implements the compressed Butterfly path "
                "(path='block_sparse', block_compression='mean') only")
        self.cfg = cfg
        self.layer_idx = int(layer_idx)
        self.scale = scale
        self._last: Any = None     # an AttentionProfile, or the raw fields it is built from on access

    @property
    def last_profile(self) -> Optional[AttentionProfile]:
        """Profile of the last call (reference: bna/mlx/attention.py:144-162), built on
        first access from the fields the call recorded (keeps the per-chunk path cheap)."""
        r = self._last
        if r is None or isinstance(r, AttentionProfile):
            return r
        t0, t1, graph_ms, path, notes, lay = r
        notes = dict(notes)
        if graph_ms is not None:
            notes["graph_ms"] = graph_ms
        if lay is not None:
            notes["stage_idx"] = lay.stage_idx
            notes["stage_count"] = lay.stage_count
        prof = AttentionProfile(graph_build_ms=float(graph_ms or 0.0), total_ms=t1 - t0, path=path, notes=notes)
        self._last = prof
        return prof

    @last_profile.setter
    def last_profile(self, value: Optional[AttentionProfile]) -> None:
        self._last = value

    def layout(self, kv_len: int, num_kv_heads: int, groups: int, device):
        c = self.cfg
        return build_block_butterfly_layout(
            seq_len=int(kv_len), block_size=int(c.block_size), num_key_value_heads=int(num_kv_heads),
            num_key_value_groups=int(groups), layer_idx=self.layer_idx,
            local_window_blocks=int(c.block_local_window_blocks), sink_count=int(c.block_sink_blocks),
            partner_count=int(c.block_partner_count), partner_rule=c.block_partner_rule, device=device)

    def fuses_qk_norm(self, cache, q_len: int, head_dim: int, dtype) -> bool:
        """Whether ``__call__`` takes ``qk_norm`` for this step: a device-counter decode step of
        bf16 rows with head_dim 128 that runs on the MFMA kernel (``bfly_decode_step_qk_norm``:
        positive scale, 32-bit positions and offsets)."""
        from .attention import _scale

        return (isinstance(cache, CompressedKVCache) and cache.device_counters is not None and q_len == 1
                and self.cfg.butterfly_decode_backend != "dense" and head_dim == 128 and dtype == torch.bfloat16
                and cache.step_on_mfma(head_dim, int(self.cfg.compressed_local_window_tokens),
                                       _scale(self.scale, head_dim), dtype))

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 cache: Optional[CompressedKVCache] = None, qk_norm=None) -> torch.Tensor:
        """``qk_norm`` (see ``CompressedKVCache.decode_step``) hands raw q/k projection rows to
        the decode step, which applies the q/k RMSNorm and RoPE itself; only where
        ``fuses_qk_norm`` holds."""
        t0 = _now_ms()
        b, hq, q_len, d = q.shape
        hkv = int(k.shape[1])
        if hq % hkv != 0:
            raise ValueError(f"query heads {hq} must be a multiple of kv heads {hkv}")
        groups = hq // hkv
        w = int(self.cfg.compressed_local_window_tokens)
        c = self.cfg
        if qk_norm is not None and not self.fuses_qk_norm(cache, q_len, d, q.dtype):
            raise ValueError("qk_norm is taken only by device-counter decode steps of bf16, head_dim 128 rows")
        if (cache is not None and cache.device_counters is not None and q_len == 1
                and c.butterfly_decode_backend != "dense"):
            # device counters: one fixed-argument launch, no host bookkeeping (graph-capturable)
            out = cache.decode_step(q, k, v, layer_idx=self.layer_idx, local_window_tokens=w,
                                    partner_rule=c.block_partner_rule, local_window_blocks=c.block_local_window_blocks,
                                    sink_count=c.block_sink_blocks, partner_count=c.block_partner_count,
                                    scale=self.scale, qk_norm=qk_norm)
            self._last = (t0, _now_ms(), None, "block_sparse_compressed_active", _DEVICE_STEP_NOTES, None)
            return out
        if cache is not None:
            cache.sync()
        k_len = q_len + (cache.offset if cache is not None else 0)
        notes: Dict[str, Any] = {"seq_len": int(k_len), "q_len": int(q_len)}
        graph_ms = None
        if cache is not None and q_len < k_len and q_len <= 2 and self.cfg.butterfly_decode_backend == "dense":
            # stock decode: dense attention over the trimmed tail only (qwen_mlx.py:1273-1293)
            cache.update(k, v)
            st = cache.ring_state()
            lay = self.layout(k_len, hkv, groups, q.device)
            out = _attend(_c(q), st.ring_k, st.ring_v, st.pool_k, st.pool_v, layout=lay, q_pos0=k_len - q_len,
                          qpos_dev=None, ring_capacity=st.ring_capacity, tail_start=st.tail_start,
                          kv_len=st.offset, summary_count=0, local_window_tokens=k_len - st.tail_start,
                          scale=self.scale)
            notes["dense_fallback_reason"] = "butterfly_decode_stock"
            path = "block_sparse_dense_fallback"
        elif cache is None or cache.offset == 0 and q_len == k_len:
            # one-shot prefill over this call's own tokens (q_len == k_len)
            tg = _now_ms()
            lay = self.layout(k_len, hkv, groups, q.device)
            graph_ms = _now_ms() - tg
            if cache is not None:
                cache.update(k, v)
            out, _ = compressed_butterfly_attention(q, k, v, layout=lay, local_window_tokens=w, scale=self.scale)
            path = "block_sparse_compressed"
        else:
            if not isinstance(cache, CompressedKVCache):
                raise TypeError("the active path needs a butterfly_amd.CompressedKVCache")
            tg = _now_ms()
            lay = self.layout(k_len, hkv, groups, q.device)
            graph_ms = _now_ms() - tg
            out = cache.update_and_attend(q, k, v, layout=lay, local_window_tokens=w, scale=self.scale)
            notes["block_sparse_active_mode"] = True
            path = "block_sparse_compressed_active"
        self._last = (t0, _now_ms(), graph_ms, path, notes, lay)
        return out


def install_compressed_kv_caches(model, prompt_cache: List[Any], *, layer_indices: Optional[Sequence[int]] = None,
                                 block_size: int = 128, local_window_tokens: int = 128,
                                 max_kv_size: Optional[int] = None, max_chunk_size: int = 512) -> List[int]:
    """Put a ``CompressedKVCache`` in ``prompt_cache[i]`` for the selected layers.

    Reference: bna/integrations/qwen_mlx.py:1795-1819.  ``layer_indices=None``
    selects every layer of ``model.layers``.
    """
    if not hasattr(model, "layers"):
        raise ValueError("Model has no .layers attribute")
    selected = range(len(model.layers)) if layer_indices is None else [int(x) for x in layer_indices]
    replaced: List[int] = []
    for idx in sorted(set(selected)):
        if idx < 0 or idx >= len(prompt_cache):
            continue
        prompt_cache[idx] = CompressedKVCache(block_size=int(block_size), local_window_tokens=int(local_window_tokens),
                                              max_kv_size=int(max_kv_size) if max_kv_size else None,
                                              max_chunk_size=int(max_chunk_size))
        replaced.append(idx)
    return replaced


def swap_qwen_attention_with_butterfly(model, *, cfg: QwenButterflyConfig,
                                       layer_indices: Optional[Sequence[int]] = None) -> List[int]:
    """Replace ``model.layers[i].self_attn`` by ``butterfly_module(self_attn, cfg, layer_idx=i)``.

    Reference: bna/integrations/qwen_mlx.py:1822-1846.  The layer's attention
    module must provide ``butterfly_module(cfg, layer_idx)`` returning its
    Butterfly replacement (the decoder in ``butterfly_amd.decoder`` does), the
    counterpart of ``QwenButterflyAttention(base_attn, cfg, layer_idx=i)``.
    """
    if not hasattr(model, "layers"):
        raise ValueError("Model has no .layers attribute")
    selected = None if layer_indices is None else {int(i) for i in layer_indices}
    replaced: List[int] = []
    for i, layer in enumerate(model.layers):
        if selected is not None and i not in selected:
            continue
        base = getattr(layer, "self_attn", None)
        if base is None:
            continue
        layer.self_attn = base.butterfly_module(cfg, layer_idx=i)
        replaced.append(i)
    return replaced


def split_chunks(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, chunk_size: int):
    """Contiguous per-chunk ``(q, k, v)`` along the sequence axis (what a model's
    projections of each prompt chunk produce)."""
    t = int(q.shape[2])
    return [(q[:, :, s:s + chunk_size].contiguous(), k[:, :, s:s + chunk_size].contiguous(),
             v[:, :, s:s + chunk_size].contiguous()) for s in range(0, t, int(chunk_size))]


def chunked_prefill(core: ButterflyAttentionCore, chunks, cache: CompressedKVCache) -> List[torch.Tensor]:
    """One layer's chunked prefill (the harness schedule); returns the per-chunk outputs.

    Reference: scripts/bench_qwen_consumer_mlx.py:567-757 (prompt fed in chunks,
    the cache updated per chunk) with the dispatch of qwen_mlx.py:1311-1318 and
    1515-1581: the first chunk is one-shot over its own tokens; each later
    chunk appends to the cache and attends from it with the layout of the live
    kv_len.  ``chunks`` yields contiguous ``(q, k, v)`` chunks in order.

    After the first chunk, runs of chunks go through ``bfly_stream_chunks`` (the same
    kernels and arguments, with the per-chunk bookkeeping in C++; a small first run
    so the GPU starts while the host prepares the next) whenever the configuration
    allows it; a chunk the loop does not cover goes through ``core``.
    """
    chunks = list(chunks)
    if not chunks:
        return []
    outs = [core(*chunks[0], cache)]
    i, native, run = 1, True, 8
    while i < len(chunks):
        got = _stream_chunks(core, chunks, i, run, cache) if native else None
        if got is None:
            native = native and _stream_possible(core, cache, chunks[i])
            outs.append(core(*chunks[i], cache))
            i += 1
            continue
        outs += got
        i += len(got)
        run = 64
    return outs


def _stream_possible(core: ButterflyAttentionCore, cache, chunk) -> bool:
    """False once the native loop cannot take any chunk of this call (cache mode or
    configuration); True when only this chunk's shape kept it out."""
    q = chunk[0]
    return (isinstance(cache, CompressedKVCache) and cache.device_counters is None and q.dtype == torch.bfloat16
            and int(q.shape[3]) in (64, 128, 256))


def _stream_chunks(core: ButterflyAttentionCore, chunks, start: int, run: int,
                   cache) -> Optional[List[torch.Tensor]]:
    """Outputs of up to ``run`` chunks from ``chunks[start]`` on, through one
    ``bfly_stream_chunks`` call (the cache already holds the first chunk), or None when
    ``chunks[start]`` must go through ``core``: a cache with device counters, a chunk of
    one or two tokens (the per-chunk path sends those to the decode kernel or, with the
    dense backend, to the stock fallback), or a configuration the loop does not cover."""
    import ctypes as C

    from . import _native
    from .attention import _dtype_code, _scale, _stream

    if not isinstance(cache, CompressedKVCache) or cache.device_counters is not None or cache.offset <= 0 \
            or cache._ring_k is None:
        return None
    q0, k0, _ = chunks[start]
    b, hq, _, d = (int(x) for x in q0.shape)
    hkv = int(k0.shape[1])
    qs, ks, vs = [], [], []
    for qc, kc, vc in chunks[start:start + run]:
        n = int(qc.shape[2])
        if (n <= 2 or tuple(qc.shape) != (b, hq, n, d) or tuple(kc.shape) != (b, hkv, n, d) or kc.shape != vc.shape
                or not (qc.dtype == kc.dtype == vc.dtype == torch.bfloat16) or not qc.is_cuda):
            break
        qs.append(_c(qc))
        ks.append(_c(kc))
        vs.append(_c(vc))
    if not qs:
        return None
    cache.sync()
    cache._apply_realign()
    ring_k, ring_v, pool_k, pool_v = cache._ring_k, cache._ring_v, cache._pool_k, cache._pool_v
    if tuple(ring_k.shape[:2]) != (b, hkv) or ring_k.shape[3] != d or ring_k.dtype != torch.bfloat16:
        raise ValueError("keys do not match the cache's batch/head/dim/dtype")
    # outputs: consecutive 16-byte aligned ranges of one allocation
    sizes = [q.numel() for q in qs]
    starts, off = [], 0
    for n in sizes:
        starts.append(off)
        off += (n + 7) // 8 * 8
    flat = torch.empty(off, dtype=torch.bfloat16, device=q0.device)
    outs = [flat[s:s + n].view(q.shape) for s, n, q in zip(starts, sizes, qs)]
    m = len(qs)
    ptrs = lambda ts: (C.c_void_p * m)(*[t.data_ptr() for t in ts])
    lens = (C.c_int64 * m)(*[int(q.shape[2]) for q in qs])
    counters = (C.c_int64 * 4)(cache.offset, cache.tail_size, cache.summary_count, cache.summary_offset)
    done = C.c_int64(0)
    c = core.cfg
    rule = _native.RULES.get(str(c.block_partner_rule))
    w = int(c.compressed_local_window_tokens)
    t0 = _now_ms()
    with _on(q0.device):
        rc = _native.lib().bfly_stream_chunks(
            m, ptrs(qs), ptrs(ks), ptrs(vs), ptrs(outs), lens, _dtype_code(q0), b, hq, hkv, d, ring_k.data_ptr(),
            ring_v.data_ptr(), cache.tail_capacity, pool_k.data_ptr(), pool_v.data_ptr(), cache.summary_capacity,
            counters, int(cache.local_window_tokens), core.layer_idx, rule, int(c.block_local_window_blocks),
            int(c.block_sink_blocks), int(c.block_partner_count), cache.block_size, w, _scale(core.scale, d),
            C.byref(done), _stream(q0))
    cache.offset, cache.tail_size, cache.summary_count, cache.summary_offset = (int(x) for x in counters)
    if rc == _native.ERR_UNSUPPORTED and done.value == 0:
        return None
    _native.check(rc, "bfly_stream_chunks")
    lay = core.layout(cache.offset, hkv, hq // hkv, q0.device)
    core._last = (t0, _now_ms(), None, "block_sparse_compressed_active",
                  {"seq_len": cache.offset, "q_len": int(qs[-1].shape[2]), "block_sparse_active_mode": True,
                   "native_chunk_loop": m}, lay)     # chunks of the last native call
    return outs
