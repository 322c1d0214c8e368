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

import gc
import time
import warnings
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple, Union

import torch
import torch.nn as nn

from .attention import (_attend, _c, _on, _require_cuda, compressed_butterfly_attention,
                        compressed_butterfly_attention_active)
from .compressed_cache import CompressedKVCache
from .layout import build_block_butterfly_layout, drop_layouts_for_other_lengths

_RULES = {"xor", "bit_reversal", "benes", "causal_shift", "fixed_stride", "random"}
_STRATEGIES = {"random", "greedy", "online_insertion", "regular_partition"}


@dataclass
class QwenButterflyConfig:
    """The layer-swap config: the reference's field set, defaults and checks
    (bna/integrations/qwen_mlx.py:84-165).

    Only ``path="block_sparse"`` with ``block_compression="mean"`` -- compressed
    Butterfly attention -- runs here; the attention modules refuse other paths
    with ``NotImplementedError``.  Fields that steer only those other paths
    (``strategy``, ``window``, ``landmark_stride``, ``num_cycles``, the permute
    chunking, retro-backfill, graph metrics, ...) are accepted, validated as the
    reference does, and otherwise ignored.  ``query_chunk_size`` bounds the
    reference's memory per query chunk; the kernels here stream keys in constant
    LDS, so it does not change results and is not used.
    ``compressed_butterfly_config()`` gives the compressed configuration.
    """

    path: str = "permute"
    strategy: str = "random"
    window: int = 64
    landmark_stride: Optional[int] = 64
    num_cycles: Union[int, str] = 1
    edge_disjoint: bool = True
    enforce_hamiltonian: bool = True
    regular_num_clusters: int = 8
    seed: int = 0
    edge_bias: bool = True
    window_drop: float = 0.0
    compiled_graph_dir: Optional[str] = None
    block_size: int = 128
    block_local_window_blocks: int = 1
    block_partner_count: int = 1
    block_sink_blocks: int = 1
    block_partner_rule: str = "xor"
    block_compression: str = "none"
    compressed_local_window_tokens: int = 128
    permute_head_chunk_size: int = 8
    query_chunk_size: int = 256
    permute_stream_o_proj: bool = False
    permute_log_chunks: bool = False
    compute_edge_utilization_proxy: bool = True
    compute_graph_metrics: bool = True
    retro_backfill_enabled: bool = False
    retro_backfill_alpha: float = 0.0
    retro_backfill_training_only: bool = True
    retro_backfill_causal_only: bool = True
    circular: bool = False
    multi_cycle_mode: str = "average"
    verify_spectral_gap: bool = False
    spectral_gap_threshold: float = 4.0
    use_fused_dispatch: bool = True
    active_dense_threshold: Optional[Union[int, str]] = None
    wayfinder_decode_backend: str = "active_permute"

    @property
    def butterfly_decode_backend(self) -> str:
        return self.wayfinder_decode_backend

    @butterfly_decode_backend.setter
    def butterfly_decode_backend(self, value: str) -> None:
        self.wayfinder_decode_backend = value

    @property
    def is_compressed(self) -> bool:
        """Whether this config selects compressed Butterfly attention (the path built here)."""
        return self.path == "block_sparse" and self.block_compression == "mean"

    def __post_init__(self) -> None:
        if self.path not in {"sparse", "permute", "block_sparse"}:
            raise ValueError(f"Unsupported Butterfly path: {self.path!r}")
        if self.strategy not in _STRATEGIES:
            raise ValueError(f"Unsupported Butterfly strategy: {self.strategy!r}")
        if int(self.window) < 0:
            raise ValueError("window must be >= 0")
        if self.num_cycles != "auto" and int(self.num_cycles) <= 0:
            raise ValueError("num_cycles must be > 0 or 'auto'")
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
        if self.path == "block_sparse" and self.strategy in {"greedy", "online_insertion"}:
            raise ValueError("block_sparse supports only static strategies ('random', 'regular_partition')")
        if self.wayfinder_decode_backend not in {"active_permute", "dense"}:
            raise ValueError(f"Unsupported butterfly_decode_backend: {self.wayfinder_decode_backend!r}")


QwenWayfinderConfig = QwenButterflyConfig


def compressed_butterfly_config(**overrides) -> QwenButterflyConfig:
    """The compressed Butterfly configuration of this build's benchmark shapes:
    ``path="block_sparse"``, ``block_compression="mean"``, ``causal_shift`` partners,
    a 64-token local window and 64-query chunks (one partner, one sink, one local
    block).  Keyword arguments override any field."""
    kw = dict(path="block_sparse", block_compression="mean", block_partner_rule="causal_shift",
              compressed_local_window_tokens=64, query_chunk_size=64)
    kw.update(overrides)
    return QwenButterflyConfig(**kw)


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
        if not cfg.is_compressed:
            raise NotImplementedError(
                "butterfly_amd implements the compressed Butterfly path "
                "(path='block_sparse', block_compression='mean') only; "
                f"got path={cfg.path!r}, block_compression={cfg.block_compression!r}")
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

    def runs_device_step(self, cache, q_len: int, head_dim: int, dtype) -> bool:
        """Whether ``__call__`` runs this step as one device-counter launch
        (``CompressedKVCache.decode_step``, capturable in a HIP graph): one new token on a
        cache with device counters, the compressed decode backend, and a step that
        ``bfly_decode_step`` takes (attention window <= 64 tokens, routed row <= 16 slots).
        Other steps with device counters read the counters back and run the host path."""
        return (isinstance(cache, CompressedKVCache) and cache.device_counters is not None and q_len == 1
                and self.device_step_fits(cache, head_dim, dtype))

    def device_step_fits(self, cache, head_dim: int, dtype) -> bool:
        """Whether this layer's one-token steps over ``cache`` can run as ``bfly_decode_step``
        once device counters are on (``runs_device_step`` without the counter condition)."""
        c = self.cfg
        row = 1 + int(c.block_local_window_blocks) + int(c.block_partner_count) + int(c.block_sink_blocks)
        return (isinstance(cache, CompressedKVCache) and c.butterfly_decode_backend != "dense"
                and cache.device_step_supported(head_dim, int(c.compressed_local_window_tokens), dtype, row))

    def fuses_qk_norm(self, cache, q_len: int, head_dim: int, dtype) -> bool:
        """Whether ``__call__`` takes ``qk_norm`` for this step: a device step
        (``runs_device_step``) of bf16 rows with head_dim 128 that runs on the MFMA kernel
        (``bfly_decode_step_qk_norm``: positive scale, 32-bit positions and offsets)."""
        from .attention import _scale

        return (self.runs_device_step(cache, q_len, head_dim, dtype) and head_dim == 128
                and dtype == torch.bfloat16
                and cache.step_on_mfma(head_dim, int(self.cfg.compressed_local_window_tokens),
                                       _scale(self.scale, head_dim), dtype))

    def step_oproj(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: CompressedKVCache, qk_norm,
                   o_proj):
        """A ``fuses_qk_norm`` device step that also applies the 4-bit output projection
        ``o_proj`` (``CompressedKVCache.decode_step_oproj``); returns the attention output and the
        projection's fp32 partial rows per kv head [Hkv, B, out_features]."""
        t0 = _now_ms()
        _require_cuda(q, k, v)
        d = int(q.shape[3])
        if not self.fuses_qk_norm(cache, int(q.shape[2]), d, q.dtype):
            raise ValueError("step_oproj takes device-counter decode steps of bf16, head_dim 128 rows only")
        c = self.cfg
        out, parts = cache.decode_step_oproj(
            q, k, v, layer_idx=self.layer_idx, local_window_tokens=int(c.compressed_local_window_tokens),
            qk_norm=qk_norm, o_proj=o_proj, partner_rule=c.block_partner_rule,
            local_window_blocks=c.block_local_window_blocks, sink_count=c.block_sink_blocks,
            partner_count=c.block_partner_count, scale=self.scale)
        self._last = (t0, _now_ms(), None, "block_sparse_compressed_active", _DEVICE_STEP_NOTES, None)
        return out, parts

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 cache: Optional[CompressedKVCache] = None, qk_norm=None) -> torch.Tensor:
        """``qk_norm`` (see ``CompressedKVCache.decode_step``) hands raw q/k projection rows to
        the decode step, which applies the q/k RMSNorm and RoPE itself; only where
        ``fuses_qk_norm`` holds."""
        t0 = _now_ms()
        _require_cuda(q, k, v)
        b, hq, q_len, d = q.shape
        hkv = int(k.shape[1])
        if hq % hkv != 0:
            raise ValueError(f"query heads {hq} must be a multiple of kv heads {hkv}")
        groups = hq // hkv
        w = int(self.cfg.compressed_local_window_tokens)
        c = self.cfg
        if qk_norm is not None and not self.fuses_qk_norm(cache, q_len, d, q.dtype):
            raise ValueError("qk_norm is taken only by device-counter decode steps of bf16, head_dim 128 rows")
        if self.runs_device_step(cache, q_len, d, q.dtype):
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

    def attend_full(self, q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        """This call's queries (the last ``q_len`` positions) over the full keys/values that a
        non-compressed cache returned from ``update_and_fetch``.  Reference: the
        ``block_sparse_active_mode`` branch without a ``CompressedKVCache``
        (bna/integrations/qwen_mlx.py:1547-1572: summaries recomputed over the full keys,
        then the active rows), the one-shot prefill when ``q_len == k_len`` (:1574-1583) and
        the stock decode fallback (dense over every cached key, :1273-1293)."""
        t0 = _now_ms()
        _require_cuda(q, keys, values)
        _, hq, q_len, d = q.shape
        hkv, k_len = int(keys.shape[1]), int(keys.shape[2])
        if hq % hkv != 0:
            raise ValueError(f"query heads {hq} must be a multiple of kv heads {hkv}")
        w = int(self.cfg.compressed_local_window_tokens)
        lay = self.layout(k_len, hkv, hq // hkv, q.device)
        notes: Dict[str, Any] = {"seq_len": k_len, "q_len": int(q_len)}
        if q_len == k_len:
            out, _ = compressed_butterfly_attention(q, keys, values, layout=lay, local_window_tokens=w,
                                                    scale=self.scale)
            path = "block_sparse_compressed"
        elif q_len <= 2 and self.cfg.butterfly_decode_backend == "dense":
            kc, vc = _c(keys), _c(values)
            out = _attend(_c(q), kc, vc, kc, vc, layout=lay, q_pos0=k_len - q_len, qpos_dev=None, ring_capacity=0,
                          tail_start=0, kv_len=k_len, summary_count=0, local_window_tokens=k_len, scale=self.scale)
            notes["dense_fallback_reason"] = "butterfly_decode_stock"
            path = "block_sparse_dense_fallback"
        else:
            qp = torch.arange(k_len - q_len, k_len)
            out, _ = compressed_butterfly_attention_active(q, keys, values, layout=lay, query_positions=qp,
                                                           local_window_tokens=w, scale=self.scale)
            notes["block_sparse_active_mode"] = True
            path = "block_sparse_compressed_active"
        self._last = (t0, _now_ms(), None, path, notes, lay)
        return out


# ----------------------------------------------------------------------------- the swapped attention module
def _attn_get_first(attn, names: Sequence[str]) -> Any:
    for name in names:
        value = getattr(attn, name, None)
        if value is not None:
            return value
    return None


def _attn_num_heads(attn) -> int:
    value = _attn_get_first(attn, ("n_heads", "num_attention_heads", "num_heads"))
    if value is None:
        raise AttributeError("Unable to resolve attention query head count.")
    return int(value)


def _attn_num_kv_heads(attn) -> int:
    value = _attn_get_first(attn, ("n_kv_heads", "num_key_value_heads", "num_kv_heads"))
    if value is None:
        raise AttributeError("Unable to resolve attention KV head count.")
    return int(value)


def _attn_scale(attn) -> float:
    value = _attn_get_first(attn, ("scale", "scaling"))
    if value is not None:
        return float(value)
    head_dim = getattr(attn, "head_dim", None)
    if head_dim is not None:
        return float(int(head_dim) ** -0.5)
    raise AttributeError("Unable to resolve attention scaling factor.")


def _attn_head_dim(attn, scale: float) -> int:
    value = getattr(attn, "head_dim", None)
    if value is not None:
        return int(value)
    return int(round(float(scale) ** -2))


def _rotate_half_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, H, L, d] with cos/sin [L, d] or [B, L, d] (rotate-half RoPE in fp32, cast back)."""
    if cos.dim() == 3:
        cos, sin = cos[:, None], sin[:, None]
    d = x.shape[-1]
    xf = x.float()
    rot = torch.cat([-xf[..., d // 2:], xf[..., : d // 2]], dim=-1)
    return (xf * cos.float() + rot * sin.float()).to(x.dtype)


def _cache_offset(cache) -> int:
    if isinstance(cache, CompressedKVCache):
        cache.sync()
    return int(getattr(cache, "offset", 0))


class QwenButterflyAttention(nn.Module):
    """A decoder attention module with its attention swapped to compressed Butterfly.

    Reference: ``QwenButterflyAttention`` (bna/integrations/qwen_mlx.py:859-975,
    1295-1792) over ``extract_qkv_from_qwen_attention`` (:288-357).  It takes the
    base module's ``q_proj``/``k_proj``/``v_proj`` (or a fused ``qkv_proj``),
    ``o_proj``, ``q_norm``/``k_norm`` and RoPE (``rope`` / ``rotary_emb``), and
    resolves head counts, scale and head_dim from the same attribute names.  A query
    projection twice the head width carries the output gate
    (``y * sigmoid(gate)`` before ``o_proj``).

    ``forward(x, mask=None, cache=None, *, position_embeddings=None)`` returns the
    post-``o_proj`` hidden states [B, L, hidden].  ``position_embeddings`` =
    ``(cos, sin)`` for the call's positions (the PyTorch convention of computing
    RoPE tables once per model step) replaces the base module's RoPE module.  With a
    ``CompressedKVCache`` the call appends to it and attends through
    ``ButterflyAttentionCore``; another cache object with ``update_and_fetch``
    returns the full keys/values and the call takes the reference's active path over
    them (``compressed_butterfly_attention_active``, summaries recomputed).
    ``mask`` is accepted and unused, as in the reference's compressed path.
    """

    def __init__(self, base_attn: nn.Module, cfg: QwenButterflyConfig, *, layer_idx: Optional[int] = None):
        super().__init__()
        self.n_heads = _attn_num_heads(base_attn)
        self.n_kv_heads = _attn_num_kv_heads(base_attn)
        self.scale = _attn_scale(base_attn)
        self.head_dim = _attn_head_dim(base_attn, self.scale)
        self.layer_idx = int(layer_idx) if layer_idx is not None else int(getattr(base_attn, "layer_idx", 0) or 0)
        for name in ("q_proj", "k_proj", "v_proj", "qkv_proj"):
            if hasattr(base_attn, name):
                setattr(self, name, getattr(base_attn, name))
        self.o_proj = base_attn.o_proj
        self.q_norm = getattr(base_attn, "q_norm", None) or nn.Identity()
        self.k_norm = getattr(base_attn, "k_norm", None) or nn.Identity()
        self.rope = _attn_get_first(base_attn, ("rope", "rotary_emb"))
        self.cfg = cfg
        self.path = cfg.path
        self.butterfly_decode_backend = str(cfg.butterfly_decode_backend)
        self.query_chunk_size = int(max(1, cfg.query_chunk_size))
        self.core = ButterflyAttentionCore(cfg, self.layer_idx, scale=self.scale)

    @property
    def last_profile(self) -> Optional[AttentionProfile]:
        return self.core.last_profile

    def project(self, x: torch.Tensor, cache=None, position_embeddings=None):
        """(q [B, Hq, L, d], k, v [B, Hkv, L, d], gate [B, L, Hq*d] or None), RoPE applied.
        Reference: bna/integrations/qwen_mlx.py:288-357 (without the cache update)."""
        b, length, _ = x.shape
        if hasattr(self, "qkv_proj") and not all(hasattr(self, n) for n in ("q_proj", "k_proj", "v_proj")):
            qkv = self.qkv_proj(x)
            kd = self.n_kv_heads * self.head_dim
            qd = int(qkv.shape[-1]) - 2 * kd
            if qd <= 0:
                raise ValueError(f"Unable to split qkv projection with shape {tuple(qkv.shape)}.")
            q = qkv[..., :qd].reshape(b, length, self.n_heads, -1)
            k = qkv[..., qd:qd + kd].reshape(b, length, self.n_kv_heads, -1)
            v = qkv[..., qd + kd:].reshape(b, length, self.n_kv_heads, -1)
        else:
            q = self.q_proj(x).reshape(b, length, self.n_heads, -1)
            k = self.k_proj(x).reshape(b, length, self.n_kv_heads, -1)
            v = self.v_proj(x).reshape(b, length, self.n_kv_heads, -1)
        gate = None
        norm_w = getattr(self.q_norm, "weight", None)
        expected = int(norm_w.shape[0]) if norm_w is not None else self.head_dim
        if int(q.shape[-1]) == 2 * expected:
            q, g = q.chunk(2, dim=-1)
            gate = g.reshape(b, length, -1)
        q = self.q_norm(q).transpose(1, 2)
        k = self.k_norm(k).transpose(1, 2)
        v = v.transpose(1, 2)
        if position_embeddings is not None:
            cos, sin = position_embeddings
            q, k = _rotate_half_rope(q, cos, sin), _rotate_half_rope(k, cos, sin)
        else:
            q, k = self._apply_rope(q, k, cache)
        return q.contiguous(), k.contiguous(), v.contiguous(), gate

    def _apply_rope(self, q, k, cache):
        """The reference's RoPE call resolution (bna/integrations/qwen_mlx.py:260-285)."""
        rope = self.rope
        if rope is None:
            raise AttributeError("Unable to resolve attention RoPE module.")
        if cache is not None:
            offset = _cache_offset(cache)
            try:
                return rope(q, offset=offset), rope(k, offset=offset)
            except TypeError:
                pass
        else:
            try:
                return rope(q), rope(k)
            except TypeError:
                pass
        start = _cache_offset(cache) if cache is not None else 0
        positions = (torch.arange(int(q.shape[2]), device=q.device) + start)[None, :]
        try:
            return rope(positions, q, k)
        except TypeError:
            return rope(positions, q), rope(positions, k)

    def attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache=None) -> torch.Tensor:
        """The attention core over this call's q/k/v: [B, Hq, L, d]."""
        if cache is None or isinstance(cache, CompressedKVCache):
            return self.core(q, k, v, cache)
        if not hasattr(cache, "update_and_fetch"):
            raise TypeError("cache must be a CompressedKVCache or provide update_and_fetch(keys, values)")
        keys, values = cache.update_and_fetch(k, v)
        return self.core.attend_full(q, keys, values)

    def forward(self, x: torch.Tensor, mask=None, cache=None, *, position_embeddings=None) -> torch.Tensor:
        b, length, _ = x.shape
        q, k, v, gate = self.project(x, cache, position_embeddings)
        y = self.attend(q, k, v, cache)
        y = y.transpose(1, 2).reshape(b, length, -1)
        if gate is not None:
            y = y * torch.sigmoid(gate[:, -length:, :]).to(y.dtype)
        return self.o_proj(y)


QwenWayfinderAttention = QwenButterflyAttention

# base attention class -> the QwenButterflyAttention subclass that swaps it (see
# register_butterfly_attention); anything else gets QwenButterflyAttention itself
_WRAPPERS: Dict[type, type] = {}


def register_butterfly_attention(base_cls: type, wrapper_cls: type) -> None:
    """Make ``swap_qwen_attention_with_butterfly`` wrap instances of ``base_cls`` (and its
    subclasses) in ``wrapper_cls``, a ``QwenButterflyAttention`` subclass with the same
    constructor -- for a model whose attention has a faster swapped form than the generic
    module (``butterfly_amd.decoder`` registers its attention this way)."""
    if not (isinstance(wrapper_cls, type) and issubclass(wrapper_cls, QwenButterflyAttention)):
        raise TypeError("wrapper_cls must subclass QwenButterflyAttention")
    _WRAPPERS[base_cls] = wrapper_cls


def _wrapper_for(base_attn) -> type:
    for cls in type(base_attn).__mro__:
        if cls in _WRAPPERS:
            return _WRAPPERS[cls]
    return QwenButterflyAttention


def get_qwen_full_attention_layer_indices(model) -> List[int]:
    """Layers with full attention: ``is_linear`` False, or a ``self_attn`` module.
    Reference: bna/integrations/qwen_mlx.py:1849-1859."""
    if not hasattr(model, "layers"):
        raise ValueError("Model has no .layers attribute; expected a Qwen-style model.")
    out: List[int] = []
    for idx, layer in enumerate(model.layers):
        if getattr(layer, "is_linear", None) is False or getattr(layer, "self_attn", None) is not None:
            out.append(int(idx))
    return out


# The full-attention layers of Qwen 3.5 (every fourth of 32); bna/integrations/qwen_mlx.py:49
EXPECTED_QWEN35_FULL_ATTENTION_LAYERS: Tuple[int, ...] = (3, 7, 11, 15, 19, 23, 27, 31)


def validate_qwen35_full_attention_layers(model, *, allow_mismatch: bool = False) -> List[int]:
    """The model's full-attention layers, checked against Qwen 3.5's layout: a different
    layout raises ``ValueError``, or with ``allow_mismatch`` warns and is returned as found.
    Reference: bna/integrations/qwen_mlx.py:1862-1877."""
    discovered = get_qwen_full_attention_layer_indices(model)
    if tuple(discovered) != EXPECTED_QWEN35_FULL_ATTENTION_LAYERS:
        message = ("Unexpected Qwen 3.5 full-attention layer layout: "
                   f"expected={list(EXPECTED_QWEN35_FULL_ATTENTION_LAYERS)} discovered={discovered}")
        if not allow_mismatch:
            raise ValueError(message)
        warnings.warn(message, stacklevel=2)
    return discovered


def _qwen_graph_cache_drop_other_keys(current_T: int) -> int:
    """The reference's name for evicting cached layouts of other sequence lengths
    (bna/integrations/qwen_mlx.py:52-81); see ``layout.drop_layouts_for_other_lengths``."""
    return drop_layouts_for_other_lengths(current_T)


def install_compressed_kv_caches(model, prompt_cache: List[Any], *, layer_indices: Optional[Sequence[int]] = None,
                                 block_size: int = 128, local_window_tokens: int = 128,
                                 max_kv_size: Optional[int] = None, max_chunk_size: int = 512) -> List[int]:
    """Put a ``CompressedKVCache`` in ``prompt_cache[i]`` for the selected layers.

    Reference: bna/integrations/qwen_mlx.py:1795-1819.  ``layer_indices=None`` selects
    the full-attention layers (``get_qwen_full_attention_layer_indices``).
    """
    if not hasattr(model, "layers"):
        raise ValueError("Model has no .layers attribute; expected a Qwen-style model.")
    selected = get_qwen_full_attention_layer_indices(model) if layer_indices is None else \
        [int(x) for x in layer_indices]
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
    """Replace ``model.layers[i].self_attn`` by ``QwenButterflyAttention(self_attn, cfg, layer_idx=i)``
    for every selected layer that has one (or by the subclass registered for the base module's
    class).  Returns the replaced indices.  Reference: bna/integrations/qwen_mlx.py:1822-1846.
    """
    if not hasattr(model, "layers"):
        raise ValueError("Model has no .layers attribute; expected a Qwen-style model.")
    selected = None if layer_indices is None else {int(i) for i in layer_indices}
    replaced: List[int] = []
    for i, layer in enumerate(model.layers):
        if selected is not None and i not in selected:
            continue
        base = getattr(layer, "self_attn", None)
        if base is None:
            continue
        layer.self_attn = _wrapper_for(base)(base, cfg, layer_idx=i)
        replaced.append(i)
    return replaced


swap_qwen_attention_with_wayfinder = swap_qwen_attention_with_butterfly


def iter_qwen_butterfly_layers(model):
    """The swapped attention modules of ``model``.  Reference: bna/integrations/qwen_mlx.py:1880-1886."""
    if not hasattr(model, "layers"):
        raise ValueError("Model has no .layers attribute; expected a Qwen-style model.")
    for layer in model.layers:
        attn = getattr(layer, "self_attn", None)
        if isinstance(attn, QwenButterflyAttention):
            yield attn


iter_qwen_wayfinder_layers = iter_qwen_butterfly_layers


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

    Python's cyclic garbage collector is paused for the loop (and resumed as it was): the
    loop makes a few objects per chunk (output views, pointer arrays), none of them cyclic,
    and each collection they would set off (several per stream, tens of microseconds each)
    holds the host while the GPU drains its queue.
    """
    chunks = list(chunks)
    if not chunks:
        return []
    collecting = gc.isenabled()
    gc.disable()
    try:
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
            run = _stream_run(cache, int(chunks[i - 1][0].shape[2]), run)
    finally:
        if collecting:
            gc.enable()
    return outs


# Chunks per bfly_stream_chunks call: a first run of 8, then each run about 1.3 times the one
# before, in whole batches of the native loop (its batches hold at most 10 chunks and half the ring
# minus two pages), up to 256.  The host prepares a call's chunks (about 2 us each) before its first
# launch, while the GPU works through the call before (about 3 us per chunk, of which about 2 are
# still queued when that call returns); a run 1.3 times the last is ready before that queue drains,
# where 1.5 times left the GPU waiting at every call boundary.  A call rarely ends in a small batch,
# whose attention launch runs alone.
_STREAM_GROWTH = 1.3
_STREAM_RUN_MAX = 256
_STREAM_BATCH_CAP = 10


def _stream_run(cache, chunk_len: int, prev: int) -> int:
    per = max(1, min(_STREAM_BATCH_CAP, (int(cache.tail_capacity) - 128) // 2 // max(1, chunk_len)))
    want = min(_STREAM_RUN_MAX, max(int(prev * _STREAM_GROWTH), per))
    return per * -(-want // per)


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
    # One pass over the chunks, each tensor's attributes read once (the host's cost per chunk
    # is what keeps the GPU fed): pointers, lengths, and the tensors themselves only where a
    # chunk needed a contiguous copy (kept alive until the launches are enqueued).
    qp, kp, vp, lens_l, copies = [], [], [], [], []
    bf16 = torch.bfloat16
    for qc, kc, vc in chunks[start:start + run]:
        sq = qc.shape
        n = sq[2]
        if (n <= 2 or sq != (b, hq, n, d) or kc.shape != (b, hkv, n, d) or vc.shape != (b, hkv, n, d)
                or qc.dtype != bf16 or kc.dtype != bf16 or vc.dtype != bf16 or not qc.is_cuda):
            break
        pq, pk, pv = qc.data_ptr(), kc.data_ptr(), vc.data_ptr()
        if (pq | pk | pv) & 15 or not (qc.is_contiguous() and kc.is_contiguous() and vc.is_contiguous()):
            qc, kc, vc = _c(qc), _c(kc), _c(vc)
            copies.append((qc, kc, vc))
            pq, pk, pv = qc.data_ptr(), kc.data_ptr(), vc.data_ptr()
        qp.append(pq)
        kp.append(pk)
        vp.append(pv)
        lens_l.append(n)
    if not qp:
        return None
    cache.sync()
    cache._apply_realign()
    ring_k, ring_v, pool_k, pool_v = cache._ring_k, cache._ring_v, cache._pool_k, cache._pool_v
    if tuple(ring_k.shape[:2]) != (b, hkv) or ring_k.shape[3] != d or ring_k.dtype != torch.bfloat16:
        raise ValueError("keys do not match the cache's batch/head/dim/dtype")
    # outputs: the leading run of chunks of one length as one [m1, b, hq, n, d] tensor unbound into
    # its rows (far cheaper for the host per chunk than a view each), the rest (a stream's short
    # last chunk, ragged lengths) as 16-byte aligned ranges of a second allocation
    m = len(qp)
    n0 = lens_l[0]
    m1 = 1
    while m1 < m and lens_l[m1] == n0:
        m1 += 1
    per = b * hq * d
    big = torch.empty((m1, b, hq, n0, d), dtype=torch.bfloat16, device=q0.device)
    outs = list(big.unbind(0))
    base, step = big.data_ptr(), per * n0 * 2
    op = [base + i * step for i in range(m1)]
    if m1 < m:
        starts, off = [], 0
        for n in lens_l[m1:]:
            starts.append(off)
            off += (per * n + 7) // 8 * 8
        flat = torch.empty(off, dtype=torch.bfloat16, device=q0.device)
        rest = [flat[s0:s0 + per * n].view(b, hq, n, d) for s0, n in zip(starts, lens_l[m1:])]
        outs += rest
        op += [o.data_ptr() for o in rest]
    ptrs = lambda xs: (C.c_void_p * m)(*xs)
    lens = (C.c_int64 * m)(*lens_l)
    counters = (C.c_int64 * 4)(cache.offset, cache.tail_size, cache.summary_count, cache.summary_offset)
    done = C.c_int64(0)
    c = core.cfg
    rule = _native.RULES.get(str(c.block_partner_rule))
    w = int(c.compressed_local_window_tokens)
    t0 = _now_ms()
    with _on(q0.device):
        rc = _native.lib().bfly_stream_chunks(
            m, ptrs(qp), ptrs(kp), ptrs(vp), ptrs(op), lens, _dtype_code(q0), b, hq, hkv, d, ring_k.data_ptr(),
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
                  {"seq_len": cache.offset, "q_len": lens_l[-1], "block_sparse_active_mode": True,
                   "native_chunk_loop": m}, lay)     # chunks of the last native call
    return outs
