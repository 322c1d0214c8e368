"""The Torch-side layer swap for HF-transformers Qwen3.5 models: compressed Butterfly attention.

Mirrors the reference's ``bna/integrations/qwen_torch.py`` surface for the
compressed path:

* ``QwenCUDAButterflyConfig`` -- field set, defaults and checks of
  ``qwen_torch.py:254-352``.  Only ``path="block_sparse"`` with
  ``block_compression="mean"`` runs here; the module refuses other paths with
  ``NotImplementedError``.
* ``QwenCUDAButterflyAttention(fallback_attention, cfg)`` -- wraps a stock HF
  full-attention module (``q_proj`` producing query and output gate,
  ``k_proj``/``v_proj``/``o_proj``, ``q_norm``/``k_norm``, ``head_dim``) with the HF
  ``forward(hidden_states, position_embeddings, attention_mask=None,
  past_key_values=None, cache_position=None, **kw) -> (out, None)``
  (``qwen_torch.py:576-657, 1187-1621``).  Prefill (``q_len == kv_len``) runs
  ``butterfly_compressed_attention``; a call with cached keys
  (``kv_len > q_len``) runs ``butterfly_compressed_attention_active`` over the full
  keys/values that ``past_key_values.update`` returns, at the call's query
  positions.  Training, ``output_attentions``, a short query without a cache, a
  missing ``layer_idx`` and a non-causal mask take the stock module instead, with
  the reason in ``last_profile``, as the reference does.
* ``swap_qwen_attention_with_butterfly_cuda``, ``restore_qwen_dense_attention``,
  ``iter_qwen_butterfly_layers`` (``qwen_torch.py:1624-1700``).

The attention runs on the HIP kernels of ``libbutterfly_amd.so``; the q/k/v
projections, norms, RoPE, gate and ``o_proj`` are the stock module's own.
"""
from __future__ import annotations

import copy
import sys
import time
from dataclasses import dataclass
from typing import Any, Dict, Iterable, List, Optional, Sequence

import torch
import torch.nn as nn

from .attention import _require_cuda, butterfly_compressed_attention, butterfly_compressed_attention_active
from .layout import build_block_butterfly_layout

_DYNAMIC_STRATEGIES = {"greedy", "online_insertion"}


@dataclass
class QwenCUDAButterflyConfig:
    """Reference: bna/integrations/qwen_torch.py:254-352 (fields, defaults, checks).

    Fields of the reference's other paths and engines are accepted, validated and
    otherwise unused; ``block_chunk_size`` and the ``sparse_*`` chunk sizes are
    memory knobs there and do not change results.
    """

    path: str = "permute"
    strategy: str = "random"
    window: int = 64
    landmark_stride: Optional[int] = 64
    num_cycles: int = 1
    edge_disjoint: bool = True
    enforce_hamiltonian: bool = True
    regular_num_clusters: int = 8
    seed: int = 0
    routing_dim: Optional[int] = None
    edge_bias: bool = False
    window_drop: float = 0.0
    compiled_graph_dir: Optional[str] = None
    engine: str = "auto"
    dense_fallback_q_len: int = 1
    fallback_on_output_attentions: bool = True
    fallback_on_mask: bool = True
    compute_graph_metrics: bool = False
    max_graph_cache_entries: int = 1
    sparse_query_chunk_size: int = 0
    sparse_kv_head_chunk_size: int = 0
    sparse_degree_chunk_size: int = 0
    sparse_chunk_temp_budget_mib: float = 160.0
    sparse_compute_dtype: str = "auto"
    sparse_precomputed_backend: str = "auto"
    sparse_trace_dir: Optional[str] = None
    sparse_trace_max_per_layer: int = 0
    sparse_trace_layer_indices: Optional[tuple] = None
    block_size: int = 128
    block_local_window_blocks: int = 1
    block_partner_count: int = 1
    block_sink_blocks: int = 1
    block_partner_rule: str = "xor"
    block_chunk_size: int = 0
    block_compression: str = "none"
    compressed_local_window_tokens: int = 128

    @property
    def is_compressed(self) -> bool:
        return self.path == "block_sparse" and self.block_compression == "mean"

    def __post_init__(self) -> None:
        if self.path not in {"permute", "sparse", "block_sparse"}:
            raise ValueError(f"Unsupported Butterfly path: {self.path!r}")
        if self.strategy not in {"random", "regular_partition", "greedy", "online_insertion"}:
            raise ValueError(f"Unsupported Butterfly strategy: {self.strategy!r}")
        if self.path == "block_sparse" and self.strategy in _DYNAMIC_STRATEGIES:
            raise ValueError("block_sparse currently supports only static strategies ('random', 'regular_partition')")
        if int(self.window) < 0:
            raise ValueError("window must be >= 0")
        if int(self.num_cycles) <= 0:
            raise ValueError("num_cycles must be > 0")
        if int(self.block_size) <= 0:
            raise ValueError("block_size must be > 0")
        if int(self.block_local_window_blocks) < 0:
            raise ValueError("block_local_window_blocks must be >= 0")
        if int(self.block_partner_count) < 0:
            raise ValueError("block_partner_count must be >= 0")
        if int(self.block_sink_blocks) < 0:
            raise ValueError("block_sink_blocks must be >= 0")
        if self.block_partner_rule not in {"xor", "bit_reversal", "benes", "causal_shift"}:
            raise ValueError(f"Unsupported block_partner_rule: {self.block_partner_rule!r}")
        if self.block_compression not in {"none", "mean"}:
            raise ValueError(f"Unsupported block_compression: {self.block_compression!r}")
        if int(self.compressed_local_window_tokens) <= 0:
            raise ValueError("compressed_local_window_tokens must be > 0")
        if int(self.dense_fallback_q_len) < 0:
            raise ValueError("dense_fallback_q_len must be >= 0")
        if int(self.max_graph_cache_entries) <= 0:
            raise ValueError("max_graph_cache_entries must be > 0")
        if int(self.sparse_query_chunk_size) < 0:
            raise ValueError("sparse_query_chunk_size must be >= 0")
        if int(self.sparse_kv_head_chunk_size) < 0:
            raise ValueError("sparse_kv_head_chunk_size must be >= 0")
        if int(self.sparse_degree_chunk_size) < 0:
            raise ValueError("sparse_degree_chunk_size must be >= 0")
        if float(self.sparse_chunk_temp_budget_mib) <= 0.0:
            raise ValueError("sparse_chunk_temp_budget_mib must be > 0")
        if self.sparse_compute_dtype not in {"auto", "model", "float32"}:
            raise ValueError(f"Unsupported sparse_compute_dtype: {self.sparse_compute_dtype!r}")
        if self.sparse_precomputed_backend not in {"auto", "triton_fused", "sdpa", "streamed_online_softmax",
                                                   "manual_matmul"}:
            raise ValueError(f"Unsupported sparse_precomputed_backend: {self.sparse_precomputed_backend!r}")
        if int(self.sparse_trace_max_per_layer) < 0:
            raise ValueError("sparse_trace_max_per_layer must be >= 0")
        if self.sparse_trace_layer_indices is not None:
            self.sparse_trace_layer_indices = tuple(sorted({int(i) for i in self.sparse_trace_layer_indices}))


QwenCUDAWayfinderConfig = QwenCUDAButterflyConfig


def _has_required_qwen_attention_attrs(module: nn.Module) -> bool:
    return all(hasattr(module, n) for n in ("q_proj", "k_proj", "v_proj", "o_proj", "head_dim"))


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _default_apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim: int = 1):
    """HF's rotate-half RoPE over the first ``cos.shape[-1]`` channels (partial rotary)."""
    cos, sin = cos.unsqueeze(unsqueeze_dim), sin.unsqueeze(unsqueeze_dim)
    r = cos.shape[-1]
    q_rot, q_pass = q[..., :r], q[..., r:]
    k_rot, k_pass = k[..., :r], k[..., r:]
    q_embed = torch.cat([q_rot * cos + _rotate_half(q_rot) * sin, q_pass], dim=-1)
    k_embed = torch.cat([k_rot * cos + _rotate_half(k_rot) * sin, k_pass], dim=-1)
    return q_embed, k_embed


def _resolve_apply_rotary_pos_emb(attn: nn.Module):
    """The model's own ``apply_rotary_pos_emb`` from the attention class's module (the stock
    module's RoPE, so the swapped layer rotates q/k exactly as the stock one); the HF rotate-half
    form when that module has none.  Reference: qwen_torch.py:418-457."""
    mod = sys.modules.get(getattr(type(attn), "__module__", "") or "")
    fn = getattr(mod, "apply_rotary_pos_emb", None) if mod is not None else None
    return fn if callable(fn) else _default_apply_rotary_pos_emb


def _get_decoder_with_layers(model: nn.Module) -> nn.Module:
    """Reference: qwen_torch.py:460-475."""
    if hasattr(model, "get_decoder"):
        dec = model.get_decoder()
        if hasattr(dec, "layers"):
            return dec
    if hasattr(model, "model") and hasattr(model.model, "language_model") and \
            hasattr(model.model.language_model, "layers"):
        return model.model.language_model
    if hasattr(model, "model") and hasattr(model.model, "layers"):
        return model.model
    if hasattr(model, "language_model") and hasattr(model.language_model, "layers"):
        return model.language_model
    if hasattr(model, "layers"):
        return model
    raise ValueError("Could not find a decoder with `.layers` on the supplied model.")


def _cache_seq_len(past_key_values: Optional[Any], layer_idx: Optional[int]) -> int:
    """Reference: qwen_torch.py:478-492."""
    if past_key_values is None or layer_idx is None:
        return 0
    getter = getattr(past_key_values, "get_seq_length", None)
    if getter is None:
        return 0
    try:
        return int(getter(layer_idx))
    except TypeError:
        try:
            return int(getter())
        except Exception:
            return 0
    except Exception:
        return 0


def _is_standard_causal_mask(attention_mask: Optional[torch.Tensor], *, q_len: int, k_len: int) -> bool:
    """Whether the mask is None, all-ones 2-D, or the additive 4-D causal mask of a square call
    (sampled corners and the diagonal).  Reference: qwen_torch.py:495-532."""
    if attention_mask is None:
        return True
    if attention_mask.dim() == 2:
        return bool(torch.all(attention_mask == 1))
    if attention_mask.dim() != 4:
        return False
    if int(attention_mask.shape[-2]) != q_len or int(attention_mask.shape[-1]) != k_len:
        return False
    if int(attention_mask.shape[1]) != 1 or q_len != k_len or not attention_mask.is_floating_point():
        return False
    lo = torch.finfo(attention_mask.dtype).min
    m = attention_mask
    if q_len > 1:
        if float(m[0, 0, 0, 1]) != lo or float(m[0, 0, 1, 0]) != 0.0:
            return False
        if float(m[0, 0, q_len - 1, 0]) != 0.0 or float(m[0, 0, 0, q_len - 1]) != lo:
            return False
    return bool(torch.all(torch.diagonal(m[0, 0]) == 0))


def extract_qkv_from_qwen_attention(attn: nn.Module, hidden_states: torch.Tensor,
                                    position_embeddings: tuple, *, past_key_values: Optional[Any] = None,
                                    cache_position: Optional[torch.LongTensor] = None):
    """(query [B, Hq, L, d], key, value [B, Hkv, kv_len, d], gate [B, L, Hq*d] or None) of a stock
    Qwen attention module after q/k norm and RoPE, with the cache updated.  Reference:
    qwen_torch.py:535-573.  A query projection twice the head width carries the output gate
    (Qwen3.5); one of the plain width has none (Qwen3)."""
    input_shape = hidden_states.shape[:-1]
    d = int(attn.head_dim)
    hidden_shape = (*input_shape, -1, d)
    apply_rope = _resolve_apply_rotary_pos_emb(attn)
    qp = attn.q_proj(hidden_states)
    n_heads = _num_heads(attn)
    gate = None
    if int(qp.shape[-1]) == 2 * n_heads * d:
        query, gate = torch.chunk(qp.view(*input_shape, -1, d * 2), 2, dim=-1)
        gate = gate.reshape(*input_shape, -1)
    else:
        query = qp
    q_norm = getattr(attn, "q_norm", None)
    k_norm = getattr(attn, "k_norm", None)
    query = query.reshape(hidden_shape)
    key = attn.k_proj(hidden_states).view(hidden_shape)
    query = (q_norm(query) if q_norm is not None else query).transpose(1, 2)
    key = (k_norm(key) if k_norm is not None else key).transpose(1, 2)
    value = attn.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    cos, sin = position_embeddings
    query, key = apply_rope(query, key, cos, sin)
    if past_key_values is not None:
        layer_idx = getattr(attn, "layer_idx", None)
        if layer_idx is None:
            raise ValueError("Attention module missing `layer_idx`; cannot update cache.")
        key, value = past_key_values.update(key, value, layer_idx,
                                            {"sin": sin, "cos": cos, "cache_position": cache_position})
    return query, key, value, gate


def _num_heads(attn: nn.Module) -> int:
    cfg = getattr(attn, "config", None)
    n = getattr(cfg, "num_attention_heads", None) if cfg is not None else None
    if n is not None:
        return int(n)
    # the reference's rule for Qwen3.5: q_proj holds query and gate
    return int(attn.q_proj.out_features) // (int(attn.head_dim) * 2)


class QwenCUDAButterflyAttention(nn.Module):
    """A stock HF Qwen full-attention layer with compressed Butterfly attention.

    Reference: ``QwenCUDAButterflyAttention`` (bna/integrations/qwen_torch.py:576-1621).
    """

    def __init__(self, fallback_attention: nn.Module, cfg: QwenCUDAButterflyConfig):
        super().__init__()
        if not _has_required_qwen_attention_attrs(fallback_attention):
            raise TypeError("fallback_attention does not look like a Qwen3.5 attention module. "
                            "Expected q_proj/k_proj/v_proj/o_proj and head_dim.")
        if not cfg.is_compressed:
            raise NotImplementedError(
                "butterfly_amd implements the compressed Butterfly path (path='block_sparse', "
                f"block_compression='mean') only; got path={cfg.path!r}, block_compression={cfg.block_compression!r}")
        self.fallback = fallback_attention
        self.cfg = copy.deepcopy(cfg)
        self.config = getattr(fallback_attention, "config", None)
        self.layer_idx = getattr(fallback_attention, "layer_idx", None)
        self.head_dim = int(fallback_attention.head_dim)
        self.num_key_value_groups = int(getattr(fallback_attention, "num_key_value_groups", 1))
        self.scaling = float(getattr(fallback_attention, "scaling", self.head_dim ** -0.5))
        self.is_causal = getattr(fallback_attention, "is_causal", True)
        self.num_heads = _num_heads(fallback_attention)
        self.num_key_value_heads = int(fallback_attention.k_proj.out_features) // self.head_dim
        self.hidden_size = int(fallback_attention.q_proj.in_features)
        self.last_profile: Dict[str, Any] = {}

    def _layout(self, kv_len: int, device):
        c = self.cfg
        return build_block_butterfly_layout(
            seq_len=int(kv_len), block_size=int(c.block_size), num_key_value_heads=self.num_key_value_heads,
            num_key_value_groups=self.num_heads // self.num_key_value_heads, layer_idx=int(self.layer_idx),
            local_window_blocks=int(c.block_local_window_blocks), sink_count=int(c.block_sink_blocks),
            partner_count=int(c.block_partner_count), partner_rule=c.block_partner_rule, device=device)

    def _fallback_reason(self, *, attention_mask, q_len: int, k_len_after: int, output_attentions: bool):
        """Reference: qwen_torch.py:1187-1219 (the compressed path's engine is always available)."""
        if self.training:
            return "training"
        cached = int(k_len_after) > int(q_len)
        if self.layer_idx is None:
            return "missing_layer_idx"
        if self.cfg.fallback_on_output_attentions and output_attentions:
            return "output_attentions"
        if q_len <= int(self.cfg.dense_fallback_q_len) and not cached:
            return "short_query"
        if self.cfg.fallback_on_mask and not _is_standard_causal_mask(attention_mask, q_len=q_len, k_len=k_len_after):
            return "attention_mask"
        return None

    def forward(self, hidden_states: torch.Tensor, position_embeddings: tuple,
                attention_mask: Optional[torch.Tensor] = None, past_key_values: Optional[Any] = None,
                cache_position: Optional[torch.LongTensor] = None, **kwargs: Any):
        q_len = int(hidden_states.shape[1])
        cache_len = _cache_seq_len(past_key_values, self.layer_idx)
        k_len_after = q_len + cache_len
        reason = self._fallback_reason(attention_mask=attention_mask, q_len=q_len, k_len_after=k_len_after,
                                       output_attentions=bool(kwargs.get("output_attentions", False)))
        if reason is not None:
            self.last_profile = {"mode": "fallback", "reason": reason, "layer_idx": self.layer_idx, "seq_len": q_len,
                                 "kv_len": k_len_after, "path": self.cfg.path, "strategy": self.cfg.strategy}
            return self.fallback(hidden_states, position_embeddings=position_embeddings,
                                 attention_mask=attention_mask, past_key_values=past_key_values,
                                 cache_position=cache_position, **kwargs)
        t0 = time.perf_counter()
        query, key, value, gate = extract_qkv_from_qwen_attention(
            self.fallback, hidden_states, position_embeddings, past_key_values=past_key_values,
            cache_position=cache_position)
        _require_cuda(query, key, value)
        cached = k_len_after > q_len
        w = int(self.cfg.compressed_local_window_tokens)
        tg = time.perf_counter()
        lay = self._layout(k_len_after if cached else q_len, query.device)
        graph_ms = (time.perf_counter() - tg) * 1e3
        ta = time.perf_counter()
        if cached:
            if cache_position is not None:
                positions = cache_position.detach().view(-1).to(device="cpu", dtype=torch.long)
                if positions.numel() != q_len or bool((positions < 0).any()) or \
                        bool((positions >= k_len_after).any()):
                    raise ValueError(f"cache_position must hold {q_len} positions in [0, {k_len_after})")
            else:
                positions = torch.arange(cache_len, cache_len + q_len, dtype=torch.long)
            out = butterfly_compressed_attention_active(query, key, value, layout=lay, query_positions=positions,
                                                        local_window_tokens=w)
            backend = "compressed_butterfly_active"
        else:
            out = butterfly_compressed_attention(query, key, value, layout=lay, local_window_tokens=w,
                                                 block_chunk_size=int(self.cfg.block_chunk_size))
            backend = "compressed_butterfly_sdpa"
        input_shape = hidden_states.shape[:-1]
        y = out.transpose(1, 2).contiguous().view(*input_shape, -1)
        if gate is not None:
            y = y * torch.sigmoid(gate)
        y = self.fallback.o_proj(y)
        attn_ms = (time.perf_counter() - ta) * 1e3
        self.last_profile = {
            "mode": "butterfly", "reason": None, "layer_idx": self.layer_idx, "seq_len": q_len,
            "kv_len": k_len_after, "path": self.cfg.path, "engine": "hip", "strategy": self.cfg.strategy,
            "graph_build_ms": graph_ms, "attn_kernel_ms_host": attn_ms,
            "elapsed_ms": (time.perf_counter() - t0) * 1e3, "block_sparse_backend": backend,
            "block_sparse_num_blocks": int(lay.num_blocks), "block_sparse_stage": int(lay.stage_idx),
            "block_sparse_stage_count": int(lay.stage_count), "block_partner_rule": self.cfg.block_partner_rule,
            "butterfly_variant": "compressed", "block_compression": "mean", "compressed_local_window_tokens": w,
        }
        return y, None


QwenCUDAWayfinderAttention = QwenCUDAButterflyAttention


def _is_full_attention_layer(layer) -> bool:
    """``layer_type`` (the reference's attribute) or ``block_type`` (the attribute name of
    transformers 5.15's Qwen3.5 decoder layer) equal to "full_attention"."""
    kind = getattr(layer, "layer_type", None) or getattr(layer, "block_type", None)
    return kind == "full_attention"


def swap_qwen_attention_with_butterfly_cuda(model: nn.Module, cfg: Optional[QwenCUDAButterflyConfig] = None, *,
                                            layer_indices: Optional[Sequence[int]] = None) -> List[int]:
    """Wrap the full-attention layers of a Qwen3.5 model in place; returns the wrapped indices.
    Reference: bna/integrations/qwen_torch.py:1652-1700."""
    config = copy.deepcopy(cfg) if cfg is not None else QwenCUDAButterflyConfig()
    decoder = _get_decoder_with_layers(model)
    selected = None if layer_indices is None else {int(i) for i in layer_indices}
    replaced: List[int] = []
    for idx, layer in enumerate(decoder.layers):
        if selected is not None and idx not in selected:
            continue
        if not _is_full_attention_layer(layer):
            continue
        attn = getattr(layer, "self_attn", None)
        if attn is None:
            continue
        if isinstance(attn, QwenCUDAButterflyAttention):
            replaced.append(idx)
            continue
        if not _has_required_qwen_attention_attrs(attn):
            continue
        if getattr(attn, "layer_idx", None) is None:
            attn.layer_idx = idx
        wrapped = QwenCUDAButterflyAttention(attn, config)
        wrapped.train(attn.training)
        layer.self_attn = wrapped
        replaced.append(idx)
    return replaced


swap_qwen_attention_with_wayfinder_cuda = swap_qwen_attention_with_butterfly_cuda


def restore_qwen_dense_attention(model: nn.Module) -> List[int]:
    """Put the stock attention back; returns the restored indices.  Reference: qwen_torch.py:1624-1641."""
    decoder = _get_decoder_with_layers(model)
    restored: List[int] = []
    for idx, layer in enumerate(decoder.layers):
        attn = getattr(layer, "self_attn", None)
        if isinstance(attn, QwenCUDAButterflyAttention):
            layer.self_attn = attn.fallback
            restored.append(idx)
    return restored


def iter_qwen_butterfly_layers(model: nn.Module) -> Iterable[QwenCUDAButterflyAttention]:
    """Reference: qwen_torch.py:1644-1649."""
    for layer in _get_decoder_with_layers(model).layers:
        attn = getattr(layer, "self_attn", None)
        if isinstance(attn, QwenCUDAButterflyAttention):
            yield attn


__all__ = [
    "QwenCUDAButterflyConfig",
    "QwenCUDAButterflyAttention",
    "QwenCUDAWayfinderConfig",
    "QwenCUDAWayfinderAttention",
    "extract_qkv_from_qwen_attention",
    "iter_qwen_butterfly_layers",
    "restore_qwen_dense_attention",
    "swap_qwen_attention_with_butterfly_cuda",
    "swap_qwen_attention_with_wayfinder_cuda",
]
