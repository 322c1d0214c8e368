"""The Torch-side layer swap on a random-init HF-transformers Qwen3.5 model (CPU part):
config surface, layer selection, the stock-fallback rules, and the refusal of CPU tensors
on the Butterfly path.  The GPU part (``test_gpu_qwen_swap.py``) runs the swapped layers."""
from __future__ import annotations

import dataclasses

import pytest
import torch

from butterfly_amd import qwen_torch as qt

transformers = pytest.importorskip("transformers", reason="transformers is not importable")
try:
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM
except ImportError:                                           # pragma: no cover - version without Qwen3.5
    Qwen3_5TextConfig = Qwen3_5ForCausalLM = None

needs_qwen35 = pytest.mark.skipif(Qwen3_5ForCausalLM is None, reason="this transformers has no Qwen3.5 model")

COMPRESSED = dict(path="block_sparse", block_compression="mean", block_partner_rule="causal_shift",
                  compressed_local_window_tokens=64)


def tiny_qwen35(head_dim=32, layers=("linear_attention", "full_attention", "linear_attention", "full_attention")):
    cfg = Qwen3_5TextConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=len(layers),
                            num_attention_heads=4, num_key_value_heads=2, head_dim=head_dim, layer_types=list(layers),
                            linear_num_key_heads=2, linear_num_value_heads=2, linear_key_head_dim=32,
                            linear_value_head_dim=32)
    torch.manual_seed(0)
    return Qwen3_5ForCausalLM(cfg).eval()


def test_config_defaults_and_checks_are_the_references():
    """bna/integrations/qwen_torch.py:254-352."""
    c = qt.QwenCUDAButterflyConfig()
    assert (c.path, c.block_partner_rule, c.block_compression, c.compressed_local_window_tokens, c.engine,
            c.dense_fallback_q_len, c.edge_bias, c.block_chunk_size) == ("permute", "xor", "none", 128, "auto", 1,
                                                                         False, 0)
    assert [f.name for f in dataclasses.fields(c)] == [
        "path", "strategy", "window", "landmark_stride", "num_cycles", "edge_disjoint", "enforce_hamiltonian",
        "regular_num_clusters", "seed", "routing_dim", "edge_bias", "window_drop", "compiled_graph_dir", "engine",
        "dense_fallback_q_len", "fallback_on_output_attentions", "fallback_on_mask", "compute_graph_metrics",
        "max_graph_cache_entries", "sparse_query_chunk_size", "sparse_kv_head_chunk_size", "sparse_degree_chunk_size",
        "sparse_chunk_temp_budget_mib", "sparse_compute_dtype", "sparse_precomputed_backend", "sparse_trace_dir",
        "sparse_trace_max_per_layer", "sparse_trace_layer_indices", "block_size", "block_local_window_blocks",
        "block_partner_count", "block_sink_blocks", "block_partner_rule", "block_chunk_size", "block_compression",
        "compressed_local_window_tokens"]
    for bad in (dict(path="dense"), dict(block_partner_rule="fixed_stride"), dict(block_partner_rule="random"),
                dict(num_cycles=0), dict(dense_fallback_q_len=-1), dict(sparse_compute_dtype="half"),
                dict(sparse_precomputed_backend="cuda"), dict(path="block_sparse", strategy="greedy"),
                dict(max_graph_cache_entries=0), dict(sparse_chunk_temp_budget_mib=0.0)):
        with pytest.raises(ValueError):
            qt.QwenCUDAButterflyConfig(**bad)
    assert qt.QwenCUDAButterflyConfig(sparse_trace_layer_indices=[3, 1, 3]).sparse_trace_layer_indices == (1, 3)
    assert qt.QwenCUDAButterflyConfig(**COMPRESSED).is_compressed


def test_causal_mask_recognition():
    lo = torch.finfo(torch.float32).min
    m = torch.full((1, 1, 5, 5), lo).triu(1)
    assert qt._is_standard_causal_mask(None, q_len=5, k_len=5)
    assert qt._is_standard_causal_mask(m, q_len=5, k_len=5)
    assert qt._is_standard_causal_mask(torch.ones(1, 5), q_len=5, k_len=5)
    assert not qt._is_standard_causal_mask(torch.zeros(1, 1, 5, 5), q_len=5, k_len=5)
    assert not qt._is_standard_causal_mask(m[..., :4, :], q_len=4, k_len=5)
    padded = torch.ones(1, 5)
    padded[0, 0] = 0
    assert not qt._is_standard_causal_mask(padded, q_len=5, k_len=5)


@needs_qwen35
def test_swap_takes_full_attention_layers_and_restores():
    model = tiny_qwen35()
    stock = [getattr(layer, "self_attn", None) for layer in model.model.layers]
    assert qt.swap_qwen_attention_with_butterfly_cuda(model, qt.QwenCUDAButterflyConfig(**COMPRESSED)) == [1, 3]
    wrapped = list(qt.iter_qwen_butterfly_layers(model))
    assert [w.layer_idx for w in wrapped] == [1, 3] and wrapped[0].fallback is stock[1]
    assert (wrapped[0].num_heads, wrapped[0].num_key_value_heads, wrapped[0].head_dim) == (4, 2, 32)
    # swapping again keeps the wrappers; layer_indices filters
    assert qt.swap_qwen_attention_with_butterfly_cuda(model, qt.QwenCUDAButterflyConfig(**COMPRESSED),
                                                      layer_indices=[3]) == [3]
    assert qt.restore_qwen_dense_attention(model) == [1, 3]
    assert model.model.layers[1].self_attn is stock[1]
    with pytest.raises(NotImplementedError):         # the reference's default path is not built here
        qt.swap_qwen_attention_with_butterfly_cuda(model)


@needs_qwen35
def test_stock_fallback_rules_on_cpu():
    """Short queries without a cache, output_attentions and training run the stock module (same
    output, reason recorded); a prefill on the Butterfly path refuses CPU tensors."""
    model = tiny_qwen35()
    ref = tiny_qwen35()
    qt.swap_qwen_attention_with_butterfly_cuda(model, qt.QwenCUDAButterflyConfig(**COMPRESSED))
    x = torch.randint(0, 256, (1, 1))
    with torch.no_grad():
        assert torch.equal(model(x).logits, ref(x).logits)
    assert model.model.layers[1].self_attn.last_profile["reason"] == "short_query"
    with torch.no_grad():
        model(torch.randint(0, 256, (1, 6)), output_attentions=True)
    assert model.model.layers[3].self_attn.last_profile["reason"] == "output_attentions"
    model.train()
    model(torch.randint(0, 256, (1, 6)))
    assert model.model.layers[1].self_attn.last_profile["reason"] == "training"
    model.eval()
    with pytest.raises(ValueError, match="GPU"), torch.no_grad():
        model(torch.randint(0, 256, (1, 6)))
