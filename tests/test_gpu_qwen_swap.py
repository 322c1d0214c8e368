"""GPU: the layer swaps on real module types.

* The Torch twin (``swap_qwen_attention_with_butterfly_cuda``) inside a random-init
  HF-transformers Qwen3.5 model (bf16, hybrid linear/full attention layers): a prefill
  and decode steps through ``DynamicCache``.  For every swapped call the test checks that
  the attention received exactly the stock module's q/k/v (projections, q/k norm, the
  model's own partial RoPE, the cache's full history), that the attention output matches
  the CPU oracle at the north_star bf16 tolerance, and that the module output is the stock
  gate and ``o_proj`` applied to it.
* The generic ``QwenButterflyAttention`` over this repository's decoder attention (the
  attribute set of mlx_lm / HF Qwen attention) against the decoder's own swapped module.
"""
from __future__ import annotations

import pytest
import torch

import butterfly_amd as bf
from butterfly_amd import qwen_torch as qt
from oracle import attention as oa, topology as tp

pytestmark = pytest.mark.gpu

BF16_MAX_ABS, BF16_REL_L2 = 2e-2, 1e-2


def _close(got, want):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs().max().item()
    rel = ((got - want).norm() / want.norm()).item()
    assert err <= BF16_MAX_ABS and rel <= BF16_REL_L2, (err, rel)


def _stock_qkv(attn, hidden, pos_emb):
    """The stock Qwen3.5 attention's q, k, v and gate (its forward, before the cache update)."""
    import sys

    shape = hidden.shape[:-1]
    d = attn.head_dim
    q, gate = torch.chunk(attn.q_proj(hidden).view(*shape, -1, d * 2), 2, dim=-1)
    gate = gate.reshape(*shape, -1)
    q = attn.q_norm(q.view(*shape, -1, d)).transpose(1, 2)
    k = attn.k_norm(attn.k_proj(hidden).view(*shape, -1, d)).transpose(1, 2)
    v = attn.v_proj(hidden).view(*shape, -1, d).transpose(1, 2)
    rope = sys.modules[type(attn).__module__].apply_rotary_pos_emb
    q, k = rope(q, k, *pos_emb)
    return q, k, v, gate


def test_torch_twin_in_a_hf_qwen35_model(monkeypatch):
    Qwen3_5TextConfig = pytest.importorskip("transformers.models.qwen3_5.configuration_qwen3_5").Qwen3_5TextConfig
    modeling = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    layers = ["linear_attention", "full_attention", "full_attention", "linear_attention", "full_attention"]
    cfg = Qwen3_5TextConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=len(layers),
                            num_attention_heads=4, num_key_value_heads=2, head_dim=128, layer_types=layers,
                            linear_num_key_heads=2, linear_num_value_heads=2, linear_key_head_dim=64,
                            linear_value_head_dim=64)
    torch.manual_seed(0)
    model = modeling.Qwen3_5ForCausalLM(cfg).to("cuda", torch.bfloat16).eval()
    bcfg = qt.QwenCUDAButterflyConfig(path="block_sparse", block_compression="mean", block_partner_rule="causal_shift",
                                      compressed_local_window_tokens=64)
    assert qt.swap_qwen_attention_with_butterfly_cuda(model, bcfg) == [1, 2, 4]

    calls = []
    real_prefill, real_active = qt.butterfly_compressed_attention, qt.butterfly_compressed_attention_active

    def rec_prefill(q, k, v, *, layout, local_window_tokens, block_chunk_size=0):
        out = real_prefill(q, k, v, layout=layout, local_window_tokens=local_window_tokens)
        calls.append(("prefill", q, k, v, None, out))
        return out

    def rec_active(q, k, v, *, layout, query_positions, local_window_tokens):
        out = real_active(q, k, v, layout=layout, query_positions=query_positions,
                          local_window_tokens=local_window_tokens)
        calls.append(("active", q, k, v, query_positions, out))
        return out

    monkeypatch.setattr(qt, "butterfly_compressed_attention", rec_prefill)
    monkeypatch.setattr(qt, "butterfly_compressed_attention_active", rec_active)
    seen = []

    def hook(mod, args, kwargs, output):
        seen.append((mod.layer_idx, kwargs["hidden_states"], kwargs["position_embeddings"], output[0],
                     dict(mod.last_profile)))

    handles = [m.register_forward_hook(hook, with_kwargs=True) for m in qt.iter_qwen_butterfly_layers(model)]
    prompt_len, steps = 700, 4
    ids = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=torch.Generator().manual_seed(1)).cuda()
    with torch.no_grad():
        out = model(ids, use_cache=True)
        tok = out.logits[:, -1:].argmax(-1)
        for _ in range(steps):
            out = model(tok, past_key_values=out.past_key_values, use_cache=True)
            tok = out.logits[:, -1:].argmax(-1)
    for h in handles:
        h.remove()
    assert len(calls) == len(seen) == 3 * (1 + steps)
    history = {}
    for (kind, q, k, v, qpos, o), (layer, hidden, pos_emb, y, prof) in zip(calls, seen):
        attn = model.model.layers[layer].self_attn
        sq, sk, sv, gate = _stock_qkv(attn.fallback, hidden, pos_emb)
        kv_len = k.shape[2]
        # the attention saw the stock q/k/v, and the cache's whole history
        assert torch.equal(q, sq)
        ks, vs = history.get(layer, (sk[:, :, :0], sv[:, :, :0]))
        history[layer] = (torch.cat([ks, sk], 2), torch.cat([vs, sv], 2))
        assert torch.equal(k, history[layer][0]) and torch.equal(v, history[layer][1])
        lay = tp.build_layout(seq_len=kv_len, block_size=128, num_key_value_heads=2, num_key_value_groups=2,
                              layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                              partner_rule="causal_shift")
        if kind == "prefill":
            assert kv_len == prompt_len
            want = oa.prefill(q.cpu(), k.cpu(), v.cpu(), layout=lay, W=64)
        else:
            assert list(torch.as_tensor(qpos).view(-1)) == [kv_len - 1]
            want = oa.active(q.cpu(), k.cpu(), v.cpu(), layout=lay, query_positions=torch.tensor([kv_len - 1]), W=64)
        _close(o, want)
        b, length = hidden.shape[:2]
        assert torch.equal(y, attn.fallback.o_proj(o.transpose(1, 2).reshape(b, length, -1) * torch.sigmoid(gate)))
        assert prof["mode"] == "butterfly" and prof["kv_len"] == kv_len
        assert prof["block_sparse_stage"] == lay.stage_idx


def test_generic_swapped_module_over_the_decoder_attention():
    """QwenButterflyAttention reads the decoder attention's attribute set and gives the same
    outputs as the decoder's registered swapped module (which adds fused projection kernels),
    through a CompressedKVCache prefill and decode steps; both against the oracle."""
    from butterfly_amd.decoder import Attention, ButterflyAttention, DecoderConfig, rope_cos_sin

    dcfg = DecoderConfig(vocab_size=256, hidden_size=512, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=128,
                         intermediate_size=512)
    g = torch.Generator(device="cuda").manual_seed(3)
    base = Attention(dcfg, generator=g, device="cuda")
    for norm in (base.q_norm, base.k_norm):
        norm.weight.data = (1 + 0.3 * torch.randn(128, generator=g, device="cuda")).bfloat16()
    bcfg = bf.compressed_butterfly_config()
    generic = bf.QwenButterflyAttention(base, bcfg, layer_idx=2)
    fused = ButterflyAttention(base, bcfg, layer_idx=2)
    assert type(generic) is bf.QwenButterflyAttention and generic.head_dim == 128 and generic.n_kv_heads == 2
    ca = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=1024)
    cb = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=1024)
    cos, sin = rope_cos_sin(torch.arange(1024, device="cuda"), 128, dcfg.rope_theta)
    t = 600
    x = torch.randn(1, t + 5, 512, generator=g, device="cuda").bfloat16()
    ya = generic(x[:, :t], cache=ca, position_embeddings=(cos[:t], sin[:t]))
    yb = fused(x[:, :t], cache=cb, position_embeddings=(cos[:t], sin[:t]))
    torch.testing.assert_close(ya.float(), yb.float(), atol=2e-2, rtol=2e-2)
    assert generic.last_profile.path == "block_sparse_compressed"
    for p in range(t, t + 5):
        ya = generic(x[:, p:p + 1], cache=ca, position_embeddings=(cos[p:p + 1], sin[p:p + 1]))
        yb = fused(x[:, p:p + 1], cache=cb, position_embeddings=(cos[p:p + 1], sin[p:p + 1]))
        torch.testing.assert_close(ya.float(), yb.float(), atol=2e-2, rtol=2e-2)
    assert generic.last_profile.path == "block_sparse_compressed_active"
    assert ca.offset == cb.offset == t + 5
