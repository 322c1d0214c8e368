"""GPU: the decode step with the q/k RMSNorm + RoPE fused in (``bfly_decode_step_qk_norm``)
against the separate launches it replaces (``bfly_qk_norm_rope`` then ``bfly_decode_step``).

The fused kernel follows the separate kernel's rounding points and summation order, so the
bar is bit-identity: every step's attention output, and the ring and pool contents after
steps that append, trim and pool blocks.
"""
from __future__ import annotations

import pytest
import torch

import butterfly_amd as bf
from butterfly_amd.decoder import Attention, DecoderConfig, rope_cos_sin

pytestmark = pytest.mark.gpu

CFG = DecoderConfig(vocab_size=256, hidden_size=512, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=128,
                    intermediate_size=512)


def _setup(prompt_len, rope_rows, seed=0, cfg=CFG, batch=1, cache_window=64):
    g = torch.Generator(device="cuda").manual_seed(seed)
    attn = Attention(cfg, generator=g, device="cuda")
    for norm in (attn.q_norm, attn.k_norm):
        norm.weight.data = (1 + 0.3 * torch.randn(cfg.head_dim, generator=g, device="cuda")).bfloat16()
    cos, sin = rope_cos_sin(torch.arange(rope_rows, device="cuda"), cfg.head_dim, cfg.rope_theta)
    k = torch.randn(batch, cfg.num_kv_heads, prompt_len, cfg.head_dim, generator=g, device="cuda").bfloat16()
    v = torch.randn(batch, cfg.num_kv_heads, prompt_len, cfg.head_dim, generator=g, device="cuda").bfloat16()
    caches = []
    for _ in range(2):
        c = bf.CompressedKVCache(block_size=128, local_window_tokens=cache_window, max_kv_size=prompt_len + 400)
        c.update_and_fetch(k, v)
        c.use_device_counters()
        caches.append(c)
    return attn, cos.contiguous(), sin.contiguous(), caches, g


def _raw(qkv, cfg=CFG):
    """Raw q, k, v rows of a fused projection output [B, 1, (Hq + 2 Hkv) d]: views for batch 1."""
    b = qkv.shape[0]
    row = qkv.view(b, -1)
    nq, nkv = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
    return (row[:, :nq].reshape(b, cfg.num_heads, 1, cfg.head_dim),
            row[:, nq:nq + nkv].reshape(b, cfg.num_kv_heads, 1, cfg.head_dim),
            row[:, nq + nkv:].reshape(b, cfg.num_kv_heads, 1, cfg.head_dim))


# GQA groups of 20 heads (two 16-column MFMA passes, the q transform redone for the
# second) and batch 3; the cache window of 128 differs from the attention window of 64
@pytest.mark.parametrize("layer_idx,heads,batch,cache_window", [(0, (4, 2), 1, 64), (5, (4, 2), 1, 64),
                                                                (2, (40, 2), 1, 64), (3, (8, 2), 3, 128)])
def test_fused_qk_norm_step_equals_separate_launches(layer_idx, heads, batch, cache_window):
    prompt = 700
    cfg = DecoderConfig(vocab_size=256, hidden_size=512, num_layers=1, num_heads=heads[0], num_kv_heads=heads[1],
                        head_dim=128, intermediate_size=512)
    attn, cos, sin, (ca, cb), g = _setup(prompt, 1024, seed=layer_idx, cfg=cfg, batch=batch,
                                         cache_window=cache_window)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), layer_idx)
    assert core.fuses_qk_norm(cb, 1, cfg.head_dim, torch.bfloat16)
    qk = (attn.q_norm.weight, attn.k_norm.weight, cos, sin, attn.q_norm.eps)
    for step in range(150):            # crosses block ends: appends, trims and pooling
        pos = prompt + step
        x = torch.randn(batch, 1, cfg.hidden_size, generator=g, device="cuda").bfloat16()
        qkv = attn.qkv(x)
        q, k, v = attn.heads(qkv, None, rope=(cos[pos:pos + 1], sin[pos:pos + 1]))
        oa = core(q, k, v, ca)
        ob = core(*_raw(qkv, cfg), cb, qk_norm=qk)
        assert torch.equal(oa, ob), (step, (oa.float() - ob.float()).abs().max().item(), oa.float().abs().max().item())
    ca.sync()
    cb.sync()
    assert ca.offset == cb.offset == prompt + 150
    sa, sb = ca.ring_state(), cb.ring_state()
    assert torch.equal(sa.ring_k, sb.ring_k) and torch.equal(sa.ring_v, sb.ring_v)
    assert torch.equal(sa.pool_k, sb.pool_k) and torch.equal(sa.pool_v, sb.pool_v)


def test_fused_step_past_the_rope_table_is_an_error_at_sync():
    prompt = 300
    attn, cos, sin, (_, cb), g = _setup(prompt, prompt + 2)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), 1)
    qk = (attn.q_norm.weight, attn.k_norm.weight, cos, sin, attn.q_norm.eps)
    for _ in range(2):                 # positions 300 and 301 are in the table
        core(*_raw(attn.qkv(torch.randn(1, 1, CFG.hidden_size, generator=g, device="cuda").bfloat16())), cb,
             qk_norm=qk)
    cb.sync()
    core(*_raw(attn.qkv(torch.randn(1, 1, CFG.hidden_size, generator=g, device="cuda").bfloat16())), cb, qk_norm=qk)
    with pytest.raises(RuntimeError, match="RoPE"):
        cb.sync()
    # the failed step changed nothing: the cache holds the last good state
    assert cb.offset == prompt + 2


def test_fused_step_refuses_bad_norm_weights():
    attn, cos, sin, (_, cb), g = _setup(200, 512)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), 0)
    raw = _raw(attn.qkv(torch.randn(1, 1, CFG.hidden_size, generator=g, device="cuda").bfloat16()))
    for qw in (attn.q_norm.weight.float(), attn.q_norm.weight[:64], attn.q_norm.weight.cpu()):
        with pytest.raises(ValueError):
            core(*raw, cb, qk_norm=(qw, attn.k_norm.weight, cos, sin, 1e-6))


def test_qk_norm_is_refused_off_the_device_counter_path():
    attn, cos, sin, (ca, _), g = _setup(200, 512)
    ca.use_device_counters(False)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), 0)
    qkv = attn.qkv(torch.randn(1, 1, CFG.hidden_size, generator=g, device="cuda").bfloat16())
    with pytest.raises(ValueError):
        core(*_raw(qkv), ca, qk_norm=(attn.q_norm.weight, attn.k_norm.weight, cos, sin, 1e-6))
