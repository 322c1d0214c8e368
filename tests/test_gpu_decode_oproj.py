"""GPU: the decode step with the attention output projection inside
(``bfly_decode_step_qk_norm_oproj``) against the launches it replaces
(``bfly_decode_step_qk_norm`` then ``bfly_q4_gemv`` of the attention row).

The step's partial rows per kv head, combined as ``(p0 + p1) + (p2 + p3)`` and rounded to bf16,
equal ``bfly_q4_gemv``'s product bit for bit (both sum a row's pieces over the same lanes in the
same tree), and ``bfly_add_rms_norm_q4_gemv_silu_parts`` over them equals
``bfly_add_rms_norm_q4_gemv_silu`` over that product.  The attention output, ring, pool and
counters equal the step without the projection, also when the two entry points take turns on
one cache.
"""
from __future__ import annotations

import pytest
import torch

import butterfly_amd as bf
from butterfly_amd.decoder import (Attention, DecoderConfig, QuantLinear, add_rms_norm_q4_gemv_silu,
                                   add_rms_norm_q4_gemv_silu_parts, q4_gemv, rope_cos_sin)

pytestmark = pytest.mark.gpu


def _setup(hidden, prompt_len, seed, cache_window=64):
    cfg = DecoderConfig(vocab_size=256, hidden_size=hidden, num_layers=1, num_heads=16, num_kv_heads=4,
                        head_dim=128, intermediate_size=512)
    g = torch.Generator(device="cuda").manual_seed(seed)
    attn = Attention(cfg, generator=g, device="cuda")
    for norm in (attn.q_norm, attn.k_norm):
        norm.weight.data = (1 + 0.3 * torch.randn(cfg.head_dim, generator=g, device="cuda")).bfloat16()
    cos, sin = rope_cos_sin(torch.arange(prompt_len + 512, device="cuda"), cfg.head_dim, cfg.rope_theta)
    k = torch.randn(1, 4, prompt_len, 128, generator=g, device="cuda").bfloat16()
    v = torch.randn(1, 4, prompt_len, 128, generator=g, device="cuda").bfloat16()
    caches = []
    for _ in range(2):
        c = bf.CompressedKVCache(block_size=128, local_window_tokens=cache_window, max_kv_size=prompt_len + 400)
        c.update_and_fetch(k, v)
        c.use_device_counters()
        caches.append(c)
    qk = (attn.q_norm.weight, attn.k_norm.weight, cos.contiguous(), sin.contiguous(), attn.q_norm.eps)
    return cfg, attn, qk, caches, g


def _raw(qkv):
    row = qkv.view(-1)
    return row[:2048].view(1, 16, 1, 128), row[2048:2560].view(1, 4, 1, 128), row[2560:].view(1, 4, 1, 128)


def _combined(parts):
    return ((parts[0] + parts[1]) + (parts[2] + parts[3])).bfloat16()


# hidden 2048 is cfg5's (64 workgroups per kv head, 32 rows each), 512 the smallest grid, 4096
# the largest (64 rows per workgroup); the cache window of 128 differs from the attention window
@pytest.mark.parametrize("hidden,layer_idx,cache_window", [(2048, 3, 64), (512, 0, 64), (4096, 7, 128)])
def test_oproj_step_equals_step_then_q4_gemv(hidden, layer_idx, cache_window):
    prompt = 700
    cfg, attn, qk, (ca, cb), g = _setup(hidden, prompt, seed=layer_idx, cache_window=cache_window)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), layer_idx)
    gate_up = None
    if hidden in (2048, 4096):
        gate_up = QuantLinear.fuse_rows(QuantLinear(hidden, 512, generator=g, device="cuda"),
                                        QuantLinear(hidden, 512, generator=g, device="cuda"))
        norm_w = (1 + 0.1 * torch.randn(hidden, generator=g, device="cuda")).bfloat16()
    for step in range(150):            # crosses block ends: appends, trims and pooling
        x = torch.randn(1, 1, hidden, generator=g, device="cuda").bfloat16()
        raw = _raw(attn.qkv(x))
        oa = core(*raw, ca, qk_norm=qk)
        y = q4_gemv(oa.reshape(1, 1, -1), attn.o_proj)
        ob, parts = core.step_oproj(*raw, cb, qk, attn.o_proj)
        assert parts.shape == (4, 1, hidden) and parts.dtype == torch.float32
        assert torch.equal(oa, ob), (step, (oa.float() - ob.float()).abs().max().item())
        assert torch.equal(_combined(parts), y.view(1, hidden)), \
            (step, (_combined(parts).float() - y.view(1, hidden).float()).abs().max().item())
        if gate_up is not None and step % 10 == 0:
            resid = torch.randn(1, 1, hidden, generator=g, device="cuda").bfloat16()
            h1, s1 = add_rms_norm_q4_gemv_silu(resid, y, norm_w, 1e-6, gate_up)
            h2, s2 = add_rms_norm_q4_gemv_silu_parts(resid, parts, norm_w, 1e-6, gate_up)
            assert torch.equal(h1, h2) and torch.equal(s1, s2), step
    ca.sync()
    cb.sync()
    assert (ca.offset, ca.tail_size, ca.summary_count, ca.summary_offset) == \
           (cb.offset, cb.tail_size, cb.summary_count, cb.summary_offset) and ca.offset == prompt + 150
    sa, sb = ca.ring_state(), cb.ring_state()
    assert torch.equal(sa.ring_k, sb.ring_k) and torch.equal(sa.ring_v, sb.ring_v)
    assert torch.equal(sa.pool_k, sb.pool_k) and torch.equal(sa.pool_v, sb.pool_v)


def test_oproj_step_batch_of_three():
    """Three sequences (12 of the 16 a state of 64 copies per sequence holds): every batch row's
    partial rows combine into bfly_q4_gemv's product of its own attention row."""
    cfg = DecoderConfig(vocab_size=256, hidden_size=2048, num_layers=1, num_heads=16, num_kv_heads=4,
                        head_dim=128, intermediate_size=512)
    g = torch.Generator(device="cuda").manual_seed(21)
    attn = Attention(cfg, generator=g, device="cuda")
    cos, sin = rope_cos_sin(torch.arange(1024, device="cuda"), 128, cfg.rope_theta)
    qk = (attn.q_norm.weight, attn.k_norm.weight, cos.contiguous(), sin.contiguous(), attn.q_norm.eps)
    k = torch.randn(3, 4, 600, 128, generator=g, device="cuda").bfloat16()
    caches = []
    for _ in range(2):
        c = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=1000)
        c.update_and_fetch(k, k.flip(2))
        c.use_device_counters()
        caches.append(c)
    ca, cb = caches
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), 6)
    for step in range(140):
        q = torch.randn(3, 16, 1, 128, generator=g, device="cuda").bfloat16()
        kn = torch.randn(3, 4, 1, 128, generator=g, device="cuda").bfloat16()
        vn = torch.randn(3, 4, 1, 128, generator=g, device="cuda").bfloat16()
        oa = core(q, kn, vn, ca, qk_norm=qk)
        ob, parts = core.step_oproj(q, kn, vn, cb, qk, attn.o_proj)
        assert parts.shape == (4, 3, 2048)
        assert torch.equal(oa, ob), step
        for b in range(3):
            y = q4_gemv(oa[b].reshape(1, 1, -1), attn.o_proj).view(1, 2048)
            assert torch.equal(_combined(parts[:, b:b + 1]), y), (step, b)
    ca.sync()
    cb.sync()
    assert ca.offset == cb.offset == 740


def test_entry_points_take_turns_on_one_cache():
    """Steps with and without the projection alternate on one cache (runs of 1, 2 and 5 across
    block ends): every step's attention output equals that of a cache stepped without it, and
    every counter copy stays equal to copy 0."""
    prompt = 500
    cfg, attn, qk, (ca, cb), g = _setup(2048, prompt, seed=11)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), 2)
    pattern = [1, 0, 0, 1, 1, 0, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0] * 10
    for step, fused in enumerate(pattern):
        raw = _raw(attn.qkv(torch.randn(1, 1, 2048, generator=g, device="cuda").bfloat16()))
        oa = core(*raw, ca, qk_norm=qk)
        if fused:
            ob, parts = core.step_oproj(*raw, cb, qk, attn.o_proj)
            assert torch.equal(_combined(parts), q4_gemv(oa.reshape(1, 1, -1), attn.o_proj).view(1, 2048)), step
        else:
            ob = core(*raw, cb, qk_norm=qk)
        assert torch.equal(oa, ob), (step, fused)
    dev = cb.device_counters.view(-1)[8:].view(-1, 32)
    assert dev.shape[0] == 4 * 64 + 8
    assert torch.equal(dev[:, :4], dev[:1, :4].expand_as(dev[:, :4])), "every copy advanced alike"
    ca.sync()
    cb.sync()
    assert ca.offset == cb.offset == prompt + len(pattern)
    sa, sb = ca.ring_state(), cb.ring_state()
    assert torch.equal(sa.pool_k, sb.pool_k) and torch.equal(sa.ring_v, sb.ring_v)


def test_oproj_step_in_a_graph_replays_like_eager_steps():
    """Captured once, replayed across block ends with eager work between replays: every replay's
    partial rows and attention output equal those of eager steps on a twin cache."""
    prompt = 600
    cfg, attn, qk, (ca, cb), g = _setup(2048, prompt, seed=4)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), 5)
    xs = torch.randn(140, 1, 1, 2048, generator=g, device="cuda").bfloat16()
    xin = torch.empty(1, 1, 2048, dtype=torch.bfloat16, device="cuda")
    xin.copy_(xs[0])
    core.step_oproj(*_raw(attn.qkv(xin)), cb, qk, attn.o_proj)        # eager first step
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            ob, parts = core.step_oproj(*_raw(attn.qkv(xin)), cb, qk, attn.o_proj)
    torch.cuda.current_stream().wait_stream(side)
    oa = core(*_raw(attn.qkv(xs[0])), ca, qk_norm=qk)
    for i in range(1, xs.shape[0]):
        xin.copy_(xs[i])
        graph.replay()
        oa = core(*_raw(attn.qkv(xs[i])), ca, qk_norm=qk)
        torch.cuda.synchronize()
        assert torch.equal(oa, ob), i
        assert torch.equal(_combined(parts), q4_gemv(oa.reshape(1, 1, -1), attn.o_proj).view(1, 2048)), i
    ca.sync()
    cb.sync()
    assert ca.offset == cb.offset == prompt + xs.shape[0]


def test_oproj_step_refuses_other_shapes():
    prompt = 300
    cfg, attn, qk, (ca, _), g = _setup(2048, prompt, seed=1)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), 0)
    raw = _raw(attn.qkv(torch.randn(1, 1, 2048, generator=g, device="cuda").bfloat16()))
    odd = QuantLinear(2048, 2040, generator=g, device="cuda")                 # not a multiple of 32
    with pytest.raises(ValueError, match="multiple of 32"):
        core.step_oproj(*raw, ca, qk, odd)
    with pytest.raises(ValueError, match="2048 inputs"):                    # in_features other than hq * d
        core.step_oproj(*raw, ca, qk, QuantLinear(1024, 2048, generator=g, device="cuda"))
    with pytest.raises(ValueError, match="parts"):
        ca.decode_step_oproj(*raw, layer_idx=0, local_window_tokens=64, qk_norm=qk, o_proj=attn.o_proj,
                             parts=torch.empty(4, 1, 2048, dtype=torch.bfloat16, device="cuda"))   # wrong dtype
    ca.use_device_counters(False)
    with pytest.raises(ValueError):
        core.step_oproj(*raw, ca, qk, attn.o_proj)
