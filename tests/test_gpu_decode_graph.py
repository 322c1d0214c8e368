"""GPU: decode with device-side cache counters (bfly_decode_step) and HIP-graph replay.

The device-counter step must reproduce the host-bookkeeping path bit for bit
(same kernels' arithmetic, same pooled summaries), and every replay of a
captured step must equal the eager step on a twin cache; replays are
interleaved with eager work and synchronisations.
"""
from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

import butterfly_amd as bf
from butterfly_amd.decoder import Decoder, DecoderConfig
from oracle import attention as oa, topology as tp

pytestmark = pytest.mark.gpu


def _rand(seed, shape, dtype):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dtype)


def _layout(t, hkv, groups, layer):
    return bf.build_block_butterfly_layout(seq_len=t, block_size=128, num_key_value_heads=hkv,
                                           num_key_value_groups=groups, layer_idx=layer, local_window_blocks=1,
                                           sink_count=1, partner_count=1, partner_rule="causal_shift")


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 64), (torch.bfloat16, 256)])
def test_device_counter_steps_equal_host_steps(dtype, d):
    b, hq, hkv, layer, prompt, steps = 2, 8, 2, 5, 333, 300
    total = prompt + steps
    q = _rand(61, (b, hq, total, d), dtype).cuda()
    k = _rand(62, (b, hkv, total, d), dtype).cuda()
    v = _rand(63, (b, hkv, total, d), dtype).cuda()
    host = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total)
    dev = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total)
    host.update(k[:, :, :prompt], v[:, :, :prompt])
    dev.update(k[:, :, :prompt], v[:, :, :prompt])
    dev.use_device_counters()
    for p in range(prompt, total):
        a = host.update_and_attend(q[:, :, p:p + 1], k[:, :, p:p + 1], v[:, :, p:p + 1],
                                   layout=_layout(p + 1, hkv, hq // hkv, layer), local_window_tokens=64)
        c = dev.decode_step(q[:, :, p:p + 1], k[:, :, p:p + 1], v[:, :, p:p + 1], layer_idx=layer,
                            local_window_tokens=64)
        assert torch.equal(a, c), p
    dev.sync()
    assert (dev.offset, dev.tail_size, dev.summary_count, dev.summary_offset) == \
           (host.offset, host.tail_size, host.summary_count, host.summary_offset)
    assert torch.equal(dev.k_summary, host.k_summary) and torch.equal(dev.values, host.values)


def test_device_counter_steps_follow_changing_arguments():
    """Each step leaves the next step's routed row in the counter array; a step whose
    layer or partner rule differs from the previous step's must not use it."""
    b, hq, hkv, d, prompt, steps = 2, 8, 2, 128, 300, 120
    total = prompt + steps
    q = _rand(81, (b, hq, total, d), torch.bfloat16).cuda()
    k = _rand(82, (b, hkv, total, d), torch.bfloat16).cuda()
    v = _rand(83, (b, hkv, total, d), torch.bfloat16).cuda()
    host = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total)
    dev = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total)
    host.update(k[:, :, :prompt], v[:, :, :prompt])
    dev.update(k[:, :, :prompt], v[:, :, :prompt])
    dev.use_device_counters()
    for p in range(prompt, total):
        layer = 4 if p % 3 == 0 else 1
        rule = "xor" if p % 7 == 0 else "causal_shift"
        lay = bf.build_block_butterfly_layout(seq_len=p + 1, block_size=128, num_key_value_heads=hkv,
                                              num_key_value_groups=hq // hkv, layer_idx=layer, local_window_blocks=1,
                                              sink_count=1, partner_count=1, partner_rule=rule)
        a = host.update_and_attend(q[:, :, p:p + 1], k[:, :, p:p + 1], v[:, :, p:p + 1], layout=lay,
                                   local_window_tokens=64)
        c = dev.decode_step(q[:, :, p:p + 1], k[:, :, p:p + 1], v[:, :, p:p + 1], layer_idx=layer,
                            partner_rule=rule, local_window_tokens=64)
        assert torch.equal(a, c), (p, layer, rule)
        if p == prompt + 50:            # host bookkeeping in between: counters pushed, cached rows cleared
            dev.sync()
            dev._push()


# From 512 sequences (batch x kv heads) the step runs decode_split_kernel (d = 128, groups
# <= 16; the host path runs the workgroup kernel), so equality pins the split kernel to it
# bit for bit.  520 and 513 sequences (3 kv heads): counts that are no multiple of the route
# workgroups; GQA groups of 4 and 16; a cache window of 128 beside the attention window of 64;
# 2048 and 4096 sequences: the batch sweep's sizes, more workgroups than the chip holds at once.
@pytest.mark.parametrize("b,hq,hkv,cw,steps", [(256, 8, 2, 64, 200), (260, 32, 2, 64, 200), (171, 12, 3, 128, 200),
                                               (1024, 8, 2, 64, 60), (2048, 8, 2, 64, 60)])
def test_split_kernel_steps_equal_host_steps(b, hq, hkv, cw, steps):
    d, layer, prompt = 128, 5, 333
    total = prompt + steps
    g = torch.Generator(device="cuda").manual_seed(b + hq)
    q = torch.randn(b, hq, total, d, generator=g, device="cuda").bfloat16()
    k = torch.randn(b, hkv, total, d, generator=g, device="cuda").bfloat16()
    v = torch.randn(b, hkv, total, d, generator=g, device="cuda").bfloat16()
    host = bf.CompressedKVCache(block_size=128, local_window_tokens=cw, max_kv_size=total)
    dev = bf.CompressedKVCache(block_size=128, local_window_tokens=cw, max_kv_size=total)
    host.update(k[:, :, :prompt], v[:, :, :prompt])
    dev.update(k[:, :, :prompt], v[:, :, :prompt])
    dev.use_device_counters()
    for p in range(prompt, total):
        a = host.update_and_attend(q[:, :, p:p + 1], k[:, :, p:p + 1], v[:, :, p:p + 1],
                                   layout=_layout(p + 1, hkv, hq // hkv, layer), local_window_tokens=64)
        c = dev.decode_step(q[:, :, p:p + 1], k[:, :, p:p + 1], v[:, :, p:p + 1], layer_idx=layer,
                            local_window_tokens=64)
        assert torch.equal(a, c), p
    dev.sync()
    assert (dev.offset, dev.tail_size, dev.summary_count, dev.summary_offset) == \
           (host.offset, host.tail_size, host.summary_count, host.summary_offset)
    assert torch.equal(dev.k_summary, host.k_summary) and torch.equal(dev.v_summary, host.v_summary)
    assert torch.equal(dev.keys, host.keys) and torch.equal(dev.values, host.values)
    # and the last row is the reference's active row
    lay = tp.build_layout(seq_len=total, block_size=128, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                          layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                          partner_rule="causal_shift")
    sel = slice(0, 4)
    ref = oa.active(q[sel, :, total - 1:].cpu(), k[sel].cpu(), v[sel].cpu(), layout=lay,
                    query_positions=torch.tensor([total - 1]), W=64)
    if cw == 64:
        err = (c[sel].float().cpu() - ref.float()).abs().max().item()
        assert err <= 2e-2, err


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_cache_window_differs_from_attention_window(dtype, d):
    """The cache's own window (128, the reference's default) decides summarising and
    trimming; the attention window (64) only the keys a query sees
    (bna/mlx/compressed_cache.py:120-164).  Device step, host path and the oracle cache
    must agree on counters, pools and outputs."""
    from oracle.cache import OracleCompressedKVCache

    b, hq, hkv, layer, prompt, steps, cw, w = 2, 8, 2, 3, 333, 300, 128, 64
    total = prompt + steps
    q = _rand(91, (b, hq, total, d), dtype)
    k = _rand(92, (b, hkv, total, d), dtype)
    v = _rand(93, (b, hkv, total, d), dtype)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    host = bf.CompressedKVCache(block_size=128, local_window_tokens=cw, max_kv_size=total)
    dev = bf.CompressedKVCache(block_size=128, local_window_tokens=cw, max_kv_size=total)
    ref = OracleCompressedKVCache(block_size=128, local_window_tokens=cw, max_kv_size=total)
    host.update(kd[:, :, :prompt], vd[:, :, :prompt])
    dev.update(kd[:, :, :prompt], vd[:, :, :prompt])
    ref.update_and_fetch(k[:, :, :prompt], v[:, :, :prompt])
    dev.use_device_counters()
    grp = hq // hkv
    rep = lambda x: x.repeat_interleave(grp, dim=1)
    for p in range(prompt, total):
        a = host.update_and_attend(qd[:, :, p:p + 1], kd[:, :, p:p + 1], vd[:, :, p:p + 1],
                                   layout=_layout(p + 1, hkv, grp, layer), local_window_tokens=w)
        c = dev.decode_step(qd[:, :, p:p + 1], kd[:, :, p:p + 1], vd[:, :, p:p + 1], layer_idx=layer,
                            local_window_tokens=w)
        assert torch.equal(a, c), p
        ref.update_and_fetch(k[:, :, p:p + 1], v[:, :, p:p + 1])
        assert (host.offset, host.tail_size, host.summary_count, host.summary_offset) == \
               (ref.offset, ref.tail_size, ref.summary_count, ref.summary_offset), p
        tk, tv, sk, sv, ts, kv_len = ref.get_compressed_state()
        lay = tp.build_layout(seq_len=kv_len, block_size=128, num_key_value_heads=hkv, num_key_value_groups=grp,
                              layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                              partner_rule="causal_shift")
        want = oa.from_cache(q[:, :, p:p + 1], rep(tk), rep(tv), rep(sk), rep(sv), layout=lay,
                             query_positions=torch.tensor([p]), W=w, tail_start=ts, kv_len=kv_len)
        got, want = c.float().cpu(), want.float()
        err = (got - want).abs().max().item()
        if dtype == torch.float32:
            assert err <= 1e-5, (p, err)
        else:
            assert err <= 2e-2 and ((got - want).norm() / want.norm()).item() <= 1e-2, (p, err)
    dev.sync()
    assert (dev.offset, dev.tail_size, dev.summary_count, dev.summary_offset) == \
           (ref.offset, ref.tail_size, ref.summary_count, ref.summary_offset)
    assert ref.tail_size >= cw                       # the tail holds the cache window, not the attention's
    assert torch.equal(dev.keys, host.keys) and torch.equal(dev.k_summary, host.k_summary)
    assert torch.equal(dev.keys.cpu(), ref.keys)
    # pooled rows: fp32 means in another summation order, within one rounding of the oracle's
    tol = 1e-6 if dtype == torch.float32 else 2 ** -7
    for got_pool, want_pool in ((dev.k_summary, ref.k_summary), (dev.v_summary, ref.v_summary)):
        diff = (got_pool.float().cpu() - want_pool.float()).abs()
        assert (diff <= tol * want_pool.float().abs().clamp_min(1.0)).all()


def test_device_counter_overflow_raises_at_sync():
    cache = bf.CompressedKVCache(block_size=4, local_window_tokens=4, max_kv_size=12)   # 7 summary slots
    kv = torch.randn(1, 1, 8, 64, device="cuda").bfloat16()
    cache.update(kv, kv)
    cache.use_device_counters()
    q = torch.randn(1, 1, 1, 64, device="cuda").bfloat16()
    with pytest.raises(RuntimeError):
        for _ in range(40):
            cache.decode_step(q, kv[:, :, :1], kv[:, :, :1], layer_idx=0, local_window_tokens=4)
            cache.sync()


@pytest.mark.parametrize("b", [4, 256])            # 512 sequences: the split kernel
def test_graph_replays_match_eager_steps(b):
    hq, hkv, d, layer, prompt, steps = 8, 2, 128, 3, 1000, 150
    total = prompt + steps
    q = _rand(71, (b, hq, total, d), torch.bfloat16).cuda()
    k = _rand(72, (b, hkv, total, d), torch.bfloat16).cuda()
    v = _rand(73, (b, hkv, total, d), torch.bfloat16).cuda()
    eager = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total)
    graphed = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total)
    for c in (eager, graphed):
        c.update(k[:, :, :prompt], v[:, :, :prompt])
        c.use_device_counters()
    # static inputs of the captured step; the step index lives on the device
    qs, ks, vs = q[:, :, prompt:prompt + 1].clone(), k[:, :, prompt:prompt + 1].clone(), v[:, :, prompt:prompt + 1].clone()
    out = torch.empty_like(qs)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            graphed.decode_step(qs, ks, vs, layer_idx=layer, local_window_tokens=64, out=out)
    torch.cuda.current_stream().wait_stream(side)
    for p in range(prompt, total):
        qs.copy_(q[:, :, p:p + 1]); ks.copy_(k[:, :, p:p + 1]); vs.copy_(v[:, :, p:p + 1])
        graph.replay()
        want = eager.decode_step(q[:, :, p:p + 1], k[:, :, p:p + 1], v[:, :, p:p + 1], layer_idx=layer,
                                 local_window_tokens=64)
        torch.cuda.synchronize()
        assert torch.equal(out, want), p
    graphed.sync(); eager.sync()
    assert graphed.offset == eager.offset == total and graphed.summary_count == eager.summary_count
    # and the result is the reference's active row at the last position
    lay = tp.build_layout(seq_len=total, block_size=128, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                          layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                          partner_rule="causal_shift")
    ref = oa.active(q[:, :, total - 1:].cpu(), k.cpu(), v.cpu(), layout=lay,
                    query_positions=torch.tensor([total - 1]), W=64)
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= 2e-2, err


@pytest.mark.parametrize("batch,head_dim", [(2, 64), (1, 128)])
def test_decoder_graph_greedy_equals_eager_greedy(batch, head_dim):
    """Batch 1 at head_dim 128: the graphed steps take the fused q/k norm + RoPE decode
    step (bfly_decode_step_qk_norm), the eager ones the separate launches; the tokens
    agree only if the fused rows are bit-identical."""
    cfg = DecoderConfig(vocab_size=2048, hidden_size=512, num_layers=3, num_heads=512 // head_dim, num_kv_heads=2,
                        head_dim=head_dim, intermediate_size=1024)
    model = Decoder(cfg, seed=11)
    bf.swap_qwen_attention_with_butterfly(model, cfg=bf.compressed_butterfly_config())
    for layer in model.layers:   # non-trivial q/k norm weights
        g = torch.Generator(device="cuda").manual_seed(len(layer.self_attn.base.q_norm.weight))
        for norm in (layer.self_attn.base.q_norm, layer.self_attn.base.k_norm):
            norm.weight.data = (1 + 0.3 * torch.randn(head_dim, generator=g, device="cuda")).bfloat16()
    prompt = torch.randint(0, cfg.vocab_size, (batch, 300), generator=torch.Generator().manual_seed(5)).cuda()

    def caches():
        c = [None] * cfg.num_layers
        bf.install_compressed_kv_caches(model, c, block_size=128, local_window_tokens=64, max_kv_size=600)
        return c

    eager = model.greedy(prompt, 40, caches())
    graphed = model.greedy_graph(prompt, 40, caches())
    assert torch.equal(eager, graphed), (eager, graphed)


@pytest.mark.parametrize("fuse", [True, False])
def test_decoder_graph_with_fused_projection_and_greedy_equals_eager(fuse):
    """cfg5's attention shapes (16 heads over 4 kv heads of 128, hidden 2048) at a small depth:
    the graphed steps take the decode step with the output projection inside and the greedy
    pick from the lm_head launch's candidates with the loop's bookkeeping in one launch
    (fuse=True), or neither; either way the tokens equal the eager loop's (separate launches,
    torch.argmax over the logits), which holds only if every fused result is bit-identical."""
    import butterfly_amd.decoder as dec

    cfg = DecoderConfig(vocab_size=4096, hidden_size=2048, num_layers=2, num_heads=16, num_kv_heads=4, head_dim=128,
                        intermediate_size=1024)
    model = Decoder(cfg, seed=3)
    bf.swap_qwen_attention_with_butterfly(model, cfg=bf.compressed_butterfly_config())
    for layer in model.layers:
        g = torch.Generator(device="cuda").manual_seed(7)
        for norm in (layer.self_attn.base.q_norm, layer.self_attn.base.k_norm):
            norm.weight.data = (1 + 0.3 * torch.randn(128, generator=g, device="cuda")).bfloat16()
    prompt = torch.randint(0, cfg.vocab_size, (1, 400), generator=torch.Generator().manual_seed(8)).cuda()

    def caches():
        c = [None] * cfg.num_layers
        bf.install_compressed_kv_caches(model, c, block_size=128, local_window_tokens=64, max_kv_size=700)
        return c

    eager = model.greedy(prompt, 150, caches())        # crosses a block end: pooling inside the steps
    saved = dec.FUSE_O_PROJ, dec.FUSE_GREEDY
    dec.FUSE_O_PROJ = dec.FUSE_GREEDY = fuse
    try:
        calls = {"oproj": 0, "greedy": 0}
        real, real_adv = bf.ButterflyAttentionCore.step_oproj, dec.greedy_advance

        def counting(core, *a, **k):
            calls["oproj"] += 1
            return real(core, *a, **k)

        def counting_adv(*a, **k):
            calls["greedy"] += 1
            return real_adv(*a, **k)

        bf.ButterflyAttentionCore.step_oproj = counting
        dec.greedy_advance = counting_adv
        graphed = model.greedy_graph(prompt, 150, caches())
    finally:
        bf.ButterflyAttentionCore.step_oproj = real
        dec.greedy_advance = real_adv
        dec.FUSE_O_PROJ, dec.FUSE_GREEDY = saved
    assert (calls["oproj"] > 0) == fuse and (calls["greedy"] > 0) == fuse, calls
    assert torch.equal(eager, graphed), (eager, graphed)


def test_default_window_128_with_device_counters_takes_the_host_path():
    """The reference's compressed defaults give a 128-token attention window, beyond the
    device step's 64: with device counters on, a one-token call of the swapped layer's
    attention reads the counters back and runs the host path; its rows match the oracle
    cache's from-cache rows, and a graph-replayed decode of such a model is refused."""
    from oracle.cache import OracleCompressedKVCache

    b, hq, hkv, d, layer, prompt, steps, w = 1, 8, 2, 128, 3, 300, 80, 128
    total = prompt + steps
    q, k, v = (_rand(121 + i, (b, h, total, d), torch.bfloat16) for i, h in enumerate((hq, hkv, hkv)))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    cfg = bf.QwenButterflyConfig(path="block_sparse", block_compression="mean", block_partner_rule="causal_shift")
    assert cfg.compressed_local_window_tokens == w
    core = bf.ButterflyAttentionCore(cfg, layer_idx=layer)
    cache = bf.CompressedKVCache(block_size=128, local_window_tokens=w, max_kv_size=total)
    ref = OracleCompressedKVCache(block_size=128, local_window_tokens=w, max_kv_size=total)
    core(qd[:, :, :prompt], kd[:, :, :prompt], vd[:, :, :prompt], cache)
    ref.update_and_fetch(k[:, :, :prompt], v[:, :, :prompt])
    cache.use_device_counters()
    grp = hq // hkv
    rep = lambda x: x.repeat_interleave(grp, dim=1)
    for p in range(prompt, total):
        assert not core.runs_device_step(cache, 1, d, torch.bfloat16)
        got = core(qd[:, :, p:p + 1], kd[:, :, p:p + 1], vd[:, :, p:p + 1], cache).float().cpu()
        ref.update_and_fetch(k[:, :, p:p + 1], v[:, :, p:p + 1])
        tk, tv, sk, sv, ts, kv_len = ref.get_compressed_state()
        lay = tp.build_layout(seq_len=kv_len, block_size=128, num_key_value_heads=hkv, num_key_value_groups=grp,
                              layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                              partner_rule="causal_shift")
        want = oa.from_cache(q[:, :, p:p + 1], rep(tk), rep(tv), rep(sk), rep(sv), layout=lay,
                             query_positions=torch.tensor([p]), W=w, tail_start=ts, kv_len=kv_len).float()
        err = (got - want).abs().max().item()
        assert err <= 2e-2 and ((got - want).norm() / want.norm()).item() <= 1e-2, (p, err)
    cache.sync()
    assert (cache.offset, cache.tail_size, cache.summary_count) == (ref.offset, ref.tail_size, ref.summary_count)

    dcfg = DecoderConfig(vocab_size=1024, hidden_size=256, num_layers=2, num_heads=2, num_kv_heads=1, head_dim=128,
                         intermediate_size=512)
    model = Decoder(dcfg, seed=3)
    bf.swap_qwen_attention_with_butterfly(model, cfg=cfg)
    caches = [None] * dcfg.num_layers
    bf.install_compressed_kv_caches(model, caches, block_size=128, local_window_tokens=w, max_kv_size=512)
    prompt_ids = torch.randint(0, dcfg.vocab_size, (1, 200), generator=torch.Generator().manual_seed(9)).cuda()
    with pytest.raises(ValueError, match="at most 64 tokens"):
        model.greedy_graph(prompt_ids, 8, caches)
