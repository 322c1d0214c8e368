"""Layer-swap surface: config validation and cache installation (CPU), and the
chunked-prefill / decode dispatch against the oracle (GPU)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import butterfly_amd as bf
from oracle import attention as oa, topology as tp


def test_config_validation_matches_reference_rules():
    bf.QwenButterflyConfig()
    for bad in [dict(path="dense"), dict(block_size=0), dict(block_local_window_blocks=-1),
                dict(block_partner_count=-1), dict(block_sink_blocks=-1), dict(block_partner_rule="zigzag"),
                dict(block_compression="max"), dict(compressed_local_window_tokens=0),
                dict(wayfinder_decode_backend="flash")]:
        with pytest.raises(ValueError):
            bf.QwenButterflyConfig(**bad)
    cfg = bf.QwenButterflyConfig()
    cfg.butterfly_decode_backend = "dense"
    assert cfg.wayfinder_decode_backend == "dense"
    with pytest.raises(NotImplementedError):
        bf.ButterflyAttentionCore(bf.QwenButterflyConfig(block_compression="none"), 0)
    with pytest.raises(NotImplementedError):
        bf.ButterflyAttentionCore(bf.QwenButterflyConfig(path="permute"), 0)


def test_install_and_swap_on_a_stub_model():
    class Attn:
        def __init__(self):
            self.swapped = None

        def butterfly_module(self, cfg, layer_idx):
            return ("butterfly", layer_idx)

    class Layer:
        def __init__(self):
            self.self_attn = Attn()

    class Model:
        layers = [Layer() for _ in range(5)]

    m = Model()
    caches = [None] * 5
    assert bf.install_compressed_kv_caches(m, caches, layer_indices=[1, 3, 9], block_size=128,
                                           local_window_tokens=64, max_kv_size=1000) == [1, 3]
    assert isinstance(caches[1], bf.CompressedKVCache) and caches[0] is None
    assert caches[3].max_kv_size == 1000 and caches[3].local_window_tokens == 64
    assert bf.swap_qwen_attention_with_butterfly(m, cfg=bf.QwenButterflyConfig(), layer_indices=[0, 4]) == [0, 4]
    assert m.layers[4].self_attn == ("butterfly", 4)
    with pytest.raises(ValueError):
        bf.install_compressed_kv_caches(object(), caches)


def _rand(seed, shape, dtype):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dtype)


def _ref_layout(t, hkv, groups, layer):
    return tp.build_layout(seq_len=t, block_size=128, num_key_value_heads=hkv, num_key_value_groups=groups,
                           layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                           partner_rule="causal_shift")


def _check(got, want, dtype):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs().max().item()
    if dtype == torch.float32:
        assert err <= 1e-5, err
    else:
        rel = ((got - want).norm() / want.norm()).item()
        assert err <= 2e-2 and rel <= 1e-2, (err, rel)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_chunked_prefill_then_decode_through_core(dtype):
    """cfg4 heads (Hq16/Hkv4/d256 for bf16) with 384-token chunks, then decode."""
    d = 256 if dtype == torch.bfloat16 else 128
    b, hq, hkv, layer, chunk, T, ndec = 1, 16, 4, 9, 384, 384 * 4 + 77, 20
    total = T + ndec
    q = _rand(41, (b, hq, total, d), dtype)
    k = _rand(42, (b, hkv, total, d), dtype)
    v = _rand(43, (b, hkv, total, d), dtype)
    cfg = bf.QwenButterflyConfig()
    core = bf.ButterflyAttentionCore(cfg, layer)
    cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total, max_chunk_size=512)
    outs = bf.chunked_prefill(core, bf.split_chunks(q[:, :, :T].cuda(), k[:, :, :T].cuda(), v[:, :, :T].cuda(),
                                                    chunk), cache)
    pos = 0
    for i, o in enumerate(outs):
        n = o.shape[2]
        lay = _ref_layout(pos + n, hkv, hq // hkv, layer)
        if i == 0:
            want = oa.prefill(q[:, :, :n], k[:, :, :n], v[:, :, :n], layout=lay, W=64)
        else:
            want = oa.active(q[:, :, pos:pos + n], k[:, :, :pos + n], v[:, :, :pos + n], layout=lay,
                             query_positions=torch.arange(pos, pos + n), W=64)
        _check(o, want, dtype)
        pos += n
    assert core.last_profile.path == "block_sparse_compressed_active"
    for p in range(T, total):
        o = core(q[:, :, p:p + 1].cuda(), k[:, :, p:p + 1].cuda(), v[:, :, p:p + 1].cuda(), cache)
        lay = _ref_layout(p + 1, hkv, hq // hkv, layer)
        want = oa.active(q[:, :, p:p + 1], k[:, :, :p + 1], v[:, :, :p + 1], layout=lay,
                         query_positions=torch.tensor([p]), W=64)
        _check(o, want, dtype)
    assert core.last_profile.notes["stage_count"] == tp.width((total + 127) // 128)


@pytest.mark.gpu
def test_stock_decode_fallback_is_dense_over_the_tail():
    dtype, d, b, hq, hkv, T = torch.bfloat16, 128, 2, 8, 2, 1000
    q = _rand(51, (b, hq, T + 1, d), dtype)
    k = _rand(52, (b, hkv, T + 1, d), dtype)
    v = _rand(53, (b, hkv, T + 1, d), dtype)
    cfg = bf.QwenButterflyConfig(wayfinder_decode_backend="dense")
    core = bf.ButterflyAttentionCore(cfg, 3)
    cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64)
    core(q[:, :, :T].cuda(), k[:, :, :T].cuda(), v[:, :, :T].cuda(), cache)
    o = core(q[:, :, T:].cuda(), k[:, :, T:].cuda(), v[:, :, T:].cuda(), cache)
    assert core.last_profile.notes["dense_fallback_reason"] == "butterfly_decode_stock"
    ts = cache.offset - cache.tail_size
    kk = k[:, :, ts:T + 1].float().repeat_interleave(4, 1)
    vv = v[:, :, ts:T + 1].float().repeat_interleave(4, 1)
    want = torch.softmax(q[:, :, T:].float() @ kk.transpose(-1, -2) / d ** 0.5, -1) @ vv
    _check(o, want, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("b,hq,hkv,d", [(1, 16, 4, 256), (2, 8, 2, 128)])
def test_native_chunk_loop_equals_per_chunk_calls(b, hq, hkv, d):
    """chunked_prefill runs chunks 2.. through bfly_stream_chunks: outputs, counters,
    ring and pool must equal those of one ButterflyAttentionCore call per chunk."""
    layer, lens = 6, [384, 384, 200, 384, 130, 3, 384, 257]
    total = sum(lens)
    q = _rand(91, (b, hq, total, d), torch.bfloat16).cuda()
    k = _rand(92, (b, hkv, total, d), torch.bfloat16).cuda()
    v = _rand(93, (b, hkv, total, d), torch.bfloat16).cuda()
    chunks, pos = [], 0
    for n in lens:
        chunks.append(tuple(t[:, :, pos:pos + n].contiguous() for t in (q, k, v)))
        pos += n
    cfg = bf.QwenButterflyConfig()
    runs = []
    for native in (True, False):
        core = bf.ButterflyAttentionCore(cfg, layer)
        cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total, max_chunk_size=512)
        outs = bf.chunked_prefill(core, chunks, cache) if native else [core(*c, cache) for c in chunks]
        runs.append((core, cache, outs))
    (ca, a, oa_), (cb, bb, ob) = runs
    assert ca.last_profile.notes.get("native_chunk_loop") == len(lens) - 1
    assert (a.offset, a.tail_size, a.summary_count, a.summary_offset) == \
           (bb.offset, bb.tail_size, bb.summary_count, bb.summary_offset)
    for x, y in zip(oa_, ob):
        assert torch.equal(x, y)
    assert torch.equal(a.k_summary, bb.k_summary) and torch.equal(a.v_summary, bb.v_summary)
    assert torch.equal(a.keys, bb.keys) and torch.equal(a.values, bb.values)


@pytest.mark.gpu
def test_native_chunk_loop_capacity_error_matches_per_chunk_calls():
    b, hq, hkv, d, layer = 1, 8, 2, 128, 2
    lens = [384] * 6
    total = sum(lens)
    q = _rand(94, (b, hq, total, d), torch.bfloat16).cuda()
    k = _rand(95, (b, hkv, total, d), torch.bfloat16).cuda()
    v = _rand(96, (b, hkv, total, d), torch.bfloat16).cuda()
    chunks = [tuple(t[:, :, i * 384:(i + 1) * 384].contiguous() for t in (q, k, v)) for i in range(6)]
    caches = []
    for native in (True, False):
        core = bf.ButterflyAttentionCore(bf.QwenButterflyConfig(), layer)
        cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=1200, max_chunk_size=512)
        with pytest.raises(RuntimeError):
            if native:
                bf.chunked_prefill(core, chunks, cache)
            else:
                for c in chunks:
                    core(*c, cache)
        caches.append(cache)
    a, bb = caches
    assert (a.offset, a.tail_size, a.summary_count, a.summary_offset) == \
           (bb.offset, bb.tail_size, bb.summary_count, bb.summary_offset)


@pytest.mark.gpu
def test_native_chunk_runs_mix_with_per_chunk_calls():
    """A run of native chunks stops at a chunk the loop does not take (two tokens): that
    chunk goes through the core, and the next run continues from the same cache."""
    b, hq, hkv, d, layer = 1, 8, 2, 128, 4
    lens = [300] + [200] * 12 + [2] + [150] * 70
    total = sum(lens)
    q = _rand(97, (b, hq, total, d), torch.bfloat16).cuda()
    k = _rand(98, (b, hkv, total, d), torch.bfloat16).cuda()
    v = _rand(99, (b, hkv, total, d), torch.bfloat16).cuda()
    chunks, pos = [], 0
    for n in lens:
        chunks.append(tuple(t[:, :, pos:pos + n].contiguous() for t in (q, k, v)))
        pos += n
    runs = []
    for native in (True, False):
        core = bf.ButterflyAttentionCore(bf.QwenButterflyConfig(), layer)
        cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total, max_chunk_size=512)
        outs = bf.chunked_prefill(core, chunks, cache) if native else [core(*c, cache) for c in chunks]
        runs.append((cache, outs))
    (a, oa_), (bb, ob) = runs
    assert len(oa_) == len(ob) == len(lens)
    for x, y in zip(oa_, ob):
        assert torch.equal(x, y)
    assert (a.offset, a.tail_size, a.summary_count, a.summary_offset) == \
           (bb.offset, bb.tail_size, bb.summary_count, bb.summary_offset)
