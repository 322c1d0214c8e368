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
                dict(wayfinder_decode_backend="flash"), dict(strategy="spiral"), dict(window=-1),
                dict(num_cycles=0), dict(path="block_sparse", strategy="greedy")]:
        with pytest.raises(ValueError):
            bf.QwenButterflyConfig(**bad)
    bf.QwenButterflyConfig(num_cycles="auto")
    cfg = bf.compressed_butterfly_config()
    cfg.butterfly_decode_backend = "dense"
    assert cfg.wayfinder_decode_backend == "dense"
    for bad_path in (bf.QwenButterflyConfig(), bf.QwenButterflyConfig(path="block_sparse"),
                     bf.QwenButterflyConfig(path="permute", block_compression="mean")):
        with pytest.raises(NotImplementedError):
            bf.ButterflyAttentionCore(bad_path, 0)
    bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), 0)


def test_config_defaults_are_the_reference_defaults():
    """bna/integrations/qwen_mlx.py:84-125: the dataclass defaults, field for field."""
    c = bf.QwenButterflyConfig()
    want = dict(path="permute", strategy="random", window=64, landmark_stride=64, num_cycles=1, edge_disjoint=True,
                enforce_hamiltonian=True, regular_num_clusters=8, seed=0, edge_bias=True, window_drop=0.0,
                compiled_graph_dir=None, block_size=128, block_local_window_blocks=1, block_partner_count=1,
                block_sink_blocks=1, block_partner_rule="xor", block_compression="none",
                compressed_local_window_tokens=128, permute_head_chunk_size=8, query_chunk_size=256,
                permute_stream_o_proj=False, permute_log_chunks=False, compute_edge_utilization_proxy=True,
                compute_graph_metrics=True, retro_backfill_enabled=False, retro_backfill_alpha=0.0,
                retro_backfill_training_only=True, retro_backfill_causal_only=True, circular=False,
                multi_cycle_mode="average", verify_spectral_gap=False, spectral_gap_threshold=4.0,
                use_fused_dispatch=True, active_dense_threshold=None, wayfinder_decode_backend="active_permute")
    import dataclasses
    assert [f.name for f in dataclasses.fields(c)] == list(want)
    assert {k: getattr(c, k) for k in want} == want
    assert bf.QwenWayfinderConfig is bf.QwenButterflyConfig


def test_harness_config_call_constructs():
    """The keyword set of the reference harness's call (scripts/bench_qwen_consumer_mlx.py:1771-1800),
    for its compressed_butterfly mode."""
    cfg = bf.QwenButterflyConfig(
        path="block_sparse", strategy="random", window=64, landmark_stride=None, num_cycles=1, edge_disjoint=True,
        enforce_hamiltonian=True, seed=0, edge_bias=True, window_drop=0.0, permute_head_chunk_size=8,
        query_chunk_size=64, compute_edge_utilization_proxy=False, compute_graph_metrics=False,
        retro_backfill_enabled=False, retro_backfill_alpha=0.0, retro_backfill_training_only=True,
        retro_backfill_causal_only=True, use_fused_dispatch=True, wayfinder_decode_backend="active_permute",
        block_size=128, block_local_window_blocks=1, block_partner_count=1, block_sink_blocks=1,
        block_partner_rule="causal_shift", block_compression="mean", compressed_local_window_tokens=64)
    assert cfg.is_compressed
    core = bf.ButterflyAttentionCore(cfg, 3)
    assert core.cfg.compressed_local_window_tokens == 64


class _Linear(torch.nn.Linear):
    pass


class _Attn(torch.nn.Module):
    """A module with the attribute set of mlx_lm / HF Qwen attention."""

    def __init__(self, hidden=64, hq=4, hkv=2, d=16, gated=False):
        super().__init__()
        self.num_attention_heads, self.num_key_value_heads, self.head_dim = hq, hkv, d
        self.scaling = d ** -0.5
        self.q_proj = _Linear(hidden, hq * d * (2 if gated else 1), bias=False)
        self.k_proj = _Linear(hidden, hkv * d, bias=False)
        self.v_proj = _Linear(hidden, hkv * d, bias=False)
        self.o_proj = _Linear(hq * d, hidden, bias=False)


class _Layer:
    def __init__(self, attn=True, is_linear=None):
        if attn:
            self.self_attn = _Attn()
        else:
            self.linear_attn = object()
        if is_linear is not None:
            self.is_linear = is_linear


class _Model:
    def __init__(self, layers):
        self.layers = layers


def test_full_attention_layers_and_install_default():
    """Hybrid models: only layers with full attention get a cache or a swap by default
    (bna/integrations/qwen_mlx.py:1795-1859)."""
    m = _Model([_Layer(False, True), _Layer(False, True), _Layer(True, False), _Layer(False, True), _Layer(True)])
    assert bf.get_qwen_full_attention_layer_indices(m) == [2, 4]
    caches = [None] * 5
    assert bf.install_compressed_kv_caches(m, caches) == [2, 4]
    assert caches[0] is None and isinstance(caches[2], bf.CompressedKVCache)
    assert caches[2].local_window_tokens == 128 and caches[2].max_chunk_size == 512
    caches = [None] * 5
    assert bf.install_compressed_kv_caches(m, caches, layer_indices=[1, 3, 9], block_size=128,
                                           local_window_tokens=64, max_kv_size=1000) == [1, 3]
    assert caches[3].max_kv_size == 1000 and caches[3].local_window_tokens == 64
    with pytest.raises(ValueError):
        bf.install_compressed_kv_caches(object(), caches)


def test_qwen35_full_attention_layout_validation():
    """validate_qwen35_full_attention_layers (bna/integrations/qwen_mlx.py:1862-1877): the
    full-attention layers of Qwen 3.5 are every fourth of 32 (3, 7, .., 31)."""
    assert bf.EXPECTED_QWEN35_FULL_ATTENTION_LAYERS == (3, 7, 11, 15, 19, 23, 27, 31)
    m = _Model([_Layer(False, True) if i % 4 != 3 else _Layer(True, False) for i in range(32)])
    assert bf.validate_qwen35_full_attention_layers(m) == [3, 7, 11, 15, 19, 23, 27, 31]
    odd = _Model([_Layer(False, True), _Layer(True, False), _Layer(False, True), _Layer(True, False)])
    with pytest.raises(ValueError, match="expected=.*discovered=\\[1, 3\\]"):
        bf.validate_qwen35_full_attention_layers(odd)
    with pytest.warns(UserWarning, match="Unexpected Qwen 3.5 full-attention layer layout"):
        assert bf.validate_qwen35_full_attention_layers(odd, allow_mismatch=True) == [1, 3]


def test_layout_cache_drops_other_lengths():
    """Per-length eviction of cached layouts (bna/integrations/qwen_mlx.py:52-81) over the
    cache's keys (sequence length first): entries of other lengths go, the current
    length's stay."""
    from butterfly_amd import integrations, layout
    saved = list(layout._LAYOUT_CACHE.items())
    layout._LAYOUT_CACHE.clear()
    try:
        for t, li in ((256, 3), (384, 3), (512, 3), (384, 4)):
            layout._LAYOUT_CACHE[(t, 128, 2, 4, li, 1, 1, 1, "causal_shift", "cuda:0")] = object()
        assert integrations._qwen_graph_cache_drop_other_keys(384) == 2
        assert sorted(k[4] for k in layout._LAYOUT_CACHE) == [3, 4] and all(k[0] == 384 for k in layout._LAYOUT_CACHE)
        assert bf.drop_layouts_for_other_lengths(384) == 0
        assert bf.drop_layouts_for_other_lengths(512) == 2 and not layout._LAYOUT_CACHE
    finally:
        layout._LAYOUT_CACHE.clear()
        layout._LAYOUT_CACHE.update(saved)


@pytest.mark.gpu
def test_layout_cache_eviction_keeps_the_current_length_shared():
    kw = dict(block_size=128, num_key_value_heads=2, num_key_value_groups=4, layer_idx=3, local_window_blocks=1,
              partner_rule="causal_shift")
    bf.clear_layout_cache()
    lays = {t: bf.build_block_butterfly_layout(seq_len=t, **kw) for t in (256, 384, 512)}
    keep = bf.build_block_butterfly_layout(seq_len=384, **dict(kw, layer_idx=4))
    assert bf.drop_layouts_for_other_lengths(384) == 2
    assert bf.build_block_butterfly_layout(seq_len=384, **kw) is lays[384]
    assert bf.build_block_butterfly_layout(seq_len=384, **dict(kw, layer_idx=4)) is keep
    rebuilt = bf.build_block_butterfly_layout(seq_len=512, **kw)
    assert rebuilt is not lays[512] and torch.equal(rebuilt.block_neighbors, lays[512].block_neighbors)
    bf.clear_layout_cache()


def test_compress_profile_counters_reset_and_dump():
    """The BNA_COMPRESS_PROFILE counters (bna/mlx/attention.py:45-79): reset zeroes them and
    dump returns a copy of the store."""
    from butterfly_amd import attention as at
    at._compress_stats["calls"] = 3
    at._compress_stats["shapes"].append({"seq_len": 1})
    d = at._compress_profile_dump()
    assert d["calls"] == 3 and d is not at._compress_stats
    at._compress_profile_reset()
    assert at._compress_profile_dump() == {"calls": 0, "summary_ms": 0.0, "attn_ms": 0.0, "shapes": []}


@pytest.mark.gpu
def test_compress_profile_counts_the_compressor_and_the_active_attention(monkeypatch):
    """With the profile on, the active entry's compressor (K and V pooled by one launch, two
    calls as the reference counts them) and its attention add wall time and shapes."""
    from butterfly_amd import attention as at
    monkeypatch.setattr(at, "_COMPRESS_PROFILE", True)
    at._compress_profile_reset()
    q = _rand(81, (1, 8, 64, 128), torch.bfloat16).cuda()
    k = _rand(82, (1, 2, 640, 128), torch.bfloat16).cuda()
    v = _rand(83, (1, 2, 640, 128), torch.bfloat16).cuda()
    lay = bf.build_block_butterfly_layout(seq_len=640, block_size=128, num_key_value_heads=2, num_key_value_groups=4,
                                          layer_idx=2, local_window_blocks=1, partner_rule="causal_shift")
    out, _ = bf.compressed_butterfly_attention_active(q, k, v, layout=lay, query_positions=list(range(576, 640)),
                                                      local_window_tokens=64)
    assert torch.isfinite(out.float()).all()
    d = at._compress_profile_dump()
    assert d["calls"] == 2 and d["summary_ms"] > 0 and d["attn_ms"] > 0
    assert d["shapes"] == [{"seq_len": 640, "block_size": 128, "num_blocks": 5, "x_shape": [1, 2, 640, 128],
                            "x_dtype": "torch.bfloat16"}] * 2
    monkeypatch.setattr(at, "_COMPRESS_PROFILE", False)
    bf.compressed_butterfly_attention_active(q, k, v, layout=lay, query_positions=list(range(576, 640)),
                                             local_window_tokens=64)
    assert at._compress_profile_dump()["calls"] == 2     # nothing counted with the profile off
    at._compress_profile_reset()


def test_swap_wraps_modules_with_the_attribute_set():
    m = _Model([_Layer(False, True), _Layer(True, False), _Layer(True, False)])
    cfg = bf.compressed_butterfly_config()
    assert bf.swap_qwen_attention_with_butterfly(m, cfg=cfg) == [1, 2]
    attn = m.layers[2].self_attn
    assert isinstance(attn, bf.QwenButterflyAttention) and attn.layer_idx == 2
    assert (attn.n_heads, attn.n_kv_heads, attn.head_dim) == (4, 2, 16) and attn.scale == 16 ** -0.5
    assert [a.layer_idx for a in bf.iter_qwen_butterfly_layers(m)] == [1, 2]
    m2 = _Model([_Layer(True, False) for _ in range(3)])
    assert bf.swap_qwen_attention_with_butterfly(m2, cfg=cfg, layer_indices=[0, 2]) == [0, 2]
    with pytest.raises(NotImplementedError):     # other Butterfly paths are not built here
        bf.swap_qwen_attention_with_butterfly(_Model([_Layer(True, False)]), cfg=bf.QwenButterflyConfig())


def test_swapped_module_projects_like_the_reference_on_cpu():
    """Projection, q/k norm, gate split and RoPE of the swapped module (qwen_mlx.py:288-357); the
    attention itself needs the GPU, and a CPU input is refused rather than computed another way."""
    torch.manual_seed(0)
    base = _Attn(gated=True)
    base.q_norm = torch.nn.RMSNorm(16, eps=1e-6)
    base.k_norm = torch.nn.RMSNorm(16, eps=1e-6)
    attn = bf.QwenButterflyAttention(base, bf.compressed_butterfly_config(), layer_idx=1)
    x = torch.randn(2, 5, 64)
    pos = torch.arange(5).float()
    inv = 1.0 / (1e4 ** (torch.arange(0, 16, 2).float() / 16))
    ang = torch.cat([pos[:, None] * inv, pos[:, None] * inv], -1)
    q, k, v, gate = attn.project(x, None, (ang.cos(), ang.sin()))
    qr, gr = base.q_proj(x).view(2, 5, 4, 32).chunk(2, -1)
    qr = base.q_norm(qr).transpose(1, 2)
    rot = lambda t: torch.cat([-t[..., 8:], t[..., :8]], -1)
    assert torch.allclose(q, qr * ang.cos() + rot(qr) * ang.sin(), atol=1e-5)
    assert torch.allclose(gate, gr.reshape(2, 5, 64))
    assert torch.allclose(v, base.v_proj(x).view(2, 5, 2, 16).transpose(1, 2))
    assert k.shape == (2, 2, 5, 16)
    with pytest.raises(ValueError):
        attn(x, position_embeddings=(ang.cos(), ang.sin()))


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
    cfg = bf.compressed_butterfly_config()
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


def test_chunked_prefill_pauses_the_cyclic_collector_and_restores_it():
    """chunked_prefill runs its loop with Python's cyclic GC paused and leaves it as it found
    it, also when a chunk raises (a stand-in core and cache: no native loop, CPU only)."""
    import gc
    seen = []

    def core(q, k, v, cache):
        seen.append(gc.isenabled())
        if q.shape[2] == 3:
            raise RuntimeError("planted")
        return q

    chunks = [tuple(torch.zeros(1, 1, n, 4) for _ in range(3)) for n in (5, 4, 6)]
    was = gc.isenabled()
    try:
        for enabled in (True, False):
            gc.enable() if enabled else gc.disable()
            seen.clear()
            outs = bf.chunked_prefill(core, chunks, object())
            assert [o.shape[2] for o in outs] == [5, 4, 6] and seen == [False] * 3
            assert gc.isenabled() == enabled
            with pytest.raises(RuntimeError, match="planted"):
                bf.chunked_prefill(core, chunks + [tuple(torch.zeros(1, 1, 3, 4) for _ in range(3))], object())
            assert gc.isenabled() == enabled
    finally:
        gc.enable() if was else gc.disable()


def test_native_call_sizes_grow_in_whole_batches():
    """Chunks per bfly_stream_chunks call after the first run: whole batches of the native loop
    (at most ten chunks, and half the ring minus two pages), about 1.3 times the run before, at
    least one batch, at most 256 chunks rounded up to a whole batch."""
    from types import SimpleNamespace

    from butterfly_amd.integrations import _stream_run

    def schedule(tail_capacity, chunk_len, first=8, total=682):
        cache = SimpleNamespace(tail_capacity=tail_capacity)
        runs, run, done = [], first, 0
        while done < total:
            runs.append(min(run, total - done))
            done += runs[-1]
            run = _stream_run(cache, chunk_len, run)
        return runs

    # cfg4: a ring of 8512 rows and chunks of 384 -> batches of ten
    assert schedule(8512, 384) == [8, 10, 20, 30, 40, 60, 80, 110, 150, 174]
    cache = SimpleNamespace(tail_capacity=8512)
    assert _stream_run(cache, 384, 200) == 260 and _stream_run(cache, 384, 260) == 260
    # a ring of 1344 rows (max_chunk_size 512): one chunk of 384 per batch, growth alone
    assert schedule(1344, 384, total=60) == [8, 10, 13, 16, 13]
    # batches bounded by the ring, not the cap of ten: (8512 - 128) // 2 // 1000 = 4 chunks
    runs = schedule(8512, 1000, total=300)
    assert all(r % 4 == 0 for r in runs[1:-1]) and runs[1] == 12
    # a chunk longer than half the ring still makes progress, one chunk per batch
    assert _stream_run(SimpleNamespace(tail_capacity=1344), 4096, 8) == 10


@pytest.mark.gpu
def test_stock_decode_fallback_is_dense_over_the_tail():
    dtype, d, b, hq, hkv, T = torch.bfloat16, 128, 2, 8, 2, 1000
    q = _rand(51, (b, hq, T + 1, d), dtype)
    k = _rand(52, (b, hkv, T + 1, d), dtype)
    v = _rand(53, (b, hkv, T + 1, d), dtype)
    cfg = bf.compressed_butterfly_config(wayfinder_decode_backend="dense")
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
@pytest.mark.parametrize("b,hq,hkv,d,max_chunk", [(1, 16, 4, 256, 512), (2, 8, 2, 128, 512), (1, 16, 4, 256, 2048),
                                                   (2, 8, 2, 128, 1024), (1, 16, 4, 256, 4096)])
def test_native_chunk_loop_equals_per_chunk_calls(b, hq, hkv, d, max_chunk):
    """chunked_prefill runs chunks 2.. through bfly_stream_chunks: outputs, counters,
    ring and pool must equal those of one ButterflyAttentionCore call per chunk.  A ring of
    a few chunks (max_chunk_size 512) gives one chunk per launch; larger rings batch several
    chunks per attention launch and per update job (blocks pooled across chunk boundaries
    inside a batch, batches fused with the next batch's update or not)."""
    _native_loop_matches_per_chunk(b, hq, hkv, d, max_chunk,
                                   [384, 384, 200, 384, 130, 3, 384, 257, 384, 384, 384, 100, 384, 384])


@pytest.mark.gpu
@pytest.mark.parametrize("b,hq,hkv,d,max_chunk", [(1, 16, 4, 256, 4096), (2, 8, 2, 128, 2048), (1, 16, 4, 256, 1024),
                                                   (4, 16, 8, 256, 4096)])
def test_native_chunk_loop_on_the_page_grid_equals_per_chunk_calls(b, hq, hkv, d, max_chunk):
    """Every chunk a multiple of 64 tokens: the batches read their own tokens from the chunk
    inputs and copy only the tail they leave to the ring; outputs, counters, tail and pool
    must still equal the one-call-per-chunk schedule's.  At batch 4 with 8 kv heads the d = 256
    batches hold two chunks per workgroup segment (the LDS page shift inside a batched launch)."""
    _native_loop_matches_per_chunk(b, hq, hkv, d, max_chunk,
                                   [384, 384, 256, 448, 64, 384, 128, 384, 384, 320, 384, 384, 192, 384, 384, 384])


def _native_loop_matches_per_chunk(b, hq, hkv, d, max_chunk, lens):
    layer = 6
    total = sum(lens)
    q = _rand(91, (b, hq, total, d), torch.bfloat16).cuda()
    k = _rand(92, (b, hkv, total, d), torch.bfloat16).cuda()
    v = _rand(93, (b, hkv, total, d), torch.bfloat16).cuda()
    chunks, pos = [], 0
    for n in lens:
        chunks.append(tuple(t[:, :, pos:pos + n].contiguous() for t in (q, k, v)))
        pos += n
    cfg = bf.compressed_butterfly_config()
    runs = []
    for native in (True, False):
        core = bf.ButterflyAttentionCore(cfg, layer)
        cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total,
                                     max_chunk_size=max_chunk)
        outs = bf.chunked_prefill(core, chunks, cache) if native else [core(*c, cache) for c in chunks]
        runs.append((core, cache, outs))
    (ca, a, oa_), (cb, bb, ob) = runs
    assert ca.last_profile.notes.get("native_chunk_loop", 0) > 0     # (chunks of the last native run)
    assert (a.offset, a.tail_size, a.summary_count, a.summary_offset) == \
           (bb.offset, bb.tail_size, bb.summary_count, bb.summary_offset)
    for x, y in zip(oa_, ob):
        assert torch.equal(x, y)
    assert torch.equal(a.k_summary, bb.k_summary) and torch.equal(a.v_summary, bb.v_summary)
    assert torch.equal(a.keys, bb.keys) and torch.equal(a.values, bb.values)


@pytest.mark.gpu
def test_native_chunk_loop_takes_non_contiguous_chunks():
    """Chunks given as strided views (slices of the whole sequence along its length) go through
    the native loop as contiguous copies: outputs and cache equal those of contiguous chunks."""
    b, hq, hkv, d, layer = 1, 16, 4, 256, 3
    lens = [384, 384, 320, 384, 200, 384, 384]
    total = sum(lens)
    q = _rand(71, (b, hq, total, d), torch.bfloat16).cuda()
    k = _rand(72, (b, hkv, total, d), torch.bfloat16).cuda()
    v = _rand(73, (b, hkv, total, d), torch.bfloat16).cuda()
    runs = []
    for contiguous in (True, False):
        chunks, pos = [], 0
        for n in lens:
            views = tuple(t[:, :, pos:pos + n] for t in (q, k, v))
            assert not any(x.is_contiguous() for x in views)
            chunks.append(tuple(x.contiguous() for x in views) if contiguous else views)
            pos += n
        core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), layer)
        cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total, max_chunk_size=4096)
        runs.append((core, cache, bf.chunked_prefill(core, chunks, cache)))
    (ca, a, oa_), (cb, bb, ob) = runs
    assert ca.last_profile.notes.get("native_chunk_loop", 0) > 0 and cb.last_profile.notes.get("native_chunk_loop", 0) > 0
    for x, y in zip(oa_, ob):
        assert torch.equal(x, y)
    assert torch.equal(a.k_summary, bb.k_summary) and torch.equal(a.keys, bb.keys)


@pytest.mark.gpu
@pytest.mark.parametrize("max_chunk", [512, 2048])     # 2048: the pool runs out inside a batch
def test_native_chunk_loop_capacity_error_matches_per_chunk_calls(max_chunk):
    b, hq, hkv, d, layer = 1, 8, 2, 128, 2
    lens = [384] * 6
    total = sum(lens)
    q = _rand(94, (b, hq, total, d), torch.bfloat16).cuda()
    k = _rand(95, (b, hkv, total, d), torch.bfloat16).cuda()
    v = _rand(96, (b, hkv, total, d), torch.bfloat16).cuda()
    chunks = [tuple(t[:, :, i * 384:(i + 1) * 384].contiguous() for t in (q, k, v)) for i in range(6)]
    caches = []
    for native in (True, False):
        core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), layer)
        cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=1200,
                                     max_chunk_size=max_chunk)
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
    assert torch.equal(a.k_summary, bb.k_summary) and torch.equal(a.keys, bb.keys)


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
        core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), layer)
        cache = bf.CompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=total, max_chunk_size=1024)
        outs = bf.chunked_prefill(core, chunks, cache) if native else [core(*c, cache) for c in chunks]
        runs.append((cache, outs))
    (a, oa_), (bb, ob) = runs
    assert len(oa_) == len(ob) == len(lens)
    for x, y in zip(oa_, ob):
        assert torch.equal(x, y)
    assert (a.offset, a.tail_size, a.summary_count, a.summary_offset) == \
           (bb.offset, bb.tail_size, bb.summary_count, bb.summary_offset)
