"""GPU: active rows, from-cache attention and the device two-pool cache vs the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import butterfly_amd as bf
from oracle import attention as oa, topology as tp
from oracle.cache import OracleCompressedKVCache

pytestmark = pytest.mark.gpu

BF16_MAX_ABS, BF16_REL_L2, F32_MAX_ABS = 2e-2, 1e-2, 1e-5


def _rand(seed, shape, dtype):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dtype)


def _layouts(t, bs, hkv, groups, layer):
    kw = dict(seq_len=t, block_size=bs, num_key_value_heads=hkv, num_key_value_groups=groups, layer_idx=layer,
              local_window_blocks=1, sink_count=1, partner_count=1, partner_rule="causal_shift")
    return bf.build_block_butterfly_layout(**kw), tp.build_layout(**kw)


def _check(got, want, dtype):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs().max().item()
    if dtype == torch.float32:
        assert err <= F32_MAX_ABS, err
    else:
        rel = ((got - want).norm() / want.norm()).item()
        assert err <= BF16_MAX_ABS and rel <= BF16_REL_L2, (err, rel)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tk,positions,layer", [
    (18, [9, 13, 17], 3),
    (4096, list(range(3712, 4096)), 2),
    (4096, [0, 1, 63, 64, 127, 128, 129, 1000, 4095], 4),
    (131072, list(range(131072 - 70, 131072)), 9),
])
def test_active_rows(dtype, tk, positions, layer):
    bs, W = (4, 4) if tk == 18 else (128, 64)
    hq, hkv, d = (2, 2, 8) if tk == 18 else (8, 2, 128)
    q = _rand(1, (1, hq, len(positions), d), dtype)
    k = _rand(2, (1, hkv, tk, d), dtype)
    v = _rand(3, (1, hkv, tk, d), dtype)
    lay, ref_lay = _layouts(tk, bs, hkv, hq // hkv, layer)
    qp = torch.tensor(positions)
    y, _ = bf.compressed_butterfly_attention_active(q.cuda(), k.cuda(), v.cuda(), layout=lay, query_positions=qp,
                                                    local_window_tokens=W)
    want = oa.active(q, k, v, layout=ref_lay, query_positions=qp, W=W)
    _check(y, want, dtype)
    # device positions take the general path; results must agree
    y2, _ = bf.compressed_butterfly_attention_active(q.cuda(), k.cuda(), v.cuda(), layout=lay,
                                                     query_positions=qp.cuda(), local_window_tokens=W)
    _check(y2, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_from_cache_matches_oracle(dtype):
    b, hq, hkv, d, bs, W, T, step = 2, 8, 2, 128, 128, 64, 3000, 384
    k = _rand(4, (b, hkv, T, d), dtype)
    v = _rand(5, (b, hkv, T, d), dtype)
    cache = OracleCompressedKVCache(block_size=bs, local_window_tokens=W)
    for s in range(0, T, step):
        cache.update_and_fetch(k[:, :, s:s + step], v[:, :, s:s + step])
    tk_, tv_, ks, vs, ts, off = cache.get_compressed_state()
    tq = T - (T // step) * step or step
    qp = torch.arange(off - tq, off)
    q = _rand(6, (b, hq, tq, d), dtype)
    lay, ref_lay = _layouts(off, bs, hkv, hq // hkv, 5)
    got, _ = bf.compressed_butterfly_attention_from_cache(q.cuda(), tk_.cuda(), tv_.cuda(), ks.cuda(), vs.cuda(),
                                                          layout=lay, query_positions=qp, local_window_tokens=W,
                                                          tail_start=ts, kv_len=off)
    g = hq // hkv
    rep = lambda x: x.repeat_interleave(g, dim=1)  # the oracle's from_cache takes broadcast heads
    want = oa.from_cache(q, rep(tk_), rep(tv_), rep(ks), rep(vs), layout=ref_lay, query_positions=qp, W=W,
                         tail_start=ts, kv_len=off)
    _check(got, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bs,W,step,T,d", [(4, 4, 3, 24, 8), (128, 64, 384, 4000, 128), (16, 8, 5, 301, 16),
                                          (128, 64, 1, 700, 128)])
def test_device_cache_tracks_oracle(dtype, bs, W, step, T, d):
    k = _rand(7, (2, 2, T, d), dtype)
    v = _rand(8, (2, 2, T, d), dtype)
    dev = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_chunk_size=max(512, step))
    ref = OracleCompressedKVCache(block_size=bs, local_window_tokens=W, max_chunk_size=max(512, step))
    for s in range(0, T, step):
        kd, vd = dev.update_and_fetch(k[:, :, s:s + step].cuda(), v[:, :, s:s + step].cuda())
        kr, vr = ref.update_and_fetch(k[:, :, s:s + step], v[:, :, s:s + step])
        assert (dev.offset, dev.tail_size, dev.summary_count, dev.summary_offset) == \
               (ref.offset, ref.tail_size, ref.summary_count, ref.summary_offset)
        assert torch.equal(kd.cpu(), kr) and torch.equal(vd.cpu(), vr)
    gk, gv = dev.k_summary.cpu().float(), dev.v_summary.cpu().float()
    wk, wv = ref.k_summary.float(), ref.v_summary.float()
    tol = 1e-6 if dtype == torch.float32 else 2 ** -7
    assert ((gk - wk).abs() <= wk.abs() * tol + 1e-6).all()
    assert ((gv - wv).abs() <= wv.abs() * tol + 1e-6).all()
    assert dev.nbytes == ref.nbytes
    st = dev.get_compressed_state()
    assert st[4] == ref.offset - ref.tail_size and st[5] == ref.offset


def test_cache_state_round_trip_and_errors():
    k = _rand(9, (1, 2, 12, 8), torch.float32).cuda()
    cache = bf.CompressedKVCache(block_size=4, local_window_tokens=4)
    cache.update_and_fetch(k, k)
    restored = bf.CompressedKVCache(block_size=1, local_window_tokens=1)
    restored.state = cache.state
    restored.meta_state = cache.meta_state
    assert (restored.offset, restored.summary_offset, restored.block_size, restored.local_window_tokens) == \
           (cache.offset, cache.summary_offset, cache.block_size, cache.local_window_tokens)
    assert torch.equal(restored.keys, cache.keys) and torch.equal(restored.k_summary, cache.k_summary)
    more = _rand(10, (1, 2, 5, 8), torch.float32).cuda()
    cache.update_and_fetch(more, more)
    restored.update_and_fetch(more, more)
    assert torch.equal(restored.keys, cache.keys)
    assert torch.equal(restored.k_summary, cache.k_summary)
    small = bf.CompressedKVCache(block_size=4, local_window_tokens=4, max_chunk_size=2)
    with pytest.raises(RuntimeError):
        small.update_and_fetch(torch.zeros(1, 1, 64, 4, device="cuda"), torch.zeros(1, 1, 64, 4, device="cuda"))
    tiny = bf.CompressedKVCache(block_size=4, local_window_tokens=4, max_kv_size=4)
    with pytest.raises(RuntimeError):
        for _ in range(20):
            tiny.update_and_fetch(torch.zeros(1, 1, 4, 4, device="cuda"), torch.zeros(1, 1, 4, 4, device="cuda"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_chunked_prefill_then_decode_matches_active(dtype):
    """cfg4-style streaming prefill (Hq16/Hkv4/d256, 384-token chunks) then decode.

    Chunk 1 takes the one-shot path; later chunks and decode read the device
    ring + pool (bna/integrations/qwen_mlx.py:1311-1318, 1515-1581).  Every
    output is checked against the oracle's active rows over the full K/V,
    with the layout rebuilt for the live kv_len.
    """
    b, hq, hkv, d, bs, W, step = 1, 16, 4, 256, 128, 64, 384
    T, ndec = 384 * 5 + 100, 40
    total = T + ndec
    q = _rand(11, (b, hq, total, d), dtype)
    k = _rand(12, (b, hkv, total, d), dtype)
    v = _rand(13, (b, hkv, total, d), dtype)
    cache = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=total, max_chunk_size=512)
    pos = 0
    layer = 7
    while pos < total:
        n = min(step, T - pos) if pos < T else 1
        kc, vc, qc = k[:, :, pos:pos + n].cuda(), v[:, :, pos:pos + n].cuda(), q[:, :, pos:pos + n].cuda()
        cache.update(kc, vc)
        kv_len = pos + n
        lay, ref_lay = _layouts(kv_len, bs, hkv, hq // hkv, layer)
        if pos == 0:
            got, _ = bf.compressed_butterfly_attention(qc, kc, vc, layout=lay, local_window_tokens=W)
            want = oa.prefill(q[:, :, :n], k[:, :, :n], v[:, :, :n], layout=ref_lay, W=W)
        else:
            got = bf.compressed_butterfly_attention_cached(qc, cache, layout=lay, local_window_tokens=W)
            want = oa.active(q[:, :, pos:pos + n], k[:, :, :kv_len], v[:, :, :kv_len], layout=ref_lay,
                             query_positions=torch.arange(pos, kv_len), W=W)
        _check(got, want, dtype)
        pos = kv_len
