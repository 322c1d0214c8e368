"""GPU: the fused decode kernel (append + attention over the two-pool cache) vs the oracle.

Every decode output is compared with the oracle's active row over the full
K/V (bna/torch/attention_wayfinder_permute.py:1125-1197), with the layout
rebuilt for the live kv_len as the reference integration does.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import butterfly_amd as bf
from oracle import attention as oa, topology as tp

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


@pytest.mark.parametrize("dtype,d,hq,hkv,b", [(torch.bfloat16, 128, 8, 2, 2), (torch.float32, 128, 8, 2, 1),
                                              (torch.bfloat16, 256, 16, 4, 1), (torch.bfloat16, 64, 4, 1, 3),
                                              (torch.float32, 64, 6, 3, 2),
                                              # GQA groups of 20 (two 16-head MFMA passes), 3 and 1
                                              (torch.bfloat16, 128, 40, 2, 1), (torch.bfloat16, 128, 3, 1, 2),
                                              (torch.bfloat16, 64, 5, 5, 1)])
def test_decode_steps_across_block_boundaries(dtype, d, hq, hkv, b):
    bs, W, prompt, ndec, layer = 128, 64, 300, 300, 6
    total = prompt + ndec
    q = _rand(21, (b, hq, total, d), dtype)
    k = _rand(22, (b, hkv, total, d), dtype)
    v = _rand(23, (b, hkv, total, d), dtype)
    cache = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=total)
    cache.update(k[:, :, :prompt].cuda(), v[:, :, :prompt].cuda())
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    summaries_seen = set()
    for pos in range(prompt, total):
        lay, ref_lay = _layouts(pos + 1, bs, hkv, hq // hkv, layer)
        got = cache.update_and_attend(qd[:, :, pos:pos + 1], kd[:, :, pos:pos + 1], vd[:, :, pos:pos + 1],
                                      layout=lay, local_window_tokens=W)
        want = oa.active(q[:, :, pos:pos + 1], k[:, :, :pos + 1], v[:, :, :pos + 1], layout=ref_lay,
                         query_positions=torch.tensor([pos]), W=W)
        _check(got, want, dtype)
        summaries_seen.add(cache.summary_count)
    assert len(summaries_seen) >= 2          # the compressor ran during decode
    # the ring holds exactly the appended tokens
    assert torch.equal(cache.keys.cpu(), k[:, :, cache.offset - cache.tail_size:cache.offset])


def test_decode_cfg3_shape_matches_from_cache_oracle():
    """cfg3 shape: 131072-token context, tail 256 + 1023 summaries, B=4, 130 decode steps."""
    b, hq, hkv, d, bs, W, ctx, steps = 4, 8, 2, 128, 128, 64, 131072, 130
    g = torch.Generator().manual_seed(5)
    tk = torch.randn(b, hkv, 256, d, generator=g).bfloat16()
    tv = torch.randn(b, hkv, 256, d, generator=g).bfloat16()
    sk = torch.randn(b, hkv, 1023, d, generator=g).bfloat16()
    sv = torch.randn(b, hkv, 1023, d, generator=g).bfloat16()
    cache = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=ctx + 256, max_chunk_size=512)
    cache.state = (tk.cuda(), tv.cuda(), sk.cuda(), sv.cuda())
    cache.meta_state = (str(bs), str(W), str(ctx), str(1023 * bs))
    kn = torch.randn(steps, b, hkv, 1, d, generator=g).bfloat16()
    vn = torch.randn(steps, b, hkv, 1, d, generator=g).bfloat16()
    qn = torch.randn(steps, b, hq, 1, d, generator=g).bfloat16()
    tail_k, tail_v = tk, tv
    pool_k, pool_v = sk, sv
    grp = hq // hkv
    rep = lambda x: x.repeat_interleave(grp, dim=1)
    for s in range(steps):
        kv_len = ctx + s + 1
        lay, ref_lay = _layouts(kv_len, bs, hkv, grp, 3)
        got = cache.update_and_attend(qn[s].cuda(), kn[s].cuda(), vn[s].cuda(), layout=lay, local_window_tokens=W)
        # oracle state: tail grows by one token, pool by the blocks the cache summarised
        tail_k = torch.cat([tail_k, kn[s]], 2)
        tail_v = torch.cat([tail_v, vn[s]], 2)
        tail_start = kv_len - tail_k.shape[2]
        while cache.summary_count > pool_k.shape[2]:
            n = pool_k.shape[2]
            r0 = n * bs - tail_start
            pool_k = torch.cat([pool_k, tail_k[:, :, r0:r0 + bs].float().mean(2, keepdim=True).bfloat16()], 2)
            pool_v = torch.cat([pool_v, tail_v[:, :, r0:r0 + bs].float().mean(2, keepdim=True).bfloat16()], 2)
        want = oa.from_cache(qn[s], rep(tail_k), rep(tail_v), rep(pool_k), rep(pool_v), layout=ref_lay,
                             query_positions=torch.tensor([kv_len - 1]), W=W, tail_start=tail_start, kv_len=kv_len)
        _check(got, want, torch.bfloat16)
    assert cache.summary_count == 1024 and pool_k.shape[2] == 1024


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_single_row_entries_use_decode_kernel(dtype):
    """Active / from-cache entry points with one query at the newest position."""
    b, hq, hkv, d, bs, W, T = 2, 8, 2, 128, 128, 64, 1000
    q = _rand(31, (b, hq, 1, d), dtype)
    k = _rand(32, (b, hkv, T, d), dtype)
    v = _rand(33, (b, hkv, T, d), dtype)
    lay, ref_lay = _layouts(T, bs, hkv, hq // hkv, 2)
    qp = torch.tensor([T - 1])
    y, _ = bf.compressed_butterfly_attention_active(q.cuda(), k.cuda(), v.cuda(), layout=lay, query_positions=qp,
                                                    local_window_tokens=W)
    want = oa.active(q, k, v, layout=ref_lay, query_positions=qp, W=W)
    _check(y, want, dtype)
    ts = T - 200
    n = ts // bs
    ksum = oa.block_mean(k, seq_len=T, block_size=bs, num_blocks=lay.num_blocks)[:, :, :n]
    vsum = oa.block_mean(v, seq_len=T, block_size=bs, num_blocks=lay.num_blocks)[:, :, :n]
    y2, _ = bf.compressed_butterfly_attention_from_cache(q.cuda(), k[:, :, ts:].cuda(), v[:, :, ts:].cuda(),
                                                         ksum.cuda(), vsum.cuda(), layout=lay, query_positions=qp,
                                                         local_window_tokens=W, tail_start=ts, kv_len=T)
    grp = hq // hkv
    rep = lambda x: x.repeat_interleave(grp, dim=1)
    want2 = oa.from_cache(q, rep(k[:, :, ts:]), rep(v[:, :, ts:]), rep(ksum), rep(vsum), layout=ref_lay,
                          query_positions=qp, W=W, tail_start=ts, kv_len=T)
    _check(y2, want2, dtype)


@pytest.mark.parametrize("rule,lwb,sinks,partners,bs,W", [("xor", 2, 2, 2, 64, 17), ("benes", 1, 3, 2, 96, 64),
                                                          ("bit_reversal", 0, 1, 3, 64, 40),
                                                          ("random", 3, 0, 1, 128, 1)])
def test_decode_routing_variants(rule, lwb, sinks, partners, bs, W):
    """Other partner rules, sink/partner counts, block sizes and windows through the
    decode kernel's in-kernel routed selection (lane per row entry, first-occurrence dedup)."""
    b, hq, hkv, d, prompt, ndec, layer = 2, 8, 2, 128, 5 * bs + 7, 2 * bs + 3, 7
    total = prompt + ndec
    q = _rand(31, (b, hq, total, d), torch.bfloat16)
    k = _rand(32, (b, hkv, total, d), torch.bfloat16)
    v = _rand(33, (b, hkv, total, d), torch.bfloat16)
    cache = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=total)
    cache.update(k[:, :, :prompt].cuda(), v[:, :, :prompt].cuda())
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    for pos in range(prompt, total):
        kw = dict(seq_len=pos + 1, block_size=bs, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                  layer_idx=layer, local_window_blocks=lwb, sink_count=sinks, partner_count=partners,
                  partner_rule=rule)
        lay, ref_lay = bf.build_block_butterfly_layout(**kw), tp.build_layout(**kw)
        got = cache.update_and_attend(qd[:, :, pos:pos + 1], kd[:, :, pos:pos + 1], vd[:, :, pos:pos + 1],
                                      layout=lay, local_window_tokens=W)
        want = oa.active(q[:, :, pos:pos + 1], k[:, :, :pos + 1], v[:, :, :pos + 1], layout=ref_lay,
                         query_positions=torch.tensor([pos]), W=W)
        _check(got, want, torch.bfloat16)
