"""GPU: compressor and one-shot prefill vs the CPU oracle.

Tolerances (north_star): fp32 <= 1e-5 max-abs; bf16 <= 2e-2 max-abs and
<= 1e-2 relative L2 against the oracle run in bf16 on the same inputs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import butterfly_amd as bf
from oracle import attention as oa, topology as tp

pytestmark = pytest.mark.gpu

BF16_MAX_ABS = 2e-2
BF16_REL_L2 = 1e-2
F32_MAX_ABS = 1e-5


def _inputs(seed, b, hq, hkv, t, d, dtype, k_scale=False):
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.standard_normal((b, hq, t, d), dtype=np.float32))
    k = torch.from_numpy(rng.standard_normal((b, hkv, t, d), dtype=np.float32))
    v = torch.from_numpy(rng.standard_normal((b, hkv, t, d), dtype=np.float32))
    if k_scale:
        k = k * torch.from_numpy(rng.uniform(0.5, 2.0, size=(d,)).astype(np.float32))
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _layouts(t, bs, hkv, groups, layer, lwb=1, sinks=1, partners=1, rule="causal_shift"):
    kw = dict(seq_len=t, block_size=bs, num_key_value_heads=hkv, num_key_value_groups=groups, layer_idx=layer,
              local_window_blocks=lwb, sink_count=sinks, partner_count=partners, partner_rule=rule)
    return bf.build_block_butterfly_layout(**kw), tp.build_layout(**kw)


def _close_bf16(got, want):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs().max().item()
    rel = ((got - want).norm() / want.norm()).item()
    assert err <= BF16_MAX_ABS and rel <= BF16_REL_L2, (err, rel)
    return err, rel


# ---------------------------------------------------------------- compressor
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("t,bs,d", [(4096, 128, 128), (1000, 128, 128), (18, 4, 8), (700, 64, 256), (129, 128, 64)])
def test_block_mean(dtype, t, bs, d):
    _, k, v = _inputs(t, 2, 2, 3, t, d, dtype)
    n = (t + bs - 1) // bs
    gk, gv = bf.block_mean_summaries(k.cuda(), seq_len=t, block_size=bs, num_blocks=n, x2=v.cuda())
    wk = oa.block_mean(k, seq_len=t, block_size=bs, num_blocks=n)
    wv = oa.block_mean(v, seq_len=t, block_size=bs, num_blocks=n)
    if dtype == torch.float32:
        assert (gk.cpu() - wk).abs().max() < 1e-6 and (gv.cpu() - wv).abs().max() < 1e-6
    else:
        # fp32 sums in a different order may round to the neighbouring bf16 value
        assert ((gk.cpu().float() - wk.float()).abs() <= wk.float().abs() * 2 ** -7 + 1e-6).all()
        assert ((gv.cpu().float() - wv.float()).abs() <= wv.float().abs() * 2 ** -7 + 1e-6).all()
        assert (gk.cpu() == wk).float().mean() > 0.97


# ---------------------------------------------------------------- cfg1: fp32 parity, layers 0..4
@pytest.mark.parametrize("layer", [0, 1, 2, 3, 4])
def test_cfg1_fp32_layers(layer):
    q, k, v = _inputs(1, 1, 8, 2, 4096, 128, torch.float32)
    lay, ref_lay = _layouts(4096, 128, 2, 4, layer)
    assert lay.stage_idx == layer and lay.stage_count == 5
    assert torch.equal(lay.block_neighbors.cpu().long(), ref_lay.block_neighbors)
    y = bf.butterfly_compressed_attention(q.cuda(), k.cuda(), v.cuda(), layout=lay, local_window_tokens=64)
    want = oa.prefill(q, k, v, layout=ref_lay, W=64)
    err = (y.cpu() - want).abs().max().item()
    assert err <= F32_MAX_ABS, err


# ---------------------------------------------------------------- cfg2: bf16 64k, all 9 stages
def test_cfg2_bf16_all_stages():
    q, k, v = _inputs(2, 1, 8, 2, 65536, 128, torch.bfloat16, k_scale=True)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    for layer in range(9):
        lay, ref_lay = _layouts(65536, 128, 2, 4, layer)
        assert lay.stage_count == 9
        y, _ = bf.compressed_butterfly_attention(qd, kd, vd, layout=lay, local_window_tokens=64)
        want = oa.prefill(q, k, v, layout=ref_lay, W=64)
        err, rel = _close_bf16(y, want)
        print(f"stage {layer}: max_abs={err:.3e} rel_l2={rel:.3e}", flush=True)


# ---------------------------------------------------------------- shapes and edge cases
CASES = [
    # (b, hq, hkv, t, d, bs, W, layer, dtype)
    (1, 8, 2, 1, 128, 128, 64, 0, torch.bfloat16),
    (1, 8, 2, 63, 128, 128, 64, 2, torch.bfloat16),
    (1, 8, 2, 129, 128, 128, 64, 1, torch.bfloat16),
    (2, 8, 2, 1000, 128, 128, 64, 3, torch.bfloat16),
    (1, 4, 4, 777, 128, 64, 64, 2, torch.bfloat16),
    (1, 16, 2, 2048, 128, 128, 17, 4, torch.bfloat16),
    (1, 2, 1, 1500, 64, 128, 64, 5, torch.bfloat16),
    (1, 16, 4, 3000, 256, 128, 64, 6, torch.bfloat16),
    # d = 256 with two / four chunks per workgroup segment: the kept page moves between the LDS
    # halves from chunk to chunk, forwards in even segments and backwards in odd ones
    (2, 16, 4, 8192, 256, 128, 64, 5, torch.bfloat16),
    (2, 16, 4, 16384, 256, 128, 64, 7, torch.bfloat16),
    (1, 8, 2, 4096, 128, 128, 100, 3, torch.bfloat16),   # W > 64: generic kernel
    (1, 8, 2, 999, 96, 32, 33, 2, torch.bfloat16),      # d=96, BS<64: generic kernel
    (1, 2, 2, 18, 8, 4, 4, 2, torch.float32),           # reference test shape
    (2, 6, 3, 333, 40, 16, 9, 7, torch.float32),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(x) for x in c))
def test_prefill_cases(case):
    b, hq, hkv, t, d, bs, W, layer, dtype = case
    q, k, v = _inputs(t + d, b, hq, hkv, t, d, dtype)
    lay, ref_lay = _layouts(t, bs, hkv, hq // hkv, layer)
    y, _ = bf.compressed_butterfly_attention(q.cuda(), k.cuda(), v.cuda(), layout=lay, local_window_tokens=W)
    want = oa.prefill(q, k, v, layout=ref_lay, W=W)
    if dtype == torch.float32:
        assert (y.cpu() - want).abs().max().item() <= F32_MAX_ABS
    else:
        _close_bf16(y, want)


def test_prefill_custom_scale_and_errors():
    q, k, v = _inputs(3, 1, 8, 2, 512, 128, torch.bfloat16)
    lay, ref_lay = _layouts(512, 128, 2, 4, 1)
    y, _ = bf.compressed_butterfly_attention(q.cuda(), k.cuda(), v.cuda(), layout=lay, local_window_tokens=64,
                                             scale=0.05)
    want = oa.prefill(q * (0.05 * 128 ** 0.5), k, v, layout=ref_lay, W=64)
    _close_bf16(y, want)
    with pytest.raises(NotImplementedError):
        bf.compressed_butterfly_attention(q.cuda(), k.cuda(), v.cuda(), layout=lay, local_window_tokens=64,
                                          return_weights=True)
    with pytest.raises(ValueError):
        bf.compressed_butterfly_attention(q.cuda(), k[:, :, :100].cuda(), v[:, :, :100].cuda(), layout=lay,
                                          local_window_tokens=64)
    lay3, _ = _layouts(511, 128, 2, 4, 1)
    with pytest.raises(ValueError):
        bf.compressed_butterfly_attention(q.cuda(), k.cuda(), v.cuda(), layout=lay3, local_window_tokens=64)


# fp32 tile kernel (attn_f32_tile_kernel): W <= 64, d 64 / 128, GQA groups of at most 4, block size a
# multiple of 16; ragged lengths, windows shorter than a tile, batch 2
F32_TILE_CASES = [
    # b, hq, hkv, t, d, bs, W, layer
    (2, 6, 2, 333, 64, 16, 17, 3),
    (1, 3, 3, 500, 128, 32, 1, 2),
    (1, 4, 1, 777, 128, 64, 64, 5),
    (2, 8, 2, 1000, 128, 128, 64, 2),
    (1, 2, 2, 100, 64, 16, 64, 1),
    (1, 8, 4, 4099, 128, 128, 48, 7),
]


@pytest.mark.parametrize("case", F32_TILE_CASES, ids=lambda c: "-".join(str(x) for x in c))
def test_f32_tile_prefill_cases(case):
    b, hq, hkv, t, d, bs, W, layer = case
    q, k, v = _inputs(t + 11 * d, b, hq, hkv, t, d, torch.float32)
    lay, ref_lay = _layouts(t, bs, hkv, hq // hkv, layer)
    y, _ = bf.compressed_butterfly_attention(q.cuda(), k.cuda(), v.cuda(), layout=lay, local_window_tokens=W)
    want = oa.prefill(q, k, v, layout=ref_lay, W=W)
    assert (y.cpu() - want).abs().max().item() <= F32_MAX_ABS


@pytest.mark.parametrize("d,W,bs,step,hq,hkv", [(128, 64, 128, 100, 8, 2), (64, 20, 16, 37, 4, 4),
                                                (128, 64, 64, 384, 4, 1)])
def test_f32_tile_ring_chunks_match_active(d, W, bs, step, hq, hkv):
    """Chunks attended from the device ring (fp32 tile kernel, ring mode): chunk starts off the
    16-position tiles, the ring wrapping, token-level summary cut-off; each chunk against the
    oracle's active rows over the full keys."""
    from butterfly_amd import CompressedKVCache

    b, layer, total = 2, 6, 2000
    q, k, v = _inputs(d + step, b, hq, hkv, total, d, torch.float32)
    cache = CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=total, max_chunk_size=512)
    pos = 0
    while pos < total:
        n = min(step, total - pos)
        kc, vc, qc = k[:, :, pos:pos + n].cuda(), v[:, :, pos:pos + n].cuda(), q[:, :, pos:pos + n].cuda()
        cache.update(kc, vc)
        kv_len = pos + n
        lay, ref_lay = _layouts(kv_len, bs, hkv, hq // hkv, layer)
        if pos == 0:
            got, _ = bf.compressed_butterfly_attention(qc, kc, vc, layout=lay, local_window_tokens=W)
            want = oa.prefill(q[:, :, :n], k[:, :, :n], v[:, :, :n], layout=ref_lay, W=W)
        else:
            got = bf.compressed_butterfly_attention_cached(qc, cache, layout=lay, local_window_tokens=W)
            want = oa.active(q[:, :, pos:kv_len], k[:, :, :kv_len], v[:, :, :kv_len], layout=ref_lay,
                             query_positions=torch.arange(pos, kv_len), W=W)
        err = (got.cpu() - want).abs().max().item()
        assert err <= F32_MAX_ABS, (pos, err)
        pos = kv_len
    assert cache.tail_capacity < total          # the ring wrapped
