"""GPU: the stream-level API (SWA stream, compressed stream in routed and HCA mode,
online-softmax merge) against the oracle restatement of bna/mlx/attention.py:304-548.

Tolerances: fp32 o <= 1e-5 max-abs, l and m <= 1e-5 relative; bf16 o <= 2e-2 max-abs
and <= 1e-2 relative L2 (l, m from fp32 scores: <= 1e-4 relative).  The reference's
own stream tests (tests/mlx/test_compressed_butterfly_{swa,hca}_stream.py,
test_online_softmax_merge.py) hold the MLX path to 3e-4.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import butterfly_amd as bf
from oracle import attention as oa, topology as tp

pytestmark = pytest.mark.gpu


def _rand(seed, *shape, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def _check_stream(got, want, dtype):
    go, gl, gm = (x.float().cpu() for x in got)
    wo, wl, wm = (x.float() for x in want)
    empty = wm < -1e20
    assert torch.equal(gm < -1e20, empty)
    assert (gl[empty] == 0).all() and (go[empty.expand_as(go)] == 0).all()
    keep = ~empty
    assert torch.allclose(gm[keep], wm[keep], rtol=1e-5, atol=1e-5)
    rtol = 1e-5 if dtype == torch.float32 else 1e-4
    assert torch.allclose(gl[keep], wl[keep], rtol=rtol, atol=1e-6)
    if dtype == torch.float32:
        assert (go - wo).abs().max() <= 1e-5
    else:
        err = (go - wo).abs().max().item()
        rel = ((go - wo).norm() / wo.norm().clamp_min(1e-12)).item()
        assert err <= 2e-2 and rel <= 1e-2, (err, rel)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,h,t,d,W", [(1, 2, 32, 8, 8), (2, 4, 300, 64, 64), (1, 1, 70, 128, 1), (1, 2, 200, 96, 150)])
def test_swa_stream(dtype, b, h, t, d, W):
    q, k, v = (_rand(s, b, h, t, d, dtype=dtype) for s in (1, 2, 3))
    scale = 1.0 / math.sqrt(d)
    got = bf.swa_stream_attention(q.cuda(), k.cuda(), v.cuda(), n_win=W, scale=scale)
    assert got[0].dtype == dtype and got[1].dtype == torch.float32 and got[1].shape == (b, h, t, 1)
    _check_stream(got, oa.swa_stream(q, k, v, W=W, scale=scale), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,h,t,d,bs", [(1, 2, 32, 8, 8), (2, 2, 1000, 64, 16), (1, 4, 333, 128, 4)])
def test_hca_stream(dtype, b, h, t, d, bs):
    nb = (t + bs - 1) // bs
    q = _rand(4, b, h, t, d, dtype=dtype)
    ks, vs = _rand(5, b, h, nb, d, dtype=dtype), _rand(6, b, h, nb, d, dtype=dtype)
    scale = 1.0 / math.sqrt(d)
    got = bf.compressed_stream_attention(q.cuda(), ks.cuda(), vs.cuda(), block_size=bs, scale=scale)
    _check_stream(got, oa.compressed_stream(q, ks, vs, block_size=bs, scale=scale), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_routed_stream_random_indices(dtype):
    b, h, t, d, bs, K = 2, 3, 257, 64, 8, 70       # K > 64: two key groups per row
    nqb = (t + bs - 1) // bs
    nb = nqb - 3                                    # fewer summaries than query blocks
    g = torch.Generator().manual_seed(9)
    routed = torch.randint(-2, nqb + 2, (h, nqb + 1, K), generator=g, dtype=torch.int32)
    q = _rand(7, b, h, t, d, dtype=dtype)
    ks, vs = _rand(8, b, h, nb, d, dtype=dtype), _rand(10, b, h, nb, d, dtype=dtype)
    got = bf.compressed_stream_attention(q.cuda(), ks.cuda(), vs.cuda(), block_size=bs, scale=0.2,
                                         routed_indices=routed.cuda())
    _check_stream(got, oa.compressed_stream(q, ks, vs, block_size=bs, scale=0.2, routed_indices=routed), dtype)


def test_routed_stream_reference_case_seed17():
    """tests/mlx/test_compressed_butterfly_hca_stream.py:62-98: block b routes to b-1 only."""
    rng = np.random.default_rng(17)
    B, H, T, dh, bs = 1, 2, 16, 8, 4
    nb = T // bs
    q = torch.from_numpy(rng.standard_normal((B, H, T, dh)).astype(np.float32))
    ks = torch.from_numpy(rng.standard_normal((B, H, nb, dh)).astype(np.float32))
    vs = torch.from_numpy(rng.standard_normal((B, H, nb, dh)).astype(np.float32))
    routed = torch.full((H, nb, 1), -1, dtype=torch.int32)
    for blk in range(1, nb):
        routed[:, blk, 0] = blk - 1
    o, l, m = bf.compressed_stream_attention(q.cuda(), ks.cuda(), vs.cuda(), block_size=bs,
                                             scale=1 / math.sqrt(dh), routed_indices=routed.cuda())
    o, l = o.cpu(), l.cpu()
    for t in range(T):
        blk = t // bs
        if blk:
            assert torch.allclose(o[0, :, t], vs[0, :, blk - 1], atol=1e-6)
            assert torch.allclose(l[0, :, t, 0], torch.ones(H))
        else:
            assert (l[0, :, t] == 0).all() and (m.cpu()[0, :, t] < -1e20).all()


def test_gqa_heads_read_their_kv_head():
    b, hq, hkv, t, d, bs = 1, 8, 2, 96, 32, 8
    q = _rand(11, b, hq, t, d)
    k, v = _rand(12, b, hkv, t, d), _rand(13, b, hkv, t, d)
    rep = lambda x: x.repeat_interleave(hq // hkv, dim=1)
    got = bf.swa_stream_attention(q.cuda(), k.cuda(), v.cuda(), n_win=20, scale=0.3)
    _check_stream(got, oa.swa_stream(q, rep(k), rep(v), W=20, scale=0.3), torch.float32)
    nb = t // bs
    ks, vs = _rand(14, b, hkv, nb, d), _rand(15, b, hkv, nb, d)
    got = bf.compressed_stream_attention(q.cuda(), ks.cuda(), vs.cuda(), block_size=bs, scale=0.3)
    _check_stream(got, oa.compressed_stream(q, rep(ks), rep(vs), block_size=bs, scale=0.3), torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_merge(dtype):
    rng = np.random.default_rng(7)
    B, H, Tq, dh = 2, 3, 50, 16
    q = torch.from_numpy(rng.standard_normal((B, H, Tq, dh)).astype(np.float32))

    def stream(nk, seed):
        r = np.random.default_rng(seed)
        k = torch.from_numpy(r.standard_normal((B, H, nk, dh)).astype(np.float32))
        v = torch.from_numpy(r.standard_normal((B, H, nk, dh)).astype(np.float32))
        s = (q @ k.transpose(-1, -2)) * 0.25
        o, l, m = oa._stream(s, torch.ones_like(s, dtype=torch.bool), v)
        return (o.to(dtype), l, m), k, v

    (a, ka, va), (c, kc, vc) = stream(5, 1), stream(9, 2)
    # one row of each stream is empty (m = -1e30, l = 0, o = 0)
    a[1][0, 0, 3] = 0.0
    a[2][0, 0, 3] = oa.NEG
    a[0][0, 0, 3] = 0.0
    got = bf.online_softmax_merge(tuple(x.cuda() for x in a), tuple(x.cuda() for x in c)).cpu()
    want = oa.merge((a[0].float(), a[1], a[2]), (c[0].float(), c[1], c[2]))
    assert got.dtype == torch.float32
    assert (got - want).abs().max() <= 1e-5
    # both empty -> 0
    e = (torch.zeros(B, H, Tq, dh), torch.zeros(B, H, Tq, 1), torch.full((B, H, Tq, 1), oa.NEG))
    z = bf.online_softmax_merge(tuple(x.cuda() for x in e), tuple(x.cuda() for x in e))
    assert (z == 0).all()


@pytest.mark.parametrize("layer", [0, 2, 4])
def test_streams_compose_to_one_shot_prefill(layer):
    """merge(swa, compressed(routed by the block-level table)) is the reference's one-shot
    entry (bna/mlx/attention.py:1455-1467): compare with the fused prefill kernel."""
    B, H, T, d, bs, W = 1, 2, 600, 64, 32, 24
    q, k, v = (_rand(20 + i, B, H, T, d) for i in range(3))
    kw = dict(seq_len=T, block_size=bs, num_key_value_heads=H, num_key_value_groups=1, layer_idx=layer,
              local_window_blocks=1, sink_count=1, partner_count=1, partner_rule="causal_shift")
    lay, ref_lay = bf.build_block_butterfly_layout(**kw), tp.build_layout(**kw)
    n = lay.num_blocks
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    ks, vs = bf.block_mean_summaries(kc, seq_len=T, block_size=bs, num_blocks=n, x2=vc)
    _, _, sidx, smask = oa.prefill_tables(ref_lay, T=T, W=W)
    routed = torch.where(smask.any(1), sidx, torch.full_like(sidx, -1)).to(torch.int32)
    routed = routed.unsqueeze(0).expand(H, -1, -1).contiguous().cuda()
    scale = d ** -0.5
    a = bf.swa_stream_attention(qc, kc, vc, n_win=W, scale=scale)
    c = bf.compressed_stream_attention(qc, ks, vs, block_size=bs, scale=scale, routed_indices=routed)
    merged = bf.online_softmax_merge(a, c)
    fused, _ = bf.compressed_butterfly_attention(qc, kc, vc, layout=lay, local_window_tokens=W)
    assert (merged - fused.float()).abs().max().item() <= 2e-5


def test_stream_argument_errors():
    q = torch.randn(1, 2, 16, 8, device="cuda")
    ks = torch.randn(1, 2, 4, 8, device="cuda")
    with pytest.raises(ValueError):
        bf.compressed_stream_attention(q, ks, ks, block_size=4, scale=1.0,
                                       routed_indices=torch.zeros(2, 3, 1, dtype=torch.int32))   # 3 < 4 blocks
    with pytest.raises(ValueError):
        bf.compressed_stream_attention(q, ks, ks, block_size=0, scale=1.0)
    with pytest.raises(ValueError):
        bf.swa_stream_attention(q, ks, ks, n_win=4, scale=1.0)
    o, l, m = bf.swa_stream_attention(q[:, :, :0], q[:, :, :0], q[:, :, :0], n_win=4, scale=1.0)
    assert o.shape == (1, 2, 0, 8) and m.shape == (1, 2, 0, 1)
