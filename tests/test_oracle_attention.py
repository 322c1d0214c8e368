"""Pins the CPU attention oracle (oracle/attention.py) against independent checks.

* the reference tests' float64 brute force (oracle/brute.py, restating
  tests/pytorch/test_compressed_butterfly_attention.py:31-85) on the
  reference's own cases (seeds 23 and 29) and on GQA / ragged / larger cases;
* block means against a float64 closed form;
* the online-softmax merge against one softmax over the union, and associativity
  (tests/mlx/test_online_softmax_merge.py:13-97 restated);
* from-cache == active rows (tests/mlx/test_compressed_butterfly_from_cache.py:16-82
  restated).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa, brute, topology as tp
from oracle.cache import OracleCompressedKVCache


def _layout(T, bs, layer, hkv=2, groups=1, rule="causal_shift"):
    return tp.build_layout(seq_len=T, block_size=bs, num_key_value_heads=hkv, num_key_value_groups=groups,
                           layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                           partner_rule=rule)


def test_reference_case_prefill_seed23():
    rng = np.random.default_rng(23)
    B, H, T, dh = 1, 2, 18, 8
    lay = _layout(T, 4, 2, hkv=H)
    q, k, v = (rng.standard_normal((B, H, T, dh), dtype=np.float32) for _ in range(3))
    y = oa.prefill(*(torch.from_numpy(x) for x in (q, k, v)), layout=lay, W=4)
    ref = brute.compressed_reference(q, k, v, lay.block_neighbors[0].numpy(), block_size=4, W=4)
    assert np.allclose(y.numpy(), ref, atol=3e-4, rtol=3e-4)
    assert np.abs(y.numpy() - ref).max() < 1e-5


def test_reference_case_active_seed29():
    rng = np.random.default_rng(29)
    B, H, Tk, Tq, dh = 1, 2, 18, 3, 8
    qp = np.asarray([9, 13, 17])
    lay = _layout(Tk, 4, 3, hkv=H)
    q = rng.standard_normal((B, H, Tq, dh), dtype=np.float32)
    k = rng.standard_normal((B, H, Tk, dh), dtype=np.float32)
    v = rng.standard_normal((B, H, Tk, dh), dtype=np.float32)
    y = oa.active(*(torch.from_numpy(x) for x in (q, k, v)), layout=lay, query_positions=torch.from_numpy(qp), W=4)
    ref = brute.compressed_reference(q, k, v, lay.block_neighbors[0].numpy(), block_size=4, W=4, query_positions=qp)
    assert np.abs(y.numpy() - ref).max() < 1e-5


@pytest.mark.parametrize("T,bs,W,layer,hkv,groups", [
    (67, 8, 5, 1, 2, 4), (64, 16, 16, 3, 1, 2), (130, 32, 20, 2, 2, 1), (45, 4, 3, 4, 2, 2)])
def test_prefill_matches_brute_force_gqa_ragged(T, bs, W, layer, hkv, groups):
    rng = np.random.default_rng(T * 7 + layer)
    hq, dh = hkv * groups, 16
    lay = _layout(T, bs, layer, hkv=hkv, groups=groups)
    q = rng.standard_normal((1, hq, T, dh), dtype=np.float32)
    k = rng.standard_normal((1, hkv, T, dh), dtype=np.float32)
    v = rng.standard_normal((1, hkv, T, dh), dtype=np.float32)
    y = oa.prefill(*(torch.from_numpy(x) for x in (q, k, v)), layout=lay, W=W)
    ref = brute.compressed_reference(q, k, v, lay.block_neighbors[0].numpy(), block_size=bs, W=W)
    assert np.abs(y.numpy() - ref).max() < 1e-5


def test_prefill_summary_terms_matter():
    # Planted mistake: dropping the routed summaries must break agreement, so the
    # brute force really exercises the compressed stream at this shape.
    rng = np.random.default_rng(5)
    T, bs, W = 96, 8, 4
    lay = _layout(T, bs, 2)
    q, k, v = (rng.standard_normal((1, 2, T, 8), dtype=np.float32) for _ in range(3))
    ref = brute.compressed_reference(q, k, v, lay.block_neighbors[0].numpy(), block_size=bs, W=W)
    no_sum = brute.compressed_reference(q, k, v, np.full_like(lay.block_neighbors[0].numpy(), -1),
                                        block_size=bs, W=W)
    assert np.abs(ref - no_sum).max() > 1e-2


@pytest.mark.parametrize("T,bs", [(18, 4), (128, 128), (130, 64), (1, 128)])
def test_block_mean_closed_form(T, bs):
    rng = np.random.default_rng(T)
    x = rng.standard_normal((2, 3, T, 8)).astype(np.float32)
    n = (T + bs - 1) // bs
    got = oa.block_mean(torch.from_numpy(x), seq_len=T, block_size=bs, num_blocks=n).numpy()
    want = brute.block_summaries(x, bs)
    assert np.abs(got - want).max() < 1e-6


def test_merge_equals_union_softmax_and_is_associative():
    rng = np.random.default_rng(0)
    d = 16
    q = torch.from_numpy(rng.standard_normal(d))
    keys = torch.from_numpy(rng.standard_normal((30, d)))
    vals = torch.from_numpy(rng.standard_normal((30, d)))
    parts = [(0, 10), (10, 22), (22, 30)]

    def stream(lo, hi):
        s = (keys[lo:hi] @ q).view(1, -1) * 0.25
        return oa._stream(s, torch.ones_like(s, dtype=torch.bool), vals[lo:hi])

    a, b, c = (stream(*p) for p in parts)

    def as_stream(o, ms):
        # (o, l, m) of a merged pair, for a second-level merge
        m = torch.maximum(ms[0][2], ms[1][2])
        l = sum(torch.exp(x[2] - m) * x[1] for x in ms)
        return o, l, m

    ab = as_stream(oa.merge(a, b), (a, b))
    left = oa.merge(ab, c)
    bc = as_stream(oa.merge(b, c), (b, c))
    right = oa.merge(a, bc)
    dense = oa.dense_union_attention(q, keys, vals, scale=0.25)
    assert torch.allclose(left.view(-1), dense, atol=1e-12)
    assert torch.allclose(right.view(-1), dense, atol=1e-12)
    empty = (torch.zeros(1, d, dtype=torch.float64), torch.zeros(1, 1, dtype=torch.float64),
             torch.full((1, 1), oa.NEG, dtype=torch.float64))
    assert torch.allclose(oa.merge(a, empty), a[0])


def test_swa_stream_is_windowed_dense():
    rng = np.random.default_rng(1)
    t, d, W = 40, 8, 5
    q, k, v = (torch.from_numpy(rng.standard_normal((1, 1, t, d))) for _ in range(3))
    o, l, m = oa.swa_stream(q, k, v, W=W, scale=0.3)
    for p in range(t):
        lo = max(0, p - W + 1)
        want = oa.dense_union_attention(q[0, 0, p], k[0, 0, lo:p + 1], v[0, 0, lo:p + 1], scale=0.3)
        assert torch.allclose(o[0, 0, p].double(), want, atol=1e-6)


def test_from_cache_equals_active_seed202():
    rng = np.random.default_rng(202)
    B, H, Tk, Tq, dh, bs, W = 1, 2, 24, 3, 8, 4, 4
    q = torch.from_numpy(rng.standard_normal((B, H, Tq, dh), dtype=np.float32))
    k = torch.from_numpy(rng.standard_normal((B, H, Tk, dh), dtype=np.float32))
    v = torch.from_numpy(rng.standard_normal((B, H, Tk, dh), dtype=np.float32))
    qp = torch.tensor([21, 22, 23])
    lay = _layout(Tk, bs, 3, hkv=H)
    ref = oa.active(q, k, v, layout=lay, query_positions=qp, W=W)
    cache = OracleCompressedKVCache(block_size=bs, local_window_tokens=W)
    for s in range(0, Tk, 3):
        cache.update_and_fetch(k[:, :, s:s + 3], v[:, :, s:s + 3])
    tk_, tv_, ks, vs, ts, off = cache.get_compressed_state()
    got = oa.from_cache(q, tk_, tv_, ks, vs, layout=lay, query_positions=qp, W=W, tail_start=ts, kv_len=off)
    assert torch.allclose(got, ref, atol=3e-4, rtol=3e-4)
    assert (got - ref).abs().max() < 1e-5


# ---- compressed stream (bna/mlx/attention.py:372-516), pinned by the reference's
# tests/mlx/test_compressed_butterfly_hca_stream.py brute forces, restated in numpy
def _softmax_rows(q, kk, vv, scale):
    s = (q @ kk.T) * scale
    w = np.exp(s - s.max())
    return (w / w.sum()) @ vv


def test_hca_stream_dense_over_prior_blocks_seed13():
    rng = np.random.default_rng(13)
    B, H, T, dh, bs = 1, 2, 32, 8, 8
    nb = T // bs
    q = rng.standard_normal((B, H, T, dh)).astype(np.float32)
    ks = rng.standard_normal((B, H, nb, dh)).astype(np.float32)
    vs = rng.standard_normal((B, H, nb, dh)).astype(np.float32)
    scale = 1.0 / math.sqrt(dh)
    o, l, m = oa.compressed_stream(torch.from_numpy(q), torch.from_numpy(ks), torch.from_numpy(vs),
                                   block_size=bs, scale=scale)
    for t in range(T):
        qb = t // bs
        for h in range(H):
            if qb == 0:
                assert l[0, h, t, 0] == 0.0 and m[0, h, t, 0] < -1e20 and (o[0, h, t] == 0).all()
                continue
            want = _softmax_rows(q[0, h, t], ks[0, h, :qb], vs[0, h, :qb], scale)
            assert np.allclose(o[0, h, t].numpy(), want, atol=3e-6)
            s = (ks[0, h, :qb] @ q[0, h, t]) * scale
            assert abs(m[0, h, t, 0].item() - s.max()) < 1e-5
            assert abs(l[0, h, t, 0].item() - np.exp(s - s.max()).sum()) < 1e-5


def test_routed_stream_via_indices_seed17():
    rng = np.random.default_rng(17)
    B, H, T, dh, bs = 1, 2, 16, 8, 4
    nb = T // bs
    q = rng.standard_normal((B, H, T, dh)).astype(np.float32)
    ks = rng.standard_normal((B, H, nb, dh)).astype(np.float32)
    vs = rng.standard_normal((B, H, nb, dh)).astype(np.float32)
    routed = np.full((H, nb, 1), -1, dtype=np.int32)
    for b in range(1, nb):
        routed[:, b, 0] = b - 1
    scale = 1.0 / math.sqrt(dh)
    o, l, m = oa.compressed_stream(torch.from_numpy(q), torch.from_numpy(ks), torch.from_numpy(vs),
                                   block_size=bs, scale=scale, routed_indices=torch.from_numpy(routed))
    for t in range(T):
        b = t // bs
        for h in range(H):
            if b == 0:
                assert l[0, h, t, 0] == 0.0 and m[0, h, t, 0] < -1e20
                continue
            assert np.allclose(o[0, h, t].numpy(), vs[0, h, b - 1], atol=1e-6)   # one key: its value
            assert abs(l[0, h, t, 0].item() - 1.0) < 1e-6


def test_routed_stream_drops_non_causal_and_invalid_entries():
    rng = np.random.default_rng(5)
    B, H, T, dh, bs = 1, 1, 12, 4, 4
    nb = 3
    q = torch.from_numpy(rng.standard_normal((B, H, T, dh)).astype(np.float32))
    ks = torch.from_numpy(rng.standard_normal((B, H, nb, dh)).astype(np.float32))
    vs = torch.from_numpy(rng.standard_normal((B, H, nb, dh)).astype(np.float32))
    routed = torch.tensor([[[0, 1, 2, -1], [1, 0, 0, 2], [2, 1, 0, 7]]], dtype=torch.int32)   # [H, 3, 4]
    o, l, m = oa.compressed_stream(q, ks, vs, block_size=bs, scale=0.5, routed_indices=routed)
    hca, lh, mh = oa.compressed_stream(q, ks, vs, block_size=bs, scale=0.5)
    # block 1 routes {1 (self, dropped), 0, 0 (duplicate, both count), 2 (future, dropped)}
    t = 5
    s0 = (ks[0, 0, 0] @ q[0, 0, t]).item() * 0.5
    assert abs(m[0, 0, t, 0].item() - s0) < 1e-6 and abs(l[0, 0, t, 0].item() - 2.0) < 1e-6
    # block 2 routes {2 (self), 1, 0, 7 (out of range)}: the same keys as HCA
    assert torch.allclose(o[0, 0, 8:], hca[0, 0, 8:], atol=1e-6)
    assert torch.allclose(l[0, 0, 8:], lh[0, 0, 8:], atol=1e-6)


def test_swa_and_routed_streams_merge_to_one_shot_prefill():
    """The reference's one-shot entry is merge(swa, compressed(routed)) with the
    block-level routing (bna/mlx/attention.py:1455-1467): check the oracle's two
    halves against its SDPA one-shot restatement."""
    rng = np.random.default_rng(29)
    B, H, T, dh, bs, W = 1, 2, 70, 8, 8, 6
    q, k, v = (torch.from_numpy(rng.standard_normal((B, H, T, dh), dtype=np.float32)) for _ in range(3))
    lay = _layout(T, bs, 3, hkv=H)
    n = lay.num_blocks
    ks = oa.block_mean(k, seq_len=T, block_size=bs, num_blocks=n)
    vs = oa.block_mean(v, seq_len=T, block_size=bs, num_blocks=n)
    _, _, sidx, smask = oa.prefill_tables(lay, T=T, W=W)
    # the Torch table pads with index 0 and a False mask; the stream takes -1 for "no entry"
    routed = torch.where(smask.any(1), sidx, torch.full_like(sidx, -1)).to(torch.int32)
    routed = routed.unsqueeze(0).expand(H, -1, -1)
    scale = dh ** -0.5
    a = oa.swa_stream(q, k, v, W=W, scale=scale)
    c = oa.compressed_stream(q, ks, vs, block_size=bs, scale=scale, routed_indices=routed)
    got = oa.merge(a, c)
    want = oa.prefill(q, k, v, layout=lay, W=W)
    assert torch.allclose(got, want, atol=2e-6)


# ---- tail-relative active routing (bna/mlx/attention.py:1601-1666)
# Three checks pin oracle.attention.active_tables_from_tail: (1) with a tail that
# holds the whole context and every block pooled it reduces to the reference-written
# active tables (tests/golden/golden.npz, bna/torch/attention_wayfinder_permute.py:969-1019);
# (2) on tiny layouts it equals a per-query enumeration over every token and every
# block (which positions the query sees, where in the tail they sit, which summary
# rows exist and lie wholly before the window); (3) planted off-by-one variants of
# the oracle fail (1) or (2).
def _from_tail_golden_failures(fn):
    from tests.golden.make_golden import ACTIVE_CASES
    import pathlib
    g = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "golden.npz")
    bad = []
    for name, _dt, _b, hq, hkv, t, _d, bs, w, layers, pos in ACTIVE_CASES:
        for layer in layers:
            lay = _layout(t, bs, layer, hkv=hkv, groups=hq // hkv)
            tabs = fn(lay, kv_len=t, tail_start=0, num_summary_blocks=lay.num_blocks, tail_len=t,
                      query_positions=torch.tensor(pos), W=w)
            for tn, got in zip(("raw_idx", "raw_mask", "summary_idx", "summary_mask"), tabs):
                want = torch.from_numpy(g[f"{name}/L{layer}/{tn}"])
                if not torch.equal(got.to(want.dtype), want):
                    bad.append((name, layer, tn))
    return bad


def _from_tail_enumerated(lay, *, kv_len, tail_start, num_summary_blocks, tail_len, query_positions, W):
    """Per-query enumeration from the definitions, over every token and block."""
    bs, n = lay.block_size, lay.num_blocks
    k = lay.block_neighbors.shape[-1]
    row_of = lay.block_neighbors[0].tolist()
    tail = list(range(tail_start, tail_start + tail_len))          # absolute position per tail slot
    out = []
    for p in query_positions:
        blk = min(p // bs, n - 1)
        first = max(0, p - W + 1)
        # raw slot j stands for absolute position first + j; it is live when that token
        # exists, is causal for p and is held in the tail
        seen = {}
        for j in range(W):
            a = first + j
            if a <= p and a < kv_len and a in tail:
                seen[j] = tail.index(a)
        ridx = [seen.get(j, min(max(first + j - tail_start, 0), max(0, tail_len - 1))) for j in range(W)]
        rmask = [j in seen for j in range(W)]
        # summary rows: entries of the block's neighbour row, in row order, that name a
        # pooled block other than the query's own whose every token precedes the window
        picks = []
        for nb in row_of[blk]:
            if nb < 0 or nb == blk or nb >= num_summary_blocks:
                continue
            if all(t < first for t in range(nb * bs, (nb + 1) * bs)) and len(picks) < k:
                picks.append(nb)
        out.append((ridx, rmask, picks + [0] * (k - len(picks)), [True] * len(picks) + [False] * (k - len(picks))))
    return out


_FROM_TAIL_TINY = [
    # (T, bs, layer, W, kv_len, tail_start, tail_len, num_summary_blocks)
    (64, 4, 2, 4, 64, 52, 12, 13), (64, 4, 3, 6, 61, 40, 21, 9), (64, 4, 1, 4, 64, 60, 4, 15),
    (40, 8, 2, 5, 40, 24, 16, 3), (40, 8, 1, 10, 37, 16, 21, 2), (33, 4, 4, 3, 33, 28, 5, 7),
    (96, 8, 3, 12, 90, 72, 18, 1), (96, 8, 2, 9, 96, 0, 96, 12), (24, 4, 0, 4, 24, 8, 16, 0),
    (64, 4, 2, 6, 64, 40, 16, 10), (48, 8, 1, 7, 45, 20, 19, 2),     # tails that end before kv_len
]


def _from_tail_enumeration_failures(fn):
    bad = []
    for T, bs, layer, W, kv_len, ts, tl, ns in _FROM_TAIL_TINY:
        lay = _layout(T, bs, layer)
        qps = [p for p in range(max(0, ts - W), kv_len)]
        got = fn(lay, kv_len=kv_len, tail_start=ts, num_summary_blocks=ns, tail_len=tl,
                 query_positions=torch.tensor(qps), W=W)
        want = _from_tail_enumerated(lay, kv_len=kv_len, tail_start=ts, num_summary_blocks=ns, tail_len=tl,
                                     query_positions=qps, W=W)
        for r, (ri, rm, si, sm) in enumerate(want):
            if (got[0][r].tolist() != ri or got[1][r].tolist() != rm or got[2][r].tolist() != si
                    or got[3][r].tolist() != sm):
                bad.append((T, bs, layer, W, kv_len, ts, tl, ns, qps[r]))
    return bad


def test_from_tail_reduces_to_reference_active_tables():
    assert _from_tail_golden_failures(oa.active_tables_from_tail) == []


def test_from_tail_equals_per_query_enumeration():
    # the cases cover tails that start mid-window, tails that end before kv_len, pools
    # that stop short of the routed partner (and an empty pool), ragged kv_len and a
    # tail holding everything
    assert _from_tail_enumeration_failures(oa.active_tables_from_tail) == []


def test_from_tail_tables_gather_the_from_cache_attention():
    # the tables drive one softmax over tail rows and pool rows; it equals the
    # from-cache entry, which the reference's from_cache == active test pins
    rng = np.random.default_rng(71)
    B, H, Tk, dh, bs, W = 1, 2, 40, 8, 4, 5
    lay = _layout(Tk, bs, 3, hkv=H)
    k = torch.from_numpy(rng.standard_normal((B, H, Tk, dh), dtype=np.float32))
    v = torch.from_numpy(rng.standard_normal((B, H, Tk, dh), dtype=np.float32))
    q = torch.from_numpy(rng.standard_normal((B, H, 6, dh), dtype=np.float32))
    cache = OracleCompressedKVCache(block_size=bs, local_window_tokens=W)
    for s in range(0, Tk, 3):
        cache.update_and_fetch(k[:, :, s:s + 3], v[:, :, s:s + 3])
    tk_, tv_, ks, vs, ts, off = cache.get_compressed_state()
    qp = torch.arange(off - 6, off)
    ri, rm, si, sm = oa.active_tables_from_tail(lay, kv_len=off, tail_start=ts, num_summary_blocks=ks.shape[2],
                                                tail_len=tk_.shape[2], query_positions=qp, W=W)
    want = oa.from_cache(q, tk_, tv_, ks, vs, layout=lay, query_positions=qp, W=W, tail_start=ts, kv_len=off)
    for r in range(6):
        keys = torch.cat([tk_[0, :, ri[r][rm[r]]], ks[0, :, si[r][sm[r]]]], 1)
        vals = torch.cat([tv_[0, :, ri[r][rm[r]]], vs[0, :, si[r][sm[r]]]], 1)
        for h in range(H):
            o = oa.dense_union_attention(q[0, h, r], keys[h], vals[h], scale=dh ** -0.5)
            assert torch.allclose(o.float(), want[0, h, r], atol=1e-5)


@pytest.mark.parametrize("old,new", [
    ("nb >= num_summary_blocks", "nb > num_summary_blocks"),          # one pool row too many
    ("(rpos < tail_end)", "(rpos <= tail_end)"),                      # one tail slot too many
    ("(rpos >= tail_start)", "(rpos > tail_start)"),                  # first tail slot dropped
    ("(rpos - tail_start)", "(rpos - tail_start + 1)"),               # tail slot index off by one
    ("(nb + 1) * bs > start", "nb * bs > start"),                     # partner inside the window
    ("start = max(0, p - W + 1)", "start = max(0, p - W)"),           # window one token wide too many
])
def test_from_tail_checks_catch_planted_mistakes(old, new):
    import inspect
    import textwrap
    src = textwrap.dedent(inspect.getsource(oa.active_tables_from_tail))
    assert src.count(old) == 1, old
    ns = dict(vars(oa))
    exec(compile(src.replace(old, new), "<planted>", "exec"), ns)
    planted = ns["active_tables_from_tail"]
    assert _from_tail_golden_failures(planted) or _from_tail_enumeration_failures(planted)


def test_from_tail_rejects_empty_context():
    lay = _layout(16, 4, 1)
    with pytest.raises(ValueError):
        oa.active_tables_from_tail(lay, kv_len=0, tail_start=0, num_summary_blocks=0, tail_len=0,
                                   query_positions=torch.tensor([0]), W=4)
