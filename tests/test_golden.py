"""The CPU oracle reproduces the reference's own Torch path bit for bit.

``tests/golden/golden.npz`` was written by ``tests/golden/make_golden.py``
from the reference (bna/torch/attention_wayfinder_permute.py:568-682,
912-1197).  Inputs are regenerated here from the recorded seeds; their
checksums guard the recipe.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as oa, topology as tp
from tests.golden.make_golden import ACTIVE_CASES, PREFILL_CASES, TABLE_NS, TABLE_PARAMS, TABLE_RULES, digest, \
    make_inputs

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")


def _tensor(a: np.ndarray, like: torch.dtype) -> torch.Tensor:
    if like == torch.bfloat16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a))


def _layout(t, bs, hkv, g, layer):
    return tp.build_layout(seq_len=t, block_size=bs, num_key_value_heads=hkv, num_key_value_groups=g,
                           layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                           partner_rule="causal_shift")


def _inputs(name, dt):
    seed, b, hq, hkv, t, d, bs, w = (int(x) for x in G[f"{name}/meta"])
    q, k, v = make_inputs(seed, b, hq, hkv, t, d, dt)
    assert [digest(x) for x in (q, k, v)] == list(G[f"{name}/digest"]), "input recipe drifted"
    return q, k, v, (b, hq, hkv, t, d, bs, w)


@pytest.mark.parametrize("case", PREFILL_CASES, ids=lambda c: c[0])
def test_prefill_matches_reference_bits(case):
    name, dt, *_ , layers = case
    q, k, v, (b, hq, hkv, t, d, bs, w) = _inputs(name, dt)
    n = (t + bs - 1) // bs
    tdt = q.dtype
    assert torch.equal(oa.block_mean(k, seq_len=t, block_size=bs, num_blocks=n), _tensor(G[f"{name}/k_summary"], tdt))
    assert torch.equal(oa.block_mean(v, seq_len=t, block_size=bs, num_blocks=n), _tensor(G[f"{name}/v_summary"], tdt))
    for layer in layers:
        lay = _layout(t, bs, hkv, hq // hkv, layer)
        assert torch.equal(lay.block_neighbors[0].int(), torch.from_numpy(G[f"{name}/L{layer}/block_neighbors"]))
        tabs = oa.prefill_tables(lay, T=t, W=w)
        for tn, got in zip(("raw_idx", "raw_mask", "summary_idx", "summary_mask"), tabs):
            want = torch.from_numpy(G[f"{name}/L{layer}/{tn}"])
            assert torch.equal(got.to(want.dtype), want), tn
        y = oa.prefill(q, k, v, layout=lay, W=w)
        assert torch.equal(y, _tensor(G[f"{name}/L{layer}/out"], tdt)), (name, layer)


@pytest.mark.parametrize("case", ACTIVE_CASES, ids=lambda c: c[0])
def test_active_matches_reference_bits(case):
    name, dt, *_, layers, pos = case
    q, k, v, (b, hq, hkv, t, d, bs, w) = _inputs(name, dt)
    qp = torch.tensor(pos)
    qa = q[:, :, : len(pos)].contiguous()
    for layer in layers:
        lay = _layout(t, bs, hkv, hq // hkv, layer)
        tabs = oa.active_tables(lay, kv_len=t, query_positions=qp, W=w)
        for tn, got in zip(("raw_idx", "raw_mask", "summary_idx", "summary_mask"), tabs):
            want = torch.from_numpy(G[f"{name}/L{layer}/{tn}"])
            assert torch.equal(got.to(want.dtype), want), tn
        y = oa.active(qa, k, v, layout=lay, query_positions=qp, W=w)
        assert torch.equal(y, _tensor(G[f"{name}/L{layer}/out"], q.dtype)), (name, layer)


def test_neighbor_tables_match_reference():
    checked = 0
    for n in TABLE_NS:
        for rule in TABLE_RULES:
            for lwb, sinks, partners in TABLE_PARAMS:
                _, count = tp.stage_meta(n, 0, rule)
                for layer in range(count + 1):
                    key = f"nbr/{rule}/N{n}/L{layer}/{lwb}-{sinks}-{partners}"
                    lay = tp.build_layout(seq_len=n * 4, block_size=4, num_key_value_heads=1, num_key_value_groups=1,
                                          layer_idx=layer, local_window_blocks=lwb, sink_count=sinks,
                                          partner_count=partners, partner_rule=rule)
                    assert torch.equal(lay.block_neighbors[0], torch.from_numpy(G[key].astype(np.int64))), key
                    assert (lay.stage_idx, lay.stage_count) == tuple(int(x) for x in G[key + "/stage"]), key
                    checked += 1
    assert checked > 500


# ------------------------------------------------------------------ HIP path against the same vectors
def _tol_check(got: torch.Tensor, want: torch.Tensor, dt: str) -> None:
    got, want = got.float().cpu(), want.float()
    err = (got - want).abs().max().item()
    if dt == "f32":
        assert err <= 1e-5, err
    else:
        rel = ((got - want).norm() / want.norm()).item()
        assert err <= 2e-2 and rel <= 1e-2, (err, rel)


@pytest.mark.gpu
@pytest.mark.parametrize("case", PREFILL_CASES, ids=lambda c: c[0])
def test_hip_prefill_matches_reference_vectors(case):
    import butterfly_amd as bf

    name, dt, *_, layers = case
    q, k, v, (b, hq, hkv, t, d, bs, w) = _inputs(name, dt)
    for layer in layers:
        lay = bf.build_block_butterfly_layout(seq_len=t, block_size=bs, num_key_value_heads=hkv,
                                              num_key_value_groups=hq // hkv, layer_idx=layer, local_window_blocks=1,
                                              sink_count=1, partner_count=1, partner_rule="causal_shift")
        assert torch.equal(lay.block_neighbors[0].cpu(), torch.from_numpy(G[f"{name}/L{layer}/block_neighbors"]))
        y = bf.butterfly_compressed_attention(q.cuda(), k.cuda(), v.cuda(), layout=lay, local_window_tokens=w)
        _tol_check(y, _tensor(G[f"{name}/L{layer}/out"], q.dtype), dt)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ACTIVE_CASES, ids=lambda c: c[0])
def test_hip_active_matches_reference_vectors(case):
    import butterfly_amd as bf

    name, dt, *_, layers, pos = case
    q, k, v, (b, hq, hkv, t, d, bs, w) = _inputs(name, dt)
    qa = q[:, :, : len(pos)].contiguous()
    for layer in layers:
        lay = bf.build_block_butterfly_layout(seq_len=t, block_size=bs, num_key_value_heads=hkv,
                                              num_key_value_groups=hq // hkv, layer_idx=layer, local_window_blocks=1,
                                              sink_count=1, partner_count=1, partner_rule="causal_shift")
        y = bf.butterfly_compressed_attention_active(qa.cuda(), k.cuda(), v.cuda(), layout=lay,
                                                     query_positions=torch.tensor(pos), local_window_tokens=w)
        _tol_check(y, _tensor(G[f"{name}/L{layer}/out"], q.dtype), dt)
