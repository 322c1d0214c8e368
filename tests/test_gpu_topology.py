"""GPU: partner/neighbour table and routing tables are bit-exact vs the oracle."""
from __future__ import annotations

import pytest
import torch

import butterfly_amd as bf
from oracle import attention as oa, topology as tp

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 2, 7, 32, 33, 512, 1025, 2048])
@pytest.mark.parametrize("rule", list(tp.RULES))
def test_neighbor_table_bit_exact(n, rule):
    w = tp.width(n)
    count = max(1, 2 * w - 2) if rule == "benes" else w
    for layer in sorted(set(list(range(count + 1)) + [37])):
        for lwb, sinks, partners in [(1, 1, 1), (4, 2, 2), (0, 0, 1), (2, 0, 0)]:
            got = bf.block_neighbor_table(num_blocks=n, layer_idx=layer, partner_rule=rule,
                                          local_window_blocks=lwb, sink_count=sinks, partner_count=partners)
            want = tp.build_layout(seq_len=n * 128, block_size=128, num_key_value_heads=1, num_key_value_groups=1,
                                   layer_idx=layer, local_window_blocks=lwb, sink_count=sinks,
                                   partner_count=partners, partner_rule=rule).block_neighbors[0]
            assert got.dtype == torch.int32
            assert torch.equal(got.cpu().long(), want), (n, rule, layer, lwb, sinks, partners)


def test_neighbor_table_matches_reference_role_rows():
    """Device tables of every rule (fixed_stride and random included) against the rows the
    reference's topology module wrote (tests/golden/golden_roles.npz)."""
    from pathlib import Path

    import numpy as np

    roles = np.load(Path(__file__).resolve().parent / "golden" / "golden_roles.npz")
    checked = 0
    for key in roles.files:
        if key.endswith("/stage"):
            continue
        _, rule, n, layer, params = key.split("/")
        lwb, sinks, partners = (int(x) for x in params.split("-"))
        got = bf.block_neighbor_table(num_blocks=int(n[1:]), layer_idx=int(layer[1:]), partner_rule=rule,
                                      local_window_blocks=lwb, sink_count=sinks, partner_count=partners)
        assert torch.equal(got.cpu().long(), torch.from_numpy(roles[key][:, :, 0].astype(np.int64))), key
        checked += 1
    assert checked >= 1500


def test_layout_metadata_and_heads():
    lay = bf.build_block_butterfly_layout(seq_len=65536, block_size=128, num_key_value_heads=2,
                                          num_key_value_groups=4, layer_idx=12, local_window_blocks=1,
                                          sink_count=1, partner_count=1, partner_rule="causal_shift")
    ref = tp.build_layout(seq_len=65536, block_size=128, num_key_value_heads=2, num_key_value_groups=4,
                          layer_idx=12, local_window_blocks=1, sink_count=1, partner_count=1,
                          partner_rule="causal_shift")
    assert (lay.num_blocks, lay.stage_idx, lay.stage_count) == (512, 3, 9)
    assert lay.block_neighbors.shape == ref.block_neighbors.shape == (8, 512, 4)
    assert torch.equal(lay.block_neighbors.cpu().long(), ref.block_neighbors)
    assert lay.metadata.partner_bits == (3,)


@pytest.mark.parametrize("T,bs,W,layer", [(18, 4, 4, 2), (4096, 128, 64, 3), (1000, 128, 64, 1),
                                          (300, 64, 17, 5), (65536, 128, 64, 7)])
def test_prefill_tables_bit_exact(T, bs, W, layer):
    lay = bf.build_block_butterfly_layout(seq_len=T, block_size=bs, num_key_value_heads=2, num_key_value_groups=4,
                                          layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                                          partner_rule="causal_shift")
    ref_lay = tp.build_layout(seq_len=T, block_size=bs, num_key_value_heads=2, num_key_value_groups=4,
                              layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                              partner_rule="causal_shift")
    got = bf.compressed_butterfly_block_index_tensors(lay, T=T, local_window_tokens=W)
    want = oa.prefill_tables(ref_lay, T=T, W=W)
    for g, w_ in zip(got, want):
        assert g.shape == w_.shape
        assert torch.equal(g.cpu().to(w_.dtype), w_)


@pytest.mark.parametrize("kv_len,bs,W,layer,positions", [
    (18, 4, 4, 3, [9, 13, 17]), (4096, 128, 64, 2, list(range(3700, 4096, 7))),
    (131073, 128, 64, 10, [131072, 131000, 64, 0, 127, 128, 191, 192])])
def test_active_tables_bit_exact(kv_len, bs, W, layer, positions):
    lay = bf.build_block_butterfly_layout(seq_len=kv_len, block_size=bs, num_key_value_heads=2,
                                          num_key_value_groups=4, layer_idx=layer, local_window_blocks=1,
                                          sink_count=1, partner_count=1, partner_rule="causal_shift")
    ref_lay = tp.build_layout(seq_len=kv_len, block_size=bs, num_key_value_heads=2, num_key_value_groups=4,
                              layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                              partner_rule="causal_shift")
    qp = torch.tensor(positions)
    got = bf.compressed_butterfly_active_index_tensors(lay, kv_len=kv_len, query_positions=qp, local_window_tokens=W)
    want = oa.active_tables(ref_lay, kv_len=kv_len, query_positions=qp, W=W)
    for g, w_ in zip(got, want):
        assert torch.equal(g.cpu().to(w_.dtype), w_)
    # tail-relative variant
    ts, tl, ns = max(0, kv_len - 256), min(256, kv_len), (kv_len - 64) // bs
    got = bf.compressed_butterfly_active_index_tensors(lay, kv_len=kv_len, query_positions=qp, local_window_tokens=W,
                                                       tail_start=ts, tail_len=tl, num_summary_blocks=ns)
    want = oa.active_tables_from_tail(ref_lay, kv_len=kv_len, tail_start=ts, num_summary_blocks=ns, tail_len=tl,
                                      query_positions=qp, W=W)
    for g, w_ in zip(got, want):
        assert torch.equal(g.cpu().to(w_.dtype), w_)
