"""Pins the CPU topology oracle (oracle/topology.py) independently of its own code.

Known answers come from the reference's tests
(tests/pytorch/test_butterfly_topology.py:316-321, :454-470, :490-525, :560-582)
and from a set-based brute force of the role map.
"""
from __future__ import annotations

import math

import pytest

from oracle import topology as tp

RULES = ["xor", "bit_reversal", "benes", "causal_shift"]


def test_stage_meta_known_answers():
    assert tp.stage_meta(16, 0, "xor") == (0, 4)
    assert tp.stage_meta(8, 0, "xor") == (0, 3)
    assert tp.stage_meta(32, 0, "xor") == (0, 5)
    assert tp.stage_meta(32, 0, "causal_shift") == (0, 5)
    assert tp.stage_meta(16, 0, "benes")[1] == 2 * 4 - 2
    # widths quoted for the configs: 32->5, 512->9, 1024->10, 1025->11, 2048->11
    for n, w in [(1, 1), (2, 1), (3, 2), (32, 5), (512, 9), (1024, 10), (1025, 11), (2048, 11)]:
        assert tp.width(n) == w
    for layer in range(12):
        assert tp.stage_meta(512, layer, "causal_shift") == (layer % 9, 9)


@pytest.mark.parametrize("n", [2, 5, 33, 100, 513])
def test_width_is_integer_ceil_log2(n):
    assert tp.width(n) == (n - 1).bit_length()


def test_causal_shift_partner_is_power_of_two_predecessor():
    w = tp.width(33)
    for b in range(33):
        for bit in range(w):
            p = tp.partner_block(b, bit, 33, "causal_shift", w)
            want = b - (1 << bit)
            assert p == (None if want < 0 else want)


def _brute_row(b, n, layer, rule, lwb, sinks, partners):
    # Independent restatement: a role set per block, then order by first role
    # position in [self, locals (nearest first), partners, sinks].
    w = max(1, math.ceil(math.log2(n))) if n > 1 else 1
    count = max(1, 2 * w - 2) if rule == "benes" else w
    s = layer % count
    seq = [b] + [b - o for o in range(1, lwb + 1)]
    for j in range(partners):
        if rule == "causal_shift":
            bit = (s + j) % w
            seq.append(b - 2 ** bit)
    seq += list(range(min(sinks, n)))
    out = []
    for v in seq:
        if 0 <= v < n and v not in out:
            out.append(v)
    return out


@pytest.mark.parametrize("n", [1, 2, 7, 32, 33, 100])
@pytest.mark.parametrize("layer", [0, 1, 2, 5])
def test_causal_shift_rows_match_brute_force(n, layer):
    lay = tp.build_layout(seq_len=n * 8, block_size=8, num_key_value_heads=1, num_key_value_groups=1,
                          layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                          partner_rule="causal_shift")
    for b in range(n):
        row = [x for x in lay.block_neighbors[0, b].tolist() if x >= 0]
        assert row == _brute_row(b, n, layer, "causal_shift", 1, 1, 1)


@pytest.mark.parametrize("rule", RULES)
@pytest.mark.parametrize("n", [8, 16, 17, 32, 33])
def test_rows_causal_degree_bounded_self_first(rule, n):
    for layer in range(6):
        lay = tp.build_layout(seq_len=n * 4, block_size=4, num_key_value_heads=2, num_key_value_groups=2,
                              layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                              partner_rule=rule)
        nb = lay.block_neighbors
        assert nb.shape[0] == 4
        for h in range(1, 4):
            assert bool((nb[h] == nb[0]).all())
        for b in range(n):
            row = [x for x in nb[0, b].tolist() if x >= 0]
            assert row[0] == b
            assert len(row) == len(set(row)) <= 4
            assert all(0 <= x <= b for x in row)
            # padding only at the end
            full = nb[0, b].tolist()
            assert full[len(row):] == [-1] * (len(full) - len(row))


def test_single_block_trivial():
    lay = tp.build_layout(seq_len=10, block_size=64, num_key_value_heads=1, num_key_value_groups=1,
                          layer_idx=0, local_window_blocks=1, sink_count=1, partner_count=1,
                          partner_rule="causal_shift")
    assert lay.num_blocks == 1 and lay.block_neighbors[0, 0].tolist() == [0]


def _reach(n, layers, rule):
    reach = {i: {i} for i in range(n)}
    for layer in range(layers):
        lay = tp.build_layout(seq_len=n * 4, block_size=4, num_key_value_heads=1, num_key_value_groups=1,
                              layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                              partner_rule=rule)
        new = {i: set(reach[i]) for i in range(n)}
        for b in range(n):
            for x in lay.block_neighbors[0, b].tolist():
                if x >= 0:
                    new[b] |= reach[x]
        reach = new
    return reach


@pytest.mark.parametrize("n", [16, 32, 33, 64, 65, 100, 129, 200, 255, 257])
def test_causal_shift_full_prefix_at_log_depth(n):
    """docs/BUTTERFLY_THEOREMS.md:59-63: every block reaches its whole causal
    prefix after exactly ceil(log2 N) causal_shift layers."""
    reach = _reach(n, tp.width(n), "causal_shift")
    for b in range(n):
        assert reach[b] >= set(range(b + 1))


def test_causal_shift_needs_every_layer():
    # One layer fewer must leave some block short of its prefix (guards a rule
    # that silently links too much, e.g. an off-by-one partner).
    n = 64
    reach = _reach(n, tp.width(n) - 1, "causal_shift")
    assert any(not reach[b] >= set(range(b + 1)) for b in range(n))


def test_partner_block_with_explicit_widths():
    """butterfly_partner_block with an explicit width: bit_reversal reverses exactly the low
    ``width`` bits (bna/topology/butterfly.py:45-49, 137-138), dropping higher bits, and width
    0 reverses nothing.  Known answers worked by hand from those lines: block 5 = 0b101 over
    2 bits is 0b01 -> 0b10, flip bit 0 -> 0b11, reversed 0b11 = 3; block 3 over 0 bits is
    0, flipped to 1, reversed over 0 bits is 0.  Every rule agrees with the oracle."""
    from butterfly_amd.topology import butterfly_partner_block

    assert butterfly_partner_block(block_idx=5, bit_idx=0, num_blocks=8, partner_rule="bit_reversal", width=2) == 3
    assert butterfly_partner_block(block_idx=3, bit_idx=0, num_blocks=8, partner_rule="bit_reversal", width=0) == 0
    assert tp.bit_reverse(0b1011, 3) == 0b110 and tp.bit_reverse(0b1011, 0) == 0
    for rule in tp.RULES:
        for n in (1, 5, 8, 33, 300):
            for w in range(0, 11):
                for b in range(n):
                    for bit in range(-1, w + 1):
                        got = butterfly_partner_block(block_idx=b, bit_idx=bit, num_blocks=n, partner_rule=rule,
                                                      width=w)
                        assert got == tp.partner_block(b, bit, n, rule, w), (rule, n, w, b, bit)
