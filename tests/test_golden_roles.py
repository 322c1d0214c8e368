"""Role-annotated neighbour rows of all six partner rules against the reference's own rows.

``tests/golden/golden_roles.npz`` was written by ``tests/golden/make_golden_roles.py``
from ``build_butterfly_neighbor_role_row`` (bna/topology/butterfly.py:219-262).  It
pins the oracle's ``fixed_stride`` and ``random`` branches, which the Torch-path
golden tables do not cover (the Torch layout builder refuses those rules), and the
role map.  The GPU test in ``test_gpu_topology.py`` checks the device table against
the same rows.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import butterfly_amd as bf
from butterfly_amd.topology import build_butterfly_neighbor_role_row
from oracle import topology as tp

R = np.load(Path(__file__).resolve().parent / "golden" / "golden_roles.npz")
BITS = {"self": 1, "local": 2, "partner": 4, "sink": 8}


def _cases(rules=None):
    for key in R.files:
        if key.endswith("/stage"):
            continue
        _, rule, n, layer, params = key.split("/")
        if rules is None or rule in rules:
            yield key, rule, int(n[1:]), int(layer[1:]), tuple(int(x) for x in params.split("-"))


RULES = ("xor", "bit_reversal", "benes", "causal_shift", "fixed_stride", "random")


@pytest.mark.parametrize("rule", RULES)
def test_oracle_role_rows_match_reference(rule):
    checked = 0
    for key, _, n, layer, (lwb, sinks, partners) in _cases({rule}):
        want = R[key]
        s, count = tp.stage_meta(n, layer, rule)
        assert (s, count) == tuple(int(x) for x in R[key + "/stage"]), key
        for b in range(n):
            row = tp.role_row(b, n, layer, rule, lwb, sinks, partners)
            k = len(row)
            assert [tuple(int(x) for x in e) for e in want[b, :k]] == row, (key, b)
            assert (want[b, k:, 0] == -1).all(), (key, b)
        checked += 1
    assert checked >= 200


@pytest.mark.parametrize("rule", ("fixed_stride", "random", "bit_reversal"))
def test_host_role_rows_match_reference(rule):
    """The product's host-side role rows (butterfly_amd.topology), over the native metadata."""
    for key, _, n, layer, (lwb, sinks, partners) in _cases({rule}):
        if n > 100:
            continue
        meta = bf.butterfly_layout_metadata(num_blocks=n, layer_idx=layer, partner_rule=rule, partner_count=partners,
                                            sink_count=sinks, local_window_blocks=lwb)
        want = R[key]
        for b in range(n):
            row = build_butterfly_neighbor_role_row(block_idx=b, metadata=meta)
            got = [(e.neighbor, sum(BITS[r] for r in e.roles)) for e in row]
            assert [tuple(int(x) for x in e) for e in want[b, :len(got)]] == got, (key, b)
