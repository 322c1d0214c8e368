"""Write role-annotated neighbour rows from the reference's topology module (build container only).

Usage: ``python tests/golden/make_golden_roles.py /path/to/Hmbown-Butterfly``

Imports ``bna.topology.butterfly`` (standard library only) from the given path and
writes ``golden_roles.npz``: for every partner rule -- including ``fixed_stride``
and ``random``, which the reference's Torch layout builder refuses and its MLX
builder accepts -- the ordered neighbour row of each block with its roles, from
``build_butterfly_neighbor_role_row`` (bna/topology/butterfly.py:219-262) over
``butterfly_layout_metadata`` (:144-180).  The file holds data only; nothing under
``tests/`` reads the reference at test time.

Encoding: ``roles/{rule}/N{n}/L{layer}/{lwb}-{sinks}-{partners}`` is an int16 array
[N, K, 2]: entry [b, j] = (neighbour, role bits) for j < len(row b), (-1, 0) after;
role bits: self 1, local 2, partner 4, sink 8.  ``.../stage`` = (stage_idx, stage_count).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUT = HERE / "golden_roles.npz"

RULES = ("xor", "bit_reversal", "benes", "causal_shift", "fixed_stride", "random")
NS = (1, 2, 3, 5, 8, 9, 16, 17, 32, 33, 100, 257, 1025)
PARAMS = ((1, 1, 1), (4, 1, 1), (2, 2, 2), (0, 0, 1), (1, 0, 3))
ROLE_BITS = {"self": 1, "local": 2, "partner": 4, "sink": 8}


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from bna.topology import butterfly as T  # noqa: E402

    data: dict[str, np.ndarray] = {}
    for rule in RULES:
        for n in NS:
            for lwb, sinks, partners in PARAMS if n <= 100 else PARAMS[:1]:
                _, count = T.butterfly_stage_meta(num_blocks=n, layer_idx=0, partner_rule=rule)
                layers = range(count + 1) if n <= 100 else (0, 1, count - 1, count, 3 * count + 2)
                for layer in layers:
                    meta = T.butterfly_layout_metadata(num_blocks=n, layer_idx=layer, partner_rule=rule,
                                                       partner_count=partners, sink_count=sinks,
                                                       local_window_blocks=lwb)
                    rows = [T.build_butterfly_neighbor_role_row(block_idx=b, metadata=meta) for b in range(n)]
                    k = max(1, max(len(r) for r in rows))
                    arr = np.full((n, k, 2), -1, dtype=np.int16)
                    arr[:, :, 1] = 0
                    for b, row in enumerate(rows):
                        for j, spec in enumerate(row):
                            arr[b, j, 0] = spec.neighbor
                            arr[b, j, 1] = sum(ROLE_BITS[r] for r in spec.roles)
                    key = f"roles/{rule}/N{n}/L{layer}/{lwb}-{sinks}-{partners}"
                    data[key] = arr
                    data[key + "/stage"] = np.array([meta.stage_idx, meta.stage_count], dtype=np.int16)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
