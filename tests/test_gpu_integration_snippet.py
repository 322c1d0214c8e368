"""GPU: the reference-side dispatch snippet of the repository's integration notes, executed
as written.

The fenced Python block under "The reference-side binding a maintainer would add" is read
from the notes (``_NOTES`` below) and run against a layout object with the fields of the
reference's Torch ``BlockHamiltonianLayout`` (bna/torch/attention_wayfinder_permute.py:382-405);
its output must match the CPU oracle of ``butterfly_compressed_attention``.
"""
from __future__ import annotations

import re
from dataclasses import dataclass
from pathlib import Path

import pytest
import torch

from oracle import attention as oa, topology as tp

pytestmark = pytest.mark.gpu


@dataclass(frozen=True)
class ReferenceShapedLayout:
    seq_len: int
    block_size: int
    num_blocks: int
    block_neighbors: torch.Tensor
    block_perm: torch.Tensor
    landmark_blocks: tuple
    sink_blocks: tuple
    num_cycles: int
    strategy: str
    topology_name: str = "hamiltonian"
    stage_idx: int = 0
    stage_count: int = 1
    local_window_blocks: int = 0
    partner_rule: str = "none"
    partner_count: int = 0


_NOTES = Path(__file__).resolve().parents[1] / "INTEGRATION.md"


def _snippet():
    text = _NOTES.read_text()
    section = text[text.index("## 2. The reference-side binding"):]
    return re.search(r"```python\n(.*?)```", section, re.S).group(1)


@pytest.mark.parametrize("layer", [3, 13])
def test_integration_snippet_runs_and_matches_the_oracle(layer):
    ns = {"torch": torch}
    exec(compile(_snippet(), _NOTES.name, "exec"), ns)
    t, hq, hkv, d = 1000, 8, 2, 128
    g = torch.Generator().manual_seed(layer)
    q = torch.randn(1, hq, t, d, generator=g).bfloat16()
    k = torch.randn(1, hkv, t, d, generator=g).bfloat16()
    v = torch.randn(1, hkv, t, d, generator=g).bfloat16()
    ref = tp.build_layout(seq_len=t, block_size=128, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                          layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                          partner_rule="causal_shift")
    lay = ReferenceShapedLayout(seq_len=t, block_size=128, num_blocks=ref.num_blocks,
                                block_neighbors=ref.block_neighbors, block_perm=torch.arange(ref.num_blocks)[None],
                                landmark_blocks=(), sink_blocks=ref.sink_blocks, num_cycles=1, strategy="random",
                                topology_name="butterfly", stage_idx=ref.stage_idx, stage_count=ref.stage_count,
                                local_window_blocks=1, partner_rule="causal_shift", partner_count=1)
    out = ns["butterfly_compressed_attention"](q.cuda(), k.cuda(), v.cuda(), layout=lay, local_window_tokens=64)
    want = oa.prefill(q, k, v, layout=ref, W=64)
    err = (out.float().cpu() - want.float()).abs().max().item()
    rel = ((out.float().cpu() - want.float()).norm() / want.float().norm()).item()
    assert err <= 2e-2 and rel <= 1e-2, (err, rel)
