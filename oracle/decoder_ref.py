"""CPU reference attention for the swapped decoder -- TEST INFRASTRUCTURE ONLY.

The reference's Torch layer swap (bna/integrations/qwen_torch.py:1221-1470)
runs the one-shot ``butterfly_compressed_attention`` when ``q_len == k_len`` and
``butterfly_compressed_attention_active`` over the full cached K/V for later
rows (the ``cached_block_sparse`` branch, :1400-1427), with the layout rebuilt
for the live ``kv_len``.  This module restates that dispatch over
``oracle.attention`` so a decoder's attention can be swapped to it on the CPU.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import attention as oa
from . import topology as tp


class OracleButterflyAttention(nn.Module):
    """Projections/norms/RoPE of ``base`` + the reference Torch compressed attention."""

    def __init__(self, base, *, layer_idx: int, block_size: int = 128, local_window_tokens: int = 64,
                 local_window_blocks: int = 1, sink_count: int = 1, partner_count: int = 1,
                 partner_rule: str = "causal_shift"):
        super().__init__()
        self.base = base
        self.layer_idx = int(layer_idx)
        self.kw = dict(block_size=block_size, local_window_blocks=local_window_blocks, sink_count=sink_count,
                       partner_count=partner_count, partner_rule=partner_rule)
        self.W = int(local_window_tokens)

    def forward(self, x: torch.Tensor, mask=None, cache=None, *, position_embeddings=None) -> torch.Tensor:
        q, k, v = self.base.project(x, None, position_embeddings)
        if cache is not None and cache:
            k = torch.cat([cache[0], k], 2)
            v = torch.cat([cache[1], v], 2)
        if cache is not None:
            cache[:] = [k, v]
        tq, tk = q.shape[2], k.shape[2]
        lay = tp.build_layout(seq_len=tk, num_key_value_heads=k.shape[1], num_key_value_groups=q.shape[1] // k.shape[1],
                              layer_idx=self.layer_idx, **self.kw)
        if tq == tk:
            o = oa.prefill(q, k, v, layout=lay, W=self.W)
        else:
            o = oa.active(q, k, v, layout=lay, query_positions=torch.arange(tk - tq, tk), W=self.W)
        return self.base.output(o)


def swap_to_oracle(model, cfg, layer_indices=None):
    """Swap every (selected) ``model.layers[i].self_attn`` to the CPU reference attention."""
    out = []
    for i, layer in enumerate(model.layers):
        if layer_indices is not None and i not in layer_indices:
            continue
        layer.self_attn = OracleButterflyAttention(
            layer.self_attn, layer_idx=i, block_size=cfg.block_size,
            local_window_tokens=cfg.compressed_local_window_tokens,
            local_window_blocks=cfg.block_local_window_blocks, sink_count=cfg.block_sink_blocks,
            partner_count=cfg.block_partner_count, partner_rule=cfg.block_partner_rule)
        out.append(i)
    return out
