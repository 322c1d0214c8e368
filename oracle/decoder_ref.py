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


# --------------------------------------------------------------------------- rounding points
def q4_weight_fp32(layer) -> torch.Tensor:
    """The layer's weights ``code * scale + bias`` in fp32, not rounded to bf16: what the GPU's
    one-row product from the 4-bit codes multiplies by (its factorised sum is this product
    up to fp32 summation order).  Cached on the layer."""
    w = getattr(layer, "_oracle_w32", None)
    if w is None:
        out_f, group = layer.packed.shape[0], layer.group
        q = torch.stack([layer.packed & 0xF, layer.packed >> 4], dim=-1).view(out_f, -1).float()
        w = (q.view(out_f, -1, group) * layer.scale.float().unsqueeze(-1)
             + layer.bias.float().unsqueeze(-1)).view(out_f, -1)
        layer._oracle_w32 = w
    return w


def q4_row(x: torch.Tensor, layer) -> torch.Tensor:
    """One activation row through a 4-bit layer with the GPU decode step's rounding points:
    fp32 weights from the codes, fp32 accumulation, one rounding of each output to bf16
    (``bfly_q4_gemv``).  Multi-row products on the GPU run over the bf16-dequantised weights, as
    the layer's own forward does on the CPU."""
    y = x.reshape(1, -1).float() @ q4_weight_fp32(layer).t()
    return y.to(x.dtype).view(*x.shape[:-1], y.shape[-1])


def match_gpu_rounding(model) -> None:
    """Give a CPU copy of ``butterfly_amd.decoder.Decoder`` the GPU's rounding points: every
    one-row product (a decode step's projections, the last position's lm_head) from the 4-bit
    codes in fp32 (``q4_row``); prefill products stay on the bf16-dequantised weights."""
    import types

    from butterfly_amd.decoder import QuantLinear

    def forward(self, x):
        if x.numel() == x.shape[-1] and not x.is_cuda:
            return q4_row(x, self)
        return type(self).forward(self, x)

    for m in model.modules():
        if isinstance(m, QuantLinear):
            m.forward = types.MethodType(forward, m)

    def logits(self, h):
        if h.numel() == h.shape[-1] and not h.is_cuda:
            return q4_row(h, self.lm_head)
        return type(self)._logits(self, h)

    model._logits = types.MethodType(logits, model)
