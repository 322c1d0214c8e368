"""Staged Butterfly block topology: host metadata and the device neighbour table.

Mirrors the reference's ``bna/topology/butterfly.py`` surface (names, argument
meaning, errors).  Scalar metadata comes from the native library's host
functions; the per-block partner/neighbour table is computed on the GPU
(``bfly_block_neighbors``).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Literal

import torch

from . import _native
from ._device import on as _on, stream_of as _stream_of

ButterflyPartnerRule = Literal["xor", "bit_reversal", "benes", "causal_shift", "fixed_stride", "random"]
ROLE_ORDER = ("self", "local", "partner", "sink")


def _rule_code(rule: str) -> int:
    code = _native.RULES.get(str(rule))
    if code is None:
        raise ValueError(f"Unsupported Butterfly partner rule: {rule!r}")
    return code


def butterfly_stage_meta(*, num_blocks: int, layer_idx: int, partner_rule: str) -> tuple[int, int]:
    """(stage_idx, stage_count).  Reference: bna/topology/butterfly.py:52-65."""
    s, c, w = C.c_int32(), C.c_int32(), C.c_int32()
    _native.call("bfly_stage_meta", int(num_blocks), int(layer_idx), _rule_code(partner_rule),
                 C.byref(s), C.byref(c), C.byref(w))
    return int(s.value), int(c.value)


def butterfly_width(num_blocks: int) -> int:
    """ceil(log2 N), 1 for N <= 1.  Reference: bna/topology/butterfly.py:39-42."""
    s, c, w = C.c_int32(), C.c_int32(), C.c_int32()
    _native.call("bfly_stage_meta", int(num_blocks), 0, 0, C.byref(s), C.byref(c), C.byref(w))
    return int(w.value)


def butterfly_stage_count(num_blocks: int, partner_rule: str) -> int:
    """Reference: bna/topology/butterfly.py:68-74."""
    return butterfly_stage_meta(num_blocks=num_blocks, layer_idx=0, partner_rule=partner_rule)[1]


def butterfly_partner_bits(*, stage_idx: int, stage_count: int, width: int, partner_count: int,
                           partner_rule: str) -> list[int]:
    """Reference: bna/topology/butterfly.py:77-105."""
    code = _rule_code(partner_rule)
    if int(width) <= 0 or int(partner_count) <= 0:
        return []
    buf = (C.c_int32 * int(partner_count))()
    _native.call("bfly_partner_bits", int(stage_idx), int(stage_count), int(width), int(partner_count),
                 code, buf)
    return [int(x) for x in buf]


@dataclass(frozen=True)
class ButterflyLayoutMetadata:
    """Reference: bna/topology/butterfly.py:26-36."""

    num_blocks: int
    width: int
    stage_idx: int
    stage_count: int
    partner_bits: tuple[int, ...]
    sink_blocks: tuple[int, ...]
    local_window_blocks: int
    partner_count: int
    partner_rule: str


def butterfly_layout_metadata(*, num_blocks: int, layer_idx: int, partner_rule: str, partner_count: int,
                              sink_count: int, local_window_blocks: int) -> ButterflyLayoutMetadata:
    """Reference: bna/topology/butterfly.py:144-180."""
    _rule_code(partner_rule)
    width = butterfly_width(num_blocks)
    stage_idx, stage_count = butterfly_stage_meta(num_blocks=num_blocks, layer_idx=layer_idx,
                                                  partner_rule=partner_rule)
    bits = butterfly_partner_bits(stage_idx=stage_idx, stage_count=stage_count, width=width,
                                  partner_count=partner_count, partner_rule=partner_rule)
    return ButterflyLayoutMetadata(
        num_blocks=int(num_blocks), width=int(width), stage_idx=int(stage_idx),
        stage_count=int(stage_count), partner_bits=tuple(bits),
        sink_blocks=tuple(range(min(int(sink_count), int(num_blocks)))),
        local_window_blocks=int(local_window_blocks), partner_count=int(partner_count),
        partner_rule=str(partner_rule),
    )


def block_neighbor_table_padded(*, num_blocks: int, layer_idx: int, partner_rule: str, local_window_blocks: int,
                                sink_count: int, partner_count: int, device=None):
    """Device (table int32 [N, kcap], degree int32 [N]) with kcap = 1 + lwb + partners + sinks.

    Row b is the ordered unique list [b, b-1..b-lwb, partners, sinks], -1 padded
    (reference: bna/torch/attention_wayfinder_permute.py:627-662,
    bna/topology/butterfly.py:219-284).  One GPU launch, no host synchronisation:
    the kernels skip -1 entries, so the padded width is equivalent to the
    reference's K = max row length.
    """
    if int(num_blocks) <= 0:
        raise ValueError("num_blocks must be positive")
    if int(local_window_blocks) < 0:
        raise ValueError("local_window_blocks must be >= 0")
    if int(sink_count) < 0:
        raise ValueError("sink_count must be >= 0")
    if int(partner_count) < 0:
        raise ValueError("partner_count must be >= 0")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    kcap = 1 + int(local_window_blocks) + int(partner_count) + int(sink_count)
    table = torch.empty((int(num_blocks), kcap), dtype=torch.int32, device=dev)
    degree = torch.empty((int(num_blocks),), dtype=torch.int32, device=dev)
    with _on(dev):
        _native.call("bfly_block_neighbors", int(num_blocks), int(layer_idx), _rule_code(partner_rule),
                     int(local_window_blocks), int(sink_count), int(partner_count), table.data_ptr(), kcap,
                     degree.data_ptr(), _stream_of(dev))
    return table, degree


def block_neighbor_table(*, num_blocks: int, layer_idx: int, partner_rule: str, local_window_blocks: int,
                         sink_count: int, partner_count: int, device=None) -> torch.Tensor:
    """Device int32 [N, K] neighbour table, -1 padded, K = max row length (the
    reference's ``block_neighbors[0]`` shape); reads K back from the device."""
    table, degree = block_neighbor_table_padded(num_blocks=num_blocks, layer_idx=layer_idx, partner_rule=partner_rule,
                                                local_window_blocks=local_window_blocks, sink_count=sink_count,
                                                partner_count=partner_count, device=device)
    k = max(1, int(degree.max().item()))
    return table[:, :k].contiguous()
