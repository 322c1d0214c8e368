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
    if dev.type != "cuda":
        raise ValueError(f"the neighbour table is built on a HIP device, not {dev}")
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


# ----------------------------------------------------------------------------- role-annotated rows
@dataclass(frozen=True)
class NeighborSpec:
    """One entry of a role-annotated neighbour row.  Reference: bna/topology/butterfly.py:20-23."""

    neighbor: int
    roles: tuple[str, ...]


def _reverse_low_bits(value: int, width: int) -> int:
    """The low ``width`` bits of ``value`` in reverse order (higher bits dropped; 0 for
    width 0).  Reference: bna/topology/butterfly.py:45-49."""
    out = 0
    for i in range(max(0, int(width))):
        out = (out << 1) | ((int(value) >> i) & 1)
    return out


def butterfly_partner_block(*, block_idx: int, bit_idx: int, num_blocks: int, partner_rule: str,
                            width: int | None = None) -> int | None:
    """Partner of ``block_idx`` along ``bit_idx`` under the rule, or None when it falls outside
    ``[0, min(block_idx, num_blocks - 1)]``.  Reference: bna/topology/butterfly.py:108-141 (the
    same function the kernels evaluate in ``bfly_topology.h``)."""
    rule = str(partner_rule)
    _rule_code(rule)
    b, bit = int(block_idx), int(bit_idx)
    w = butterfly_width(num_blocks) if width is None else int(width)
    if bit < 0 or bit >= max(1, w):
        return None
    if rule == "causal_shift":
        p = b - (1 << bit)
    elif rule in ("xor", "benes"):
        p = b ^ (1 << bit)
    elif rule == "fixed_stride":
        p = b - 1
    elif rule == "random":
        if b <= 0:
            return None
        p = ((b * 2654435761 + bit * 374761393) & 0xFFFFFFFF) % b
    else:                                                     # bit_reversal over the low w bits
        p = _reverse_low_bits(_reverse_low_bits(b, w) ^ (1 << bit), w)
    if p < 0 or p >= int(num_blocks) or p > b:
        return None
    return int(p)


def build_butterfly_role_map(*, block_idx: int, num_blocks: int, local_window_blocks: int, sink_blocks,
                             partner_bits, partner_rule: str, width: int | None = None) -> dict[int, set[str]]:
    """Neighbour block -> the roles it plays for ``block_idx`` (self, local, partner, sink).
    Reference: bna/topology/butterfly.py:183-216."""
    roles: dict[int, set[str]] = {int(block_idx): {"self"}}
    for off in range(1, int(local_window_blocks) + 1):
        if int(block_idx) - off < 0:
            break
        roles.setdefault(int(block_idx) - off, set()).add("local")
    for bit in partner_bits:
        p = butterfly_partner_block(block_idx=block_idx, bit_idx=bit, num_blocks=num_blocks,
                                    partner_rule=partner_rule, width=width)
        if p is not None:
            roles.setdefault(p, set()).add("partner")
    for s in sink_blocks:
        if 0 <= int(s) < int(num_blocks):
            roles.setdefault(int(s), set()).add("sink")
    return roles


def ordered_roles(roles) -> tuple[str, ...]:
    """Roles in ``ROLE_ORDER``.  Reference: bna/topology/butterfly.py:264-265."""
    return tuple(r for r in ROLE_ORDER if r in roles)


def build_butterfly_neighbor_role_row(*, block_idx: int, metadata: ButterflyLayoutMetadata) -> list[NeighborSpec]:
    """The ordered unique row ``[b, b-1..b-lwb, partners, sinks]`` (entries in ``[0, N)``, first
    occurrence kept) with each entry's roles.  The neighbour order is the row of the device
    table ``bfly_block_neighbors``.  Reference: bna/topology/butterfly.py:219-262, 275-284."""
    m = metadata
    b = int(block_idx)
    role_map = build_butterfly_role_map(block_idx=b, num_blocks=m.num_blocks,
                                        local_window_blocks=m.local_window_blocks, sink_blocks=m.sink_blocks,
                                        partner_bits=m.partner_bits, partner_rule=m.partner_rule, width=m.width)
    cand = [b] + [b - off for off in range(1, m.local_window_blocks + 1)]
    for bit in m.partner_bits:
        p = butterfly_partner_block(block_idx=b, bit_idx=bit, num_blocks=m.num_blocks, partner_rule=m.partner_rule,
                                    width=m.width)
        if p is not None:
            cand.append(p)
    cand += [int(s) for s in m.sink_blocks]
    seen: set[int] = set()
    row: list[NeighborSpec] = []
    for v in cand:
        if v < 0 or v >= m.num_blocks or v in seen:
            continue
        seen.add(v)
        row.append(NeighborSpec(neighbor=v, roles=ordered_roles(role_map.get(v, {"self"}))))
    return row
