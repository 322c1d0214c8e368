"""CPU restatement of the staged Butterfly block topology (test infrastructure).

Follows ``bna/topology/butterfly.py`` (reference) and the Torch layout builder
``build_block_butterfly_layout`` (``bna/torch/attention_wayfinder_permute.py:568-682``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

RULES = ("xor", "bit_reversal", "benes", "causal_shift", "fixed_stride", "random")


def width(num_blocks: int) -> int:
    """ceil(log2 N), 1 for N <= 1.  butterfly.py:39-42 (float log2, as there)."""
    n = int(num_blocks)
    if n <= 1:
        return 1
    return int(math.ceil(math.log2(n)))


def bit_reverse(value: int, nbits: int) -> int:
    """butterfly.py:45-49."""
    out = 0
    for i in range(int(nbits)):
        out = (out << 1) | ((int(value) >> i) & 1)
    return out


def stage_meta(num_blocks: int, layer_idx: int, rule: str) -> tuple[int, int]:
    """(stage_idx, stage_count).  butterfly.py:52-65."""
    if rule not in RULES:
        raise ValueError(rule)
    w = width(num_blocks)
    count = max(1, 2 * w - 2) if rule == "benes" else w
    return int(layer_idx) % count, count


def partner_bits(stage_idx: int, stage_count: int, w: int, partner_count: int, rule: str) -> list[int]:
    """butterfly.py:77-105."""
    if w <= 0 or partner_count <= 0:
        return []
    if rule == "benes":
        base = 0 if stage_count <= 1 else stage_idx % stage_count

        def to_bit(phase: int) -> int:
            if w <= 1:
                return 0
            return phase if phase < w else 2 * w - 2 - phase

        return [to_bit((base + j) % stage_count) for j in range(partner_count)]
    return [(stage_idx + j) % w for j in range(partner_count)]


def partner_block(block: int, bit: int, num_blocks: int, rule: str, w: int | None = None) -> int | None:
    """butterfly.py:108-141."""
    ew = width(num_blocks) if w is None else int(w)
    if bit < 0 or bit >= max(1, ew):
        return None
    if rule == "causal_shift":
        p = block - (1 << bit)
    elif rule in ("xor", "benes"):
        p = block ^ (1 << bit)
    elif rule == "fixed_stride":
        p = block - 1
    elif rule == "random":
        if block <= 0:
            return None
        seed = (block * 2654435761 + bit * 374761393) & 0xFFFFFFFF
        p = seed % block
    else:  # bit_reversal
        p = bit_reverse(bit_reverse(block, ew) ^ (1 << bit), ew)
    if p < 0 or p >= num_blocks or p > block:
        return None
    return int(p)


def neighbor_row(block: int, num_blocks: int, layer_idx: int, rule: str, local_window_blocks: int,
                 sink_count: int, partner_count: int) -> list[int]:
    """Ordered, de-duplicated row [self, b-1..b-lwb, partners, sinks].

    Torch builder: attention_wayfinder_permute.py:627-650 (the local walk stops
    at the first negative block; dedup keeps first occurrence; out-of-range
    entries dropped).
    """
    w = width(num_blocks)
    s, count = stage_meta(num_blocks, layer_idx, rule)
    bits = partner_bits(s, count, w, partner_count, rule)
    row = [block]
    for off in range(1, local_window_blocks + 1):
        if block - off < 0:
            break
        row.append(block - off)
    for bit in bits:
        p = partner_block(block, bit, num_blocks, rule, w)
        if p is not None:
            row.append(p)
    row.extend(range(min(sink_count, num_blocks)))
    seen: set[int] = set()
    out: list[int] = []
    for v in row:
        if v in seen or not (0 <= v < num_blocks):
            continue
        seen.add(v)
        out.append(v)
    return out


@dataclass(frozen=True)
class Layout:
    """Torch ``BlockHamiltonianLayout`` subset used by the compressed path."""

    seq_len: int
    block_size: int
    num_blocks: int
    block_neighbors: torch.Tensor  # [Hq, N, K] int64, -1 padded
    stage_idx: int
    stage_count: int
    local_window_blocks: int
    partner_rule: str
    partner_count: int
    sink_blocks: tuple[int, ...]


def build_layout(*, seq_len: int, block_size: int, num_key_value_heads: int, num_key_value_groups: int,
                 layer_idx: int, local_window_blocks: int = 4, sink_count: int = 1, partner_count: int = 1,
                 partner_rule: str = "xor") -> Layout:
    """attention_wayfinder_permute.py:568-682 (Torch ``build_block_butterfly_layout``)."""
    if seq_len <= 0 or block_size <= 0:
        raise ValueError("seq_len and block_size must be positive")
    n = (seq_len + block_size - 1) // block_size
    rows = [neighbor_row(b, n, layer_idx, partner_rule, local_window_blocks, sink_count, partner_count)
            for b in range(n)]
    k = max(1, max(len(r) for r in rows))
    kv = torch.full((n, k), -1, dtype=torch.long)
    for b, r in enumerate(rows):
        kv[b, : len(r)] = torch.tensor(r, dtype=torch.long)
    hq = num_key_value_heads * num_key_value_groups
    s, count = stage_meta(n, layer_idx, partner_rule)
    return Layout(
        seq_len=seq_len, block_size=block_size, num_blocks=n,
        block_neighbors=kv.unsqueeze(0).repeat(hq, 1, 1),
        stage_idx=s, stage_count=count, local_window_blocks=local_window_blocks,
        partner_rule=partner_rule, partner_count=partner_count,
        sink_blocks=tuple(range(min(sink_count, n))),
    )


ROLE_BITS = {"self": 1, "local": 2, "partner": 4, "sink": 8}


def role_row(block: int, num_blocks: int, layer_idx: int, rule: str, local_window_blocks: int, sink_count: int,
             partner_count: int) -> list[tuple[int, int]]:
    """``neighbor_row`` with each entry's role bits (self 1, local 2, partner 4, sink 8).

    butterfly.py:183-262: a block's roles are every reason it enters the row (a
    partner that is also the previous block is local and partner).
    """
    w = width(num_blocks)
    s, count = stage_meta(num_blocks, layer_idx, rule)
    bits = partner_bits(s, count, w, partner_count, rule)
    roles = {block: ROLE_BITS["self"]}
    for off in range(1, local_window_blocks + 1):
        if block - off < 0:
            break
        roles[block - off] = roles.get(block - off, 0) | ROLE_BITS["local"]
    for bit in bits:
        p = partner_block(block, bit, num_blocks, rule, w)
        if p is not None:
            roles[p] = roles.get(p, 0) | ROLE_BITS["partner"]
    for sk in range(min(sink_count, num_blocks)):
        roles[sk] = roles.get(sk, 0) | ROLE_BITS["sink"]
    return [(v, roles[v]) for v in neighbor_row(block, num_blocks, layer_idx, rule, local_window_blocks,
                                                sink_count, partner_count)]
