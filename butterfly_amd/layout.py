"""Block Butterfly layout (the reference's ``build_block_butterfly_layout``).

Reference: bna/torch/attention_wayfinder_permute.py:568-682 (Torch,
``BlockHamiltonianLayout`` :382-405) and bna/mlx/attention.py:196-301 (MLX,
``BlockSparseButterflyLayout`` :105-141).  The layout holds the device
neighbour table once ([N, K] int32); ``block_neighbors`` exposes it as the
reference's [Hq, N, K] tensor (identical across heads) without copying.

Tables are shared across layouts with the same block count and topology
(the reference shares layouts across layers through a keyed cache,
bna/integrations/qwen_mlx.py:47-48, 790-820): during decode the sequence
length grows by one token per step but the table only changes when the block
count does.
"""
from __future__ import annotations

import ctypes as C
from collections import OrderedDict
from dataclasses import dataclass

import torch

from . import _native
from .topology import ButterflyLayoutMetadata, block_neighbor_table_padded, butterfly_layout_metadata

_TABLE_CACHE: "OrderedDict[tuple, torch.Tensor]" = OrderedDict()
_TABLE_CACHE_MAX = 256


class _Table:
    """A device neighbour table, its row degrees, (lazily) its exact width K, and
    the host topology struct the decode kernel computes rows from."""

    __slots__ = ("padded", "degree", "_exact", "topology")

    def __init__(self, padded: torch.Tensor, degree: torch.Tensor, topology) -> None:
        self.padded = padded
        self.degree = degree
        self._exact = None
        self.topology = topology

    def exact(self) -> torch.Tensor:
        if self._exact is None:
            k = max(1, int(self.degree.max().item()))
            self._exact = self.padded[:, :k].contiguous()
        return self._exact


@dataclass(frozen=True)
class BlockButterflyLayout:
    seq_len: int
    block_size: int
    num_blocks: int
    num_query_heads: int
    table: _Table
    metadata: ButterflyLayoutMetadata
    topology_name: str = "butterfly"

    @property
    def neighbors(self) -> torch.Tensor:
        """Device int32 [N, kcap] table the kernels read (kcap = 1 + lwb + partners + sinks,
        -1 padded); no host synchronisation."""
        return self.table.padded

    @property
    def block_neighbors(self) -> torch.Tensor:
        """The reference's [Hq, N, K] tensor (K = max row length), identical for every
        query head; the first access reads K back from the device."""
        return self.table.exact().unsqueeze(0).expand(self.num_query_heads, -1, -1)

    @property
    def num_neighbors(self) -> int:
        return int(self.table.exact().shape[1])

    @property
    def stage_idx(self) -> int:
        return self.metadata.stage_idx

    @property
    def stage_count(self) -> int:
        return self.metadata.stage_count

    @property
    def local_window_blocks(self) -> int:
        return self.metadata.local_window_blocks

    @property
    def partner_rule(self) -> str:
        return self.metadata.partner_rule

    @property
    def partner_count(self) -> int:
        return self.metadata.partner_count

    @property
    def sink_blocks(self) -> tuple[int, ...]:
        return self.metadata.sink_blocks


_LAYOUT_CACHE: "OrderedDict[tuple, BlockButterflyLayout]" = OrderedDict()
_LAYOUT_CACHE_MAX = 8192


def build_block_butterfly_layout(*, seq_len: int, block_size: int, num_key_value_heads: int,
                                 num_key_value_groups: int, layer_idx: int, local_window_blocks: int = 4,
                                 sink_count: int = 1, partner_count: int = 1, partner_rule: str = "xor",
                                 device=None) -> BlockButterflyLayout:
    """Build (or fetch) the staged Butterfly block layout of one layer."""
    dev = device if device is not None else torch.cuda.current_device()
    args = (seq_len, block_size, num_key_value_heads, num_key_value_groups, layer_idx, local_window_blocks,
            sink_count, partner_count, partner_rule, str(dev))
    hit = _LAYOUT_CACHE.get(args)
    if hit is not None:
        return hit
    lay = _build_layout(seq_len=seq_len, block_size=block_size, num_key_value_heads=num_key_value_heads,
                        num_key_value_groups=num_key_value_groups, layer_idx=layer_idx,
                        local_window_blocks=local_window_blocks, sink_count=sink_count, partner_count=partner_count,
                        partner_rule=partner_rule, device=device)
    _LAYOUT_CACHE[args] = lay
    while len(_LAYOUT_CACHE) > _LAYOUT_CACHE_MAX:
        _LAYOUT_CACHE.popitem(last=False)
    return lay


def _build_layout(*, seq_len: int, block_size: int, num_key_value_heads: int, num_key_value_groups: int,
                  layer_idx: int, local_window_blocks: int, sink_count: int, partner_count: int, partner_rule: str,
                  device) -> BlockButterflyLayout:
    if int(seq_len) <= 0:
        raise ValueError("seq_len must be positive")
    if int(block_size) <= 0:
        raise ValueError("block_size must be positive")
    if int(num_key_value_heads) <= 0:
        raise ValueError("num_key_value_heads must be positive")
    if int(num_key_value_groups) <= 0:
        raise ValueError("num_key_value_groups must be positive")
    if int(local_window_blocks) < 0:
        raise ValueError("local_window_blocks must be >= 0")
    if int(sink_count) < 0:
        raise ValueError("sink_count must be >= 0")
    if int(partner_count) < 0:
        raise ValueError("partner_count must be >= 0")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    n = (int(seq_len) + int(block_size) - 1) // int(block_size)
    meta = butterfly_layout_metadata(num_blocks=n, layer_idx=layer_idx, partner_rule=partner_rule,
                                     partner_count=partner_count, sink_count=sink_count,
                                     local_window_blocks=local_window_blocks)
    key = (n, meta.stage_idx, meta.partner_rule, meta.partner_bits, int(local_window_blocks), int(sink_count),
           int(partner_count), str(dev))
    table = _TABLE_CACHE.get(key)
    if table is None:
        topo = _native.Topology()
        _native.call("bfly_topology_init", n, int(layer_idx), _native.RULES[meta.partner_rule],
                     int(local_window_blocks), int(sink_count), int(partner_count), C.byref(topo))
        table = _Table(*block_neighbor_table_padded(num_blocks=n, layer_idx=layer_idx, partner_rule=partner_rule,
                                                    local_window_blocks=local_window_blocks, sink_count=sink_count,
                                                    partner_count=partner_count, device=dev), topo)
        _TABLE_CACHE[key] = table
        while len(_TABLE_CACHE) > _TABLE_CACHE_MAX:
            _TABLE_CACHE.popitem(last=False)
    else:
        _TABLE_CACHE.move_to_end(key)
    return BlockButterflyLayout(
        seq_len=int(seq_len), block_size=int(block_size), num_blocks=n,
        num_query_heads=int(num_key_value_heads) * int(num_key_value_groups),
        table=table, metadata=meta,
    )


def clear_layout_cache() -> None:
    _TABLE_CACHE.clear()
    _LAYOUT_CACHE.clear()


def drop_layouts_for_other_lengths(current_T: int) -> int:
    """Evict every cached layout whose sequence length is not ``current_T``; returns how
    many were dropped.  Chunked prefill builds one layout per live kv_len, so without this
    the cache holds one entry per chunk; the layers of one chunk, which share a length,
    keep sharing theirs.  (The neighbour tables behind the layouts are keyed by block count
    and stay, bounded by their own LRU.)

    Reference: _qwen_graph_cache_drop_other_keys (bna/integrations/qwen_mlx.py:52-81),
    called per chunk by the harness (scripts/bench_qwen_consumer_mlx.py:650-651).
    """
    drop = [key for key in _LAYOUT_CACHE if int(key[0]) != int(current_T)]
    for key in drop:
        _LAYOUT_CACHE.pop(key, None)
    return len(drop)
