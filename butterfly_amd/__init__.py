"""butterfly_amd: Butterfly compressed attention for AMD MI355X (gfx950).

PyTorch-ROCm host code over hand-written HIP kernels reached through a C ABI
(``include/butterfly_amd.h``, ``butterfly_amd/_lib/libbutterfly_amd.so``).
"""
from .attention import (
    block_mean_summaries,
    butterfly_compressed_attention,
    butterfly_compressed_attention_active,
    compressed_butterfly_active_index_tensors,
    compressed_butterfly_attention,
    compressed_butterfly_attention_active,
    compressed_butterfly_attention_cached,
    compressed_butterfly_attention_from_cache,
    compressed_butterfly_block_index_tensors,
)
from .compressed_cache import CompressedKVCache
from .integrations import (
    AttentionProfile,
    ButterflyAttentionCore,
    QwenButterflyConfig,
    chunked_prefill,
    install_compressed_kv_caches,
    split_chunks,
    swap_qwen_attention_with_butterfly,
)
from .layout import BlockButterflyLayout, build_block_butterfly_layout, clear_layout_cache
from .streams import compressed_stream_attention, online_softmax_merge, swa_stream_attention
from .topology import (
    ROLE_ORDER,
    ButterflyLayoutMetadata,
    NeighborSpec,
    block_neighbor_table,
    build_butterfly_neighbor_role_row,
    build_butterfly_role_map,
    butterfly_partner_block,
    ordered_roles,
    butterfly_layout_metadata,
    butterfly_partner_bits,
    butterfly_stage_count,
    butterfly_stage_meta,
    butterfly_width,
)

__all__ = [
    "compressed_stream_attention",
    "online_softmax_merge",
    "swa_stream_attention",
    "AttentionProfile",
    "ButterflyAttentionCore",
    "QwenButterflyConfig",
    "chunked_prefill",
    "install_compressed_kv_caches",
    "split_chunks",
    "swap_qwen_attention_with_butterfly",
    "BlockButterflyLayout",
    "ButterflyLayoutMetadata",
    "NeighborSpec",
    "ROLE_ORDER",
    "build_butterfly_neighbor_role_row",
    "build_butterfly_role_map",
    "butterfly_partner_block",
    "ordered_roles",
    "CompressedKVCache",
    "block_mean_summaries",
    "block_neighbor_table",
    "build_block_butterfly_layout",
    "butterfly_compressed_attention",
    "butterfly_compressed_attention_active",
    "butterfly_layout_metadata",
    "butterfly_partner_bits",
    "butterfly_stage_count",
    "butterfly_stage_meta",
    "butterfly_width",
    "clear_layout_cache",
    "compressed_butterfly_active_index_tensors",
    "compressed_butterfly_attention",
    "compressed_butterfly_attention_active",
    "compressed_butterfly_attention_cached",
    "compressed_butterfly_attention_from_cache",
    "compressed_butterfly_block_index_tensors",
]
