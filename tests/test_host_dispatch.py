"""CPU: host-side dispatch rules that pick a kernel or refuse a call before any GPU work."""
from __future__ import annotations

import pytest
import torch

import butterfly_amd as bf
from butterfly_amd.decoder import QuantLinear


@pytest.mark.parametrize("in_f,group,codes", [(2048, 64, True), (8192, 64, True), (6144, 32, True),
                                              (9728, 64, False), (2048, 16, False)])
def test_q4_gemv_only_for_shapes_it_takes(in_f, group, codes):
    """One-row products read the 4-bit codes only where bfly_q4_gemv accepts the shape
    (groups of a multiple of 32 codes, at most 8192 inputs); other layers use the
    dequantised weight."""
    layer = QuantLinear(in_f, 8, generator=torch.Generator().manual_seed(0), group=group)
    assert layer.gemv_from_codes is codes
    x = torch.randn(1, 1, in_f).bfloat16()
    y = layer(x)                                   # CPU: always the dequantised product
    want = torch.nn.functional.linear(x.float(), layer.weight.float())
    assert torch.allclose(y.float(), want, atol=2e-2 * want.abs().max().item())


def test_mfma_step_eligibility_mirrors_the_kernel_limits():
    """CompressedKVCache.step_on_mfma: bf16, positive scale, 32-bit positions and offsets."""
    c = bf.CompressedKVCache(block_size=128, local_window_tokens=128, max_kv_size=131072 + 512)
    assert not c.step_on_mfma(128, 64, 0.088, torch.bfloat16)          # not allocated yet
    c._allocate(1, 2, 128, torch.bfloat16, "cpu")
    assert c.step_on_mfma(128, 64, 0.088, torch.bfloat16)
    assert not c.step_on_mfma(128, 64, -0.088, torch.bfloat16)
    assert not c.step_on_mfma(128, 64, 0.0, torch.bfloat16)
    assert not c.step_on_mfma(128, 64, 0.088, torch.float32)
    big = bf.CompressedKVCache(block_size=128, local_window_tokens=128, max_kv_size=1 << 30)
    big.tail_capacity, big.summary_capacity = 1600, (1 << 30) // 128 + 4       # pool rows * d >= 2^30
    big._ring_k = torch.empty(0)
    assert not big.step_on_mfma(128, 64, 0.088, torch.bfloat16)


@pytest.mark.parametrize("window,row_blocks,device_step", [
    (64, (1, 1, 1), True), (128, (1, 1, 1), False), (65, (1, 1, 1), False), (1, (1, 1, 1), True),
    (64, (10, 3, 2), True), (64, (12, 3, 2), False)])
def test_device_decode_step_only_where_the_kernel_takes_it(window, row_blocks, device_step):
    """A q_len == 1 call on a cache with device counters runs bfly_decode_step only for an
    attention window of at most 64 tokens and a routed row (1 + local blocks + partners +
    sinks) of at most 16 slots; other steps take the host path, and the fused q/k norm step
    follows the same rule.  The reference default window (128 tokens) is one of them."""
    lwb, partners, sinks = row_blocks
    cfg = bf.compressed_butterfly_config(compressed_local_window_tokens=window, block_local_window_blocks=lwb,
                                         block_partner_count=partners, block_sink_blocks=sinks)
    core = bf.ButterflyAttentionCore(cfg, layer_idx=3)
    c = bf.CompressedKVCache(block_size=128, local_window_tokens=window, max_kv_size=4096)
    assert not core.runs_device_step(c, 1, 128, torch.bfloat16)          # no device counters
    c._allocate(1, 2, 128, torch.bfloat16, "cpu")
    assert core.device_step_fits(c, 128, torch.bfloat16) is device_step  # counters not needed for this one
    assert not core.runs_device_step(c, 1, 128, torch.bfloat16)
    c._dev = torch.zeros(8, dtype=torch.int64)                            # counters present
    assert core.runs_device_step(c, 1, 128, torch.bfloat16) is device_step
    assert core.fuses_qk_norm(c, 1, 128, torch.bfloat16) is device_step
    assert not core.runs_device_step(c, 2, 128, torch.bfloat16)          # two new tokens
    assert not core.runs_device_step(c, 1, 96, torch.bfloat16)           # head_dim the kernel lacks
    assert core.runs_device_step(c, 1, 256, torch.float32) is False      # d = 256 is bf16 only
    dense = bf.ButterflyAttentionCore(
        bf.compressed_butterfly_config(compressed_local_window_tokens=window, wayfinder_decode_backend="dense"), 3)
    assert not dense.runs_device_step(c, 1, 128, torch.bfloat16)


def test_reference_default_window_is_beyond_the_device_step():
    """QwenButterflyConfig's compressed defaults give a 128-token window
    (bna/integrations/qwen_mlx.py:84-165); the device step takes 64 at most."""
    cfg = bf.QwenButterflyConfig(path="block_sparse", block_compression="mean")
    assert cfg.compressed_local_window_tokens == 128
    core = bf.ButterflyAttentionCore(cfg, layer_idx=0)
    c = bf.CompressedKVCache(block_size=128, local_window_tokens=128, max_kv_size=4096)
    c._allocate(1, 2, 128, torch.bfloat16, "cpu")
    c._dev = torch.zeros(8, dtype=torch.int64)
    assert not core.runs_device_step(c, 1, 128, torch.bfloat16)
