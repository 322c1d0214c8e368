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
