"""Pins the CPU cache oracle (oracle/cache.py) on the reference tests' invariants
(tests/mlx/test_compressed_kv_cache.py:12-53 restated) and capacity errors."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import brute
from oracle.cache import OracleCompressedKVCache


@pytest.mark.parametrize("bs,W,step,T", [(4, 4, 3, 24), (128, 64, 384, 131072 // 64), (16, 8, 5, 301)])
def test_cache_invariants_and_summaries(bs, W, step, T):
    rng = np.random.default_rng(101)
    xk = rng.standard_normal((1, 2, T, 8), dtype=np.float32)
    xv = rng.standard_normal((1, 2, T, 8), dtype=np.float32)
    cache = OracleCompressedKVCache(block_size=bs, local_window_tokens=W, max_chunk_size=max(512, step))
    for s in range(0, T, step):
        cache.update_and_fetch(torch.from_numpy(xk[:, :, s:s + step]), torch.from_numpy(xv[:, :, s:s + step]))
        tk, _tv, ks, vs, ts, off = cache.get_compressed_state()
        last = min(step, T - s)
        assert off == min(T, s + step)
        assert ts % bs == 0
        assert tk.shape[2] >= min(W, off)
        assert tk.shape[2] < W + max(last, step) + bs
        # the tail holds exactly the raw tokens [ts, off)
        assert np.array_equal(tk.numpy(), xk[:, :, ts:off])
        # every complete block older than the window is summarised, none else
        assert cache.summary_count == max(0, (off - W) // bs)
    n = cache.summary_count
    want = brute.block_summaries(xk[:, :, : n * bs], bs)
    assert np.abs(ks.numpy() - want).max() < 1e-6
    assert np.abs(vs.numpy() - brute.block_summaries(xv[:, :, : n * bs], bs)).max() < 1e-6


def test_cache_capacity_errors():
    cache = OracleCompressedKVCache(block_size=4, local_window_tokens=4, max_chunk_size=2)
    with pytest.raises(RuntimeError):
        cache.update_and_fetch(torch.zeros(1, 1, 64, 4), torch.zeros(1, 1, 64, 4))
    small = OracleCompressedKVCache(block_size=4, local_window_tokens=4, max_kv_size=4)
    with pytest.raises(RuntimeError):
        for _ in range(20):
            small.update_and_fetch(torch.zeros(1, 1, 4, 4), torch.zeros(1, 1, 4, 4))


def test_cfg3_prefill_schedule_counters():
    # cfg3: 131072 tokens in 384-token chunks (max_chunk = 512) then decode.
    cache = OracleCompressedKVCache(block_size=128, local_window_tokens=64, max_kv_size=131328, max_chunk_size=512)
    z = torch.zeros(1, 1, 384, 1)
    t = 0
    while t < 131072:
        step = min(384, 131072 - t)
        cache.update_and_fetch(z[:, :, :step], z[:, :, :step])
        t += step
    assert cache.tail_capacity == 64 + 1024 + 256
    assert cache.summary_capacity == 131328 // 128 + 4
    assert cache.tail_size == 256 and cache.summary_count == 1023
    one = torch.zeros(1, 1, 1, 1)
    for _ in range(64):
        cache.update_and_fetch(one, one)
        assert 64 <= cache.tail_size <= 191
    assert cache.summary_count == 1024
