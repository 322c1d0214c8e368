"""CPU restatement of the two-pool ``CompressedKVCache`` (test infrastructure).

Follows ``bna/mlx/compressed_cache.py:9-302``: a tail buffer of recent raw tokens
(slide-and-trim by whole blocks) and a summary pool with one fp32-mean row per
completed block.  Buffers are torch CPU tensors; the arithmetic on the counters
is the reference's, line for line in meaning.
"""
from __future__ import annotations

import torch


class OracleCompressedKVCache:
    def __init__(self, *, block_size: int = 128, local_window_tokens: int = 128,
                 max_kv_size: int | None = None, max_chunk_size: int = 512) -> None:
        self.block_size = int(block_size)
        self.local_window_tokens = int(local_window_tokens)
        self.max_kv_size = int(max_kv_size) if max_kv_size else None
        self.max_chunk_size = int(max_chunk_size)
        self.tk = self.tv = self.sk = self.sv = None
        self.tail_capacity = self.summary_capacity = 0
        self.tail_size = self.summary_count = self.offset = self.summary_offset = 0

    def _allocate(self, b, h, d, dtype):
        # compressed_cache.py:69-92
        self.tail_capacity = self.local_window_tokens + 2 * self.max_chunk_size + 2 * self.block_size
        self.summary_capacity = (self.max_kv_size // self.block_size + 4) if self.max_kv_size else 2048
        self.tk = torch.zeros((b, h, self.tail_capacity, d), dtype=dtype)
        self.tv = torch.zeros_like(self.tk)
        self.sk = torch.zeros((b, h, self.summary_capacity, d), dtype=dtype)
        self.sv = torch.zeros_like(self.sk)

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        # compressed_cache.py:94-172
        step = keys.shape[2]
        if self.tk is None:
            self._allocate(keys.shape[0], keys.shape[1], keys.shape[3], keys.dtype)
        bs, lw = self.block_size, self.local_window_tokens
        if self.tail_size + step > self.tail_capacity:
            raise RuntimeError("tail capacity exceeded")
        self.tk[:, :, self.tail_size:self.tail_size + step] = keys
        self.tv[:, :, self.tail_size:self.tail_size + step] = values
        self.tail_size += step
        self.offset += step
        while self.summary_offset + bs <= self.offset - lw:
            start = self.summary_offset - (self.offset - self.tail_size)
            if start < 0 or start + bs > self.tail_size:
                break
            if self.summary_count >= self.summary_capacity:
                raise RuntimeError("summary capacity exhausted")
            slot = self.summary_count
            self.sk[:, :, slot] = self.tk[:, :, start:start + bs].float().mean(dim=2).to(self.tk.dtype)
            self.sv[:, :, slot] = self.tv[:, :, start:start + bs].float().mean(dim=2).to(self.tv.dtype)
            self.summary_count += 1
            self.summary_offset += bs
        target = max(lw, step + lw - 1)
        while self.tail_size - bs >= target:
            keep = self.tail_size - bs
            self.tk[:, :, :keep] = self.tk[:, :, bs:bs + keep].clone()
            self.tv[:, :, :keep] = self.tv[:, :, bs:bs + keep].clone()
            self.tail_size = keep
        return self.keys, self.values

    @property
    def keys(self):
        return None if self.tk is None else self.tk[:, :, : self.tail_size]

    @property
    def values(self):
        return None if self.tv is None else self.tv[:, :, : self.tail_size]

    @property
    def k_summary(self):
        return None if self.sk is None else self.sk[:, :, : self.summary_count]

    @property
    def v_summary(self):
        return None if self.sv is None else self.sv[:, :, : self.summary_count]

    def get_compressed_state(self):
        if self.tk is None:
            raise ValueError("empty cache")
        return (self.keys, self.values, self.k_summary, self.v_summary,
                self.offset - self.tail_size, self.offset)

    @property
    def nbytes(self) -> int:
        # compressed_cache.py:231-244 (valid slices only)
        if self.tk is None:
            return 0
        b, h, _, d = self.tk.shape
        e = self.tk.element_size()
        return 2 * b * h * d * e * (self.tail_size + self.summary_count)
