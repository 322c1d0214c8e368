"""Two-pool KV cache for compressed Butterfly attention, resident in HBM.

Contract: the reference's ``CompressedKVCache`` (bna/mlx/compressed_cache.py:9-302):
constructor arguments, capacity formulas, the counters ``offset``,
``tail_size``, ``summary_count``, ``summary_offset`` and their update rules,
the logical views (``keys``/``values`` = the tail, ``k_summary``/``v_summary``
= completed block means), ``get_compressed_state``, ``nbytes``, ``state`` /
``meta_state`` round trip and the capacity ``RuntimeError``s.

Physical layout (MI355X-specific): the tail is a ring of
``tail_capacity = W + 2*max_chunk + 2*BS`` slots per (batch, kv head) in which
position ``p`` lives at slot ``p mod tail_capacity``; trimming the tail is a
counter update (no data moves).  The summary pool is
``[B, H, summary_capacity, d]``.  Appends and block means run as HIP kernels
(``bfly_cache_append``, ``bfly_cache_compress``); the host only does the
reference's integer bookkeeping.  The logical tail always fits the ring because
``tail_size <= tail_capacity`` (the reference's own capacity check).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional

import torch

from . import _native
from .attention import _c, _dtype_code, _on, _stream

# int64 words per counter copy in the device counter array of bfly_decode_step:
# an 8-word header, then _dev_copies(n) copies per sequence (n = batch * Hkv
# sequences: 64 when n <= 16, for the attending workgroups of
# bfly_decode_step_qk_norm_oproj, else 1) and eight for the step's route
# workgroups, so bfly_decode_state_words(1, 1) == 8 + (64 + 8) * _DEV_SLOT.
_DEV_SLOT = 32


def _dev_copies(n: int) -> int:
    return 64 if n <= 16 else 1
# device error word (state[4]) of a failed step: 1 = tail or pool capacity, 2 = a
# position past the RoPE tables of the fused q/k norm step
_DEV_ERR_CAPACITY, _DEV_ERR_ROPE = 1, 2
# the bf16 MFMA decode kernel works in 32-bit positions and offsets below this
_POS_LIMIT = 1 << 30
# what bfly_decode_step takes (decode.hip kDecMaxWin, kDecMaxSum): an attention window of
# at most 64 tokens and a routed row (self, local blocks, partners, sinks) of at most 16
_DEC_MAX_WIN, _DEC_MAX_ROW = 64, 16


@dataclass(frozen=True)
class RingState:
    ring_k: torch.Tensor
    ring_v: torch.Tensor
    ring_capacity: int
    tail_start: int
    offset: int
    pool_k: torch.Tensor
    pool_v: torch.Tensor
    summary_count: int


class CompressedKVCache:
    def __init__(self, *, block_size: int = 128, local_window_tokens: int = 128,
                 max_kv_size: Optional[int] = None, max_chunk_size: int = 512) -> None:
        self.block_size = int(block_size)
        self.local_window_tokens = int(local_window_tokens)
        self.max_kv_size = int(max_kv_size) if max_kv_size else None
        self.max_chunk_size = int(max_chunk_size)
        self._ring_k: Optional[torch.Tensor] = None
        self._ring_v: Optional[torch.Tensor] = None
        self._pool_k: Optional[torch.Tensor] = None
        self._pool_v: Optional[torch.Tensor] = None
        self._realign = False   # tail stored at slots [0, tail_size) by the state setter
        self._dev: Optional[torch.Tensor] = None   # device counters (use_device_counters)
        self._dev_dirty = False
        self.tail_capacity = 0
        self.summary_capacity = 0
        self.tail_size = 0
        self.summary_count = 0
        self.offset = 0
        self.summary_offset = 0

    # ------------------------------------------------------------------ allocation
    def _allocate(self, b: int, h: int, d: int, dtype: torch.dtype, device) -> None:
        # compressed_cache.py:69-92 (same capacity formulas)
        self.tail_capacity = self.local_window_tokens + 2 * self.max_chunk_size + 2 * self.block_size
        self.summary_capacity = (self.max_kv_size // self.block_size + 4) if self.max_kv_size is not None else 2048
        # the two rings and the two pools as views of one zeroed allocation (one allocation and one
        # fill instead of four of each, on the path of a stream's first chunk); each view starts on a
        # 256-element boundary
        shapes = [(b, h, self.tail_capacity, d)] * 2 + [(b, h, self.summary_capacity, d)] * 2
        sizes = [b * h * n * d for _, _, n, d in shapes]
        starts, off = [], 0
        for n in sizes:
            starts.append(off)
            off += -(-n // 256) * 256
        flat = torch.zeros(off, dtype=dtype, device=device)
        self._ring_k, self._ring_v, self._pool_k, self._pool_v = (
            flat[s:s + n].view(shape) for s, n, shape in zip(starts, sizes, shapes))

    def _apply_realign(self) -> None:
        if self._realign and self._ring_k is not None:
            shift = (self.offset - self.tail_size) % self.tail_capacity
            if shift:
                self._ring_k = torch.roll(self._ring_k, shifts=shift, dims=2).contiguous()
                self._ring_v = torch.roll(self._ring_v, shifts=shift, dims=2).contiguous()
        self._realign = False

    # ------------------------------------------------------------------ device counters
    def use_device_counters(self, enable: bool = True) -> None:
        """Keep the counters in device memory so ``decode_step`` runs with fixed
        arguments (no host bookkeeping, capturable in a HIP graph).

        Every other method first reads the counters back (a device synchronisation)
        and writes them again after changing them.
        """
        if not enable:
            self.sync()
            self._dev = None
            return
        if self._ring_k is None:
            raise ValueError("allocate the cache with a first update before enabling device counters")
        self._apply_realign()
        b, h = int(self._ring_k.shape[0]), int(self._ring_k.shape[1])
        words = int(_native.lib().bfly_decode_state_words(b, h))
        self._dev = torch.zeros(words, dtype=torch.int64, device=self._ring_k.device)
        self._dev_dirty = False
        self._push()

    def device_step_supported(self, head_dim: int, window: int, dtype: torch.dtype, row_slots: int) -> bool:
        """Whether ``decode_step`` takes a step of this cache: ``window`` (the attention window)
        in [1, 64], head_dim 64 or 128 (256 for bf16), a routed row of at most 16 slots
        (1 + local blocks + partners + sinks) and the cache's own window below 2^20.  Other
        steps run on the host-counter path (``update_and_attend``), which cannot be captured."""
        return (self._ring_k is not None and 0 < int(window) <= _DEC_MAX_WIN
                and (head_dim in (64, 128) or (head_dim == 256 and dtype == torch.bfloat16))
                and dtype in (torch.bfloat16, torch.float32) and 0 < int(row_slots) <= _DEC_MAX_ROW
                and 0 < self.local_window_tokens < (1 << 20))

    def step_on_mfma(self, head_dim: int, window: int, scale: float, dtype: torch.dtype) -> bool:
        """Whether ``decode_step`` of this cache runs on the bf16 MFMA kernel: a positive
        scale and every position, row and element offset of the ring and pool below 2^30
        (the host-side mirror of decode.hip's ``decode_on_mfma``).  The fused q/k norm step
        exists only there."""
        if self._ring_k is None or dtype != torch.bfloat16 or not scale > 0.0:
            return False
        lim = _POS_LIMIT
        ring, pool, bs = self.tail_capacity, self.summary_capacity, self.block_size
        return (ring * head_dim < lim and pool * head_dim < lim and ring < lim
                and (pool + 2) * bs + ring + max(int(window), self.local_window_tokens) < lim)

    @property
    def device_counters(self) -> Optional[torch.Tensor]:
        """The device counter array, or None: word 4 is the error flag; sequence g
        (= batch * Hkv + kv head) of n keeps copies of ``_DEV_SLOT`` words at
        8 + _DEV_SLOT * (g + n * j), j < _dev_copies(n) (eight more copies follow for the
        kernel's route workgroups): {offset, tail_size, summary_count, summary_offset} in
        their first four words (all copies equal), then the kernel's cache of the next
        step's routed row."""
        return self._dev

    def sync(self) -> None:
        """Read device counters back; raise the error a device step recorded.

        A failing step and every step after it leave the counters as they were, so
        the cache keeps the last good state (the counters read back here) and the
        error word is cleared before raising.
        """
        if self._dev is None or not self._dev_dirty:
            return
        head = self._dev[:12].tolist()
        err = int(head[4])
        off, ts, sc, so = (int(x) for x in head[8:12])
        self._dev_dirty = False
        self.offset, self.tail_size, self.summary_count, self.summary_offset = off, ts, sc, so
        if err:
            self._push()
            if err == _DEV_ERR_ROPE:
                raise RuntimeError(
                    f"decode step at position {off} is past the RoPE tables given to the fused q/k norm "
                    f"step; pass cos/sin tables with more rows.")
            raise RuntimeError(
                f"CompressedKVCache capacity exceeded in a device decode step at offset={off} "
                f"(tail_capacity={self.tail_capacity}, summary_capacity={self.summary_capacity}); "
                f"raise max_chunk_size / max_kv_size at construction time.")

    def _push(self) -> None:
        """Write the host counters into every copy; the kernel's routed-row cache is cleared."""
        if self._dev is not None:
            g = (self._dev.numel() - 8) // _DEV_SLOT
            copy = torch.zeros(_DEV_SLOT, dtype=torch.int64)
            copy[:4] = torch.tensor([self.offset, self.tail_size, self.summary_count, self.summary_offset],
                                    dtype=torch.int64)
            self._dev.copy_(torch.cat([torch.zeros(8, dtype=torch.int64), copy.repeat(g)]))
            self._dev_dirty = False

    def decode_step(self, q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, *, layer_idx: int,
                    local_window_tokens: int, partner_rule: str = "causal_shift", local_window_blocks: int = 1,
                    sink_count: int = 1, partner_count: int = 1, scale: Optional[float] = None,
                    out: Optional[torch.Tensor] = None, qk_norm=None) -> torch.Tensor:
        """One token per sequence with device counters: ``update_and_attend`` of one step,
        with the layer's layout at the live kv_len computed on the device.

        q [B, Hq, 1, d]; keys/values [B, Hkv, 1, d].  One kernel launch, fixed
        arguments; the host counters are stale until ``sync()``.  The cache's own
        ``local_window_tokens`` decides which blocks are summarised and how far the
        tail is trimmed (compressed_cache.py:120-164); ``local_window_tokens`` here is
        the attention window.  ``qk_norm`` =
        ``(q_norm_weight, k_norm_weight, rope_cos, rope_sin, eps)``: q and keys are raw
        projection rows, normed and rotated at position ``offset`` inside the launch
        (``bfly_decode_step_qk_norm``: bf16, d = 128; rope tables [rows, 128] fp32).
        """
        from .attention import _scale

        if self._dev is None:
            raise ValueError("call use_device_counters() first")
        b, hq, tq, d = q.shape
        if tq != 1 or keys.shape[2] != 1 or keys.shape != values.shape:
            raise ValueError("decode_step takes one new token per sequence")
        if tuple(keys.shape[:2]) != tuple(self._ring_k.shape[:2]) or keys.shape[3] != self._ring_k.shape[3] or \
                keys.dtype != self._ring_k.dtype or q.dtype != keys.dtype:
            raise ValueError("q/keys do not match the cache's batch/head/dim/dtype")
        dev = self._ring_k.device
        if q.device != dev or keys.device != dev or values.device != dev or (out is not None and out.device != dev):
            raise ValueError(f"decode_step tensors must be on the cache's device {dev}")
        rule = _native.RULES.get(str(partner_rule))
        if rule is None:
            raise ValueError(f"Unsupported Butterfly partner rule: {partner_rule!r}")
        q, keys, values = _c(q), _c(keys), _c(values)
        if out is None:
            out = torch.empty_like(q)
        if qk_norm is not None:
            qw, kw, cos, sin, eps = qk_norm
            if cos.dtype != torch.float32 or cos.shape != sin.shape or cos.dim() != 2 or cos.shape[-1] != d or \
                    not cos.is_contiguous() or not sin.is_contiguous() or cos.device != q.device or \
                    sin.device != q.device:
                raise ValueError("rope tables must be contiguous fp32 [rows, head_dim] on q's device")
            for w in (qw, kw):
                if w.dtype != torch.bfloat16 or tuple(w.shape) != (d,) or not w.is_contiguous() or w.device != q.device:
                    raise ValueError("q/k norm weights must be contiguous bf16 [head_dim] on q's device")
            _native.call("bfly_decode_step_qk_norm", q.data_ptr(), _dtype_code(q), b, hq, int(keys.shape[1]), d,
                         keys.data_ptr(), values.data_ptr(), self._ring_k.data_ptr(), self._ring_v.data_ptr(),
                         self.tail_capacity, self._pool_k.data_ptr(), self._pool_v.data_ptr(), self.summary_capacity,
                         self._dev.data_ptr(), int(layer_idx), rule, int(local_window_blocks), int(sink_count),
                         int(partner_count), self.block_size, int(local_window_tokens), self.local_window_tokens,
                         _scale(scale, d), qw.data_ptr(), kw.data_ptr(), cos.data_ptr(), sin.data_ptr(), int(cos.shape[0]), float(eps),
                         out.data_ptr(), _stream(q))
            self._dev_dirty = True
            return out
        _native.call("bfly_decode_step", q.data_ptr(), _dtype_code(q), b, hq, int(keys.shape[1]), d, keys.data_ptr(),
                     values.data_ptr(), self._ring_k.data_ptr(), self._ring_v.data_ptr(), self.tail_capacity,
                     self._pool_k.data_ptr(), self._pool_v.data_ptr(), self.summary_capacity, self._dev.data_ptr(),
                     int(layer_idx), rule, int(local_window_blocks), int(sink_count), int(partner_count),
                     self.block_size, int(local_window_tokens), self.local_window_tokens, _scale(scale, d),
                     out.data_ptr(), _stream(q))
        self._dev_dirty = True
        return out

    def decode_step_oproj(self, q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, *, layer_idx: int,
                          local_window_tokens: int, qk_norm, o_proj, partner_rule: str = "causal_shift",
                          local_window_blocks: int = 1, sink_count: int = 1, partner_count: int = 1,
                          scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                          parts: Optional[torch.Tensor] = None):
        """``decode_step`` with ``qk_norm`` and the attention output projection ``o_proj`` (a 4-bit
        ``QuantLinear`` over the hq * d attention row) in the same launch
        (``bfly_decode_step_qk_norm_oproj``).  Returns ``(out, parts)``: the attention output
        [B, Hq, 1, d] and the projection's fp32 partial rows per kv head
        [Hkv, B, o_proj.out_features], whose ``bf16((p0 + p1) + (p2 + p3))`` is ``o_proj`` of
        ``out`` bit for bit.  16 query heads over 4 kv heads of 128, batch * 4 <= 16,
        ``out_features`` a multiple of 32 up to 2048 or of 64 up to 4096."""
        from .attention import _scale

        if self._dev is None:
            raise ValueError("call use_device_counters() first")
        b, hq, tq, d = q.shape
        hkv = int(keys.shape[1])
        if tq != 1 or keys.shape[2] != 1 or keys.shape != values.shape:
            raise ValueError("decode_step_oproj takes one new token per sequence")
        if tuple(keys.shape[:2]) != tuple(self._ring_k.shape[:2]) or d != self._ring_k.shape[3] or \
                keys.dtype != self._ring_k.dtype or q.dtype != keys.dtype:
            raise ValueError("q/keys do not match the cache's batch/head/dim/dtype")
        rule = _native.RULES.get(str(partner_rule))
        if rule is None:
            raise ValueError(f"Unsupported Butterfly partner rule: {partner_rule!r}")
        qw, kw, cos, sin, eps = qk_norm
        dev = self._ring_k.device
        if q.device != dev or keys.device != dev or values.device != dev:
            raise ValueError(f"decode_step_oproj tensors must be on the cache's device {dev}")
        if cos.dtype != torch.float32 or cos.shape != sin.shape or cos.dim() != 2 or cos.shape[-1] != d or \
                not cos.is_contiguous() or not sin.is_contiguous() or cos.device != dev or sin.device != dev:
            raise ValueError("rope tables must be contiguous fp32 [rows, head_dim] on the cache's device")
        for w in (qw, kw):
            if w.dtype != torch.bfloat16 or tuple(w.shape) != (d,) or not w.is_contiguous() or w.device != dev:
                raise ValueError("q/k norm weights must be contiguous bf16 [head_dim] on the cache's device")
        n_out = int(o_proj.out_features)
        if int(o_proj.in_features) != hq * d or o_proj.packed.device != dev or o_proj.scale_bias.device != dev \
                or not o_proj.packed.is_contiguous() or not o_proj.scale_bias.is_contiguous():
            raise ValueError(f"o_proj must be a 4-bit layer of hq * head_dim = {hq * d} inputs on the cache's "
                             f"device (contiguous codes and scales)")
        q, keys, values = _c(q), _c(keys), _c(values)
        if out is None:
            out = torch.empty_like(q)
        if parts is None:
            parts = torch.empty(hkv, b, n_out, dtype=torch.float32, device=q.device)
        elif (parts.dtype != torch.float32 or tuple(parts.shape) != (hkv, b, n_out) or not parts.is_contiguous()
              or parts.device != dev):
            raise ValueError(f"parts must be a contiguous fp32 [{hkv}, {b}, {n_out}] tensor on the cache's device")
        _native.call("bfly_decode_step_qk_norm_oproj", q.data_ptr(), _dtype_code(q), b, hq, hkv, d,
                     keys.data_ptr(), values.data_ptr(), self._ring_k.data_ptr(), self._ring_v.data_ptr(),
                     self.tail_capacity, self._pool_k.data_ptr(), self._pool_v.data_ptr(), self.summary_capacity,
                     self._dev.data_ptr(), int(layer_idx), rule, int(local_window_blocks), int(sink_count),
                     int(partner_count), self.block_size, int(local_window_tokens), self.local_window_tokens,
                     _scale(scale, d), qw.data_ptr(), kw.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                     int(cos.shape[0]), float(eps), o_proj.packed.data_ptr(), o_proj.scale_bias.data_ptr(), n_out,
                     int(o_proj.group), parts.data_ptr(), out.data_ptr(), _stream(q))
        self._dev_dirty = True
        return out, parts

    # ------------------------------------------------------------------ update
    def _advance(self, keys: torch.Tensor, values: torch.Tensor):
        """Validate, allocate, and advance the counters for one appended chunk.

        Returns ``(step, first_pos, first_slot, n_new, overflow)``: the blocks
        ``[first_pos, first_pos + n_new*BS)`` are due to be summarised into pool
        slots ``[first_slot, first_slot + n_new)`` (compressed_cache.py:94-149).
        """
        if not keys.is_cuda or keys.shape != values.shape or keys.dtype != values.dtype:
            raise ValueError("keys/values must be matching GPU tensors [B, H, step, d]")
        step = int(keys.shape[2])
        b, h, d = int(keys.shape[0]), int(keys.shape[1]), int(keys.shape[3])
        if self._ring_k is None:
            self._allocate(b, h, d, keys.dtype, keys.device)
        self._apply_realign()
        if tuple(self._ring_k.shape[:2]) != (b, h) or self._ring_k.shape[3] != d or keys.dtype != self._ring_k.dtype:
            raise ValueError("keys do not match the cache's batch/head/dim/dtype")
        bs, lw = self.block_size, self.local_window_tokens
        if self.tail_size + step > self.tail_capacity:
            raise RuntimeError(
                f"CompressedKVCache.tail_capacity={self.tail_capacity} too small to fit "
                f"tail_size={self.tail_size} + step={step}; raise max_chunk_size or "
                f"local_window_tokens to make room.")
        self.tail_size += step
        self.offset += step
        first_pos, first_slot, n_new = self.summary_offset, self.summary_count, 0
        overflow = False
        while self.summary_offset + bs <= self.offset - lw:
            tail_start = self.offset - self.tail_size
            block_start = self.summary_offset - tail_start
            if block_start < 0 or block_start + bs > self.tail_size:
                break
            if self.summary_count + n_new >= self.summary_capacity:
                overflow = True
                break
            n_new += 1
            self.summary_offset += bs
        return step, first_pos, first_slot, n_new, overflow

    def _compress(self, first_pos: int, first_slot: int, n_new: int, overflow: bool, st: int) -> None:
        """Pool the due blocks (they predate the new tokens) and raise on overflow."""
        b, h, _, d = self._ring_k.shape
        if n_new:
            with _on(self._ring_k.device):
                _native.call("bfly_cache_compress", self._ring_k.data_ptr(), self._ring_v.data_ptr(),
                             _dtype_code(self._ring_k), b, h, d, self.tail_capacity, first_pos, n_new,
                             self.block_size, self._pool_k.data_ptr(), self._pool_v.data_ptr(),
                             self.summary_capacity, first_slot, st)
            self.summary_count += n_new
        if overflow:
            raise RuntimeError(
                f"CompressedKVCache.summary_capacity={self.summary_capacity} exhausted "
                f"at offset={self.offset}; raise max_kv_size at construction time.")

    def _trim(self, step: int) -> None:
        """Drop whole blocks from the tail (compressed_cache.py:151-164); a counter update here."""
        bs, lw = self.block_size, self.local_window_tokens
        target = max(lw, step + lw - 1)
        while self.tail_size - bs >= target:
            self.tail_size -= bs

    def update(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Append, summarise completed blocks, trim (compressed_cache.py:94-172).

        The append and the pooling of the blocks that became due run as one
        launch (``bfly_cache_update``); an overflowing pool raises after the
        blocks that fit were pooled, as the reference does.
        """
        self.sync()
        offset0 = self.offset
        step, first_pos, first_slot, n_new, overflow = self._advance(keys, values)
        b, h, d = int(keys.shape[0]), int(keys.shape[1]), int(keys.shape[3])
        keys, values = _c(keys), _c(values)
        with _on(keys.device):
            _native.call("bfly_cache_update", keys.data_ptr(), values.data_ptr(), _dtype_code(keys), b, h, step, d,
                         self._ring_k.data_ptr(), self._ring_v.data_ptr(), self.tail_capacity, offset0, first_pos,
                         n_new, self.block_size, self._pool_k.data_ptr(), self._pool_v.data_ptr(),
                         self.summary_capacity, first_slot, _stream(keys))
        self.summary_count += n_new
        if overflow:
            raise RuntimeError(
                f"CompressedKVCache.summary_capacity={self.summary_capacity} exhausted "
                f"at offset={self.offset}; raise max_kv_size at construction time.")
        self._trim(step)
        self._push()

    def update_and_attend(self, q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, *, layout,
                          local_window_tokens: int, scale: Optional[float] = None) -> torch.Tensor:
        """Append this step's keys/values and attend its queries (the last ``step`` positions).

        Same result as ``update`` followed by
        ``compressed_butterfly_attention_from_cache`` over ``get_compressed_state()``
        (bna/integrations/qwen_mlx.py:1515-1581).  A single-token step runs
        as one fused launch (append + attention; plus the block compressor on the
        steps that complete a block); longer steps append, then attend.
        """
        from .attention import _attend, _require_cuda, _scale

        _require_cuda(q)
        self.sync()
        step = int(keys.shape[2])
        d = int(q.shape[3])
        w = int(local_window_tokens)
        fused = (step == 1 and int(q.shape[2]) == 1 and q.dtype == keys.dtype and w <= 64
                 and layout.neighbors.shape[1] <= 16
                 and (d in (64, 128) or (d == 256 and q.dtype == torch.bfloat16)))
        if not fused:
            self.update(keys, values)
            return _attend(_c(q), self._ring_k, self._ring_v, self._pool_k, self._pool_v, layout=layout,
                           q_pos0=self.offset - int(q.shape[2]), qpos_dev=None, ring_capacity=self.tail_capacity,
                           tail_start=self.offset - self.tail_size, kv_len=self.offset,
                           summary_count=self.summary_count, local_window_tokens=w, scale=scale)
        _, first_pos, first_slot, n_new, overflow = self._advance(keys, values)
        keys, values, q = _c(keys), _c(values), _c(q)
        st = _stream(q)
        self._compress(first_pos, first_slot, n_new, overflow, st)
        self._trim(1)
        self._push()
        b, hq = int(q.shape[0]), int(q.shape[1])
        out = torch.empty_like(q)
        nb = layout.neighbors
        with _on(q.device):
            _native.call("bfly_decode", q.data_ptr(), _dtype_code(q), b, hq, int(keys.shape[1]), d,
                         keys.data_ptr(), values.data_ptr(), self._ring_k.data_ptr(), self._ring_v.data_ptr(),
                         self.tail_capacity, self.offset - self.tail_size, self.offset, self._pool_k.data_ptr(),
                         self._pool_v.data_ptr(), self.summary_capacity, self.summary_count, layout.table.topology,
                         nb.shape[0], layout.block_size, w, _scale(scale, d), out.data_ptr(), st)
        return out

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        self.update(keys, values)
        return self.keys, self.values

    # ------------------------------------------------------------------ views
    def _tail_view(self, ring: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        if ring is None:
            return None
        self.sync()
        if self._realign:
            return ring[:, :, : self.tail_size]
        start = self.offset - self.tail_size
        idx = (torch.arange(start, self.offset, device=ring.device) % self.tail_capacity)
        return ring.index_select(2, idx)

    @property
    def keys(self) -> Optional[torch.Tensor]:
        return self._tail_view(self._ring_k)

    @property
    def values(self) -> Optional[torch.Tensor]:
        return self._tail_view(self._ring_v)

    @property
    def k_summary(self) -> Optional[torch.Tensor]:
        self.sync()
        return None if self._pool_k is None else self._pool_k[:, :, : self.summary_count]

    @property
    def v_summary(self) -> Optional[torch.Tensor]:
        self.sync()
        return None if self._pool_v is None else self._pool_v[:, :, : self.summary_count]

    def get_compressed_state(self):
        self.sync()
        if self._ring_k is None:
            raise ValueError("CompressedKVCache is empty")
        return (self.keys, self.values, self.k_summary, self.v_summary,
                int(self.offset - self.tail_size), int(self.offset))

    def ring_state(self) -> RingState:
        """Device buffers and counters for the attention kernel (no copies)."""
        if self._ring_k is None:
            raise ValueError("CompressedKVCache is empty")
        self.sync()
        self._apply_realign()
        return RingState(self._ring_k, self._ring_v, self.tail_capacity, self.offset - self.tail_size,
                         self.offset, self._pool_k, self._pool_v, self.summary_count)

    # ------------------------------------------------------------------ mlx_lm cache protocol
    def size(self) -> int:
        self.sync()
        return int(self.offset)

    def is_trimmable(self) -> bool:
        return False

    def trim(self, n: int) -> int:
        return 0

    def make_mask(self, N: int, window_size: Optional[int] = None, return_array: bool = False):
        """Causal mask for N new queries (mlx_lm ``create_causal_mask`` semantics)."""
        if N == 1 and window_size is None:
            return None
        if return_array or N > 1:
            dev = self._ring_k.device if self._ring_k is not None else None
            r = torch.arange(self.offset + N, device=dev)
            l = torch.arange(self.offset, self.offset + N, device=dev)[:, None]
            mask = l >= r[None]
            if window_size is not None:
                mask = mask & (l < r[None] + window_size)
            return mask
        return None

    def empty(self) -> bool:
        self.sync()
        return self._ring_k is None or self.tail_size == 0

    @property
    def nbytes(self) -> int:
        """Bytes of the valid slices only (compressed_cache.py:231-244)."""
        if self._ring_k is None:
            return 0
        self.sync()
        b, h, _, d = self._ring_k.shape
        e = self._ring_k.element_size()
        return 2 * b * h * d * e * (self.tail_size + self.summary_count)

    @property
    def allocated_bytes(self) -> int:
        """Device bytes the cache holds: the K and V rings at their full capacity and the K and
        V summary pools (this build's physical layout; ``nbytes`` counts the valid slices)."""
        if self._ring_k is None:
            return 0
        return sum(t.numel() * t.element_size() for t in (self._ring_k, self._ring_v, self._pool_k, self._pool_v))

    @property
    def state(self) -> tuple[Any, Any, Any, Any]:
        self.sync()
        return self.keys, self.values, self.k_summary, self.v_summary

    @state.setter
    def state(self, v) -> None:
        keys, values, k_summary, v_summary = v
        if keys is None or values is None:
            self._ring_k = self._ring_v = None
            self.tail_size = 0
        else:
            b, h, t, d = keys.shape
            if self._ring_k is None or self._ring_k.shape[2] < t:
                self._allocate(int(b), int(h), int(d), keys.dtype, keys.device)
            self._ring_k[:, :, :t] = keys
            self._ring_v[:, :, :t] = values
            self.tail_size = int(t)
            self._realign = True
        if k_summary is None or v_summary is None:
            self.summary_count = 0
        else:
            b, h, s, d = k_summary.shape
            if self._pool_k is None or self._pool_k.shape[2] < s:
                cap = max(int(s), self.summary_capacity)
                self._pool_k = torch.zeros((b, h, cap, d), dtype=k_summary.dtype, device=k_summary.device)
                self._pool_v = torch.zeros_like(self._pool_k)
                self.summary_capacity = cap
            self._pool_k[:, :, :s] = k_summary
            self._pool_v[:, :, :s] = v_summary
            self.summary_count = int(s)
        self._push()

    @property
    def meta_state(self) -> tuple[str, str, str, str]:
        self.sync()
        return tuple(map(str, (self.block_size, self.local_window_tokens, self.offset, self.summary_offset)))

    @meta_state.setter
    def meta_state(self, v) -> None:
        self.sync()
        self.block_size, self.local_window_tokens, self.offset, self.summary_offset = map(int, v)
        self._push()
