"""A random-init Qwen3-style decoder in PyTorch, the model the layer swap plugs into.

The reference swaps attention inside third-party decoders (mlx_lm / HF
transformers Qwen models, bna/integrations/qwen_mlx.py:1822-1846,
qwen_torch.py:1652-1700); none can be downloaded here, so this module
provides the same structure with random weights: ``model.layers[i].self_attn``
with q/k/v/o projections, per-head q/k RMSNorm and RoPE (qwen_mlx.py:260-357),
SwiGLU MLP, RMSNorm, tied embeddings.  Linear weights and the tied embedding
are stored 4-bit affine (group 64 along the input dimension, bf16 scale and
bias per group: w = q * scale + bias, q in [0, 15]).  A single activation row
on the GPU (a decode step, the prefill's last-position logits) is multiplied
straight from the 4-bit codes by ``bfly_q4_gemv`` (``bfly_q4_gemv_silu`` for
the gate|up projection with SiLU * up); larger products run through
PyTorch-ROCm's GEMMs over the weights dequantized once to bf16 (q/k/v and
gate/up as one GEMM each).  On the GPU (bf16) the row-wise
and elementwise steps -- residual add + RMSNorm, q/k norm + RoPE + the move to
heads-first, SiLU * up -- run as single HIP launches
(include/butterfly_amd_decoder.h) with the rounding points of the PyTorch
forms written below, which are the model's definition and what a CPU copy of
the model runs.

``swap_qwen_attention_with_butterfly(model, cfg=...)`` replaces every
attention by :class:`ButterflyAttention` (registered for :class:`Attention`), a
``QwenButterflyAttention`` that keeps the projections, norms and RoPE, routes
the attention core through the HIP kernels
(:class:`butterfly_amd.ButterflyAttentionCore`) and adds this model's fused
projection paths.  The attention exposes the attribute set the generic swapped
module reads (``n_heads``, ``n_kv_heads``, ``head_dim``, ``scale``, the
projections and norms), so ``QwenButterflyAttention`` itself also wraps it.  The
stock attention that it replaces is plain causal GQA softmax attention (PyTorch
SDPA).  Attention modules take ``(x, mask=None, cache=None, *,
position_embeddings=(cos, sin))``, the RoPE rows of the call's positions.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass
from typing import Callable, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native
from ._device import on, stream_of
from .compressed_cache import CompressedKVCache
from .integrations import QwenButterflyAttention, QwenButterflyConfig, register_butterfly_attention


@dataclass
class DecoderConfig:
    vocab_size: int = 151936
    hidden_size: int = 2048
    num_layers: int = 24
    num_heads: int = 16
    num_kv_heads: int = 4
    head_dim: int = 128
    intermediate_size: int = 6144
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    quant_group: int = 64
    quant_bits: int = 4


# ----------------------------------------------------------------------------- 4-bit affine weights
def quantize_affine(w: torch.Tensor, group: int = 64, bits: int = 4):
    """Per-group affine quantisation along the input dimension.

    Returns ``(packed uint8 [out, in/2], scale bf16 [out, in/group], bias bf16 [out, in/group])``
    with ``w ~= q * scale + bias``; two 4-bit codes per byte, low nibble first.
    """
    out_f, in_f = w.shape
    if in_f % group != 0 or bits != 4:
        raise ValueError("in_features must be a multiple of the group; only 4-bit codes are supported")
    g = w.float().view(out_f, in_f // group, group)
    lo = g.amin(-1, keepdim=True)
    hi = g.amax(-1, keepdim=True)
    scale = ((hi - lo) / 15.0).clamp_min(1e-8)
    scale_b, bias_b = scale.to(torch.bfloat16), lo.to(torch.bfloat16)
    q = torch.round((g - bias_b.float()) / scale_b.float()).clamp_(0, 15).to(torch.uint8).view(out_f, in_f)
    packed = q[:, 0::2] | (q[:, 1::2] << 4)
    return packed.contiguous(), scale_b.view(out_f, -1).contiguous(), bias_b.view(out_f, -1).contiguous()


def dequantize_affine(packed: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor, group: int = 64) -> torch.Tensor:
    out_f = packed.shape[0]
    q = torch.stack([packed & 0xF, packed >> 4], dim=-1).view(out_f, -1).float()
    w = q.view(out_f, -1, group) * scale.float().unsqueeze(-1) + bias.float().unsqueeze(-1)
    return w.view(out_f, -1).to(torch.bfloat16)


_Q4_TENSORS = ("packed", "scale", "bias", "scale_bias", "weight")


class QuantLinear(nn.Module):
    """Linear layer with 4-bit affine weights.

    Buffers: ``packed`` (two codes per byte, low nibble first), ``scale`` and ``bias``
    (bf16 per group), ``scale_bias`` (the same pairs interleaved, [out, in/group, 2], the
    layout ``bfly_q4_gemv`` reads) and ``weight`` (dequantized once to bf16, for the
    multi-row GEMMs and for CPU copies of the model)."""

    def __init__(self, in_features: int, out_features: int, *, generator: Optional[torch.Generator] = None,
                 device=None, group: int = 64, weight: Optional[torch.Tensor] = None):
        super().__init__()
        if weight is None:
            weight = torch.randn(out_features, in_features, generator=generator, device=device) / math.sqrt(in_features)
        self.group = group
        self._set(*quantize_affine(weight, group))

    def _set(self, packed, scale, bias):
        self.register_buffer("packed", packed)
        self.register_buffer("scale", scale)
        self.register_buffer("bias", bias)
        self.register_buffer("scale_bias", torch.stack([scale, bias], -1).contiguous())
        self.register_buffer("weight", dequantize_affine(packed, scale, bias, self.group))

    @property
    def in_features(self) -> int:
        return int(self.packed.shape[1]) * 2

    @property
    def out_features(self) -> int:
        return int(self.packed.shape[0])

    @classmethod
    def fuse_rows(cls, *parts: "QuantLinear") -> "QuantLinear":
        """One layer whose output rows are the given layers' rows in order (q|k|v, gate|up):
        each part's tensors become views of their row range, so memory is not doubled."""
        fused = cls.__new__(cls)
        nn.Module.__init__(fused)
        fused.group = parts[0].group
        for name in _Q4_TENSORS:
            fused.register_buffer(name, torch.cat([getattr(m, name) for m in parts]))
        row = 0
        for m in parts:
            n = m.out_features
            for name in _Q4_TENSORS:
                setattr(m, name, getattr(fused, name)[row:row + n])
            row += n
        return fused

    @property
    def gemv_from_codes(self) -> bool:
        """Whether ``bfly_q4_gemv`` takes this layer's shape: groups of a multiple of 32 codes
        and at most 8192 inputs (the kernel keeps a lane's inputs in registers)."""
        return self.group % Q4_PIECE_CODES == 0 and self.in_features <= Q4_MAX_IN

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _one_row(x) and self.gemv_from_codes:
            return q4_gemv(x, self)
        return _linear(x, self.weight)


# shape limits of bfly_q4_gemv / bfly_q4_gemv_silu (include/butterfly_amd_decoder.h)
Q4_PIECE_CODES, Q4_MAX_IN = 32, 8192
# decode steps of a swapped layer run its output projection in the decode-step launch where
# the shapes allow (ButterflyAttention.takes_o_proj); False keeps it a launch of its own
FUSE_O_PROJ = True
# graph-replayed greedy steps of one sequence pick the token from the lm_head launch's
# per-workgroup candidates and advance token, output, counters and the next input in one more
# launch (GreedyState); False keeps torch's embedding, index_copy and add and the argmax passes
FUSE_GREEDY = True


def _one_row(x: torch.Tensor) -> bool:
    """A single bf16 activation row on the GPU: the product runs from the 4-bit codes."""
    return x.is_cuda and x.dtype == torch.bfloat16 and x.numel() == x.shape[-1]


def _row16(x: torch.Tensor) -> torch.Tensor:
    x = x.reshape(-1)
    if not x.is_contiguous() or x.data_ptr() % 16:
        x = x.clone()
    return x


def q4_gemv(x: torch.Tensor, layer: QuantLinear) -> torch.Tensor:
    """``layer(x)`` for one bf16 row ``x`` [..., in] through ``bfly_q4_gemv`` (reads the
    4-bit codes and the (scale, bias) pairs; fp32 accumulation, bf16 out)."""
    xr = _row16(x)
    out = torch.empty(*x.shape[:-1], layer.out_features, dtype=torch.bfloat16, device=x.device)
    with on(x.device):
        _native.call("bfly_q4_gemv", xr.data_ptr(), layer.packed.data_ptr(), layer.scale_bias.data_ptr(),
                     layer.out_features, layer.in_features, layer.group, out.data_ptr(), stream_of(x))
    return out


def q4_gemv_silu(x: torch.Tensor, gate_up: QuantLinear) -> torch.Tensor:
    """``SiLU(gate(x)) * up(x)`` for one bf16 row through ``bfly_q4_gemv_silu``; ``gate_up``
    holds the gate rows, then as many up rows.  Same rounding points as the two projections'
    bf16 outputs followed by ``bfly_silu_mul``."""
    xr = _row16(x)
    f = gate_up.out_features // 2
    out = torch.empty(*x.shape[:-1], f, dtype=torch.bfloat16, device=x.device)
    with on(x.device):
        _native.call("bfly_q4_gemv_silu", xr.data_ptr(), gate_up.packed.data_ptr(), gate_up.scale_bias.data_ptr(),
                     f, gate_up.in_features, gate_up.group, f, out.data_ptr(), stream_of(x))
    return out


NORM_Q4_DIMS = (2048, 4096, 6144)   # row lengths of bfly_add_rms_norm_q4_gemv(_silu)


def norm_q4_fits(x: torch.Tensor, layer: QuantLinear) -> bool:
    """Whether one row ``x`` takes the fused residual add + RMSNorm + 4-bit product."""
    return _one_row(x) and layer.gemv_from_codes and layer.in_features in NORM_Q4_DIMS \
        and int(x.shape[-1]) == layer.in_features


def add_rms_norm_q4_gemv(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
                         layer: QuantLinear):
    """``(h, layer(n))`` with ``h, n = add_rms_norm(x, residual, weight, eps)`` for one bf16 row, in
    one launch of ``bfly_add_rms_norm_q4_gemv`` (bit-identical to the two launches; ``h`` is
    computed even when the caller drops it)."""
    xr = _row16(x)
    rr = _row16(residual) if residual is not None else None
    h = torch.empty_like(xr)
    out = torch.empty(*x.shape[:-1], layer.out_features, dtype=torch.bfloat16, device=x.device)
    with on(x.device):
        _native.call("bfly_add_rms_norm_q4_gemv", xr.data_ptr(), rr.data_ptr() if rr is not None else None,
                     weight.data_ptr(), float(eps), h.data_ptr() if rr is not None else None,
                     layer.packed.data_ptr(), layer.scale_bias.data_ptr(), layer.out_features, layer.in_features,
                     layer.group, out.data_ptr(), stream_of(x))
    return (h.view(x.shape) if rr is not None else x), out


def add_rms_norm_q4_gemv_silu(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
                              gate_up: QuantLinear):
    """``(h, SiLU(gate(n)) * up(n))`` with ``h, n = add_rms_norm(...)`` for one bf16 row, in one
    launch of ``bfly_add_rms_norm_q4_gemv_silu`` (bit-identical to the two launches)."""
    xr = _row16(x)
    rr = _row16(residual) if residual is not None else None
    h = torch.empty_like(xr)
    f = gate_up.out_features // 2
    out = torch.empty(*x.shape[:-1], f, dtype=torch.bfloat16, device=x.device)
    with on(x.device):
        _native.call("bfly_add_rms_norm_q4_gemv_silu", xr.data_ptr(), rr.data_ptr() if rr is not None else None,
                     weight.data_ptr(), float(eps), h.data_ptr() if rr is not None else None,
                     gate_up.packed.data_ptr(), gate_up.scale_bias.data_ptr(), f, gate_up.in_features,
                     gate_up.group, f, out.data_ptr(), stream_of(x))
    return (h.view(x.shape) if rr is not None else x), out


def add_rms_norm_q4_gemv_silu_parts(x: torch.Tensor, parts: torch.Tensor, weight: torch.Tensor, eps: float,
                                    gate_up: QuantLinear):
    """``add_rms_norm_q4_gemv_silu(x, a, ...)`` where the residual branch ``a`` is given as four fp32
    partial rows ``parts`` [4, 1, hidden] (``a = bf16((p0 + p1) + (p2 + p3))``, the output
    projection of ``CompressedKVCache.decode_step_oproj``), in one launch of
    ``bfly_add_rms_norm_q4_gemv_silu_parts``: ``x`` is this layer's residual input, ``h = x + a``."""
    xr = _row16(x)
    if parts.dtype != torch.float32 or not parts.is_contiguous() or parts.numel() != 4 * xr.numel() or \
            parts.data_ptr() % 16:
        raise ValueError("parts must be a contiguous, 16-byte aligned fp32 [4, 1, hidden] tensor")
    h = torch.empty_like(xr)
    f = gate_up.out_features // 2
    out = torch.empty(*x.shape[:-1], f, dtype=torch.bfloat16, device=x.device)
    with on(x.device):
        _native.call("bfly_add_rms_norm_q4_gemv_silu_parts", parts.data_ptr(), 4, xr.data_ptr(), weight.data_ptr(),
                     float(eps), h.data_ptr(), gate_up.packed.data_ptr(), gate_up.scale_bias.data_ptr(), f,
                     gate_up.in_features, gate_up.group, f, out.data_ptr(), stream_of(x))
    return h.view(x.shape), out


def add_rms_norm_q4_gemv_argmax(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor,
                                eps: float, layer: QuantLinear, workspace: torch.Tensor) -> torch.Tensor:
    """``add_rms_norm_q4_gemv(...)[1]`` through ``bfly_add_rms_norm_q4_gemv_argmax``, which also leaves
    its per-workgroup greedy candidates in ``workspace`` (uint8, ``bfly_q4_argmax_workspace_bytes``
    bytes) for ``greedy_advance``."""
    xr = _row16(x)
    rr = _row16(residual) if residual is not None else None
    h = torch.empty_like(xr) if rr is not None else None
    out = torch.empty(*x.shape[:-1], layer.out_features, dtype=torch.bfloat16, device=x.device)
    with on(x.device):
        _native.call("bfly_add_rms_norm_q4_gemv_argmax", xr.data_ptr(), rr.data_ptr() if rr is not None else None,
                     weight.data_ptr(), float(eps), h.data_ptr() if h is not None else None,
                     layer.packed.data_ptr(), layer.scale_bias.data_ptr(), layer.out_features, layer.in_features,
                     layer.group, out.data_ptr(), workspace.data_ptr(), workspace.numel(), stream_of(x))
    return out


class GreedyState:
    """What ``bfly_greedy_advance`` updates after each graph-replayed decode step of one sequence:
    ``tok`` [1, 1] int64 (the pick), ``out`` [1, n] int64 (picks by column), ``ctr`` int64
    [position, column], ``x`` [1, 1, hidden] bf16 (the next step's embedded input), and the
    candidate workspace of ``add_rms_norm_q4_gemv_argmax``."""

    def __init__(self, tok, out, ctr, x, workspace):
        self.tok, self.out, self.ctr, self.x, self.workspace = tok, out, ctr, x, workspace


def greedy_advance(g: GreedyState, embed: torch.Tensor) -> None:
    """The greedy pick from ``g.workspace`` and the step's bookkeeping in one launch
    (``bfly_greedy_advance``): ``g.tok``, ``g.out[0, col]``, ``g.ctr`` + 1 and ``g.x = embed[pick]``."""
    with on(g.x.device):
        _native.call("bfly_greedy_advance", g.workspace.data_ptr(), g.workspace.numel(), embed.data_ptr(),
                     int(embed.shape[0]),
                     int(embed.shape[1]), g.x.data_ptr(), g.tok.data_ptr(), g.out.data_ptr(), int(g.out.numel()),
                     g.ctr.data_ptr(), stream_of(g.x))


def _linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``x @ w^T``.  One row of activations on the GPU (a decode step at batch 1) runs as
    ``w @ x^T``, which PyTorch-ROCm hands to a GEMV kernel that streams the weight at close
    to HBM rate; its ``F.linear`` form is a skinny GEMM that spreads a small weight over too
    few workgroups."""
    if x.is_cuda and x.numel() == x.shape[-1]:
        return torch.matmul(w, x.reshape(-1, 1)).view(*x.shape[:-1], w.shape[0])
    return F.linear(x, w)


def _hip(x: torch.Tensor) -> bool:
    """bf16 tensors on the GPU take the HIP kernels of the decoder steps."""
    return x.is_cuda and x.dtype == torch.bfloat16


def add_rms_norm(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor, eps: float):
    """``(h, n)``: ``h = x + residual`` (bf16; ``x`` when no residual) and ``n = RMSNorm(h) * weight``,
    one launch of ``bfly_add_rms_norm``."""
    xc = x.contiguous()
    dim = int(xc.shape[-1])
    n = torch.empty_like(xc)
    rc = residual.contiguous() if residual is not None else None
    h = torch.empty_like(xc) if rc is not None else None
    with on(xc.device):
        _native.call("bfly_add_rms_norm", xc.data_ptr(), rc.data_ptr() if rc is not None else None,
                     weight.data_ptr(), xc.numel() // dim, dim, float(eps), h.data_ptr() if h is not None else None,
                     n.data_ptr(), stream_of(xc))
    return (h if h is not None else xc), n


def argmax_rows(x: torch.Tensor, parallel: bool = True) -> torch.Tensor:
    """``x.argmax(-1, keepdim=True)`` for a 2-D bf16 GPU tensor (any strides) through
    ``bfly_argmax_rows``: torch's argmax reduction records a memset node when captured in a
    graph, these kernels write their results directly.  ``parallel=False`` passes no
    workspace (one workgroup per row)."""
    rows, n = x.shape
    out = torch.empty(rows, 1, dtype=torch.long, device=x.device)
    ws = torch.empty(rows * 3072 + 8 if parallel else 0, dtype=torch.uint8, device=x.device)
    with on(x.device):
        _native.call("bfly_argmax_rows", x.data_ptr(), rows, n, x.stride(0), x.stride(1),
                     ws.data_ptr() if parallel else None, ws.numel(), out.data_ptr(), stream_of(x))
    return out


def argmax_rows_noalloc(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``argmax_rows`` for at most 64 rows through ``bfly_argmax_rows_noalloc``: no workspace and
    no allocation besides the output (the library's static device workspace holds the
    per-workgroup candidates; calls that overlap on one GPU race).  ``out``: a contiguous int64
    [rows, 1] tensor to write instead of a new one."""
    rows, n = x.shape
    if out is None:
        out = torch.empty(rows, 1, dtype=torch.long, device=x.device)
    elif out.shape != (rows, 1) or out.dtype != torch.long or not out.is_contiguous() or out.device != x.device:
        raise ValueError("out must be a contiguous int64 [rows, 1] tensor on the input's device")
    with on(x.device):
        _native.call("bfly_argmax_rows_noalloc", x.data_ptr(), rows, n, x.stride(0), x.stride(1), out.data_ptr(),
                     stream_of(x))
    return out


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float, device):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=torch.bfloat16), requires_grad=False)
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _hip(x) and x.shape[-1] % 256 == 0:
            return add_rms_norm(x, None, self.weight, self.eps)[1]
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float):
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=positions.device, dtype=torch.float32) / head_dim))
    ang = positions.float()[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos(), emb.sin()


class RopeTable:
    """RoPE for one decode step whose position lives on the device: the full cos/sin tables
    [rows, d] (fp32) and the position tensor [1].  ``rows()`` gives the ``(cos, sin)`` rows a
    projection needs; a swapped attention with a device-counter cache passes the tables to
    the decode step instead, which reads the row of its own position."""

    def __init__(self, cos_tab: torch.Tensor, sin_tab: torch.Tensor, pos: torch.Tensor):
        self.cos_tab, self.sin_tab, self.pos = cos_tab, sin_tab, pos

    def rows(self):
        return self.cos_tab.index_select(0, self.pos), self.sin_tab.index_select(0, self.pos)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, H, T, d]; rotate-half RoPE in fp32."""
    d = x.shape[-1]
    xf = x.float()
    rot = torch.cat([-xf[..., d // 2:], xf[..., : d // 2]], dim=-1)
    return (xf * cos + rot * sin).to(x.dtype)


# ----------------------------------------------------------------------------- attention
class Attention(nn.Module):
    """Stock attention: projections, q/k RMSNorm, RoPE and causal GQA softmax attention."""

    def __init__(self, cfg: DecoderConfig, *, generator: torch.Generator, device):
        super().__init__()
        h, d = cfg.hidden_size, cfg.head_dim
        self.cfg = cfg
        self.q_proj = QuantLinear(h, cfg.num_heads * d, generator=generator, device=device, group=cfg.quant_group)
        self.k_proj = QuantLinear(h, cfg.num_kv_heads * d, generator=generator, device=device, group=cfg.quant_group)
        self.v_proj = QuantLinear(h, cfg.num_kv_heads * d, generator=generator, device=device, group=cfg.quant_group)
        self.o_proj = QuantLinear(cfg.num_heads * d, h, generator=generator, device=device, group=cfg.quant_group)
        self.q_norm = RMSNorm(d, cfg.rms_eps, device)
        self.k_norm = RMSNorm(d, cfg.rms_eps, device)
        self.n_heads, self.n_kv_heads, self.head_dim = cfg.num_heads, cfg.num_kv_heads, d
        self.scale = d ** -0.5
        # q, k and v weights as row ranges of one [Hq*d + 2*Hkv*d, hidden] layer: one product per
        # projection on the GPU path, whose kernels read q, k and v as column ranges of its output.
        self.qkv = QuantLinear.fuse_rows(self.q_proj, self.k_proj, self.v_proj)

    def project(self, x: torch.Tensor, positions: torch.Tensor, rope=None):
        """x [B, T, hidden] -> q [B, Hq, T, d], k/v [B, Hkv, T, d] (normed, RoPE applied).

        ``rope`` is an optional precomputed ``(cos, sin)`` for ``positions``."""
        b, t, _ = x.shape
        c = self.cfg
        if isinstance(rope, RopeTable):
            rope = rope.rows()
        if _hip(x) and c.head_dim in (128, 256):
            return self.heads(self.qkv(x), positions, rope)
        q = self.q_proj(x).view(b, t, c.num_heads, c.head_dim).transpose(1, 2)
        k = self.k_proj(x).view(b, t, c.num_kv_heads, c.head_dim).transpose(1, 2)
        v = self.v_proj(x).view(b, t, c.num_kv_heads, c.head_dim).transpose(1, 2)
        q, k = self.q_norm(q), self.k_norm(k)
        cos, sin = rope if rope is not None else rope_cos_sin(positions, c.head_dim, c.rope_theta)
        return apply_rope(q, cos, sin).contiguous(), apply_rope(k, cos, sin).contiguous(), v.contiguous()

    def heads(self, qkv: torch.Tensor, positions: torch.Tensor, rope=None):
        """The fused projection output [B, T, (Hq + 2 Hkv) d] (bf16, GPU, d in {128, 256}) ->
        q [B, Hq, T, d], k/v [B, Hkv, T, d]: q/k RMSNorm and RoPE in one ``bfly_qk_norm_rope``."""
        b, t, _ = qkv.shape
        c = self.cfg
        if isinstance(rope, RopeTable):
            rope = rope.rows()
        nq, nkv = c.num_heads * c.head_dim, c.num_kv_heads * c.head_dim
        base, ld, es = qkv.data_ptr(), qkv.shape[-1], qkv.element_size()
        cos, sin = rope if rope is not None else rope_cos_sin(positions, c.head_dim, c.rope_theta)
        cos, sin = cos.float().contiguous(), sin.float().contiguous()
        qo = torch.empty(b, c.num_heads, t, c.head_dim, dtype=qkv.dtype, device=qkv.device)
        ko = torch.empty(b, c.num_kv_heads, t, c.head_dim, dtype=qkv.dtype, device=qkv.device)
        vo = torch.empty_like(ko)
        with on(qkv.device):
            _native.call("bfly_qk_norm_rope", base, base + nq * es, base + (nq + nkv) * es, ld, ld, ld,
                         self.q_norm.weight.data_ptr(), self.k_norm.weight.data_ptr(), cos.data_ptr(),
                         sin.data_ptr(), b, t, c.num_heads, c.num_kv_heads, c.head_dim, float(self.q_norm.eps),
                         qo.data_ptr(), ko.data_ptr(), vo.data_ptr(), stream_of(qkv))
        return qo, ko, vo

    def output(self, o: torch.Tensor) -> torch.Tensor:
        b, _, t, _ = o.shape
        return self.o_proj(o.transpose(1, 2).reshape(b, t, -1))

    def forward(self, x: torch.Tensor, mask=None, cache=None, *, position_embeddings=None) -> torch.Tensor:
        """``cache``: a list ``[k, v]`` of the full history (empty before the first call);
        ``position_embeddings``: ``(cos, sin)`` rows of the call's positions (or a ``RopeTable``),
        else computed from the cache length."""
        positions = None
        if position_embeddings is None:
            start = int(cache[0].shape[2]) if cache else 0
            positions = torch.arange(start, start + x.shape[1], device=x.device)
        q, k, v = self.project(x, positions, position_embeddings)
        if cache is not None:           # a list cache [k, v] of the full history
            if cache:
                k = torch.cat([cache[0], k], 2)
                v = torch.cat([cache[1], v], 2)
            cache[:] = [k, v]
        groups = q.shape[1] // k.shape[1]
        kk = k.repeat_interleave(groups, 1)
        vv = v.repeat_interleave(groups, 1)
        tq, tk = q.shape[2], kk.shape[2]
        mask = torch.ones(tq, tk, dtype=torch.bool, device=q.device).tril(tk - tq)
        o = F.scaled_dot_product_attention(q, kk, vv, attn_mask=mask)
        return self.output(o)

class ButterflyAttention(QwenButterflyAttention):
    """The swapped attention of this decoder: ``QwenButterflyAttention`` over the base
    module's fused projection (q, k and v read as column ranges of one product, q/k norm
    and RoPE in one launch) and, for a graph-replayed decode step with device counters,
    the decode step that applies the q/k norm and RoPE itself at its device position.

    Counterpart of ``QwenButterflyAttention`` (bna/integrations/qwen_mlx.py:1295-1792)
    and ``QwenCUDAButterflyAttention.forward`` (qwen_torch.py:1221-1622).
    """

    def __init__(self, base: Attention, cfg: QwenButterflyConfig, *, layer_idx: Optional[int] = None):
        super().__init__(base, cfg, layer_idx=layer_idx)
        self.base = base

    def forward(self, x: torch.Tensor, mask=None, cache=None, *, position_embeddings=None) -> torch.Tensor:
        base, c = self.base, self.base.cfg
        rope = position_embeddings
        if rope is None:
            raise ValueError("the decoder passes the RoPE rows of the call's positions (position_embeddings)")
        if self.takes_qkv_row(x, cache, rope):
            # one decode step with device counters: the raw q|k|v row goes to the decode
            # step, which applies q/k RMSNorm and RoPE at its own position (one launch fewer)
            return self.forward_qkv_row(base.qkv(x), cache, rope)
        q, k, v = base.project(x, None, rope)
        return base.output(self.attend(q, k, v, cache))

    def takes_qkv_row(self, x: torch.Tensor, cache, rope) -> bool:
        """Whether this call is a device-counter decode step fed with the raw q|k|v row."""
        c = self.base.cfg
        return (isinstance(rope, RopeTable) and _one_row(x)
                and self.core.fuses_qk_norm(cache, 1, c.head_dim, x.dtype))

    def _qkv_row(self, qkv: torch.Tensor, rope):
        base, c = self.base, self.base.cfg
        row = qkv.view(-1)
        nq, nkv = c.num_heads * c.head_dim, c.num_kv_heads * c.head_dim
        q = row[:nq].view(1, c.num_heads, 1, c.head_dim)
        k = row[nq:nq + nkv].view(1, c.num_kv_heads, 1, c.head_dim)
        v = row[nq + nkv:].view(1, c.num_kv_heads, 1, c.head_dim)
        qk = (base.q_norm.weight, base.k_norm.weight, rope.cos_tab, rope.sin_tab, base.q_norm.eps)
        return q, k, v, qk

    def forward_qkv_row(self, qkv: torch.Tensor, cache, rope) -> torch.Tensor:
        """The decode step from the fused projection's raw output row (``base.qkv`` of the
        normed input; ``takes_qkv_row`` held), through the output projection."""
        q, k, v, qk = self._qkv_row(qkv, rope)
        return self.base.output(self.core(q, k, v, cache, qk_norm=qk))

    def takes_o_proj(self, x: torch.Tensor, cache, rope) -> bool:
        """Whether this decode step also runs the output projection in its launch
        (``forward_qkv_row_parts``): a ``takes_qkv_row`` step of 16 query heads over 4 kv heads of
        128 whose o_proj is a 4-bit layer of 2048 inputs, a power-of-two group and a multiple of 32
        outputs up to 2048 or of 64 up to 4096 (``bfly_decode_step_qk_norm_oproj``)."""
        c, o = self.base.cfg, self.base.o_proj
        n = o.out_features if isinstance(o, QuantLinear) else 0
        return (FUSE_O_PROJ and c.num_heads == 16 and c.num_kv_heads == 4 and c.head_dim == 128
                and isinstance(o, QuantLinear) and o.gemv_from_codes and o.in_features == 2048
                and ((n % 32 == 0 and 0 < n <= 2048) or (n % 64 == 0 and 0 < n <= 4096))
                and o.group & (o.group - 1) == 0 and self.takes_qkv_row(x, cache, rope))

    def forward_qkv_row_parts(self, qkv: torch.Tensor, cache, rope) -> torch.Tensor:
        """``forward_qkv_row`` with the output projection inside the decode step
        (``takes_o_proj`` held): returns its four fp32 partial rows [4, 1, hidden], which
        ``add_rms_norm_q4_gemv_silu_parts`` combines into the projection's bf16 row."""
        q, k, v, qk = self._qkv_row(qkv, rope)
        return self.core.step_oproj(q, k, v, cache, qk, self.base.o_proj)[1]


register_butterfly_attention(Attention, ButterflyAttention)


class MLP(nn.Module):
    def __init__(self, cfg: DecoderConfig, *, generator: torch.Generator, device):
        super().__init__()
        h, f = cfg.hidden_size, cfg.intermediate_size
        self.gate_proj = QuantLinear(h, f, generator=generator, device=device, group=cfg.quant_group)
        self.up_proj = QuantLinear(h, f, generator=generator, device=device, group=cfg.quant_group)
        self.down_proj = QuantLinear(f, h, generator=generator, device=device, group=cfg.quant_group)
        self.gate_up = QuantLinear.fuse_rows(self.gate_proj, self.up_proj)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _one_row(x) and self.gate_up.gemv_from_codes:
            return self.down_proj(q4_gemv_silu(x, self.gate_up))
        if _hip(x):
            gu = self.gate_up(x)                           # [..., 2f]: gate columns, then up columns
            f = gu.shape[-1] // 2
            s = gu.new_empty(*gu.shape[:-1], f)
            with on(x.device):
                _native.call("bfly_silu_mul", gu.data_ptr(), gu.data_ptr() + f * gu.element_size(),
                             gu.numel() // (2 * f), f, 2 * f, s.data_ptr(), stream_of(x))
            return self.down_proj(s)
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, cfg: DecoderConfig, *, generator: torch.Generator, device):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_eps, device)
        self.self_attn = Attention(cfg, generator=generator, device=device)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_eps, device)
        self.mlp = MLP(cfg, generator=generator, device=device)

    def forward(self, x: torch.Tensor, positions: torch.Tensor, cache=None, rope=None) -> torch.Tensor:
        if _hip(x) and x.shape[-1] % 256 == 0:
            a = self.self_attn(self.input_layernorm(x), cache=cache, position_embeddings=rope)
            h, n = add_rms_norm(x, a, self.post_attention_layernorm.weight, self.post_attention_layernorm.eps)
            return h + self.mlp(n)
        x = x + self.self_attn(self.input_layernorm(x), cache=cache, position_embeddings=rope)
        return x + self.mlp(self.post_attention_layernorm(x))

    def forward_split(self, x: torch.Tensor, pending: Optional[torch.Tensor], positions: torch.Tensor, cache=None,
                      rope=None):
        """The HIP form of ``forward`` with the last residual add left pending: returns ``(h, m)``
        whose sum is the layer's output.  ``pending`` is the previous layer's ``m`` (or None); it
        is added to ``x`` in the launch that computes the input RMSNorm, which rounds the sum to
        bf16 before normalising it, as the separate add would."""
        attn, mlp = self.self_attn, self.mlp
        ln, post = self.input_layernorm, self.post_attention_layernorm
        if (isinstance(attn, ButterflyAttention) and attn.takes_qkv_row(x, cache, rope)
                and norm_q4_fits(x, attn.base.qkv)):
            # a decode step: each norm rides in the launch of the product that consumes it
            x, qkv = add_rms_norm_q4_gemv(x, pending, ln.weight, ln.eps, attn.base.qkv)
            if (attn.takes_o_proj(x, cache, rope) and norm_q4_fits(x, mlp.gate_up)
                    and mlp.down_proj.gemv_from_codes):
                # and the output projection rides in the decode step: its partial rows go
                # straight into the post-attention norm of the gate|up launch
                parts = attn.forward_qkv_row_parts(qkv, cache, rope)
                h, s = add_rms_norm_q4_gemv_silu_parts(x, parts, post.weight, post.eps, mlp.gate_up)
                return h, mlp.down_proj(s)
            a = attn.forward_qkv_row(qkv, cache, rope)
        else:
            x, n = add_rms_norm(x, pending, ln.weight, ln.eps)
            a = attn(n, cache=cache, position_embeddings=rope)
        if norm_q4_fits(x, mlp.gate_up) and mlp.down_proj.gemv_from_codes:
            h, s = add_rms_norm_q4_gemv_silu(x, a, post.weight, post.eps, mlp.gate_up)
            return h, mlp.down_proj(s)
        h, n = add_rms_norm(x, a, post.weight, post.eps)
        return h, mlp(n)


class Decoder(nn.Module):
    """Random-init decoder; ``forward(tokens, caches, start)`` returns last-position logits."""

    def __init__(self, cfg: DecoderConfig, *, seed: int = 0, device=None):
        super().__init__()
        device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        g = torch.Generator(device=device).manual_seed(seed)
        self.cfg = cfg
        # tied embedding, 4-bit like every other weight: the lookup reads the dequantized
        # table, the lm_head the same layer (from the codes for one row on the GPU)
        self.lm_head = QuantLinear(cfg.hidden_size, cfg.vocab_size, group=cfg.quant_group,
                                   weight=torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=device) * 0.02)
        self.embed_tokens = nn.Parameter(self.lm_head.weight, requires_grad=False)
        self.layers = nn.ModuleList(DecoderLayer(cfg, generator=g, device=device) for _ in range(cfg.num_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_eps, device)

    def _logits(self, h: torch.Tensor) -> torch.Tensor:
        """Tied lm_head for a few rows [B, hidden]: one row on the GPU from the 4-bit codes,
        else embed @ h^T over the dequantized table."""
        if _one_row(h) and self.lm_head.gemv_from_codes:
            return q4_gemv(h, self.lm_head)
        return torch.matmul(self.embed_tokens, h.t()).t()

    def _rope(self, start: int, t: int, device):
        """cos/sin rows for positions [start, start+t) from a table grown on demand."""
        need = start + t
        tab = getattr(self, "_rope_tab", None)
        if tab is None or tab[0].shape[0] < need or tab[0].device != device:
            n = max(need, 2 * (tab[0].shape[0] if tab is not None else 0), 4096)
            tab = rope_cos_sin(torch.arange(n, device=device), self.cfg.head_dim, self.cfg.rope_theta)
            self._rope_tab = tab
        return tab[0][start:need], tab[1][start:need]

    def _last_logits(self, x: torch.Tensor, positions: torch.Tensor, caches: List, rope,
                     greedy: Optional[GreedyState] = None) -> torch.Tensor:
        """Run every layer over the embedded ``x`` [B, T, hidden]; returns the logits of the last
        position (final RMSNorm, tied lm_head).  On the HIP path each layer's closing residual
        add is folded into the next layer's (or the final) RMSNorm launch, and for one row the
        final norm rides in the lm_head product's launch.  ``greedy``: also pick the token and
        advance the decode loop's state (``greedy_advance``; one row)."""
        if _hip(x) and x.shape[-1] % 256 == 0:
            m = None
            for layer, cache in zip(self.layers, caches):
                x, m = layer.forward_split(x, m, positions, cache, rope)
            xl, ml = x[:, -1], (m[:, -1] if m is not None else None)
            if greedy is not None:
                lg = add_rms_norm_q4_gemv_argmax(xl, ml, self.norm.weight, self.norm.eps, self.lm_head,
                                                 greedy.workspace)
                greedy_advance(greedy, self.embed_tokens)
                return lg
            if norm_q4_fits(xl, self.lm_head):
                return add_rms_norm_q4_gemv(xl, ml, self.norm.weight, self.norm.eps, self.lm_head)[1]
            return self._logits(add_rms_norm(xl, ml, self.norm.weight, self.norm.eps)[1])
        for layer, cache in zip(self.layers, caches):
            x = layer(x, positions, cache, rope)
        return self._logits(self.norm(x[:, -1]))

    @torch.no_grad()
    def forward(self, tokens: torch.Tensor, caches: List, start: int) -> torch.Tensor:
        """tokens [B, T] at positions [start, start+T); returns logits [B, vocab] of the last position."""
        x = F.embedding(tokens, self.embed_tokens)
        positions = torch.arange(start, start + tokens.shape[1], device=tokens.device)
        rope = self._rope(start, tokens.shape[1], tokens.device)
        return self._last_logits(x, positions, caches, rope).float()

    @torch.no_grad()
    def greedy_graph(self, prompt: torch.Tensor, new_tokens: int, caches: List) -> torch.Tensor:
        """``greedy`` with the decode steps replayed from one captured HIP graph.

        ``caches`` must be ``CompressedKVCache`` objects; the prompt is prefilled
        eagerly, then the caches switch to device counters; the first decode step
        runs eagerly and the next one (every layer, argmax, position advance) is
        captured and replayed ``new_tokens - 2`` times with no host
        synchronisation in between.
        """
        logits = self.forward(prompt, caches, 0)
        return self.greedy_graph_from_logits(logits, prompt.shape[1], new_tokens, caches)

    @torch.no_grad()
    def greedy_graph_from_logits(self, logits: torch.Tensor, t: int, new_tokens: int, caches: List,
                                 timed: bool = False, on_step: Optional[Callable[[int], None]] = None) -> torch.Tensor:
        """The decode part of ``greedy_graph`` after a prefill of ``t`` tokens that produced ``logits``.

        With ``timed`` the replays are bracketed by device synchronisations and
        their wall time is kept in ``self.last_graph_decode_s``.  ``on_step(i)`` is called after
        replay ``i`` (the step at position ``t + 1 + i``) with the device synchronised, for
        inspection of what the replay wrote."""
        dev = logits.device
        b = logits.shape[0]
        for i, (layer, c) in enumerate(zip(self.layers, caches)):
            attn = layer.self_attn
            if not isinstance(c, CompressedKVCache) or not (
                    isinstance(attn, ButterflyAttention)
                    and attn.core.device_step_fits(c, self.cfg.head_dim, self.embed_tokens.dtype)):
                raise ValueError(
                    f"greedy_graph: layer {i} cannot run its decode step as one device launch (it needs a swapped "
                    f"layer over a CompressedKVCache, an attention window of at most 64 tokens and a routed row "
                    f"of at most 16 blocks); use greedy() for this configuration")
        for c in caches:
            c.use_device_counters()
        self._rope(0, t + new_tokens + 1, dev)               # table sized before capture
        tok = logits.argmax(-1, keepdim=True)
        out = torch.empty(b, new_tokens, dtype=torch.long, device=dev)
        out[:, :1] = tok
        ctr = torch.tensor([t, 1], dtype=torch.long, device=dev)   # position, output column: one add per step
        pos, step = ctr[0:1], ctr[1:2]
        cos_tab, sin_tab = self._rope_tab
        greedy = None
        hid = self.cfg.hidden_size
        if (FUSE_GREEDY and b == 1 and _hip(self.embed_tokens) and hid in NORM_Q4_DIMS
                and self.lm_head.gemv_from_codes and self.lm_head.in_features == hid):
            ws = torch.empty(int(_native.lib().bfly_q4_argmax_workspace_bytes(self.cfg.vocab_size, hid)),
                             dtype=torch.uint8, device=dev)
            greedy = GreedyState(tok, out, ctr, F.embedding(tok, self.embed_tokens).contiguous(), ws)

        def one_step():
            if greedy is not None:
                # the token, its output column, the counters and the next step's input row are
                # advanced inside the launches after the lm_head
                self._last_logits(greedy.x, pos, caches, RopeTable(cos_tab, sin_tab, pos), greedy=greedy)
                return
            x = F.embedding(tok, self.embed_tokens)
            rope = RopeTable(cos_tab, sin_tab, pos)
            lg = self._last_logits(x, pos, caches, rope)
            if _hip(lg) and lg.shape[0] <= 64:
                nxt = argmax_rows_noalloc(lg, out=tok)    # the next step's token, written in place
            else:
                nxt = argmax_rows(lg) if _hip(lg) else lg.argmax(-1, keepdim=True)
                tok.copy_(nxt)
            out.index_copy_(1, step, nxt)
            ctr.add_(1)

        if new_tokens > 1:
            one_step()           # eager first step: every op meets its decode shapes before capture
        if new_tokens > 2:
            graph = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                with torch.cuda.graph(graph, stream=side):
                    one_step()   # recorded, not run
            torch.cuda.current_stream(dev).wait_stream(side)
            if timed:
                torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            for i in range(new_tokens - 2):
                graph.replay()
                if on_step is not None:
                    torch.cuda.synchronize(dev)
                    on_step(i)
            if timed:
                torch.cuda.synchronize(dev)
            self.last_graph_decode_s = time.perf_counter() - t0
        for c in caches:
            c.use_device_counters(False)
        return out

    @torch.no_grad()
    def greedy(self, prompt: torch.Tensor, new_tokens: int, caches: List,
               on_token: Optional[Callable[[int], None]] = None) -> torch.Tensor:
        """Prefill ``prompt`` [B, T] in one call, then ``new_tokens`` greedy steps; returns [B, new_tokens]."""
        logits = self.forward(prompt, caches, 0)
        out = []
        pos = prompt.shape[1]
        for i in range(new_tokens):
            nxt = logits.argmax(-1, keepdim=True)
            out.append(nxt)
            if on_token is not None:
                on_token(i)
            if i + 1 == new_tokens:
                break
            logits = self.forward(nxt, caches, pos)
            pos += 1
        return torch.cat(out, 1)
