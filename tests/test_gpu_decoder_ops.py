"""GPU: the decoder's HIP steps (include/butterfly_amd_decoder.h) against the PyTorch forms of
butterfly_amd/decoder.py that define the model (run here on the CPU, bf16 rounding per op).

The kernels round at the same points; they may differ from the PyTorch forms by the fp32
summation order of a mean square and the last bit of rsqrt/exp, so the bar is: at most one
bf16 unit in the last place anywhere, and at least 99 % of the elements bit-identical.  The
residual add and the v move are exact.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from butterfly_amd import _native
from butterfly_amd.decoder import RMSNorm, add_rms_norm, apply_rope, argmax_rows, rope_cos_sin

pytestmark = pytest.mark.gpu


def _rand(seed, *shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).bfloat16()


def _close(got: torch.Tensor, want: torch.Tensor):
    got, want = got.float(), want.float()
    ulp = torch.clamp(want.abs(), min=1e-30) * 2.0 ** -7
    diff = (got - want).abs()
    assert bool((diff <= ulp + 1e-30).all()), float((diff - ulp).max())
    assert float((diff == 0).float().mean()) >= 0.99


@pytest.mark.parametrize("dim,rows", [(2048, 37), (1024, 5), (6144, 3), (512, 4), (768, 2)])
def test_add_rms_norm(dim, rows):
    x, y = _rand(1, rows, dim), _rand(2, rows, dim, scale=0.5)
    norm = RMSNorm(dim, 1e-6, "cpu")
    norm.weight.data = _rand(3, dim, scale=0.2) + 1
    h, n = add_rms_norm(x.cuda(), y.cuda(), norm.weight.cuda(), 1e-6)
    assert torch.equal(h.cpu(), x + y)
    _close(n.cpu(), norm(x + y))
    _, n0 = add_rms_norm(x.cuda(), None, norm.weight.cuda(), 1e-6)
    _close(n0.cpu(), norm(x))
    # rows that start 2 bytes off a 16-byte boundary take the element-wise path
    xo = torch.cat([torch.zeros(rows, 1, dtype=x.dtype), x], 1).cuda()[:, 1:]
    yo = torch.cat([torch.zeros(rows, 1, dtype=x.dtype), y], 1).cuda()[:, 1:]
    h2, n2 = add_rms_norm(xo, yo, norm.weight.cuda(), 1e-6)
    assert torch.equal(h2.cpu(), x + y)
    _close(n2.cpu(), norm(x + y))


@pytest.mark.parametrize("d", [128, 256])
def test_qk_norm_rope(d):
    B, T, hq, hkv = 2, 7, 4, 2
    qp, kp, vp = _rand(4, B, T, hq * d), _rand(5, B, T, hkv * d), _rand(6, B, T, hkv * d)
    qn, kn = RMSNorm(d, 1e-6, "cpu"), RMSNorm(d, 1e-6, "cpu")
    qn.weight.data = _rand(7, d, scale=0.2) + 1
    kn.weight.data = _rand(8, d, scale=0.2) + 1
    cos, sin = rope_cos_sin(torch.arange(100, 100 + T), d, 1e6)
    want_q = apply_rope(qn(qp.view(B, T, hq, d).transpose(1, 2)), cos, sin)
    want_k = apply_rope(kn(kp.view(B, T, hkv, d).transpose(1, 2)), cos, sin)
    want_v = vp.view(B, T, hkv, d).transpose(1, 2).contiguous()
    qo = torch.empty(B, hq, T, d, dtype=torch.bfloat16, device="cuda")
    ko = torch.empty(B, hkv, T, d, dtype=torch.bfloat16, device="cuda")
    vo = torch.empty_like(ko)
    qc, kc, vc, cc, sc = qp.cuda(), kp.cuda(), vp.cuda(), cos.cuda().contiguous(), sin.cuda().contiguous()
    qw, kw = qn.weight.cuda(), kn.weight.cuda()
    _native.call("bfly_qk_norm_rope", qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), hq * d, hkv * d, hkv * d,
                 qw.data_ptr(), kw.data_ptr(), cc.data_ptr(), sc.data_ptr(), B, T, hq, hkv, d, 1e-6, qo.data_ptr(),
                 ko.data_ptr(), vo.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _close(qo.cpu(), want_q)
    _close(ko.cpu(), want_k)
    assert torch.equal(vo.cpu(), want_v)
    # q, k and v as column ranges of one fused projection output [B, T, (hq + 2 hkv) d]
    fused = torch.cat([qp, kp, vp], -1).cuda()
    ld, es, base = fused.shape[-1], fused.element_size(), fused.data_ptr()
    qo2, ko2, vo2 = torch.empty_like(qo), torch.empty_like(ko), torch.empty_like(vo)
    _native.call("bfly_qk_norm_rope", base, base + hq * d * es, base + (hq + hkv) * d * es, ld, ld, ld,
                 qw.data_ptr(), kw.data_ptr(), cc.data_ptr(), sc.data_ptr(), B, T, hq, hkv, d, 1e-6, qo2.data_ptr(),
                 ko2.data_ptr(), vo2.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(qo2, qo) and torch.equal(ko2, ko) and torch.equal(vo2, vo)
    # a fused output whose row stride is not a multiple of 8 takes the element-wise kernel
    ld3 = ld + 1
    fused3 = torch.zeros(B, T, ld3, dtype=torch.bfloat16)
    fused3[..., :ld] = torch.cat([qp, kp, vp], -1)
    fused3 = fused3.cuda()
    base3 = fused3.data_ptr()
    qo3, ko3, vo3 = torch.empty_like(qo), torch.empty_like(ko), torch.empty_like(vo)
    _native.call("bfly_qk_norm_rope", base3, base3 + hq * d * es, base3 + (hq + hkv) * d * es, ld3, ld3, ld3,
                 qw.data_ptr(), kw.data_ptr(), cc.data_ptr(), sc.data_ptr(), B, T, hq, hkv, d, 1e-6, qo3.data_ptr(),
                 ko3.data_ptr(), vo3.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _close(qo3.cpu(), want_q)
    _close(ko3.cpu(), want_k)
    assert torch.equal(vo3.cpu(), want_v)


def test_silu_mul():
    g, u = _rand(9, 3, 6144, scale=3.0), _rand(10, 3, 6144)
    out = torch.empty(3, 6144, dtype=torch.bfloat16, device="cuda")
    gc, uc = g.cuda(), u.cuda()
    _native.call("bfly_silu_mul", gc.data_ptr(), uc.data_ptr(), 3, 6144, 6144, out.data_ptr(),
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _close(out.cpu(), F.silu(g) * u)
    # gate and up as the two column halves of one fused [3, 2 * 6144] output
    gu = torch.cat([g, u], -1).cuda()
    out2 = torch.empty_like(out)
    _native.call("bfly_silu_mul", gu.data_ptr(), gu.data_ptr() + 6144 * 2, 3, 6144, 2 * 6144, out2.data_ptr(),
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
    # columns that are not a multiple of 8: the element-wise kernel, same values
    out3 = torch.empty(3, 6141, dtype=torch.bfloat16, device="cuda")
    _native.call("bfly_silu_mul", gc.data_ptr(), uc.data_ptr(), 3, 6141, 6144, out3.data_ptr(),
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out3.cpu(), out.cpu()[:, :6141])


@pytest.mark.parametrize("rows,n", [(1, 151936), (3, 1000), (2, 7), (1, 8), (2, 4096 * 300 + 5)])
def test_argmax_rows(rows, n):
    x = _rand(11, rows, n)
    x[:, n // 3] = 9.0                      # ties: the lower index wins
    x[:, n // 2] = 9.0
    if rows > 1:
        x[1, n - 1] = float("nan")          # NaN above every number
        x[1, n // 4] = float("nan")
    want = torch.argmax(x, -1, keepdim=True)
    assert torch.equal(argmax_rows(x.cuda()).cpu(), want)
    assert torch.equal(argmax_rows(x.cuda(), parallel=False).cpu(), want)
    # a column-major [rows, n] view, as the lm_head's GEMV form leaves its logits
    xt = x.t().contiguous().cuda().t()
    assert torch.equal(argmax_rows(xt).cpu(), want)
    # one row whose view carries a row stride of 1 (the lm_head's GEMV output, transposed)
    x1 = x[:1].t().contiguous().cuda().t()
    assert torch.equal(argmax_rows(x1).cpu(), want[:1])
    # a row start that is not 16-byte aligned (element path)
    xo = torch.cat([torch.zeros(rows, 1, dtype=x.dtype), x], 1).cuda()[:, 1:]
    assert torch.equal(argmax_rows(xo).cpu(), want)


def test_decoder_ops_reject_bad_shapes():
    x = torch.zeros(2, 100, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        add_rms_norm(x, None, x[0], 1e-6)          # dim 100 is not a multiple of 256
    with pytest.raises(ValueError):
        _native.call("bfly_add_rms_norm", x.data_ptr(), x.data_ptr(), x.data_ptr(), 2, 256, 1e-6, None,
                     x.data_ptr(), 0)             # residual without h_out
