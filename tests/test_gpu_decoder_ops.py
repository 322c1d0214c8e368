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
from butterfly_amd.decoder import RMSNorm, add_rms_norm, apply_rope, rope_cos_sin

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
    _native.call("bfly_qk_norm_rope", qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), qw.data_ptr(), kw.data_ptr(),
                 cc.data_ptr(), sc.data_ptr(), B, T, hq, hkv, d, 1e-6, qo.data_ptr(), ko.data_ptr(), vo.data_ptr(),
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _close(qo.cpu(), want_q)
    _close(ko.cpu(), want_k)
    assert torch.equal(vo.cpu(), want_v)


def test_silu_mul():
    g, u = _rand(9, 3, 6144, scale=3.0), _rand(10, 3, 6144)
    out = torch.empty(3, 6144, dtype=torch.bfloat16, device="cuda")
    gc, uc = g.cuda(), u.cuda()
    _native.call("bfly_silu_mul", gc.data_ptr(), uc.data_ptr(), g.numel(), out.data_ptr(),
                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _close(out.cpu(), F.silu(g) * u)


def test_decoder_ops_reject_bad_shapes():
    x = torch.zeros(2, 100, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        add_rms_norm(x, None, x[0], 1e-6)          # dim 100 is not a multiple of 256
    with pytest.raises(ValueError):
        _native.call("bfly_add_rms_norm", x.data_ptr(), x.data_ptr(), x.data_ptr(), 2, 256, 1e-6, None,
                     x.data_ptr(), 0)             # residual without h_out
