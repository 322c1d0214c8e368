"""GPU: one-row products from 4-bit affine codes (``bfly_q4_gemv``, ``bfly_q4_gemv_silu``).

The reference is the product with the fp32 weights ``code * scale + bias`` in float64 on
the CPU: the kernel accumulates in fp32 in another order and rounds once to bf16, so every
output lies within half a bf16 unit of the reference plus the fp32 summation error, and
nearly all of them equal the reference rounded to bf16.  The fused SiLU variant is checked
against the two projections followed by ``bfly_silu_mul`` (the same rounding points).
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from butterfly_amd import _native
from butterfly_amd.decoder import QuantLinear, q4_gemv, q4_gemv_silu

pytestmark = pytest.mark.gpu


def _layer(out_f, in_f, group, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(out_f, in_f, generator=g) / in_f ** 0.5
    # a few outlier groups, so scales differ widely between groups
    w[:, : min(in_f, group)] *= 8
    return QuantLinear(in_f, out_f, group=group, weight=w).cuda()


def _fp32_weights(layer: QuantLinear) -> torch.Tensor:
    p = layer.packed.cpu()
    codes = torch.stack([p & 0xF, p >> 4], -1).view(p.shape[0], -1).double()
    s = layer.scale.cpu().double().repeat_interleave(layer.group, 1)
    b = layer.bias.cpu().double().repeat_interleave(layer.group, 1)
    return codes * s + b


def _x(in_f, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, in_f, generator=g).bfloat16()


# (out_features, in_features, group): one lane piece (64, 2048), partial second and third
# pieces per lane (2112, 4160), three and four pieces (6144, 8192), groups of 32 / 64 / 128,
# two rows per wave (small outputs) and four (9000 rows; 8195 ends in a partial set), the lm_head's shape.
CASES = [(1, 64, 64), (100, 96, 32), (7, 2048, 64), (3072, 2048, 64), (9000, 2048, 64), (8195, 2048, 64),
         (5, 2112, 32), (2048, 6144, 64), (5, 4160, 64), (33, 8192, 128), (151936, 2048, 64)]


@pytest.mark.parametrize("out_f,in_f,group", CASES)
def test_q4_gemv_matches_fp32_weight_product(out_f, in_f, group):
    layer = _layer(out_f, in_f, group, seed=out_f + in_f)
    x = _x(in_f, seed=in_f)
    y = q4_gemv(x.cuda(), layer).cpu()
    assert y.shape == (1, out_f) and y.dtype == torch.bfloat16
    w = _fp32_weights(layer)
    ref = (x.double() @ w.t())[0]
    mag = (x.double().abs() @ w.abs().t())[0]
    got = y[0].double()
    bound = ref.abs() * 2.0 ** -8 + mag * 2.0 ** -20 + 1e-30
    assert bool(((got - ref).abs() <= bound).all()), float(((got - ref).abs() - bound).max())
    same = (y[0] == ref.float().bfloat16()).float().mean().item()
    assert same >= 0.97, same


@pytest.mark.parametrize("f,in_f", [(6144, 2048), (4097, 2048), (100, 2048), (1, 64), (2048, 6144), (300, 8192)])
def test_q4_gemv_silu_equals_projections_then_silu_mul(f, in_f):
    gate_up = _layer(2 * f, in_f, 64, seed=f)
    x = _x(in_f, seed=f + 1).cuda()
    s = q4_gemv_silu(x, gate_up)
    gu = q4_gemv(x, gate_up)                              # gate rows, then up rows
    want = torch.empty(1, f, dtype=torch.bfloat16, device="cuda")
    _native.call("bfly_silu_mul", gu.data_ptr(), gu.data_ptr() + f * 2, 1, f, 2 * f, want.data_ptr(),
                 torch.cuda.current_stream().cuda_stream)
    got, ref = s.cpu().float(), want.cpu().float()
    diff = (got - ref).abs()
    assert bool((diff <= ref.abs() * 2.0 ** -7 + 1e-30).all())
    assert (diff == 0).float().mean().item() >= 0.99


def test_quant_linear_row_paths_agree():
    """One row through the 4-bit codes vs the same row through the dequantized bf16 GEMM."""
    layer = _layer(3072, 2048, 64, seed=5)
    x = _x(2048, seed=6).cuda()
    one = layer(x.view(1, 1, 2048))
    two = F.linear(torch.cat([x, x]).view(1, 2, 2048), layer.weight)[:, :1]
    assert one.shape == two.shape == (1, 1, 3072)
    err = (one.float() - two.float()).abs().max().item()
    assert err <= 2e-2 * two.float().abs().max().item()


def test_q4_gemv_unaligned_row_is_copied():
    layer = _layer(64, 128, 64, seed=9)
    buf = _x(129, seed=10).cuda()
    x = buf[:, 1:]                                        # 2-byte offset: the wrapper copies it
    assert x.data_ptr() % 16
    y = q4_gemv(x, layer)
    assert torch.equal(y, q4_gemv(x.clone(), layer))



@pytest.mark.parametrize("out_f,in_f,residual", [(3072, 2048, True), (9000, 2048, True), (151936, 2048, True),
                                                 (100, 2048, False), (2048, 4096, True), (33, 6144, True)])
def test_add_rms_norm_q4_gemv_equals_two_launches(out_f, in_f, residual):
    """The residual add + RMSNorm inside the product's launch gives the same h and the same
    outputs, bit for bit, as bfly_add_rms_norm followed by bfly_q4_gemv."""
    from butterfly_amd.decoder import add_rms_norm, add_rms_norm_q4_gemv

    layer = _layer(out_f, in_f, 64, seed=out_f)
    g = torch.Generator().manual_seed(in_f + out_f)
    x = (torch.randn(1, in_f, generator=g) * 3).bfloat16().cuda()
    r = torch.randn(1, in_f, generator=g).bfloat16().cuda() if residual else None
    w = (1 + 0.5 * torch.randn(in_f, generator=g)).bfloat16().cuda()
    h, y = add_rms_norm_q4_gemv(x, r, w, 1e-6, layer)
    h2, n = add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(h, h2)
    assert torch.equal(y, q4_gemv(n, layer))


@pytest.mark.parametrize("f,in_f", [(6144, 2048), (4097, 2048), (100, 4096), (300, 6144)])
def test_add_rms_norm_q4_gemv_silu_equals_two_launches(f, in_f):
    from butterfly_amd.decoder import add_rms_norm, add_rms_norm_q4_gemv_silu

    gate_up = _layer(2 * f, in_f, 64, seed=f)
    g = torch.Generator().manual_seed(f)
    x = torch.randn(1, in_f, generator=g).bfloat16().cuda()
    r = torch.randn(1, in_f, generator=g).bfloat16().cuda()
    w = (1 + 0.5 * torch.randn(in_f, generator=g)).bfloat16().cuda()
    h, s = add_rms_norm_q4_gemv_silu(x, r, w, 1e-6, gate_up)
    h2, n = add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(h, h2)
    assert torch.equal(s, q4_gemv_silu(n, gate_up))


@pytest.mark.parametrize("out_f,tie", [(151936, False), (4096, True), (50000, True), (300, False)])
def test_argmax_variant_and_greedy_advance(out_f, tie):
    """``bfly_add_rms_norm_q4_gemv_argmax`` writes the same logits as ``bfly_add_rms_norm_q4_gemv``
    and leaves candidates whose pick (``bfly_greedy_advance``) is torch.argmax of those logits;
    with two equal top rows the lower index wins.  The advance also writes the token, its
    output column, both counters and the next input row (the pick's embedding row)."""
    from butterfly_amd.decoder import GreedyState, add_rms_norm_q4_gemv, add_rms_norm_q4_gemv_argmax, greedy_advance

    g = torch.Generator().manual_seed(out_f)
    w = torch.randn(out_f, 2048, generator=g) / 2048 ** 0.5
    x = torch.randn(1, 2048, generator=g).bfloat16().cuda()
    r = torch.randn(1, 2048, generator=g).bfloat16().cuda()
    nw = (1 + 0.1 * torch.randn(2048, generator=g)).bfloat16().cuda()
    layer = QuantLinear(2048, out_f, group=64, weight=w).cuda()
    want = add_rms_norm_q4_gemv(x, r, nw, 1e-6, layer)[1]
    expect = None
    if tie:
        # the top row copied to a lower index: identical codes, identical logits, the lower index wins
        top = int(torch.argmax(want.float()))
        dup = top // 2 if top > 0 else out_f - 1
        w[dup] = w[top]
        layer = QuantLinear(2048, out_f, group=64, weight=w).cuda()
        want = add_rms_norm_q4_gemv(x, r, nw, 1e-6, layer)[1]
        assert want[0, dup] == want[0, top]
        expect = min(dup, top)
    ws = torch.empty(int(_native.lib().bfly_q4_argmax_workspace_bytes(out_f, 2048)), dtype=torch.uint8,
                     device="cuda")
    got = add_rms_norm_q4_gemv_argmax(x, r, nw, 1e-6, layer, ws)
    assert torch.equal(got, want)
    embed = torch.randn(out_f, 256, generator=g).bfloat16().cuda()
    tok = torch.full((1, 1), -5, dtype=torch.long, device="cuda")
    out = torch.full((1, 6), -1, dtype=torch.long, device="cuda")
    ctr = torch.tensor([1000, 2], dtype=torch.long, device="cuda")
    xn = torch.empty(1, 1, 256, dtype=torch.bfloat16, device="cuda")
    greedy_advance(GreedyState(tok, out, ctr, xn, ws), embed)
    pick = int(torch.argmax(want.float()))
    if tie:
        assert pick == expect
    assert int(tok) == pick
    assert out.tolist() == [[-1, -1, pick, -1, -1, -1]] and ctr.tolist() == [1001, 3]
    assert torch.equal(xn.view(-1), embed[pick])
    ctr.fill_(6)                                    # a column past the output: nothing written there
    greedy_advance(GreedyState(tok, out, ctr, xn, ws), embed)
    assert out.tolist() == [[-1, -1, pick, -1, -1, -1]] and ctr.tolist() == [7, 7]
