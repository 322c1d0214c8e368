"""The swapped random-init decoder: 4-bit affine weights (CPU), and greedy decoding
through the HIP Butterfly path vs the CPU reference Torch path (GPU)."""
from __future__ import annotations

import copy

import pytest
import torch

import butterfly_amd as bf
from butterfly_amd.decoder import Decoder, DecoderConfig, dequantize_affine, quantize_affine
from oracle.decoder_ref import swap_to_oracle


def test_quantize_affine_round_trip_and_packing():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(16, 256, generator=g)
    packed, scale, bias = quantize_affine(w, 64)
    assert packed.dtype == torch.uint8 and packed.shape == (16, 128)
    assert scale.shape == bias.shape == (16, 4) and scale.dtype == torch.bfloat16
    wd = dequantize_affine(packed, scale, bias, 64).float()
    # every value is one of the 16 levels of its group, and within half a step of w
    step = scale.float().repeat_interleave(64, 1)
    assert ((wd - w).abs() <= step * 0.5 + step * 0.02 + 1e-3).all()
    codes = torch.stack([packed & 0xF, packed >> 4], -1).view(16, 256)
    assert int(codes.max()) <= 15
    # dequantisation is codes * scale + bias, rounded once to bf16
    exact = codes.float() * step + bias.float().repeat_interleave(64, 1)
    assert torch.equal(wd.bfloat16(), exact.bfloat16())


SMALL = DecoderConfig(vocab_size=2048, hidden_size=512, num_layers=4, num_heads=8, num_kv_heads=2, head_dim=64,
                      intermediate_size=1024)
# head_dim 128: decode steps take the fused one-row path (add + RMSNorm inside the projections)
SMALL128 = DecoderConfig(vocab_size=2048, hidden_size=512, num_layers=4, num_heads=4, num_kv_heads=2, head_dim=128,
                         intermediate_size=1024)


@pytest.mark.gpu
@pytest.mark.parametrize("cfg_", [SMALL, SMALL128], ids=["d64", "d128"])
def test_swapped_decoder_tracks_cpu_reference_teacher_forced(cfg_):
    """Same tokens into both paths (the CPU reference's greedy continuation): the
    HIP path's logits stay within bf16 noise of the reference's at every step, and
    the argmax agrees wherever the reference's top-2 margin exceeds that noise."""
    model = Decoder(cfg_, seed=7)
    cpu_model = copy.deepcopy(model).to("cpu")
    cfg = bf.compressed_butterfly_config()
    assert bf.swap_qwen_attention_with_butterfly(model, cfg=cfg) == [0, 1, 2, 3]
    swap_to_oracle(cpu_model, cfg)
    prompt = torch.randint(0, cfg_.vocab_size, (1, 700), generator=torch.Generator().manual_seed(3))
    steps = 12
    caches = [None] * cfg_.num_layers
    bf.install_compressed_kv_caches(model, caches, block_size=128, local_window_tokens=64, max_kv_size=800)
    ref_caches = [[] for _ in range(cfg_.num_layers)]
    lc = cpu_model.forward(prompt, ref_caches, 0)
    lg = model.forward(prompt.cuda(), caches, 0).cpu()
    pos, diffs, checked = 700, [], 0
    for step in range(steps):
        diffs.append((lg - lc).abs().max().item())
        top2 = lc[0].topk(2).values
        if (top2[0] - top2[1]).item() > 2 * diffs[-1]:
            assert lg.argmax().item() == lc.argmax().item(), (step, diffs)
            checked += 1
        tok = lc.argmax(-1, keepdim=True)
        lc = cpu_model.forward(tok, ref_caches, pos)
        lg = model.forward(tok.cuda(), caches, pos).cpu()
        pos += 1
    spread = lc.std().item()
    print(f"logit max-abs diffs {diffs}; logit std {spread:.3f}; argmax checked at {checked} steps", flush=True)
    assert max(diffs) <= 0.25 * spread, (diffs, spread)
    assert checked >= steps // 2
    prof = model.layers[2].self_attn.last_profile
    assert prof.path == "block_sparse_compressed_active" and prof.notes["q_len"] == 1


def test_fuse_rows_gives_views_and_the_same_products():
    from butterfly_amd.decoder import QuantLinear

    g = torch.Generator().manual_seed(1)
    parts = [QuantLinear(128, n, generator=g, device="cpu") for n in (64, 32, 32)]
    want_w = torch.cat([p.weight for p in parts])
    fused = QuantLinear.fuse_rows(*parts)
    assert torch.equal(fused.weight, want_w) and fused.out_features == 128 and fused.in_features == 128
    # each part's tensors are views of its row range of the fused layer
    assert parts[1].weight.data_ptr() == fused.weight[64:].data_ptr()
    assert parts[2].packed.data_ptr() == fused.packed[96:].data_ptr()
    # the interleaved (scale, bias) pairs the 4-bit kernel reads
    assert torch.equal(fused.scale_bias[..., 0], fused.scale) and torch.equal(fused.scale_bias[..., 1], fused.bias)
    x = torch.randn(3, 128, generator=g).bfloat16()
    torch.testing.assert_close(fused(x).float(), torch.cat([p(x) for p in parts], -1).float(), atol=2e-2, rtol=1e-2)


def test_rope_table_rows_select_the_position():
    from butterfly_amd.decoder import RopeTable, rope_cos_sin

    cos, sin = rope_cos_sin(torch.arange(10), 8, 1e4)
    c, s = RopeTable(cos, sin, torch.tensor([3])).rows()
    assert torch.equal(c, cos[3:4]) and torch.equal(s, sin[3:4])


def test_cpu_reference_one_row_products_take_the_gpu_rounding_points():
    """oracle.decoder_ref.match_gpu_rounding: a one-row product runs over the fp32 weights
    code * scale + bias (which round to the layer's bf16 weights), accumulates in fp32 and
    rounds once, i.e. equals the float64 product rounded to bf16 up to fp32 summation order;
    multi-row products and the layer's own forward are untouched."""
    from butterfly_amd.decoder import QuantLinear
    from oracle.decoder_ref import match_gpu_rounding, q4_row, q4_weight_fp32

    g = torch.Generator().manual_seed(4)
    layer = QuantLinear(2048, 96, generator=g)
    w32 = q4_weight_fp32(layer)
    assert torch.equal(w32.to(torch.bfloat16), layer.weight)          # the bf16 weights are its rounding
    assert not torch.equal(w32, layer.weight.float())                # and it keeps bits they drop
    x = torch.randn(1, 1, 2048, generator=g).bfloat16()
    y = q4_row(x, layer)
    exact = (x.double().view(1, -1) @ w32.double().t()).view(1, 1, -1)
    assert torch.equal(y, exact.to(torch.bfloat16)) or \
        ((y.double() - exact).abs() <= exact.abs() * 2 ** -8 + 1e-30).all()
    model = Decoder(DecoderConfig(vocab_size=256, hidden_size=256, num_layers=1, num_heads=2, num_kv_heads=1,
                                  head_dim=128, intermediate_size=512), seed=1, device="cpu")
    rows = torch.randn(1, 3, 256, generator=g).bfloat16()
    before = model.layers[0].mlp.gate_proj(rows)
    match_gpu_rounding(model)
    q = model.layers[0].self_attn.q_proj
    one = rows[:, :1]
    assert torch.equal(q(one), q4_row(one, q))
    assert torch.equal(model.layers[0].mlp.gate_proj(rows), before)  # three rows: the bf16 GEMM
    h = torch.randn(1, 256, generator=g).bfloat16()
    assert torch.equal(model._logits(h), q4_row(h, model.lm_head))
