"""GPU: the Torch twin's swapped module against vectors written by the reference's own swap.

``tests/golden/golden_swap.npz`` (``tests/golden/make_golden_swap.py``) holds every call the
reference's ``QwenCUDAButterflyAttention`` (bna/integrations/qwen_torch.py:1187-1470) made in
a tiny random-init HF Qwen3.5 model on the CPU: input hidden states, RoPE rows, output and
profile.  Here the same model (rebuilt from its seed, digest checked) runs on the GPU with
the twin's swap (``butterfly_amd.qwen_torch``), and each swapped layer replays its recorded
calls in order through a ``DynamicCache``: one-shot prefill, greedy decode rows, a chunked
prefill whose masked second chunk takes the stock module, and the direct fallback calls.
Every output meets the north_star bf16 bar against the reference's (its projections run
as GPU GEMMs here, so bits differ within rounding) and every profile (mode, reason, kv_len,
stage, backend) equals the reference's.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from butterfly_amd import qwen_torch as qt

pytestmark = pytest.mark.gpu
pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5", reason="this transformers has no Qwen3.5 model")

from tests.golden.make_golden_swap import (FALLBACK_LAYER, PROFILE_KEYS, SWAP_CONFIG, SWAPPED,  # noqa: E402
                                           causal_mask, from_np, model_digest, tiny_model)

G = np.load(Path(__file__).resolve().parent / "golden" / "golden_swap.npz")
BF16_MAX_ABS, BF16_REL_L2 = 2e-2, 1e-2


def _close(got, want, what):
    got, want = got.float().cpu(), want.float()
    err = (got - want).abs().max().item()
    rel = ((got - want).norm() / want.norm()).item()
    assert err <= BF16_MAX_ABS and rel <= BF16_REL_L2, (what, err, rel)


@pytest.fixture(scope="module")
def model():
    m = tiny_model()
    assert model_digest(m) == G["meta/model_digest"][0], "tiny_model() drifted from the fixture's model"
    m = m.to("cuda")
    assert qt.swap_qwen_attention_with_butterfly_cuda(m, qt.QwenCUDAButterflyConfig(**SWAP_CONFIG)) == list(SWAPPED)
    return m


@pytest.mark.parametrize("tag", ["oneshot", "chunked"])
def test_swapped_layers_replay_the_reference_calls(model, tag):
    from transformers import DynamicCache

    modes = set()
    for layer in SWAPPED:
        mod = model.model.layers[layer].self_attn
        assert isinstance(mod, qt.QwenCUDAButterflyAttention)
        cache = DynamicCache(config=model.config)
        kv = 0
        for f in range(int(G[f"{tag}/calls"][0])):
            p = f"{tag}/f{f}/L{layer}"
            x = from_np(G[f"{p}/hidden"]).cuda()
            positions = torch.from_numpy(G[f"{tag}/f{f}/positions"]).long()
            kind = str(G[f"{tag}/f{f}/causal_mask"][0])
            mask = None if kind == "none" else causal_mask(positions, kv + x.shape[1], getattr(torch, kind)).cuda()
            pe = (from_np(G[f"{tag}/f{f}/cos"]).cuda(), from_np(G[f"{tag}/f{f}/sin"]).cuda())
            print(f"replay {p} q_len={x.shape[1]} kv={kv}", flush=True)
            with torch.no_grad():
                y = mod(hidden_states=x, position_embeddings=pe, attention_mask=mask, past_key_values=cache,
                        position_ids=positions.view(1, -1).cuda())[0]
            torch.cuda.synchronize()
            assert [str(mod.last_profile.get(k)) for k in PROFILE_KEYS] == list(G[f"{p}/profile"]), p
            modes.add((mod.last_profile["mode"], str(mod.last_profile.get("block_sparse_backend"))))
            _close(y, from_np(G[f"{p}/out"]), p)
            kv += x.shape[1]
    want = {("butterfly", "compressed_butterfly_sdpa"), ("butterfly", "compressed_butterfly_active")}
    if tag == "chunked":
        want.add(("fallback", "None"))
    assert modes == want


@pytest.mark.parametrize("name", ["short_query", "output_attentions", "attention_mask", "training"])
def test_fallback_calls_replay_the_reference(model, name):
    mod = model.model.layers[FALLBACK_LAYER].self_attn
    x = from_np(G[f"fallback/{name}/hidden"]).cuda()
    n = x.shape[1]
    mask = torch.zeros(1, 1, n, n, dtype=torch.bfloat16, device="cuda") if name == "attention_mask" else None
    kw = {"output_attentions": True} if name == "output_attentions" else {}
    pe = (from_np(G[f"fallback/{name}/cos"]).cuda(), from_np(G[f"fallback/{name}/sin"]).cuda())
    mod.train(name == "training")
    try:
        with torch.no_grad():
            y = mod(hidden_states=x, position_embeddings=pe, attention_mask=mask, **kw)[0]
    finally:
        mod.train(False)
    assert [str(mod.last_profile.get(k)) for k in PROFILE_KEYS] == list(G[f"fallback/{name}/profile"])
    _close(y, from_np(G[f"fallback/{name}/out"]), name)
