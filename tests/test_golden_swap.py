"""CPU: the layer-swap dispatch against vectors written by the reference's own Torch swap.

``tests/golden/golden_swap.npz`` holds, for a tiny random-init HF Qwen3.5 model whose
full-attention layers the reference's ``swap_qwen_attention_with_butterfly_cuda`` swapped
(bna/integrations/qwen_torch.py:1187-1470, 1652-1700), every swapped call's input, RoPE rows,
output and profile, and the model's logits (``tests/golden/make_golden_swap.py``).

* ``oracle/decoder_ref.py`` (the cfg5 CPU reference's dispatch: one-shot prefill when the
  call holds every key, else the active rows over the cached keys) reproduces every call
  the reference ran on its Butterfly path bit for bit, and the whole one-shot run's logits
  bit for bit when the model's full-attention layers are swapped to it;
* the Torch twin (``butterfly_amd.qwen_torch``) takes the reference's fallback decisions on
  every recorded call, and its fallback calls (which run the stock module, on the CPU here)
  reproduce the reference's outputs bit for bit.  Its HIP calls are compared in
  ``test_gpu_golden_swap.py``.

bf16 CPU arithmetic can round differently between host CPUs, so these checks belong to the
build container, like ``test_golden.py``.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from butterfly_amd import qwen_torch as qt
from oracle.decoder_ref import OracleButterflyAttention

pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5", reason="this transformers has no Qwen3.5 model")

from tests.golden.make_golden_swap import (CHUNKS, FALLBACK_LAYER, PROFILE_KEYS, SWAP_CONFIG, SWAPPED,  # noqa: E402
                                           WINDOW, causal_mask, from_np, model_digest, tiny_model)

G = np.load(Path(__file__).resolve().parent / "golden" / "golden_swap.npz")


def _calls(tag):
    return int(G[f"{tag}/calls"][0])


def _pe(prefix):
    return from_np(G[f"{prefix}/cos"]), from_np(G[f"{prefix}/sin"])


class _StockProjection:
    """The stock Qwen3.5 attention's projections, q/k norm, RoPE (``project``) and output gate
    with ``o_proj`` (``output``): the steps the reference's swapped module takes around its
    attention call (qwen_torch.py:535-573, 1588-1596), as the interface decoder_ref expects."""

    def __init__(self, attn):
        self.attn, self.gate = attn, None

    def project(self, x, _mask, position_embeddings):
        import sys

        a, shape, d = self.attn, x.shape[:-1], self.attn.head_dim
        q, gate = torch.chunk(a.q_proj(x).view(*shape, -1, d * 2), 2, dim=-1)
        self.gate = gate.reshape(*shape, -1)
        q = a.q_norm(q.view(*shape, -1, d)).transpose(1, 2)
        k = a.k_norm(a.k_proj(x).view(*shape, -1, d)).transpose(1, 2)
        v = a.v_proj(x).view(*shape, -1, d).transpose(1, 2)
        rope = sys.modules[type(a).__module__].apply_rotary_pos_emb
        q, k = rope(q, k, *position_embeddings)
        return q, k, v

    def output(self, o):
        b, _, t, _ = o.shape
        return self.attn.o_proj(o.transpose(1, 2).contiguous().view(b, t, -1) * torch.sigmoid(self.gate))


def _oracle_layer(attn, layer):
    return OracleButterflyAttention(_StockProjection(attn), layer_idx=layer, block_size=128,
                                    local_window_tokens=WINDOW, local_window_blocks=1, sink_count=1, partner_count=1,
                                    partner_rule="causal_shift")


@pytest.fixture(scope="module")
def model():
    m = tiny_model()
    assert model_digest(m) == G["meta/model_digest"][0], "tiny_model() drifted from the fixture's model"
    return m


def test_fixture_covers_every_dispatch_branch():
    kinds = {(str(G[f"{t}/f{f}/L{l}/profile"][0]), str(G[f"{t}/f{f}/L{l}/profile"][4]))
             for t in ("oneshot", "chunked") for f in range(_calls(t)) for l in SWAPPED}
    assert kinds == {("butterfly", "compressed_butterfly_sdpa"), ("butterfly", "compressed_butterfly_active"),
                     ("fallback", "None")}
    reasons = {str(G[f"fallback/{n}/profile"][1]) for n in ("short_query", "output_attentions", "attention_mask",
                                                            "training")}
    assert reasons == {"short_query", "output_attentions", "attention_mask", "training"}


@pytest.mark.parametrize("tag", ["oneshot", "chunked"])
def test_oracle_dispatch_reproduces_every_butterfly_call(model, tag):
    compared = 0
    for layer in SWAPPED:
        attn = model.model.layers[layer].self_attn
        ref = _oracle_layer(attn, layer)
        history: list = []
        for f in range(_calls(tag)):
            p = f"{tag}/f{f}/L{layer}"
            x = from_np(G[f"{p}/hidden"])
            with torch.no_grad():
                y = ref(x, cache=history, position_embeddings=_pe(f"{tag}/f{f}"))
            prof = G[f"{p}/profile"]
            assert int(prof[2]) == history[0].shape[2]                   # kv_len after the call
            if prof[0] == "butterfly":
                assert torch.equal(y, from_np(G[f"{p}/out"])), p
                compared += 1
    assert compared == 3 * (_calls(tag) - (1 if tag == "chunked" else 0))


def test_oracle_swapped_model_reproduces_the_reference_logits(model):
    """Every full-attention layer swapped to decoder_ref's dispatch: the one-shot prompt and
    the greedy steps give the reference-swapped model's logits bit for bit."""
    from transformers import DynamicCache

    stock = {i: model.model.layers[i].self_attn for i in SWAPPED}
    caches = {i: [] for i in SWAPPED}

    class Swapped(torch.nn.Module):
        def __init__(self, i):
            super().__init__()
            self.i, self.layer = i, _oracle_layer(stock[i], i)

        def forward(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None, **kw):
            y = self.layer(hidden_states, cache=caches[self.i], position_embeddings=position_embeddings)
            # the model reads its positions from the cache's length: append this call's keys there too
            n = hidden_states.shape[1]
            past_key_values.update(caches[self.i][0][:, :, -n:], caches[self.i][1][:, :, -n:], self.i)
            return y, None

    try:
        for i in SWAPPED:
            model.model.layers[i].self_attn = Swapped(i)
        cache = DynamicCache(config=model.config)
        with torch.no_grad():
            for f in range(_calls("oneshot")):
                ids = torch.from_numpy(G[f"oneshot/f{f}/ids"]).long()
                out = model(ids, past_key_values=cache, use_cache=True)
                assert torch.equal(out.logits[:, -1].float(), from_np(G[f"oneshot/f{f}/logits"])), f
    finally:
        for i in SWAPPED:
            model.model.layers[i].self_attn = stock[i]


def test_twin_takes_the_reference_fallback_decisions(model):
    """The Torch twin's fallback rule (qwen_torch.py:1187-1219) on every recorded call."""
    twin = qt.QwenCUDAButterflyAttention(model.model.layers[FALLBACK_LAYER].self_attn,
                                         qt.QwenCUDAButterflyConfig(**SWAP_CONFIG)).eval()
    for tag in ("oneshot", "chunked"):
        kv = 0
        for f in range(_calls(tag)):
            q_len = int(G[f"{tag}/f{f}/ids"].shape[1])
            positions = torch.from_numpy(G[f"{tag}/f{f}/positions"]).long()
            kind = str(G[f"{tag}/f{f}/causal_mask"][0])
            mask = None if kind == "none" else causal_mask(positions, kv + q_len, getattr(torch, kind))
            got = twin._fallback_reason(attention_mask=mask, q_len=q_len, k_len_after=kv + q_len,
                                        output_attentions=False)
            assert str(got) == str(G[f"{tag}/f{f}/L{FALLBACK_LAYER}/profile"][1]), (tag, f)
            kv += q_len
    assert kv == sum(CHUNKS) + _calls("chunked") - len(CHUNKS)


@pytest.mark.parametrize("name", ["short_query", "output_attentions", "attention_mask", "training"])
def test_twin_fallback_calls_equal_the_reference(model, name):
    """Direct calls that take the stock module: same reason, same output bits (CPU)."""
    twin = qt.QwenCUDAButterflyAttention(model.model.layers[FALLBACK_LAYER].self_attn,
                                         qt.QwenCUDAButterflyConfig(**SWAP_CONFIG))
    x = from_np(G[f"fallback/{name}/hidden"])
    n = x.shape[1]
    mask = torch.zeros(1, 1, n, n, dtype=torch.bfloat16) if name == "attention_mask" else None
    kw = {"output_attentions": True} if name == "output_attentions" else {}
    twin.train(name == "training")
    with torch.no_grad():
        y = twin(hidden_states=x, position_embeddings=_pe(f"fallback/{name}"), attention_mask=mask, **kw)[0]
    twin.train(False)
    prof = G[f"fallback/{name}/profile"]
    assert [str(twin.last_profile.get(k)) for k in PROFILE_KEYS] == list(prof)
    assert torch.equal(y, from_np(G[f"fallback/{name}/out"]))


def test_twin_chunked_masked_call_falls_back_like_the_reference(model):
    """The second prefill chunk (144 rows over 400 keys) arrives with transformers' boolean
    causal mask, which the reference's mask rule does not accept (qwen_torch.py:495-532):
    the reference and the twin both run the stock module, and the outputs agree bit for bit."""
    from transformers import DynamicCache

    layer = SWAPPED[0]
    twin = qt.QwenCUDAButterflyAttention(model.model.layers[layer].self_attn,
                                         qt.QwenCUDAButterflyConfig(**SWAP_CONFIG)).eval()
    cache = DynamicCache(config=model.config)
    # the first chunk's keys, as the stock module caches them (the twin's Butterfly path needs HIP)
    with torch.no_grad():
        twin.fallback(hidden_states=from_np(G["chunked/f0/L%d/hidden" % layer]), position_embeddings=_pe("chunked/f0"),
                      attention_mask=None, past_key_values=cache)
        positions = torch.from_numpy(G["chunked/f1/positions"]).long()
        mask = causal_mask(positions, sum(CHUNKS), torch.bool)
        y = twin(hidden_states=from_np(G[f"chunked/f1/L{layer}/hidden"]), position_embeddings=_pe("chunked/f1"),
                 attention_mask=mask, past_key_values=cache, position_ids=positions.view(1, -1))[0]
    assert twin.last_profile["reason"] == "attention_mask"
    assert torch.equal(y, from_np(G[f"chunked/f1/L{layer}/out"]))
