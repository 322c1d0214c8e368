"""Write golden vectors for the Torch layer swap from the reference's own module
(run in the build container only).

Usage: ``python tests/golden/make_golden_swap.py /path/to/Hmbown-Butterfly``

The reference repository is imported from the given path.  Its
``swap_qwen_attention_with_butterfly_cuda`` (bna/integrations/qwen_torch.py:1652-1700)
swaps the full-attention layers of a tiny random-init HF-transformers Qwen3.5 model
(CPU, bf16) to ``QwenCUDAButterflyAttention`` with the compressed configuration, and
the model runs:

* ``oneshot``: a 400-token prompt in one call, then 4 greedy steps through a
  ``DynamicCache`` (the one-shot branch, qwen_torch.py:1452-1470, then the cached
  branch, :1400-1427);
* ``chunked``: the same prompt as chunks of 256 and 144 tokens, then 2 greedy steps (the
  cached branch with several query rows and ``cache_position``);
* ``fallback``: direct calls of one swapped module that take the stock module by the
  reference's rules (:1187-1219): a one-token query without a cache, ``output_attentions``,
  a non-causal mask, and training mode.

For every swapped call the fixture keeps the call's input hidden states, the
position embeddings, the output and the reference's ``last_profile`` mode, reason,
kv_len, stage and backend; for every model call the last position's logits.  The
committed ``golden_swap.npz`` is data only; the model is rebuilt by the tests from
``tiny_model()`` (seeded init, checked against the recorded digest).  Nothing under
``tests/golden`` reads the reference at test time.

Why an import: the dispatch of the swapped module (which entry runs with which
query positions and layout, the output gate and ``o_proj``, the fallback rules)
is the reference's own code; no reference test writes its outputs.

transformers 5.15 names the decoder layer's kind ``block_type``; the reference's swap
selects layers by ``layer_type``, so the script copies the one to the other before
swapping.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
OUT = HERE / "golden_swap.npz"

LAYER_TYPES = ("linear_attention", "full_attention", "full_attention", "linear_attention", "full_attention")
SWAPPED = (1, 2, 4)
PROMPT, STEPS, CHUNKS, CHUNKED_STEPS = 400, 4, (256, 144), 2
WINDOW = 64
FALLBACK_LAYER = 2
SWAP_CONFIG = dict(path="block_sparse", block_compression="mean", block_partner_rule="causal_shift",
                   compressed_local_window_tokens=WINDOW)
PROFILE_KEYS = ("mode", "reason", "kv_len", "block_sparse_stage", "block_sparse_backend")


def tiny_model():
    """The random-init Qwen3.5 the fixture was written with (CPU, bf16, eval mode)."""
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM

    cfg = Qwen3_5TextConfig(vocab_size=512, hidden_size=64, intermediate_size=128, num_hidden_layers=len(LAYER_TYPES),
                            num_attention_heads=4, num_key_value_heads=2, head_dim=128, layer_types=list(LAYER_TYPES),
                            linear_num_key_heads=2, linear_num_value_heads=2, linear_key_head_dim=32,
                            linear_value_head_dim=32, initializer_range=0.1)
    torch.manual_seed(0)
    return Qwen3_5ForCausalLM(cfg).to(torch.bfloat16).eval()


def prompt_ids(vocab: int) -> torch.Tensor:
    return torch.randint(0, vocab, (1, PROMPT), generator=torch.Generator().manual_seed(1))


def model_digest(model) -> str:
    h = hashlib.sha256()
    for name, t in sorted(model.state_dict().items()):
        h.update(name.encode())
        h.update(t.detach().cpu().contiguous().flatten().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()[:16]


def to_np(t: torch.Tensor) -> np.ndarray:
    """bf16 as its uint16 bit pattern, fp32 as float32, integers as int32."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    if t.dtype in (torch.int64, torch.int32):
        return t.numpy().astype(np.int32)
    return t.float().numpy()


def from_np(a: np.ndarray) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a))


def causal_mask(positions: torch.Tensor, kv_len: int, dtype) -> torch.Tensor:
    """The causal mask [1, 1, len(positions), kv_len] that transformers passes to the attention
    of a multi-row call with a cache: boolean (True where the key is at or before the query),
    or additive (0 there, else the dtype's lowest value)."""
    allowed = (torch.arange(kv_len).view(1, -1) <= positions.view(-1, 1)).view(1, 1, len(positions), kv_len)
    if dtype == torch.bool:
        return allowed
    return torch.zeros(allowed.shape, dtype=dtype).masked_fill_(~allowed, torch.finfo(dtype).min)


def fallback_cases(hidden: int, rotary, generator: torch.Generator):
    """(name, hidden_states, position ids, mask, kwargs, train) of the direct fallback calls."""
    x8 = torch.randn(1, 8, hidden, generator=generator).bfloat16()
    x1 = torch.randn(1, 1, hidden, generator=generator).bfloat16()
    full = torch.zeros(1, 1, 8, 8, dtype=torch.bfloat16)          # attend everywhere: not causal
    return [("short_query", x1, torch.arange(1), None, {}, False),
            ("output_attentions", x8, torch.arange(8), None, {"output_attentions": True}, False),
            ("attention_mask", x8, torch.arange(8), full, {}, False),
            ("training", x8, torch.arange(8), None, {}, True)]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from bna.integrations import qwen_torch as RQ  # noqa: E402
    from transformers import DynamicCache

    torch.set_num_threads(1)
    model = tiny_model()
    data: dict[str, np.ndarray] = {"meta/model_digest": np.array([model_digest(model)])}
    decoder = model.model
    for layer in decoder.layers:
        layer.layer_type = layer.block_type
    cfg = RQ.QwenCUDAButterflyConfig(**SWAP_CONFIG)
    assert RQ.swap_qwen_attention_with_butterfly_cuda(model, cfg) == list(SWAPPED)
    calls: list = []

    def hook(mod, args, kwargs, output):
        prof = mod.last_profile
        mask = kwargs.get("attention_mask")
        calls.append((mod.layer_idx, kwargs["hidden_states"].clone(), output[0].clone(),
                      np.array([str(prof.get(k)) for k in PROFILE_KEYS]), kwargs["position_embeddings"],
                      kwargs.get("cache_position"), mask))

    handles = [m.register_forward_hook(hook, with_kwargs=True) for m in RQ.iter_qwen_butterfly_layers(model)]
    ids = prompt_ids(model.config.vocab_size)

    def run(tag, pieces, steps):
        cache = DynamicCache(config=model.config)
        start = 0
        seq = []
        for piece in pieces:
            seq.append(ids[:, start:start + piece])
            start += piece
        f = 0
        pos = 0
        with torch.no_grad():
            tok = None
            for i in range(len(seq) + steps):
                x = seq[i] if i < len(seq) else tok
                del calls[:]
                out = model(x, past_key_values=cache, use_cache=True)
                positions = torch.arange(pos, pos + x.shape[1])
                cos, sin = calls[0][4]
                # the layers' call arguments: one set of RoPE rows, the call's positions, and
                # either no mask or the additive causal mask of these positions over the cache
                assert all(torch.equal(c[4][0], cos) and torch.equal(c[4][1], sin) for c in calls)
                assert all(c[5] is None or torch.equal(c[5].view(-1), positions) for c in calls)
                masked = [c[6] is not None for c in calls]
                assert len(set(masked)) == 1
                for c in calls:
                    if c[6] is not None:
                        assert torch.equal(c[6], causal_mask(positions, pos + x.shape[1], c[6].dtype))
                kind = "none" if calls[0][6] is None else str(calls[0][6].dtype).replace("torch.", "")
                data[f"{tag}/f{f}/causal_mask"] = np.array([kind])
                data[f"{tag}/f{f}/ids"] = to_np(x)
                data[f"{tag}/f{f}/positions"] = to_np(positions)
                data[f"{tag}/f{f}/cos"], data[f"{tag}/f{f}/sin"] = to_np(cos), to_np(sin)
                data[f"{tag}/f{f}/logits"] = to_np(out.logits[:, -1].float())
                assert [c[0] for c in calls] == list(SWAPPED)
                for layer, h, y, prof, *_ in calls:
                    data[f"{tag}/f{f}/L{layer}/hidden"] = to_np(h)
                    data[f"{tag}/f{f}/L{layer}/out"] = to_np(y)
                    data[f"{tag}/f{f}/L{layer}/profile"] = prof
                tok = out.logits[:, -1:].argmax(-1)
                pos += x.shape[1]
                f += 1
        data[f"{tag}/calls"] = np.array([f])

    run("oneshot", (PROMPT,), STEPS)
    run("chunked", CHUNKS, CHUNKED_STEPS)
    for h in handles:
        h.remove()
    mod = decoder.layers[FALLBACK_LAYER].self_attn
    g = torch.Generator().manual_seed(7)
    for name, x, positions, mask, kw, train in fallback_cases(model.config.hidden_size, decoder.rotary_emb, g):
        cos, sin = decoder.rotary_emb(x, positions.view(1, -1))
        mod.train(train)
        with torch.no_grad():
            y = mod(hidden_states=x, position_embeddings=(cos, sin), attention_mask=mask, **kw)[0]
        mod.train(False)
        data[f"fallback/{name}/hidden"] = to_np(x)
        data[f"fallback/{name}/cos"], data[f"fallback/{name}/sin"] = to_np(cos), to_np(sin)
        data[f"fallback/{name}/out"] = to_np(y)
        data[f"fallback/{name}/profile"] = np.array([str(mod.last_profile.get(k)) for k in PROFILE_KEYS])
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({len(data)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
