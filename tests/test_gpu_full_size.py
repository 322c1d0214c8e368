"""GPU parity at the benchmark configurations' full sizes (4 and 5).

* cfg4: the whole 262144-token streaming prefill (683 chunks of 384, Hq16/Hkv4/d256) through
  ``chunked_prefill`` and the native chunk loop, with chunks compared against the oracle's
  active rows over the full K/V: the first (one-shot) chunk, every chunk at which
  ceil(log2 N) grows, chunks whose routed partner lies 2^10 blocks back, and the last; the
  final counters, tail and pool against the oracle cache fed the same chunks.
* cfg3: caches filled from 131072 tokens with the 384-token chunk schedule, then the
  device-counter decode step captured 64 times in one HIP graph (as the benchmark runs it)
  for B = 1, 8 and 32; every step against ``oracle.from_cache`` over the oracle cache.
* cfg5: the 24-layer, hidden-2048 decoder with a 32768-token prompt: every swapped layer's
  attention output against the oracle on the same q/k/v, for the prefill and decode steps with
  host counters, and for the graph-replayed decode steps (``bfly_decode_step_qk_norm`` inside the
  captured step the benchmark times).

Tolerances are the north_star's bf16 bar (2e-2 max-abs, 1e-2 relative L2).  The cfg5 decoder's
attention outputs reach several units, where one bf16 step of the output is 2^-5 = 0.031: there
the bar is held against the oracle evaluated in float32 (on the same bf16 q/k/v and the same bf16
summary rows), i.e. the error of the kernel plus the rounding of its own output; the difference
from the oracle's bf16 output, which adds the oracle's rounding, is printed beside it.
"""
from __future__ import annotations

import math

import pytest
import torch

import butterfly_amd as bf
from oracle import attention as oa, topology as tp
from oracle.cache import OracleCompressedKVCache

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-2, 1e-2


def _err(got, want):
    got, want = got.float().cpu(), want.float().cpu()
    return (got - want).abs().max().item(), ((got - want).norm() / want.norm()).item()


def _layout(t, hkv, groups, layer):
    return tp.build_layout(seq_len=t, block_size=128, num_key_value_heads=hkv, num_key_value_groups=groups,
                           layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                           partner_rule="causal_shift")


def _width(n):
    return 1 if n <= 1 else (n - 1).bit_length()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("max_chunk", [512, 2048, 4096])   # 2048: five chunks per launch; 4096: eight (the bench's ring)
def test_cfg4_full_stream_matches_oracle_at_stage_changes(max_chunk):
    hq, hkv, d, bs, W, T, chunk, layer = 16, 4, 256, 128, 64, 262144, 384, 10
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(41)
    q = torch.randn(1, hq, T, d, generator=g, device=dev).bfloat16()
    k = torch.randn(1, hkv, T, d, generator=g, device=dev).bfloat16()
    v = torch.randn(1, hkv, T, d, generator=g, device=dev).bfloat16()
    chunks = bf.split_chunks(q, k, v, chunk)
    cache = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=T, max_chunk_size=max_chunk)
    core = bf.ButterflyAttentionCore(bf.compressed_butterfly_config(), layer)
    outs = bf.chunked_prefill(core, chunks, cache)
    torch.cuda.synchronize()
    assert len(outs) == 683 and core.last_profile.notes.get("native_chunk_loop", 0) > 1
    print(f"cfg4 stream done: offset={cache.offset} tail={cache.tail_size} summaries={cache.summary_count}", flush=True)

    check, prev = {0, 682, 400, 555}, None        # chunks 400 and 555: N > 1024 -> stage 10, partner b - 1024
    for c in range(683):
        n = math.ceil(min(T, (c + 1) * chunk) / bs)
        if _width(n) != prev:
            check.add(c)
            prev = _width(n)
    kc, vc = k.cpu(), v.cpu()
    nall = T // bs
    ksum = oa.block_mean(kc, seq_len=T, block_size=bs, num_blocks=nall)   # every chunk ends on a block edge
    vsum = oa.block_mean(vc, seq_len=T, block_size=bs, num_blocks=nall)
    for c in sorted(check):
        s0, e = c * chunk, min(T, (c + 1) * chunk)
        lay = _layout(e, hkv, hq // hkv, layer)
        qc = q[:, :, s0:e].cpu()
        if c == 0:
            want = oa.prefill(qc, kc[:, :, :e], vc[:, :, :e], layout=lay, W=W)
        else:
            n = lay.num_blocks
            want = oa.active(qc, kc[:, :, :e], vc[:, :, :e], layout=lay, query_positions=torch.arange(s0, e), W=W,
                             k_summary=ksum[:, :, :n], v_summary=vsum[:, :, :n])
        err, rel = _err(outs[c], want)
        print(f"cfg4 chunk {c}: N={lay.num_blocks} stage={lay.stage_idx}/{lay.stage_count} "
              f"max_abs={err:.3e} rel_l2={rel:.3e}", flush=True)
        assert err <= MAX_ABS and rel <= REL_L2, (c, err, rel)
        if c in (400, 555):
            assert lay.stage_idx == 10                 # the routed partner is block b - 2^10
    # cache state against the oracle cache fed the same chunks
    oc = OracleCompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=T, max_chunk_size=512)
    for s0 in range(0, T, chunk):
        oc.update_and_fetch(kc[:, :, s0:s0 + chunk], vc[:, :, s0:s0 + chunk])
    assert (cache.offset, cache.tail_size, cache.summary_count, cache.summary_offset) == \
           (oc.offset, oc.tail_size, oc.summary_count, oc.summary_offset) == (T, 384, 2047, 2047 * bs)
    assert cache.nbytes == oc.nbytes
    assert torch.equal(cache.keys.cpu(), oc.keys) and torch.equal(cache.values.cpu(), oc.values)
    for got_pool, want_pool in ((cache.k_summary, oc.k_summary), (cache.v_summary, oc.v_summary)):
        diff = (got_pool.float().cpu() - want_pool.float()).abs()
        assert (diff <= 2 ** -8 * want_pool.float().abs() + 1e-6).all()     # one bf16 rounding apart at most


@pytest.mark.timeout(600)
@pytest.mark.parametrize("B", [1, 8, 32])
def test_cfg3_graph_decode_matches_from_cache_every_step(B):
    hq, hkv, d, bs, W, ctx, steps, layer, kv_step = 8, 2, 128, 128, 64, 131072, 64, 3, 384
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(300 + B)
    k = torch.randn(B, hkv, ctx + steps, d, generator=g, device=dev).bfloat16()
    v = torch.randn(B, hkv, ctx + steps, d, generator=g, device=dev).bfloat16()
    qn = torch.randn(steps, B, hq, 1, d, generator=g, device=dev).bfloat16()
    prealloc = -(-(ctx + steps) // kv_step) * kv_step            # 131328, as the harness rounds it
    cache = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=prealloc, max_chunk_size=512)
    for s in range(0, ctx, kv_step):
        cache.update(k[:, :, s:min(ctx, s + kv_step)], v[:, :, s:min(ctx, s + kv_step)])
    assert (cache.tail_size, cache.summary_count, cache.summary_capacity) == (256, 1023, 1030)
    kc, vc = k.cpu(), v.cpu()
    oc = OracleCompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=prealloc, max_chunk_size=512)
    for s in range(0, ctx, kv_step):
        oc.update_and_fetch(kc[:, :, s:min(ctx, s + kv_step)], vc[:, :, s:min(ctx, s + kv_step)])
    print(f"cfg3 B={B}: caches filled (tail {cache.tail_size}, {cache.summary_count} summaries)", flush=True)
    kn = [k[:, :, ctx + s:ctx + s + 1].contiguous() for s in range(steps)]
    vn = [v[:, :, ctx + s:ctx + s + 1].contiguous() for s in range(steps)]
    cache.use_device_counters()
    outs = torch.empty(steps, B, hq, 1, d, dtype=torch.bfloat16, device=dev)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for s in range(steps):
                cache.decode_step(qn[s], kn[s], vn[s], layer_idx=layer, local_window_tokens=W, out=outs[s])
    torch.cuda.current_stream(dev).wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    cache.sync()
    rep = lambda x: x.repeat_interleave(hq // hkv, dim=1)
    worst = (0.0, 0.0)
    for s in range(steps):
        oc.update_and_fetch(kc[:, :, ctx + s:ctx + s + 1], vc[:, :, ctx + s:ctx + s + 1])
        tk, tv, sk, sv, ts, kv_len = oc.get_compressed_state()
        want = oa.from_cache(qn[s].cpu(), rep(tk), rep(tv), rep(sk), rep(sv), layout=_layout(kv_len, hkv, hq // hkv, layer),
                             query_positions=torch.tensor([kv_len - 1]), W=W, tail_start=ts, kv_len=kv_len)
        err, rel = _err(outs[s], want)
        worst = (max(worst[0], err), max(worst[1], rel))
        assert err <= MAX_ABS and rel <= REL_L2, (B, s, err, rel)
    print(f"cfg3 B={B}: 64 graph-replayed steps, worst max_abs={worst[0]:.3e} rel_l2={worst[1]:.3e}", flush=True)
    assert (cache.offset, cache.tail_size, cache.summary_count, cache.summary_offset) == \
           (oc.offset, oc.tail_size, oc.summary_count, oc.summary_offset)
    assert cache.summary_count == 1024


@pytest.mark.timeout(900)
def test_cfg5_every_layer_matches_oracle_at_32768(monkeypatch):
    from butterfly_amd.decoder import Decoder, DecoderConfig

    cfg = DecoderConfig()
    prompt_len, steps, W = 32768, 2, 64
    model = Decoder(cfg, seed=5, device="cuda")
    assert bf.swap_qwen_attention_with_butterfly(model, cfg=bf.compressed_butterfly_config()) == list(range(24))
    caches = [None] * cfg.num_layers
    bf.install_compressed_kv_caches(model, caches, block_size=128, local_window_tokens=W,
                                    max_kv_size=prompt_len + 64, max_chunk_size=prompt_len + 64)
    history, results = {}, []
    real_call = bf.ButterflyAttentionCore.__call__

    def checked(core, q, k, v, cache=None, qk_norm=None):
        out = real_call(core, q, k, v, cache, qk_norm=qk_norm)
        layer = core.layer_idx
        kh, vh = history.get(layer, (None, None))
        kh = k.cpu() if kh is None else torch.cat([kh, k.cpu()], 2)
        vh = v.cpu() if vh is None else torch.cat([vh, v.cpu()], 2)
        history[layer] = (kh, vh)
        tq, tk = q.shape[2], kh.shape[2]
        lay = _layout(tk, cfg.num_kv_heads, cfg.num_heads // cfg.num_kv_heads, layer)
        want, want32 = _oracle_rows(q.cpu(), kh, vh, lay, tq, W)
        results.append((layer, tk, *_err(out, want32), want.float().abs().max().item(), _err(out, want)[0]))
        return out

    monkeypatch.setattr(bf.ButterflyAttentionCore, "__call__", checked)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=torch.Generator().manual_seed(9)).cuda()
    logits = model.forward(prompt, caches, 0)
    print(f"cfg5 prefill: {len(results)} layers checked, worst max_abs="
          f"{max(r[2] for r in results):.3e} rel_l2={max(r[3] for r in results):.3e} "
          f"(largest |o| {max(r[4] for r in results):.2f})", flush=True)
    pos = prompt_len
    for _ in range(steps):
        tok = logits.argmax(-1, keepdim=True)
        logits = model.forward(tok, caches, pos)
        pos += 1
    assert len(results) == cfg.num_layers * (1 + steps)
    for layer, tk, err, rel, amax, err_bf16 in results:
        assert err <= MAX_ABS and rel <= REL_L2, (layer, tk, err, rel, amax)
    print(f"cfg5: {len(results)} layer calls (prefill + {steps} decode steps), worst vs the fp32 oracle "
          f"max_abs={max(r[2] for r in results):.3e} rel_l2={max(r[3] for r in results):.3e}; vs the oracle's "
          f"bf16 output max_abs={max(r[5] for r in results):.3e} (largest |o| {max(r[4] for r in results):.2f})",
          flush=True)


def _oracle_rows(q, kh, vh, lay, tq, W):
    """The oracle's rows for the last ``tq`` positions of ``kh``/``vh``: its bf16 output, and the
    same evaluated in float32 over the bf16 inputs and the bf16 summary rows (block means
    rounded as the kernels pool them)."""
    tk = kh.shape[2]
    ks = oa.block_mean(kh, seq_len=tk, block_size=128, num_blocks=lay.num_blocks)
    vs = oa.block_mean(vh, seq_len=tk, block_size=128, num_blocks=lay.num_blocks)
    if tq == tk:
        want = oa.prefill(q, kh, vh, layout=lay, W=W)
        want32 = oa.prefill(q.float(), kh.float(), vh.float(), layout=lay, W=W, k_summary=ks.float(),
                            v_summary=vs.float())
    else:
        qp = torch.arange(tk - tq, tk)
        want = oa.active(q, kh, vh, layout=lay, query_positions=qp, W=W)
        want32 = oa.active(q.float(), kh.float(), vh.float(), layout=lay, query_positions=qp, W=W,
                           k_summary=ks.float(), v_summary=vs.float())
    return want, want32


@pytest.mark.timeout(900)
def test_cfg5_graph_replayed_steps_match_oracle_at_32768(monkeypatch):
    """The decode steps the benchmark times: after a 32768-token prompt, every layer's
    ``bfly_decode_step_qk_norm_oproj`` inside the captured greedy step (replayed from one HIP
    graph, device counters) against the oracle's active row over that layer's full key history,
    and its output projection's partial rows against ``bfly_q4_gemv`` of that row."""
    from butterfly_amd.decoder import Decoder, DecoderConfig

    cfg = DecoderConfig()
    prompt_len, new_tokens, W = 32768, 6, 64
    model = Decoder(cfg, seed=5, device="cuda")
    assert bf.swap_qwen_attention_with_butterfly(model, cfg=bf.compressed_butterfly_config()) == list(range(24))
    caches = [None] * cfg.num_layers
    bf.install_compressed_kv_caches(model, caches, block_size=128, local_window_tokens=W,
                                    max_kv_size=prompt_len + 64, max_chunk_size=prompt_len + 64)
    prompt_kv, rows, bufs = {}, {l: [] for l in range(cfg.num_layers)}, {}
    real_call = bf.ButterflyAttentionCore.__call__
    real_step = bf.ButterflyAttentionCore.step_oproj

    def record(layer, ts):
        if layer not in bufs:                                  # the eager first step, before capture
            bufs[layer] = [torch.empty_like(t) for t in ts]
        for b_, t_ in zip(bufs[layer], ts):
            b_.copy_(t_)                                       # recorded into the graph as well
        if not torch.cuda.is_current_stream_capturing():
            rows[layer].append([t_.cpu() for t_ in bufs[layer]])

    def recording(core, q, k, v, cache=None, qk_norm=None):
        out = real_call(core, q, k, v, cache, qk_norm=qk_norm)
        if q.shape[2] > 1:                                     # the prompt: normed, rotated k and v
            prompt_kv[core.layer_idx] = (k.cpu(), v.cpu())
            return out
        assert qk_norm is not None, "a device-counter decode step takes the raw q|k|v rows"
        record(core.layer_idx, (q, k, v, out))
        return out

    def recording_oproj(core, q, k, v, cache, qk_norm, o_proj):
        # the step with the output projection inside: its attention row and partial rows
        out, parts = real_step(core, q, k, v, cache, qk_norm, o_proj)
        record(core.layer_idx, (q, k, v, out, parts))
        return out, parts

    monkeypatch.setattr(bf.ButterflyAttentionCore, "__call__", recording)
    monkeypatch.setattr(bf.ButterflyAttentionCore, "step_oproj", recording_oproj)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=torch.Generator().manual_seed(9)).cuda()
    logits = model.forward(prompt, caches, 0)
    torch.cuda.synchronize()

    def on_step(i):
        for layer in range(cfg.num_layers):
            rows[layer].append([t_.cpu() for t_ in bufs[layer]])
        print(f"cfg5 graph replay {i} recorded", flush=True)

    model.greedy_graph_from_logits(logits, prompt_len, new_tokens, caches, on_step=on_step)
    monkeypatch.undo()
    steps = new_tokens - 1
    worst = [0.0, 0.0, 0.0]
    from butterfly_amd.decoder import q4_gemv

    for layer in range(cfg.num_layers):
        assert len(rows[layer]) == steps
        base = model.layers[layer].self_attn.base
        kh, vh = prompt_kv[layer]
        for s_, rec in enumerate(rows[layer]):
            qr, kr, vr, out = rec[:4]
            # cfg5's shapes take the output projection into the step: its partial rows combine
            # into bfly_q4_gemv's product of the attention row bit for bit
            assert len(rec) == 5, "cfg5's decode steps run the output projection inside"
            pr = rec[4]
            y = q4_gemv(out.reshape(1, -1).cuda(), base.o_proj).cpu()
            assert torch.equal(((pr[0] + pr[1]) + (pr[2] + pr[3])).bfloat16(), y.view(pr.shape[1:])), (layer, s_)
            p = prompt_len + s_
            # the raw rows normed and rotated by the separate launch (bit-identical to the fused step)
            qkv = torch.cat([qr.view(-1), kr.view(-1), vr.view(-1)]).view(1, 1, -1).cuda()
            q, k, v = base.heads(qkv, torch.tensor([p], device="cuda"))
            kh, vh = torch.cat([kh, k.cpu()], 2), torch.cat([vh, v.cpu()], 2)
            lay = _layout(p + 1, cfg.num_kv_heads, cfg.num_heads // cfg.num_kv_heads, layer)
            want, want32 = _oracle_rows(q.cpu(), kh, vh, lay, 1, W)
            err, rel = _err(out, want32)
            assert err <= MAX_ABS and rel <= REL_L2, (layer, p, err, rel)
            worst = [max(worst[0], err), max(worst[1], rel), max(worst[2], _err(out, want)[0])]
    print(f"cfg5 graph-replayed: {cfg.num_layers} layers x {steps} steps (1 eager + {steps - 1} replays), worst vs "
          f"the fp32 oracle max_abs={worst[0]:.3e} rel_l2={worst[1]:.3e}; vs its bf16 output {worst[2]:.3e}",
          flush=True)
