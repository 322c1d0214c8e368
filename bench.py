"""Benchmark: Butterfly compressed attention on one MI355X.

Headline: single-layer bf16 prefill at T=65536,
Hq=8, Hkv=2, d=128, BS=128, W=64, causal_shift, sweeping the 9 stages
(step i runs layer i mod 9).  A step = compressor (K and V, one launch) +
fused prefill over inputs already resident in HBM.  The layer layouts are
built once before timing (the reference caches them per sequence length).

Secondary: batched decode at 131072 context, B in {1, 8, 32},
64 steps each (append + compress-at-boundary + attention per step).

Prints ONE JSON line.  `python bench.py --gpus 1 --steps K --warmup W`.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
TRAFFIC_PROFILE = ROOT / "profiles" / "prefill_cfg2_hbm_traffic.md"


def measured_traffic():
    """HBM bytes per prefill launch from the committed rocprofv3 --pmc summary (None if absent)."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip().replace(",", ""))
    except OSError:
        pass
    return None
MFMA_BF16_PEAK_TFLOPS = 2500.0


def _host_threads() -> int:
    """Host threads for the CPU legs: the job's share (OMP_NUM_THREADS, as the GPU boxes set it)
    rather than every core the machine reports."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def _log(msg: str) -> None:
    """A progress line on stderr (stdout carries only the JSON result line): names the leg that
    is running, so a failed run can be attributed to it."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def prefill_workload(seed=0, T=65536, hq=8, hkv=2, d=128):
    import numpy as np
    import torch

    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.standard_normal((1, hq, T, d), dtype=np.float32))
    k = torch.from_numpy(rng.standard_normal((1, hkv, T, d), dtype=np.float32))
    v = torch.from_numpy(rng.standard_normal((1, hkv, T, d), dtype=np.float32))
    k = k * torch.from_numpy(rng.uniform(0.5, 2.0, size=(d,)).astype(np.float32))
    return q.bfloat16(), k.bfloat16(), v.bfloat16()


def prefill_algorithmic(T, hq, hkv, d, bs, W, e, neighbors_rows):
    """Algorithmic bytes and FLOPs of one prefill launch (and of the compressor).

    bytes: read Q, K, V; write O; read the routed summary rows (K and V) once
    per kv head.  flops: 4*d*Hq*sum_t [min(W, t+1) + n_sum(t)].
    """
    n = (T + bs - 1) // bs
    prefill_bytes = e * (2 * T * hq * d + 2 * T * hkv * d) + 2 * n * hkv * d * e
    compress_bytes = e * 2 * T * hkv * d + 2 * n * hkv * d * e
    keys = 0
    for b, n_sum in enumerate(neighbors_rows):
        t0, t1 = b * bs, min(T, (b + 1) * bs)
        for t in range(t0, t1):
            keys += min(W, t + 1) + n_sum
    flops = 4 * d * hq * keys
    return prefill_bytes, compress_bytes, flops


def summary_counts(layout_ref, T, W):
    """Eligible summaries per query block (block-level cut-off), from the oracle layout."""
    bs, n = layout_ref.block_size, layout_ref.num_blocks
    out = []
    nb = layout_ref.block_neighbors[0].tolist()
    for b in range(n):
        start = max(0, b * bs - W + 1)
        out.append(sum(1 for x in nb[b] if 0 <= x < b and (x + 1) * bs <= start))
    return out


def bench_prefill(args, torch, bf, tp):
    T, hq, hkv, d, bs, W = 65536, 8, 2, 128, 128, 64
    dev = torch.device("cuda:0")
    q, k, v = prefill_workload(args.seed, T, hq, hkv, d)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    stages = 9
    lays = []
    for layer in range(stages):
        kw = dict(seq_len=T, block_size=bs, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                  layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1, partner_rule="causal_shift")
        lays.append(bf.build_block_butterfly_layout(**kw))
    assert all(l.stage_count == stages for l in lays)
    ref_lays = [tp.build_layout(seq_len=T, block_size=bs, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                                layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                                partner_rule="causal_shift") for layer in range(stages)]
    from butterfly_amd import _native
    from butterfly_amd.attention import _dtype_code

    n = lays[0].num_blocks
    ksum = torch.empty((1, hkv, n, d), dtype=torch.bfloat16, device=dev)
    vsum = torch.empty_like(ksum)
    out = torch.empty_like(qd)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    lib = _native.lib()
    dt = _dtype_code(qd)
    scale = 1.0 / (d ** 0.5)

    def step(i, ev=None, sh=sh):
        lay = lays[i % stages]
        nb = lay.neighbors
        _native.check(lib.bfly_block_mean(kd.data_ptr(), ksum.data_ptr(), vd.data_ptr(), vsum.data_ptr(), dt, hkv, T,
                                          d, bs, n, sh), "bfly_block_mean")
        if ev is not None:
            ev[0].record(stream)
        _native.check(lib.bfly_prefill(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ksum.data_ptr(), vsum.data_ptr(),
                                       dt, 1, hq, hkv, T, d, nb.data_ptr(), n, nb.shape[1], bs, W, scale,
                                       out.data_ptr(), sh), "bfly_prefill")
        if ev is not None:
            ev[1].record(stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # eager steps, events around every prefill launch (same stream): per-launch view
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    eager_wall = time.perf_counter() - t0
    prefill_in_step_ms = [a.elapsed_time(b) for a, b in evs]
    # timed region: the same K steps captured in one HIP graph (launch gaps between the
    # compressor and the prefill removed), replayed once between device synchronisations
    side = torch.cuda.Stream(device=dev)
    graph = torch.cuda.CUDAGraph()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for i in range(args.steps):
                step(i, sh=side.cuda_stream)
    stream.wait_stream(side)
    graph.replay()                      # warm replay
    start_ev, end_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start_ev.record(stream)
    graph.replay()
    end_ev.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start_ev.elapsed_time(end_ev)
    # Kernel duration: back-to-back prefill launches (all stages) between two events on
    # the launch stream, so dispatch overlaps execution as in a kernel trace.
    kl0, kl1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 4 * stages
    kl0.record(stream)
    for i in range(reps):
        lay = lays[i % stages]
        nb = lay.neighbors
        _native.check(lib.bfly_prefill(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ksum.data_ptr(), vsum.data_ptr(),
                                       dt, 1, hq, hkv, T, d, nb.data_ptr(), n, nb.shape[1], bs, W, scale,
                                       out.data_ptr(), sh), "bfly_prefill")
    kl1.record(stream)
    torch.cuda.synchronize()
    prefill_ms = [kl0.elapsed_time(kl1) / reps]
    # The same kernel from cold caches: each launch follows a read-only pass over
    # 1 GiB, which leaves nothing of Q/K/V in L2 or the 256 MB MALL (the
    # back-to-back figure above re-reads inputs the previous launch left there).
    flush = torch.ones(256 << 20, dtype=torch.float32, device=dev)
    cold = []
    for i in range(2 * stages):
        flush.sum()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        nb = lays[i % stages].neighbors
        c0.record(stream)
        _native.check(lib.bfly_prefill(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ksum.data_ptr(), vsum.data_ptr(),
                                       dt, 1, hq, hkv, T, d, nb.data_ptr(), n, nb.shape[1], bs, W, scale,
                                       out.data_ptr(), sh), "bfly_prefill")
        c1.record(stream)
        torch.cuda.synchronize()
        cold.append(c0.elapsed_time(c1))
    del flush
    ms_per_step = wall * 1e3 / args.steps
    # correctness spot check of the last layer against the oracle is done in tests;
    # here only make sure outputs are finite
    assert torch.isfinite(out.float()).all()
    counts = summary_counts(ref_lays[(args.steps - 1) % stages], T, W)
    pbytes, cbytes, flops = prefill_algorithmic(T, hq, hkv, d, bs, W, 2, counts)
    avg_prefill_s = statistics.mean(prefill_ms) / 1e3
    res = {
        "T": T, "ms_per_step": ms_per_step, "gpu_ms_per_step": gpu_ms / args.steps,
        "eager_ms_per_step": eager_wall * 1e3 / args.steps,
        "prefill_kernel_ms_avg": statistics.mean(prefill_ms),
        "prefill_kernel_ms_cold": statistics.median(cold),
        "prefill_event_ms_in_step_avg": statistics.mean(prefill_in_step_ms),
        "prefill_event_ms_in_step_min": min(prefill_in_step_ms),
        "prefill_bytes": pbytes, "compress_bytes": cbytes, "prefill_flops": flops,
        "achieved_gbs": pbytes / avg_prefill_s / 1e9,
        "achieved_tflops": flops / avg_prefill_s / 1e12,
        "tok_s": T * args.steps / wall,
        "inputs": (q, k, v, ref_lays),
    }
    return res


def prefill_launches(args, torch, bf):
    """cfg2 (stage 3): ``--prefill-launches`` times the compressor (K and V) then one prefill launch."""
    T, hq, hkv, d, bs, W = 65536, 8, 2, 128, 128, 64
    dev = torch.device("cuda:0")
    q, k, v = (x.to(dev) for x in prefill_workload(args.seed, T, hq, hkv, d))
    lay = bf.build_block_butterfly_layout(seq_len=T, block_size=bs, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                                          layer_idx=3, local_window_blocks=1, sink_count=1, partner_count=1,
                                          partner_rule="causal_shift")
    n = lay.num_blocks
    ks, vs = bf.block_mean_summaries(k, seq_len=T, block_size=bs, num_blocks=n, x2=v)
    out = torch.empty_like(q)
    from butterfly_amd import _native
    from butterfly_amd.attention import _dtype_code
    lib, nb, sh = _native.lib(), lay.neighbors, torch.cuda.current_stream(dev).cuda_stream
    for _ in range(args.prefill_launches):
        _native.check(lib.bfly_block_mean(k.data_ptr(), ks.data_ptr(), v.data_ptr(), vs.data_ptr(), _dtype_code(k), hkv,
                                          T, d, bs, n, sh), "bfly_block_mean")
        _native.check(lib.bfly_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), ks.data_ptr(), vs.data_ptr(),
                                       _dtype_code(q), 1, hq, hkv, T, d, nb.data_ptr(), n, nb.shape[1], bs, W,
                                       1.0 / d ** 0.5, out.data_ptr(), sh), "bfly_prefill")
    torch.cuda.synchronize()
    print(json.dumps({"prefill_launches": args.prefill_launches}), flush=True)


def decode_steps_only(args, torch, bf, steps=64):
    """cfg3 shapes at batch ``--decode-steps``: a restored 131072-token cache, then ``steps``
    eager device-counter decode steps (one ``bfly_decode_step`` launch each), for counter
    collection."""
    hq, hkv, d, bs, W, ctx, B = 8, 2, 128, 128, 64, 131072, args.decode_steps
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    c = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=131328, max_chunk_size=512)
    c.state = tuple(torch.randn(B, hkv, n, d, generator=g, device=dev).bfloat16() for n in (256, 256, 1023, 1023))
    c.meta_state = (str(bs), str(W), str(ctx), str(1023 * bs))
    c.ring_state()
    c.use_device_counters()
    qn = torch.randn(steps, B, hq, 1, d, generator=g, device=dev).bfloat16()
    kn = torch.randn(steps, B, hkv, 1, d, generator=g, device=dev).bfloat16()
    vn = torch.randn(steps, B, hkv, 1, d, generator=g, device=dev).bfloat16()
    out = torch.empty(B, hq, 1, d, dtype=torch.bfloat16, device=dev)
    for s in range(steps):
        c.decode_step(qn[s], kn[s], vn[s], layer_idx=3, local_window_tokens=W, out=out)
    torch.cuda.synchronize()
    c.sync()
    print(json.dumps({"decode_steps": steps, "batch": B, "summaries": c.summary_count}), flush=True)


def _replay_steady(torch, graph, counters, reps=6):
    """Median wall time of ``reps`` replays of a captured decode graph, each from the same
    starting device counters (``counters`` is reset to its value at entry before every
    replay: a replay rewrites the same ring slots and pool rows with the same values)."""
    import statistics

    init = counters.clone()
    ts = []
    for _ in range(reps):
        counters.copy_(init)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def bench_decode(torch, bf, batches=(1, 8, 32), steps=64, seed=0):
    """cfg3: decode at 131072 context from a prefilled two-pool cache."""
    hq, hkv, d, bs, W, ctx = 8, 2, 128, 128, 64, 131072
    dev = torch.device("cuda:0")
    out = {}
    g = torch.Generator(device=dev).manual_seed(seed)
    # warm-up: load the decode/compress kernels outside the timed loops
    wc = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=4096)
    wk = torch.randn(1, hkv, 300, d, generator=g, device=dev).bfloat16()
    wc.update(wk[:, :, :256], wk[:, :, :256])
    for s in range(256, 300):
        lay = bf.build_block_butterfly_layout(seq_len=s + 1, block_size=bs, num_key_value_heads=hkv,
                                              num_key_value_groups=hq // hkv, layer_idx=3, local_window_blocks=1,
                                              sink_count=1, partner_count=1, partner_rule="causal_shift")
        wc.update_and_attend(torch.randn(1, hq, 1, d, generator=g, device=dev).bfloat16(), wk[:, :, s:s + 1],
                             wk[:, :, s:s + 1], layout=lay, local_window_tokens=W)
    torch.cuda.synchronize()
    for B in batches:
        # State after a 384-chunked prefill of 131072 tokens (reference schedule):
        # tail = 256 tokens, 1023 summaries, summary_offset = 1023*128.
        tail = 256
        tk = torch.randn(B, hkv, tail, d, generator=g, device=dev).bfloat16()
        tv = torch.randn(B, hkv, tail, d, generator=g, device=dev).bfloat16()
        sk = torch.randn(B, hkv, 1023, d, generator=g, device=dev).bfloat16()
        sv = torch.randn(B, hkv, 1023, d, generator=g, device=dev).bfloat16()

        def restored():
            c = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=131328, max_chunk_size=512)
            c.state = (tk, tv, sk, sv)
            c.meta_state = (str(bs), str(W), str(ctx), str(1023 * bs))
            c.ring_state()          # place the restored tail in ring order before timing
            return c

        cache = restored()
        kn = torch.randn(steps, B, hkv, 1, d, generator=g, device=dev).bfloat16()
        vn = torch.randn(steps, B, hkv, 1, d, generator=g, device=dev).bfloat16()
        qn = torch.randn(steps, B, hq, 1, d, generator=g, device=dev).bfloat16()

        def layout_for(kv_len):
            return bf.build_block_butterfly_layout(seq_len=kv_len, block_size=bs, num_key_value_heads=hkv,
                                                   num_key_value_groups=hq // hkv, layer_idx=3,
                                                   local_window_blocks=1, sink_count=1, partner_count=1,
                                                   partner_rule="causal_shift")

        # warm the layout cache for the block counts the steps will see
        for s in range(steps):
            layout_for(ctx + s + 1)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(steps):
            o = cache.update_and_attend(qn[s], kn[s], vn[s], layout=layout_for(cache.offset + 1),
                                        local_window_tokens=W)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        assert torch.isfinite(o.float()).all()
        assert cache.summary_count == 1024
        # Device counters + one HIP graph holding all `steps` decode steps (one launch each,
        # fixed arguments): the same work without host bookkeeping between steps.
        gcache = restored()
        gcache.use_device_counters()
        gouts = torch.empty(steps, B, hq, 1, d, dtype=torch.bfloat16, device=dev)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for s in range(steps):
                    gcache.decode_step(qn[s], kn[s], vn[s], layer_idx=3, local_window_tokens=W, out=gouts[s])
        torch.cuda.current_stream(dev).wait_stream(side)
        init_counters = gcache.device_counters.clone()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        first = (time.perf_counter() - t0) / steps
        gcache.sync()
        assert gcache.summary_count == 1024 and torch.equal(gouts[-1], o)
        # steady state: the same 64 steps replayed again from the same starting counters
        gcache.device_counters.copy_(init_counters)
        gdt = _replay_steady(torch, graph, gcache.device_counters) / steps
        assert torch.equal(gouts[-1], o)
        bytes_step = B * (2 * hq * d * 2 + 2 * hkv * W * d * 2 + 2 * hkv * 2 * d * 2 + 2 * hkv * d * 2)
        out[str(B)] = {"ms_per_step": gdt * 1e3, "tok_s": B / gdt, "alg_bytes_per_step": bytes_step,
                       "wall_gbs": bytes_step / gdt / 1e9,
                       "mode": "device counters, 64 steps in one HIP graph; median of 6 replays",
                       "first_replay_ms_per_step": first * 1e3,
                       "eager_ms_per_step": dt * 1e3, "eager_tok_s": B / dt}
    return out


def bench_decode_sweep(torch, bf, batches=(128, 512, 1024, 2048), steps=64, seed=1):
    """cfg3 shapes at batch sizes beyond the config (labelled as such): the same
    device-counter decode step, 64 steps in one HIP graph, to show where the
    per-step latency floor gives way to HBM bandwidth."""
    hq, hkv, d, bs, W, ctx = 8, 2, 128, 128, 64, 131072
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    out = {}
    for B in batches:
        tk = torch.randn(B, hkv, 256, d, generator=g, device=dev).bfloat16()
        tv = torch.randn(B, hkv, 256, d, generator=g, device=dev).bfloat16()
        sk = torch.randn(B, hkv, 1023, d, generator=g, device=dev).bfloat16()
        sv = torch.randn(B, hkv, 1023, d, generator=g, device=dev).bfloat16()
        c = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=131328, max_chunk_size=512)
        c.state = (tk, tv, sk, sv)
        c.meta_state = (str(bs), str(W), str(ctx), str(1023 * bs))
        c.ring_state()
        del tk, tv, sk, sv
        c.use_device_counters()
        qn = torch.randn(steps, B, hq, 1, d, generator=g, device=dev).bfloat16()
        kn = torch.randn(steps, B, hkv, 1, d, generator=g, device=dev).bfloat16()
        vn = torch.randn(steps, B, hkv, 1, d, generator=g, device=dev).bfloat16()
        outs = torch.empty(steps, B, hq, 1, d, dtype=torch.bfloat16, device=dev)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for s in range(steps):
                    c.decode_step(qn[s], kn[s], vn[s], layer_idx=3, local_window_tokens=W, out=outs[s])
        torch.cuda.current_stream(dev).wait_stream(side)
        init_counters = c.device_counters.clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        c.sync()
        assert c.summary_count == 1024 and torch.isfinite(outs[-1].float()).all()
        c.device_counters.copy_(init_counters)
        gdt = _replay_steady(torch, graph, c.device_counters) / steps
        bytes_step = B * (2 * hq * d * 2 + 2 * hkv * W * d * 2 + 2 * hkv * 2 * d * 2 + 2 * hkv * d * 2)
        out[str(B)] = {"ms_per_step": gdt * 1e3, "tok_s": B / gdt, "alg_bytes_per_step": bytes_step,
                       "wall_gbs": bytes_step / gdt / 1e9,
                       "mode": "device counters, 64 steps in one HIP graph; median of 6 replays",
                       "note": "batch beyond the config: bandwidth ramp, not a config result"}
        del c, graph, qn, kn, vn, outs
        torch.cuda.empty_cache()
    return out


def bench_stream(torch, bf, seed=0, T=262144, chunk=384, layer=5, max_chunk=4096):
    """cfg4: streaming chunked prefill, Hq=16, Hkv=4, d=256, bf16, 384-token chunks.

    Per chunk (the harness schedule): cache update (append + compress due
    blocks), layout for the live kv_len, attention (first chunk one-shot, later
    chunks from the device ring + pool).  Inputs are per-chunk contiguous
    tensors resident in HBM (what each chunk's projections would produce).
    """
    hq, hkv, d, bs, W = 16, 4, 256, 128, 64
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    chunks = []
    for s in range(0, T, chunk):
        n = min(chunk, T - s)
        chunks.append(tuple(torch.randn(1, h, n, d, generator=g, device=dev).bfloat16() for h in (hq, hkv, hkv)))
    cfg = bf.compressed_butterfly_config()

    def run():
        # a ring of 8512 rows (about 22 chunks): the native loop then runs ten chunks (its cap) per
        # attention launch and per update job (the outputs and the cache equal the one-chunk schedule's)
        cache = bf.CompressedKVCache(block_size=bs, local_window_tokens=W, max_kv_size=T, max_chunk_size=max_chunk)
        core = bf.ButterflyAttentionCore(cfg, layer)
        outs = bf.chunked_prefill(core, chunks, cache)
        return cache, outs

    cache, outs = run()                 # warm: kernels loaded, layouts for every kv_len built
    # five timed streams, each from an empty cache (the median is reported, every sample listed:
    # one stream takes about 2 ms, so a single sample moves with the host's scheduling)
    walls, peak = [], 0
    for i in range(5):
        del cache, outs
        torch.cuda.synchronize()
        if i == 0:
            base = torch.cuda.memory_allocated()
            torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        cache, outs = run()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        if i == 0:
            peak = torch.cuda.max_memory_allocated() - base
    wall = sorted(walls)[len(walls) // 2]
    assert all(torch.isfinite(o[:, :, -1].float()).all() for o in outs[-3:])
    dense = 2 * hkv * T * d * 2
    out_bytes = sum(o.numel() * o.element_size() for o in outs)
    return {"T": T, "chunks": len(chunks), "e2e_s": wall, "e2e_s_runs": walls, "e2e_timing": "median of 5 streams",
            "tok_s": T / wall, "ms_per_chunk": wall * 1e3 / len(chunks),
            "peak_hbm_bytes_above_inputs": int(peak),
            "peak_hbm_note": "the harness keeps every chunk's output: the peak is the retained outputs plus the cache",
            "retained_outputs_bytes": int(out_bytes), "cache_allocated_bytes": int(cache.allocated_bytes),
            "retained_kv_bytes": int(cache.nbytes),
            "dense_kv_bytes": int(dense), "retained_over_dense": cache.nbytes / dense,
            "final_tail": cache.tail_size, "final_summaries": cache.summary_count}


def bench_decoder(torch, bf, seed=0, prompt_len=32768, new_tokens=32, agree_prompt=32768, agree_tokens=32,
                  cpu_agreement=True):
    """cfg5: random-init 24-layer decoder (4-bit affine weights, group 64), every attention
    layer swapped to Butterfly; 32768-token prompt then 32 greedy tokens.

    Greedy agreement with the CPU reference Torch path (the same decoder on the host with the
    oracle attention) over the same 32768-token prompt and ``agree_tokens`` greedy steps.  The
    CPU side takes the GPU's rounding points for the 4-bit products (one-row products from the
    codes in fp32, prefill products over the bf16-dequantised weights), so that what remains
    between the two sides is attention and fp32 summation order.
    """
    import copy

    from butterfly_amd.decoder import Decoder, DecoderConfig
    from oracle.decoder_ref import match_gpu_rounding, swap_to_oracle

    dev = torch.device("cuda:0")
    cfg = DecoderConfig()
    model = Decoder(cfg, seed=seed, device=dev)
    cpu_model = copy.deepcopy(model).to("cpu") if cpu_agreement else None
    bcfg = bf.compressed_butterfly_config()
    bf.swap_qwen_attention_with_butterfly(model, cfg=bcfg)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=torch.Generator().manual_seed(seed + 1))
    pd = prompt.to(dev)

    def fresh(max_kv):
        # the one-shot prompt is one update: the tail must hold it (capacity W + 2*max_chunk + 2*BS)
        caches = [None] * cfg.num_layers
        bf.install_compressed_kv_caches(model, caches, block_size=128, local_window_tokens=64, max_kv_size=max_kv,
                                        max_chunk_size=max(512, max_kv))
        return caches

    model.greedy(pd[:, :512], 4, fresh(1024))           # warm-up: kernels, layouts
    torch.cuda.synchronize()
    caches = fresh(prompt_len + new_tokens)
    t0 = time.perf_counter()
    logits = model.forward(pd, caches, 0)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    toks = [logits.argmax(-1, keepdim=True)]
    t0 = time.perf_counter()
    pos = prompt_len
    for _ in range(new_tokens - 1):
        logits = model.forward(toks[-1], caches, pos)
        toks.append(logits.argmax(-1, keepdim=True))
        pos += 1
    torch.cuda.synchronize()
    eager_decode_s = time.perf_counter() - t0
    # the same prompt and decode with the decode steps replayed from one captured HIP graph
    gcaches = fresh(prompt_len + new_tokens)
    logits = model.forward(pd, gcaches, 0)
    torch.cuda.synchronize()
    gtoks = model.greedy_graph_from_logits(logits, prompt_len, new_tokens, gcaches, timed=True)
    decode_s = model.last_graph_decode_s
    assert torch.equal(gtoks.cpu(), torch.cat(toks, 1).cpu()), "graph decode diverged from eager decode"
    res = {"prompt": prompt_len, "new_tokens": new_tokens, "prefill_s": prefill_s, "prefill_tok_s": prompt_len / prefill_s,
           "decode_ms_per_token": decode_s * 1e3 / (new_tokens - 2), "decode_tok_s": (new_tokens - 2) / decode_s,
           "decode_mode": "device counters, graph-replayed steps (first decode step eager)",
           "eager_decode_ms_per_token": eager_decode_s * 1e3 / (new_tokens - 1),
           "retained_kv_bytes": int(sum(c.nbytes for c in caches)),
           "peak_hbm_bytes": int(torch.cuda.max_memory_allocated())}
    if cpu_agreement:
        swap_to_oracle(cpu_model, bcfg)
        match_gpu_rounding(cpu_model)
        torch.set_num_threads(_host_threads())
        gp = model.greedy(pd[:, :agree_prompt], agree_tokens, fresh(agree_prompt + agree_tokens)).cpu()
        # teacher-forced: both paths fed the reference's greedy tokens, logits compared per step
        gcache, ccache = fresh(agree_prompt + agree_tokens), [[] for _ in range(cfg.num_layers)]
        t0 = time.perf_counter()
        lc = cpu_model.forward(prompt[:, :agree_prompt], ccache, 0)
        lg = model.forward(pd[:, :agree_prompt], gcache, 0).cpu()
        cp, top1, diffs, margins, pos = [], [], [], [], agree_prompt
        for i in range(agree_tokens):
            tok = lc.argmax(-1, keepdim=True)
            cp.append(int(tok))
            top1.append(int(lg.argmax()) == int(tok))
            diffs.append(float((lg - lc).abs().max()))
            t2 = lc[0].topk(2).values
            margins.append(float(t2[0] - t2[1]))
            if i + 1 < agree_tokens:
                lc = cpu_model.forward(tok, ccache, pos)
                lg = model.forward(tok.to(dev), gcache, pos).cpu()
                pos += 1
        cpu_s = time.perf_counter() - t0
        same = [int(a) == b for a, b in zip(gp[0].tolist(), cp)]
        prefix = next((i for i, m in enumerate(same) if not m), len(same))
        decisive = [a for a, m, dd in zip(top1, margins, diffs) if m > 2 * dd]
        # up to the first free-running mismatch both runs hold the same tokens, so the teacher-forced
        # step there is the diverging step: the reference's top-2 margin against the logit noise
        first = None if prefix == len(same) else {
            "step": prefix, "reference_top2_margin": margins[prefix], "logit_max_abs_diff": diffs[prefix],
            "gpu_top1_is_reference_top1": top1[prefix],
            "near_tie": margins[prefix] <= 2 * diffs[prefix]}
        res["agreement"] = {"prompt": agree_prompt, "tokens": agree_tokens,
                            "cpu_rounding": "one-row 4-bit products from the codes in fp32 (as the GPU's decode "
                                            "steps), prefill products over the bf16-dequantised weights",
                            "free_running_match_rate": sum(same) / len(same), "identical_prefix": prefix,
                            "teacher_forced_top1_agreement": sum(top1) / len(top1),
                            "teacher_forced_top1_where_margin_exceeds_2x_noise":
                                (sum(decisive) / len(decisive)) if decisive else None,
                            "decisive_steps": len(decisive), "min_reference_top2_margin": min(margins),
                            "first_divergence": first,
                            "logit_max_abs_diff": max(diffs), "logit_std": float(lc.std()),
                            "gpu": gp[0].tolist(), "cpu": cp, "cpu_s": cpu_s,
                            "cpu_threads": torch.get_num_threads()}
    return res


def cpu_baseline(q, k, v, ref_lays, repeats=3, max_seconds=30.0):
    """The CPU oracle (PyTorch restatement of the reference Torch path) on the host cores."""
    import torch

    from oracle import attention as oa

    torch.set_num_threads(_host_threads())
    lay = ref_lays[3]
    T = q.shape[2]
    times = []
    t_start = time.perf_counter()
    oa.prefill(q, k, v, layout=lay, W=64)  # warmup
    for _ in range(repeats):
        t0 = time.perf_counter()
        oa.prefill(q, k, v, layout=lay, W=64)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > max_seconds:
            break
    med = statistics.median(times)
    return {"value": T / med, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"full cfg2 layer (T={T}, bf16, stage 3), 1 warmup + median of {len(times)}; "
                      f"{_cpu_model()}"}


def _timed(fn, repeats):
    fn()                                         # warmup
    ts = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), len(ts)


def cpu_baseline_cfg1(seed=0):
    """cfg1: fp32 prefill, T=4096, Hq8/Hkv2, d128, layers 0..4 (the CPU oracle, host cores)."""
    import torch

    from oracle import attention as oa, topology as tp

    g = torch.Generator().manual_seed(seed)
    T, hq, hkv, d = 4096, 8, 2, 128
    q, k, v = (torch.randn(1, h, T, d, generator=g) for h in (hq, hkv, hkv))
    per_layer = []
    for layer in range(5):
        lay = tp.build_layout(seq_len=T, block_size=128, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                              layer_idx=layer, local_window_blocks=1, sink_count=1, partner_count=1,
                              partner_rule="causal_shift")
        per_layer.append(_timed(lambda: oa.prefill(q, k, v, layout=lay, W=64), 3)[0])
    med = statistics.median(per_layer)
    return {"value": T / med, "unit": "tok/s", "ms_per_layer": med * 1e3, "cores": torch.get_num_threads(),
            "kind": "port", "sample": "full cfg1: fp32 T=4096 prefill, layers 0..4, 1 warmup + median of 3 each"}


def cpu_baseline_cfg3(torch_gpu, batches=(1, 8, 32), seed=0):
    """cfg3: one decode row per sequence at position 131072 through the CPU oracle's active rows,
    which recompute the block summaries over the full context every call as the reference's Torch
    active path does (bna/torch/attention_wayfinder_permute.py:1125-1197).  K/V are drawn on the
    GPU and copied to the host (drawing 10^9 normals on one host core would take longer than the
    measurement)."""
    import torch

    from oracle import attention as oa, topology as tp

    hq, hkv, d, ctx = 8, 2, 128, 131073
    lay = tp.build_layout(seq_len=ctx, block_size=128, num_key_value_heads=hkv, num_key_value_groups=hq // hkv,
                          layer_idx=3, local_window_blocks=1, sink_count=1, partner_count=1, partner_rule="causal_shift")
    g = torch_gpu.Generator(device="cuda:0").manual_seed(seed)
    out = {}
    for B in batches:
        k = torch_gpu.randn(B, hkv, ctx, d, generator=g, device="cuda:0").bfloat16().cpu()
        v = torch_gpu.randn(B, hkv, ctx, d, generator=g, device="cuda:0").bfloat16().cpu()
        q = torch_gpu.randn(B, hq, 1, d, generator=g, device="cuda:0").bfloat16().cpu()
        reps = 3 if B == 1 else 2 if B == 8 else 1
        med, n = _timed(lambda: oa.active(q, k, v, layout=lay, query_positions=torch.tensor([ctx - 1]), W=64), reps)
        out[str(B)] = {"ms_per_step": med * 1e3, "tok_s": B / med, "steps_timed": n}
        del k, v
    return {"value": out["32"]["tok_s"] if "32" in out else None, "unit": "tok/s (B=32)", "per_batch": out,
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": "one decode step per batch size at context 131072 (1 warmup + median of 3/2/1 for B=1/8/32); "
                      "summaries recomputed over the full context each step, as the reference's Torch active path"}


def cpu_baseline_cfg4(torch_gpu, seed=0, T=262144, chunk=384, samples=(1, 171, 341, 511, 682)):
    """cfg4: the reference's Torch chunked path on the CPU oracle -- chunk 0 one-shot, every later
    chunk the active rows over the full prefix (summaries recomputed per call, the Torch layer
    swap's cached branch, bna/integrations/qwen_torch.py:1400-1427).  A labelled sample: the
    listed chunks are timed once each and the per-chunk time, linear in the prefix length, is
    fitted and summed over all 683 chunks."""
    import torch

    from oracle import attention as oa, topology as tp

    hq, hkv, d = 16, 4, 256
    g = torch_gpu.Generator(device="cuda:0").manual_seed(seed)
    k = torch_gpu.randn(1, hkv, T, d, generator=g, device="cuda:0").bfloat16().cpu()
    v = torch_gpu.randn(1, hkv, T, d, generator=g, device="cuda:0").bfloat16().cpu()
    kw = dict(block_size=128, num_key_value_heads=hkv, num_key_value_groups=hq // hkv, layer_idx=5,
              local_window_blocks=1, sink_count=1, partner_count=1, partner_rule="causal_shift")
    q0 = torch_gpu.randn(1, hq, chunk, d, generator=g, device="cuda:0").bfloat16().cpu()
    lay0 = tp.build_layout(seq_len=chunk, **kw)
    t_first, _ = _timed(lambda: oa.prefill(q0, k[:, :, :chunk], v[:, :, :chunk], layout=lay0, W=64), 1)
    pts = []
    for c in samples:
        s0, e = c * chunk, min(T, (c + 1) * chunk)
        lay = tp.build_layout(seq_len=e, **kw)
        qc = torch_gpu.randn(1, hq, e - s0, d, generator=g, device="cuda:0").bfloat16().cpu()
        t0 = time.perf_counter()
        oa.active(qc, k[:, :, :e], v[:, :, :e], layout=lay, query_positions=torch.arange(s0, e), W=64)
        pts.append((e, time.perf_counter() - t0))
    n = len(pts)
    mx = sum(e for e, _ in pts) / n
    my = sum(t for _, t in pts) / n
    slope = sum((e - mx) * (t - my) for e, t in pts) / max(1e-9, sum((e - mx) ** 2 for e, _ in pts))
    icpt = my - slope * mx
    total = t_first + sum(icpt + slope * min(T, (c + 1) * chunk) for c in range(1, -(-T // chunk)))
    return {"value": T / total, "unit": "tok/s", "e2e_s_extrapolated": total, "first_chunk_s": t_first,
            "sampled_chunks": {str(c): round(t, 4) for c, (_, t) in zip(samples, pts)},
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"chunks {list(samples)} timed once each (plus the one-shot first chunk); per-chunk time "
                      "fitted linearly in the prefix length and summed over all 683 chunks (extrapolated)"}


def gpu_cfg1(torch, bf, seed=0, reps=20):
    """cfg1 on the GPU: the fp32 prefill (T=4096, layers 0..4), summaries + attention per layer."""
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    T, hq, hkv, d = 4096, 8, 2, 128
    q, k, v = (torch.randn(1, h, T, d, generator=g, device="cuda:0") for h in (hq, hkv, hkv))
    lays = [bf.build_block_butterfly_layout(seq_len=T, block_size=128, num_key_value_heads=hkv,
                                            num_key_value_groups=hq // hkv, layer_idx=layer, local_window_blocks=1,
                                            sink_count=1, partner_count=1, partner_rule="causal_shift")
            for layer in range(5)]
    for lay in lays:
        bf.compressed_butterfly_attention(q, k, v, layout=lay, local_window_tokens=64)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        bf.compressed_butterfly_attention(q, k, v, layout=lays[i % 5], local_window_tokens=64)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    # the same five layers captured once in a HIP graph: the GPU work without the host's dispatch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for lay in lays:
                bf.compressed_butterfly_attention(q, k, v, layout=lay, local_window_tokens=64)
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    replays = []
    for _ in range(5):
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        replays.append(e0.elapsed_time(e1) / len(lays))
    gms = statistics.median(replays)
    return {"ms_per_layer": gms, "tok_s": T / (gms / 1e3), "dtype": "f32",
            "mode": "graph-replayed layers 0..4 (compressor + fp32 attention kernel each), median of 5 replays",
            "eager_ms_per_layer": ms, "eager_mode": "eager calls, events around 20 calls"}


def hbm_ceiling(torch, nbytes: int = 1 << 30, reps: int = 10) -> dict:
    """Streaming rates of torch's own kernels over buffers 4x the 256 MB MALL:
    the practical ceilings the roofline fractions are read against."""
    src = torch.ones(nbytes // 2, dtype=torch.bfloat16, device="cuda:0")
    dst = torch.empty_like(src)
    cases = {
        "read_amax": (lambda: torch.amax(src), nbytes),
        "read_sum": (lambda: src.sum(dtype=torch.float32), nbytes),
        "write_fill": (lambda: dst.fill_(1.0), nbytes),
        "copy": (lambda: dst.copy_(src), 2 * nbytes),
    }
    out = {"bytes_per_buffer": nbytes, "reps": reps}
    for name, (fn, moved) in cases.items():
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / reps
        out[name + "_tbs"] = moved / sec / 1e12
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=45)
    ap.add_argument("--warmup", type=int, default=9)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-stream", action="store_true", help="skip the cfg4 streaming chunked-prefill leg")
    ap.add_argument("--no-model", action="store_true", help="skip the cfg5 swapped-decoder leg")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy (scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only time torch's streaming kernels (read-only reductions, fill, copy) on 1 GiB tensors")
    ap.add_argument("--decode-steps", type=int, default=0,
                    help="only run 64 eager device-counter decode steps at this batch size (counter collection)")
    ap.add_argument("--prefill-launches", type=int, default=0,
                    help="only run the cfg2 compressor once and this many prefill launches (counter collection)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (the hot path needs no collectives); "
                                   "run with --gpus 1"}), flush=True)
        sys.exit(2)
    import torch

    import butterfly_amd as bf
    from oracle import topology as tp

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP GPU visible"}), flush=True)
        sys.exit(1)
    if args.copy_calibration:
        src = torch.ones(128 << 20, dtype=torch.bfloat16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2,
                          "launches": args.steps}), flush=True)
        return
    if args.hbm_ceiling:
        print(json.dumps(hbm_ceiling(torch)), flush=True)
        return
    if args.prefill_launches:
        prefill_launches(args, torch, bf)
        return
    if args.decode_steps:
        decode_steps_only(args, torch, bf)
        return
    _log("cfg2 prefill leg")
    pre = bench_prefill(args, torch, bf, tp)
    q, k, v, ref_lays = pre.pop("inputs")
    _log("cfg1 fp32 leg")
    cfg1 = gpu_cfg1(torch, bf)
    decode = decode_sweep = stream = model = cpu = None
    if not args.no_decode:
        _log("cfg3 decode leg")
        decode = bench_decode(torch, bf)
        _log("cfg3 batch sweep leg")
        decode_sweep = bench_decode_sweep(torch, bf)
    if not args.no_stream:
        _log("cfg4 streaming leg")
        stream = bench_stream(torch, bf)
    if not args.no_model:
        _log("cfg5 decoder leg")
        model = bench_decoder(torch, bf, cpu_agreement=not args.no_cpu_baseline)
    if not args.no_cpu_baseline:
        _log("CPU baselines (cfg2, cfg1, cfg3, cfg4)")
        cpu = cpu_baseline(q, k, v, ref_lays)
        cpu["other_configs"] = {"cfg1": cpu_baseline_cfg1(), "cfg3": cpu_baseline_cfg3(torch),
                                "cfg4": cpu_baseline_cfg4(torch)}
    _log("done")
    line = {
        "metric": "prefill tok/s @64k (1 layer, bf16, 9-stage sweep)",
        "value": pre["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pre["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1), K channel-scaled U(0.5,2))",
        "config": {"workload": "cfg2: single Butterfly layer prefill, T=65536, Hq=8, Hkv=2, d=128, BS=128, W=64, "
                               "causal_shift, stages 0..8", "global_batch": 1, "seq_len": 65536,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": pre["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": pre["achieved_gbs"] / HBM_PEAK_GBS, "traffic": measured_traffic(),
                     "traffic_source": "profiles/prefill_cfg2_hbm_traffic.md (rocprofv3 --pmc, copy-calibrated)",
                     "kernel": "attn_mfma_kernel<128>", "kernel_ms_avg": pre["prefill_kernel_ms_avg"],
                     "kernel_ms_cold": pre["prefill_kernel_ms_cold"],
                     "achieved_cold": pre["prefill_bytes"] / (pre["prefill_kernel_ms_cold"] / 1e3) / 1e9,
                     "frac_cold": pre["prefill_bytes"] / (pre["prefill_kernel_ms_cold"] / 1e3) / 1e9 / HBM_PEAK_GBS,
                     "alg_bytes_per_launch": pre["prefill_bytes"],
                     "mfma_tflops": pre["achieved_tflops"],
                     "mfma_frac": pre["achieved_tflops"] / MFMA_BF16_PEAK_TFLOPS},
        "cpu_baseline": cpu,
        "extra": {"step_mode": "K steps (compressor + prefill each) in one HIP graph", "gpu_ms_per_step": pre["gpu_ms_per_step"],
                  "eager_ms_per_step": pre["eager_ms_per_step"],
                  "prefill_event_ms_in_step_avg": pre["prefill_event_ms_in_step_avg"],
                  "prefill_event_ms_in_step_min": pre["prefill_event_ms_in_step_min"],
                  "compress_alg_bytes": pre["compress_bytes"], "prefill_cfg1_f32": cfg1, "decode_cfg3": decode,
                  "decode_batch_sweep": decode_sweep,
                  "stream_cfg4": stream, "model_cfg5": model},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
