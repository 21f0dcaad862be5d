"""Benchmark of the paged attention hot path on one MI355X.

One step = the decode step of one attention layer at Qwen2.5-0.5B shape
(bf16_decode_qwen05b_b64: batch 64, 14 q / 2 KV heads, head_dim 64, block 16,
contexts U[128, 4096], 24576-block pool): the batched KV write of the 64 new
tokens through slot_mapping and the split-KV paged decode, one launch
(mlr_paged_decode_append: the write folded in, the splits merged in place).

Timing: inputs are resident in HBM. Consecutive steps use consecutive layers
of a 24-layer cache (24 distinct 201 MB K+V pools, 4.8 GB), so a layer's pool
is evicted from the 256 MB Infinity Cache (MALL) before it is read again and
the figure is an HBM figure. Exactly ``--steps`` steps are captured into one
HIP graph; after at least ``--warmup`` steps and 0.25 s of untimed replays of
it, one replay is bracketed by HIP events on its stream (with device
synchronisation on both sides). ``value`` is whole-step algorithmic bytes /
time; ``config.us_per_step_10_replays`` repeats the graph ten times as a
cross-check.

The roofline object is for that launch: its algorithmic bytes (K and V rows
of every context token, q, out, block ids, lengths, the written rows) over
its event-timed average duration, against the 8 TB/s HBM peak.

The CPU baselines time the oracle (a CPU restatement of the reference's
PyTorch path: write_slots + paged_attention_decode_batch_parallel, and
paged_attention_prefill_chunk_tiled) on the same inputs with all host cores:
the decode step above, fp32_decode_b4 (FP32, batch 4), and the chunk prefill.

Secondary objects: BF16 chunk prefill (8 x 512-token chunks on prefixes
U[0, 3584]) in TFLOP/s against the 2.5 PFLOP/s bf16 MFMA peak; the decode
step the serving runtime runs (rotary embedding, KV write and decode in one
launch) and the same step as two launches (fused pre-attention kernel, then
decode); the read floor of the decode step (config.read_floor: a read-only
pass over the same K/V rows through the same block tables,
mlr_paged_kv_read_floor); the 8 x 32K decode over rotated pools, with its
own read floor; the fused pre-attention step; the KV
write on its own (``kv_write``); the FP32 batch-4 decode step;
``reference_shapes``, the reference's own decode-kernel benchmark shape (one
request, 32 q / 8 KV heads, head_dim 128, 512 to 16384 tokens, bf16 and fp16)
beside its published latencies; ``decode_runtime``, the reference's own
full-model batched decode-step cases (Qwen2.5-0.5B shape, B=8 at contexts
288..512 and B=16 at 128, BF16 and FP32), eager and replayed from a HIP graph,
beside its published step times; and ``serving`` / ``serving_graphs``,
end-to-end continuous-batching steps of a random-init Qwen2.5-0.5B-shape model
in BF16 (workloads.qwen05b_serving: about 48 decodes + 2 x 1024-token
prefills per step, 128 steps after the warm-up), eager and with the decode
forward and repeated packed prefills replayed from HIP graphs. ``provenance`` names the sources and
library the numbers come from.

    python bench.py [--gpus 1] [--steps 240] [--warmup 48]

``--serving`` runs only the serving steps (eager; with ``--graphs``, the
decode forward and repeated prefills replayed from HIP graphs) and prints
their line.

``--profile`` launches the same kernels eagerly and untimed, for rocprofv3:
``--steps`` decode steps over the rotated layers, one decode without the
fused write and one one-launch served step per layer, the read floor per
layer, ten prefill calls, the
fused pre-attention kernel, the 8 x 32K decode, the FP32 batch-4 step, and a
plain 1 GiB device copy whose FETCH_SIZE / WRITE_SIZE counters calibrate the
traffic counters (the copy reads and writes exactly 1 GiB). With
``--contiguous-only`` it launches only the contiguous-placement comparators
of the decode step.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _path in (REPO, os.path.join(REPO, "mini-llm-runtime_amd")):
    if _path not in sys.path:
        sys.path.insert(0, _path)

METRIC = ("paged decode attn GB/s (% of HBM peak); "
          "chunk-prefill attn TFLOP/s (% MFMA)")
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_PEAK_TFLOPS = 157.3
LAYERS = 24


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=240)
    p.add_argument("--warmup", type=int, default=48)
    p.add_argument("--cpu-budget", type=float, default=20.0,
                   help="seconds of CPU-baseline work (bounded sample)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-pre-attention", action="store_true",
                   help="skip the fused pre-attention (bias + RoPE + KV write) timing")
    p.add_argument("--tokens-per-split", type=int, default=0)
    p.add_argument("--profile", action="store_true",
                   help="launch the kernels eagerly, untimed (for rocprofv3)")
    p.add_argument("--serving", action="store_true",
                   help="time only the end-to-end serving steps (qwen05b_serving, BF16)")
    p.add_argument("--graphs", action="store_true",
                   help="with --serving: replay the decode forward, and repeated packed "
                        "prefills, from HIP graphs")
    p.add_argument("--no-serving", action="store_true",
                   help="leave the serving steps out of the default run")
    p.add_argument("--no-contiguous", action="store_true",
                   help="leave out the contiguous-placement comparators of the decode step "
                        "(they launch the step's own kernel, which a kernel trace would "
                        "then lump with it)")
    p.add_argument("--contiguous-only", action="store_true",
                   help="with --profile: launch only the contiguous-placement comparators")
    return p.parse_args()


def warm_graph(graph, stream, min_replays=1, seconds=0.25):
    """Untimed replays of `graph`, at least `min_replays` and at least
    `seconds` of them, so the timed region starts with the shader clock
    already up; returns the number of replays."""
    import torch
    done = 0
    end = time.perf_counter() + seconds
    with torch.cuda.stream(stream):
        while done < min_replays or time.perf_counter() < end:
            for _ in range(4):
                graph.replay()
            done += 4
            torch.cuda.synchronize()
    return done


def timed_graph(graph, replays, stream):
    """Seconds for `replays` graph launches, bracketed by events on `stream`.

    CUDAGraph.replay() launches on the current stream, so the replays run
    inside `torch.cuda.stream(stream)`: events and kernels share one stream.
    """
    import torch
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3  # seconds


def sample_sclk(replay, seconds=1.5):
    """Shader clock while `replay()` keeps the GPU busy: `amd-smi metric
    --clock` polled from a second thread; the median, min and max over every
    sample of every XCD's gfx clock (MHz), and the part's maximum. None when
    amd-smi is absent or its output cannot be read."""
    import shutil
    import subprocess
    import threading

    import torch

    tool = shutil.which("amd-smi") or "/opt/rocm/bin/amd-smi"
    if not os.path.exists(tool):
        return None
    clocks, max_clk, stop = [], [], threading.Event()

    def poll():
        while not stop.is_set():
            try:
                res = subprocess.run([tool, "metric", "--clock", "--json"],
                                     capture_output=True, text=True, timeout=10)
                data = json.loads(res.stdout)
                gpu = (data["gpu_data"] if isinstance(data, dict) else data)[0]
                for name, clk in gpu["clock"].items():
                    if name.startswith("gfx_"):
                        clocks.append(float(clk["clk"]["value"]))
                        max_clk.append(float(clk["max_clk"]["value"]))
            except Exception:  # tool output not understood: report nothing
                return

    thread = threading.Thread(target=poll, daemon=True)
    thread.start()
    end = time.perf_counter() + seconds
    while time.perf_counter() < end:
        for _ in range(4):
            replay()
        torch.cuda.synchronize()
    stop.set()
    thread.join(timeout=15)
    if not clocks:
        return None
    return {"median": statistics.median(clocks), "min": min(clocks), "max": max(clocks),
            "part_max": max(max_clk), "samples": len(clocks),
            "source": "amd-smi metric --clock (gfx clock of every XCD), polled while "
                      "the workload's graph replays untimed"}


def contiguous_tables(wl, device):
    """Contiguous placements of a decode workload's K/V rows (the reference
    times dense attention on contiguous K/V beside its paged decode): the same
    context lengths with each sequence's blocks consecutive in the pool
    (bt_seq, with the new token's slots slots_seq), and the same token rows as
    one run of consecutive blocks (bt_flat, one sequence of ctx_flat tokens)."""
    import torch

    need = [-(-int(n) // 16) for n in wl.context_lens.tolist()]
    batch = len(need)
    starts = [sum(need[:b]) for b in range(batch)]
    bt_seq = torch.full_like(wl.block_tables, -1)
    for b, (s0, n) in enumerate(zip(starts, need)):
        bt_seq[b, :n] = torch.arange(s0, s0 + n)
    slots_seq = torch.tensor([int(bt_seq[b, (n - 1) // 16]) * 16 + (n - 1) % 16
                              for b, n in enumerate(wl.context_lens.tolist())])
    total_tokens = int(wl.context_lens.sum())
    bt_flat = torch.arange(-(-total_tokens // 16)).unsqueeze(0)
    ctx_flat = torch.tensor([total_tokens])
    return tuple(t.to(device) for t in (bt_seq, slots_seq, bt_flat, ctx_flat))


def profile_run(args, device):
    """Eager, untimed launches of the benchmarked kernels (for rocprofv3)."""
    import torch

    from mini_llm_runtime_amd import workloads
    from mini_llm_runtime_amd.kernels import paged_attention as kpa
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache

    wl = workloads.bf16_decode_qwen05b_b64()
    nb = wl.k_cache.shape[0]
    cache = PagedKVCache(LAYERS, nb, 16, 2, 64, dtype=torch.bfloat16, device=device)
    for layer in range(LAYERS):
        cache.k_cache[layer].copy_(wl.k_cache.to(device))
        cache.v_cache[layer].copy_(wl.v_cache.to(device))
    q, bt, ctx = wl.q.to(device), wl.block_tables.to(device), wl.context_lens.to(device)
    slots, new_k, new_v = (t.to(device) for t in (wl.slot_mapping, wl.new_k, wl.new_v))
    out = torch.empty_like(q)
    ws = torch.zeros(kpa.decode_workspace_bytes(64, 14, 64, bt.shape[1] * 16, torch.bfloat16),
                     dtype=torch.uint8, device=device)
    if args.contiguous_only:
        # The decode step on per-sequence contiguous blocks, the read floor
        # on those tables, and the read floor over the same rows as one run.
        bt_seq, slots_seq, bt_flat, ctx_flat = contiguous_tables(wl, device)
        seq_out = torch.empty(64 * -(-bt.shape[1] * 16 // 96), dtype=torch.int32, device=device)
        flat_out = torch.empty(-(-bt_flat.shape[1] * 16 // 96), dtype=torch.int32,
                               device=device)
        for i in range(args.steps):
            k_layer, v_layer = cache.get_layer_cache(i % LAYERS)
            kpa.paged_decode_launch(q, k_layer, v_layer, bt_seq, ctx, out, workspace=ws,
                                    new_k=new_k, new_v=new_v, slot_mapping=slots_seq)
        for i in range(args.steps):
            k_layer, v_layer = cache.get_layer_cache(i % LAYERS)
            kpa.paged_kv_read_floor(k_layer, v_layer, bt_seq, ctx, tokens_per_item=96,
                                    out=seq_out)
        for i in range(args.steps):
            k_layer, v_layer = cache.get_layer_cache(i % LAYERS)
            kpa.paged_kv_read_floor(k_layer, v_layer, bt_flat, ctx_flat, tokens_per_item=96,
                                    out=flat_out)
        torch.cuda.synchronize()
        print(f"profile: {args.steps} each of the contiguous-block step, the contiguous-block "
              "read floor and the one-run read floor", flush=True)
        return
    for i in range(args.steps):
        k_layer, v_layer = cache.get_layer_cache(i % LAYERS)
        kpa.paged_decode_launch(q, k_layer, v_layer, bt, ctx, out, workspace=ws, new_k=new_k,
                                new_v=new_v, slot_mapping=slots)
    # The decode without the fused write (the two-launch step's decode; its
    # own instantiation, one workgroup per pair of KV heads).
    for i in range(LAYERS):
        k_layer, v_layer = cache.get_layer_cache(i)
        kpa.paged_decode_launch(q, k_layer, v_layer, bt, ctx, out, workspace=ws)
    # The served step in one launch (rotary embedding + KV write + decode:
    # mlr_paged_decode_qkv, its own instantiation).
    from mini_llm_runtime_amd.kernels import pre_attention as kpre
    from mini_llm_runtime_amd.model.qwen2_attention import Qwen2RotaryEmbedding
    gen = torch.Generator().manual_seed(64)
    qkv = torch.randn(64, 18 * 64, generator=gen).to(torch.bfloat16).to(device)
    inv_freq = Qwen2RotaryEmbedding(64, 1_000_000.0).inv_freq.to(device)
    for i in range(LAYERS):
        kpre.qkv_rope_decode(qkv, inv_freq, cache, i % LAYERS, slots, bt, ctx, 14, out=out,
                             workspace=ws)
    floor_out = torch.empty(64 * -(-bt.shape[1] * 16 // 96), dtype=torch.int32, device=device)
    for i in range(LAYERS):
        k_layer, v_layer = cache.get_layer_cache(i)
        kpa.paged_kv_read_floor(k_layer, v_layer, bt, ctx, tokens_per_item=96, out=floor_out)
    torch.cuda.synchronize()
    print(f"profile: {args.steps} decode steps, {LAYERS} decode-only steps, {LAYERS} one-launch "
          f"served steps, {LAYERS} read-floor passes (96-token items)", flush=True)
    del cache
    if not args.no_prefill:
        pw = workloads.bf16_prefill_chunk512_x8()
        kc, vc = pw.k_cache.clone(), pw.v_cache.clone()
        kc.view(-1, 2, 64).index_copy_(0, pw.slot_mapping, pw.chunk_k)
        vc.view(-1, 2, 64).index_copy_(0, pw.slot_mapping, pw.chunk_v)
        kc, vc, pq = kc.to(device), vc.to(device), pw.q.to(device)
        pbt, qsl, pctx = (t.to(device) for t in (pw.block_tables, pw.query_start_loc,
                                                  pw.context_lens))
        pout = torch.empty_like(pq)
        for _ in range(10):
            kpa.paged_prefill_launch(pq, kc, vc, pbt, qsl, pctx, 512, tile_size=64, out=pout)
        torch.cuda.synchronize()
        print("profile: 10 prefill calls", flush=True)
    if not args.no_pre_attention:
        from mini_llm_runtime_amd.kernels import pre_attention as kpre
        from mini_llm_runtime_amd.model.qwen2_attention import Qwen2RotaryEmbedding
        pcache = PagedKVCache(1, 4096, 16, 2, 64, dtype=torch.bfloat16, device=device)
        inv_freq = Qwen2RotaryEmbedding(64, 1_000_000.0).inv_freq.to(device)
        gen = torch.Generator().manual_seed(2048)
        qkv = torch.randn(2048, 18 * 64, generator=gen).to(torch.bfloat16).to(device)
        pos = torch.randint(0, 4096, (2048,), generator=gen).to(device)
        pslots = torch.randperm(4096 * 16, generator=gen)[:2048].to(device)
        for _ in range(20):
            kpre.qkv_rope_write(qkv, pos, inv_freq, pcache, 0, pslots, 14)
        # Duration against token count (told apart by grid size in the trace).
        for tokens in (1, 48, 512, 8192, 32768):
            g = torch.Generator().manual_seed(tokens)
            x = torch.randn(tokens, 18 * 64, generator=g).to(torch.bfloat16).to(device)
            p_t = torch.randint(0, 4096, (tokens,), generator=g).to(device)
            s_t = torch.randint(0, 4096 * 16, (tokens,), generator=g).to(device)
            for _ in range(10):
                kpre.qkv_rope_write(x, p_t, inv_freq, pcache, 0, s_t, 14)
        torch.cuda.synchronize()
        print("profile: 20 fused pre-attention calls (2048 tokens), 10 each at "
              "1/48/512/8192/32768 tokens", flush=True)
    # 8 x 32K decode over rotated pools (its own kernel instantiation).
    lw = workloads.bf16_decode_qwen7b_32k()
    pools = [(lw.k_cache.to(device), lw.v_cache.to(device)) for _ in range(POOLS_32K)]
    lq, lbt, lctx = lw.q.to(device), lw.block_tables.to(device), lw.context_lens.to(device)
    lslots, lnk, lnv = (t.to(device) for t in (lw.slot_mapping, lw.new_k, lw.new_v))
    lout = torch.empty_like(lq)
    lws = torch.zeros(kpa.decode_workspace_bytes(8, 28, 128, lbt.shape[1] * 16, torch.bfloat16),
                      dtype=torch.uint8, device=device)
    for i in range(12):
        lkc, lvc = pools[i % POOLS_32K]
        kpa.paged_decode_launch(lq, lkc, lvc, lbt, lctx, lout, workspace=lws, new_k=lnk,
                                new_v=lnv, slot_mapping=lslots)
    torch.cuda.synchronize()
    print(f"profile: 12 decode calls of {lw.name} over {POOLS_32K} pools", flush=True)
    del pools
    # The FP32 batch-4 decode step (write folded in, one launch).
    fw = workloads.fp32_decode_b4()
    fkc, fvc = fw.k_cache.to(device), fw.v_cache.to(device)
    fq, fbt, fctx = fw.q.to(device), fw.block_tables.to(device), fw.context_lens.to(device)
    fslots, fnk, fnv = (t.to(device) for t in (fw.slot_mapping, fw.new_k, fw.new_v))
    fout = torch.empty_like(fq)
    fws = torch.zeros(kpa.decode_workspace_bytes(4, 14, 64, fbt.shape[1] * 16, torch.float32),
                      dtype=torch.uint8, device=device)
    for _ in range(20):
        kpa.paged_decode_launch(fq, fkc, fvc, fbt, fctx, fout, workspace=fws, new_k=fnk,
                                new_v=fnv, slot_mapping=fslots)
    torch.cuda.synchronize()
    print(f"profile: 20 {fw.name} steps", flush=True)
    src = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("profile: 3 copies of 1 GiB", flush=True)


def check_decode_outputs(kpa, workspace, out, stream, what):
    """A split merge that gave up waiting writes only NaN. After a timed
    region, the workspace's merge-failure flag (mlr_paged_decode_workspace_check,
    which raises DecodeMergeError) and the last outputs must be clean."""
    import torch

    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        kpa.check_workspace(workspace)
    if not bool(torch.isfinite(out).all()):
        raise RuntimeError(f"{what}: non-finite decode outputs after the timed region")


def bench_decode(args, device):
    import torch

    from mini_llm_runtime_amd import workloads
    from mini_llm_runtime_amd.kernels import paged_attention as kpa
    from mini_llm_runtime_amd.kernels import pre_attention as kpre
    from mini_llm_runtime_amd.model.qwen2_attention import Qwen2RotaryEmbedding
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache

    wl = workloads.bf16_decode_qwen05b_b64()
    nb = wl.k_cache.shape[0]
    cache = PagedKVCache(LAYERS, nb, 16, 2, 64, dtype=torch.bfloat16, device=device)
    layer0_k, layer0_v = wl.k_cache.to(device), wl.v_cache.to(device)
    for layer in range(LAYERS):
        cache.k_cache[layer].copy_(layer0_k)
        cache.v_cache[layer].copy_(layer0_v)
    del layer0_k, layer0_v
    q = wl.q.to(device)
    bt = wl.block_tables.to(device)
    ctx = wl.context_lens.to(device)
    slots = wl.slot_mapping.to(device)
    new_k, new_v = wl.new_k.to(device), wl.new_v.to(device)
    out = torch.empty_like(q)
    ts = args.tokens_per_split
    ws_bytes = kpa.decode_workspace_bytes(64, 14, 64, bt.shape[1] * 16, torch.bfloat16, ts)
    workspace = torch.zeros(ws_bytes, dtype=torch.uint8, device=device)
    # The step the serving runtime runs (Qwen2Attention.forward_decode_batch_with_cache):
    # the fused pre-attention kernel (bias-free projection output -> rotated q,
    # rotated k and v written to the cache), then the decode without the
    # append. Synthetic projection output of the 64 tokens.
    gen = torch.Generator().manual_seed(64)
    qkv = torch.randn(64, 18 * 64, generator=gen).to(torch.bfloat16).to(device)
    positions = (ctx - 1).contiguous()
    inv_freq = Qwen2RotaryEmbedding(64, 1_000_000.0).inv_freq.to(device)
    q_rot = torch.empty_like(q)
    floor_items = (64, 96, 160, 320)
    floor_out = torch.empty(64 * -(-bt.shape[1] * 16 // min(floor_items)), dtype=torch.int32,
                            device=device)
    # Contiguous comparators of the same step and rows.
    bt_seq, slots_seq, bt_flat, ctx_flat = contiguous_tables(wl, device)
    flat_out = torch.empty(-(-bt_flat.shape[1] * 16 // 96), dtype=torch.int32, device=device)

    def step(layer, kind="step"):
        k_layer, v_layer = cache.get_layer_cache(layer)
        if kind == "step":      # KV write folded into the decode (mlr_paged_decode_append)
            kpa.paged_decode_launch(q, k_layer, v_layer, bt, ctx, out, tokens_per_split=ts,
                                    workspace=workspace, new_k=new_k, new_v=new_v,
                                    slot_mapping=slots)
        elif kind == "decode":  # decode only
            kpa.paged_decode_launch(q, k_layer, v_layer, bt, ctx, out,
                                    tokens_per_split=ts, workspace=workspace)
        elif kind == "contig":  # the step on per-sequence contiguous blocks
            kpa.paged_decode_launch(q, k_layer, v_layer, bt_seq, ctx, out, tokens_per_split=ts,
                                    workspace=workspace, new_k=new_k, new_v=new_v,
                                    slot_mapping=slots_seq)
        elif kind == "floor_seq":  # read floor on per-sequence contiguous blocks
            kpa.paged_kv_read_floor(k_layer, v_layer, bt_seq, ctx, tokens_per_item=96,
                                    out=floor_out)
        elif kind == "floor_flat":  # the same rows as one contiguous run
            kpa.paged_kv_read_floor(k_layer, v_layer, bt_flat, ctx_flat, tokens_per_item=96,
                                    out=flat_out)
        elif kind.startswith("floor"):  # read-only pass over the same K/V rows
            kpa.paged_kv_read_floor(k_layer, v_layer, bt, ctx,
                                    tokens_per_item=int(kind[5:]), out=floor_out)
        elif kind == "served1":  # served step in one launch (mlr_paged_decode_qkv)
            kpre.qkv_rope_decode(qkv, inv_freq, cache, layer, slots, bt, ctx, 14, out=out,
                                 tokens_per_split=ts, workspace=workspace)
        else:                   # served pair
            kpre.qkv_rope_write(qkv, positions, inv_freq, cache, layer, slots, 14, out=q_rot)
            kpa.paged_decode_launch(q_rot, k_layer, v_layer, bt, ctx, out,
                                    tokens_per_split=ts, workspace=workspace)

    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for layer in range(LAYERS):   # eager warm-up: loads code objects
            step(layer)
            step(layer, "served")
            step(layer, "served1")
    torch.cuda.current_stream(device).wait_stream(stream)
    torch.cuda.synchronize()

    def capture(kind, n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n):
                step(i % LAYERS, kind)
        return g

    # The headline: exactly --steps steps (consecutive layers, so the MALL
    # never serves a layer twice) in one graph, after at least --warmup steps
    # and at least 0.25 s of untimed replays of it; one bracketed replay.
    steps = max(1, args.steps)
    g_steps = capture("step", steps)
    warm = warm_graph(g_steps, stream, max(1, -(-args.warmup // steps)))
    t_step = timed_graph(g_steps, 1, stream)
    # A larger sample of the same graph (10 replays) as a cross-check.
    t_step10 = timed_graph(g_steps, 10, stream) / 10
    contiguous = () if args.no_contiguous else ("contig", "floor_seq", "floor_flat")
    graphs = {kind: capture(kind, LAYERS)
              for kind in ("decode", "served", "served1", *contiguous,
                           *(f"floor{n}" for n in floor_items))}
    res = {}
    for kind, g in graphs.items():
        warm_graph(g, stream)
        res[kind] = timed_graph(g, 10, stream) / (10 * LAYERS)
    sclk = sample_sclk(g_steps.replay)
    g_steps.replay()  # the last graph to write `out` is the timed step's
    check_decode_outputs(kpa, workspace, out, stream, wl.name)
    decode_bytes = wl.algorithmic_bytes()
    step_bytes = decode_bytes + wl.write_bytes()
    sec_per_step = t_step / steps
    # The read floor: every context token's K and V rows read through the
    # same block tables (mlr_paged_kv_read_floor), no compute, best item size.
    kv_bytes = int(wl.context_lens.sum()) * 2 * 2 * 64 * 2
    floor_us = {n: res[f"floor{n}"] * 1e6 for n in floor_items}
    best = min(floor_us, key=floor_us.get)
    read_floor = {
        "kernel": "mlr_paged_kv_read_floor (kv_read_floor_kernel): read-only pass over the "
                  "step's K/V rows through the same block tables, XOR checksum",
        "kv_bytes": kv_bytes,
        "us_by_tokens_per_item": {str(n): round(v, 3) for n, v in floor_us.items()},
        "us": round(floor_us[best], 3),
        "GBps": round(kv_bytes / (floor_us[best] * 1e-6) / 1e9, 1),
        "frac_of_hbm_peak": round(kv_bytes / (floor_us[best] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "step_us_over_floor_us": round(sec_per_step * 1e6 / floor_us[best], 3),
        "contiguous": None if args.no_contiguous else {
            "what": "the same step and the same K/V rows with contiguous placement: "
                    "step_us = mlr_paged_decode_append with each sequence's blocks consecutive "
                    "in the pool; floor_seq_us = the read floor on those tables (96-token "
                    "items); floor_flat_us = the read floor over the same number of token "
                    "rows as one run of consecutive blocks (one sequence)",
            "step_us": round(res["contig"] * 1e6, 3),
            "floor_seq_us": round(res["floor_seq"] * 1e6, 3),
            "floor_flat_us": round(res["floor_flat"] * 1e6, 3),
            "floor_flat_frac_of_hbm_peak": round(
                kv_bytes / res["floor_flat"] / 1e9 / HBM_PEAK_GBS, 4),
        },
    }
    return {
        "wl": wl,
        "steps": steps,
        "warmup": warm * steps,
        "ms_per_step": sec_per_step * 1e3,
        "value_gbs": step_bytes / sec_per_step / 1e9,
        "us_per_step_10_replays": t_step10 / steps * 1e6,
        "decode_us": res["decode"] * 1e6,
        "decode_gbs": decode_bytes / res["decode"] / 1e9,
        "served_us": res["served"] * 1e6,
        "served1_us": res["served1"] * 1e6,
        "read_floor": read_floor,
        "decode_bytes": decode_bytes,
        "step_bytes": step_bytes,
        "stream": stream,
        "sclk": sclk,
    }


def bench_prefill(device, reps=5, calls_per_graph=10, dtype=None):
    """bf16_prefill_chunk512_x8 through mlr_paged_prefill (varlen, one launch
    per call). The call passes the reference's tile_size (64); it only orders
    the FP32 accumulation, and the matrix-core kernel steps by its own 64-key
    tile whatever it is, so there is one timing: the median over `reps`
    bracketed replays of a graph of `calls_per_graph` calls. `dtype` runs the
    same inputs cast to another type (fp16)."""
    import torch

    from mini_llm_runtime_amd import workloads
    from mini_llm_runtime_amd.kernels import paged_attention as kpa

    wl = workloads.bf16_prefill_chunk512_x8()
    kc, vc = wl.k_cache.clone(), wl.v_cache.clone()
    kc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.chunk_k)
    vc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.chunk_v)
    dtype = dtype or wl.q.dtype
    kc, vc = kc.to(device, dtype), vc.to(device, dtype)
    q = wl.q.to(device, dtype)
    bt, qsl, ctx = (t.to(device) for t in (wl.block_tables, wl.query_start_loc,
                                            wl.context_lens))
    out = torch.empty_like(q)

    def call():
        kpa.paged_prefill_launch(q, kc, vc, bt, qsl, ctx, 512, tile_size=64, out=out)

    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        call()
    torch.cuda.synchronize()
    # Several back-to-back calls per graph (as consecutive layers run), so
    # the per-call time is the kernel's, not the graph launch's.
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(calls_per_graph):
            call()
    warm_graph(g, stream)
    times = [timed_graph(g, 1, stream) / calls_per_graph for _ in range(reps)]
    secs = statistics.median(times)
    sclk = sample_sclk(g.replay)
    flops = wl.causal_flops()
    return {
        "workload": "bf16_prefill_chunk512_x8",
        "flops_per_call": flops,
        "us_per_call": round(secs * 1e6, 3),
        "us_per_call_min_max": [round(min(times) * 1e6, 3), round(max(times) * 1e6, 3)],
        "tflops": flops / secs / 1e12,
        "wl": wl,
        "sclk": sclk,
    }


def bench_pre_attention(device, reps=4, calls_per_graph=100):
    """The step before attention at a Qwen2.5-0.5B layer (hidden 896, 14/2
    heads, head_dim 64, BF16) for a decode batch (48 tokens) and a prefill
    step (2048 tokens): the fused mlr_qkv_rope_write kernel alone, the fused
    step (one GEMM over the concatenated projections + the kernel), and the
    reference's unfused sequence (three projection GEMMs, rotary embedding in
    PyTorch ops, then the KV write).

    Each figure is the event-timed average over `reps` replays of a graph of
    `calls_per_graph` calls: long enough that the host's graph launches keep
    ahead of the GPU (with 10-call graphs they do not, and the per-call time
    grows by ~2 us). `graph_node_us` is the same measurement for a one-element
    fill kernel: the per-launch cost a graph node adds, which the `_net`
    figures subtract. `same_bytes_elementwise_us` times a PyTorch elementwise
    kernel that reads the projection output and writes a tensor of its size
    (torch.mul(qkv, 1, out=...)): about the bytes the fused kernel moves, with
    no rotation, scatter or position loads, as a comparator."""
    import types

    import torch

    from mini_llm_runtime_amd.kernels import pre_attention as kpre
    from mini_llm_runtime_amd.model.qwen2_attention import Qwen2Attention
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache

    cfg = types.SimpleNamespace(hidden_size=896, num_attention_heads=14, num_key_value_heads=2,
                                head_dim=64, rope_theta=1_000_000.0)
    torch.manual_seed(0)
    attn = Qwen2Attention(cfg).to(device=device, dtype=torch.bfloat16)
    cache = PagedKVCache(1, 4096, 16, 2, 64, dtype=torch.bfloat16, device=device)
    inv_freq = attn.rotary_embedding.inv_freq
    bytes_per_token = 2 * (14 + 2 * 2) * 64 + 2 * 14 * 64 + 2 * 2 * 2 * 64 + 8 + 8
    stream = torch.cuda.Stream(device)

    def graph_us(fn):
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(calls_per_graph):
                fn()
        warm_graph(g, stream, seconds=0.25)
        return timed_graph(g, reps, stream) / (reps * calls_per_graph) * 1e6

    node = torch.zeros(1, device=device)
    node_us = graph_us(lambda: node.zero_())
    out = {}
    for tokens in (48, 2048):
        gen = torch.Generator().manual_seed(tokens)
        hidden = torch.randn(tokens, 896, generator=gen).to(torch.bfloat16).to(device)
        positions = torch.randint(0, 4096, (tokens,), generator=gen).to(device)
        slots = torch.randperm(cache.num_blocks * 16, generator=gen)[:tokens].to(device)
        weight, bias = attn._qkv_weights()
        qkv = torch.nn.functional.linear(hidden, weight, bias)

        def kernel():
            kpre.qkv_rope_write(qkv, positions, inv_freq, cache, 0, slots, 14)

        def fused():
            attn._fused_qkv_rope_write(hidden, positions, cache, 0, slots)

        def unfused():
            _, k, v = attn._qkv_rope(hidden.unsqueeze(0), positions.unsqueeze(0))
            cache.write_slots(slots, k[0], v[0], 0, validate=False)

        k_us = graph_us(kernel)
        dst = torch.empty_like(qkv)
        copy_us = graph_us(lambda: torch.mul(qkv, 1, out=dst))
        out[str(tokens)] = {
            "fused_kernel_us": round(k_us, 3),
            "fused_kernel_net_us": round(k_us - node_us, 3),
            "fused_step_us": round(graph_us(fused), 3),
            "unfused_step_us": round(graph_us(unfused), 3),
            "kernel_bytes": tokens * bytes_per_token,
            "kernel_GBps": round(tokens * bytes_per_token / k_us / 1e3, 1),
            "kernel_net_GBps": round(tokens * bytes_per_token / (k_us - node_us) / 1e3, 1),
            "same_bytes_elementwise_us": round(copy_us, 3),
            "same_bytes_elementwise_bytes": 2 * qkv.numel() * qkv.element_size(),
        }
    big = out["2048"]
    return {
        "workload": "qwen05b_layer_pre_attention_bf16",
        "calls_per_graph": calls_per_graph,
        "graph_node_us": round(node_us, 3),
        "by_tokens": out,
        "roofline": {"bound": "hbm", "kernel": "mlr_qkv_rope_write (2048 tokens)",
                     "achieved": big["kernel_GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(big["kernel_GBps"] / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes_per_launch": big["kernel_bytes"]},
    }


def bench_kv_write(device, reps=4, calls_per_graph=100):
    """PagedKVCache.write_slots on its own (mlr_kv_write, BF16 into a BF16 layer
    pool of 24,576 blocks x 16 slots, Qwen2.5-0.5B KV heads): 64 tokens, the
    decode step's write, and 4096 tokens, the eight 512-token chunks of the
    chunk-prefill workload; distinct random slots. Timed like the
    pre-attention leg (graphs of `calls_per_graph` calls), with the graph
    node's own cost (a one-element fill) beside it. Algorithmic bytes per
    call: 2 T Hkv D (2 + 2) + 8 T (K and V read and written, int64 slots)."""
    import torch

    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache

    hkv, d = 2, 64
    cache = PagedKVCache(1, 24576, 16, hkv, d, dtype=torch.bfloat16, device=device)
    stream = torch.cuda.Stream(device)

    def graph_us(fn):
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(calls_per_graph):
                fn()
        warm_graph(g, stream, seconds=0.25)
        return timed_graph(g, reps, stream) / (reps * calls_per_graph) * 1e6

    node = torch.zeros(1, device=device)
    node_us = graph_us(lambda: node.zero_())
    out = {}
    for tokens in (64, 4096):
        gen = torch.Generator().manual_seed(tokens)
        k = torch.randn(tokens, hkv, d, generator=gen).to(torch.bfloat16).to(device)
        v = torch.randn(tokens, hkv, d, generator=gen).to(torch.bfloat16).to(device)
        slots = torch.randperm(cache.num_blocks * 16, generator=gen)[:tokens].to(device)
        us = graph_us(lambda: cache.write_slots(slots, k, v, 0, validate=False))
        nbytes = 2 * tokens * hkv * d * (2 + 2) + 8 * tokens
        out[str(tokens)] = {"us": round(us, 3), "net_us": round(us - node_us, 3),
                            "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1)}
    del cache
    return {"workload": "kv_write_qwen05b_bf16", "calls_per_graph": calls_per_graph,
            "graph_node_us": round(node_us, 3), "by_tokens": out,
            "note": "latency-bound: at 64 tokens a call costs about one graph node; "
                    "every call rewrites the same rows from the same sources, which stay "
                    "in the 256 MB MALL, so GBps is a cache figure, not an HBM one; in "
                    "the decode step the write runs inside the decode launch "
                    "(mlr_paged_decode_append)"}


SPLITS_32K = (0, 4, 8, 16, 32, 64)
POOLS_32K = 3


def bench_decode_32k(device, reps=4, calls_per_graph=6):
    """Long-context split-KV decode, bf16_decode_qwen7b_32k: 8 sequences of
    32,768 tokens, 28 q / 4 KV heads, head_dim 128, with the step's KV write
    folded in. Consecutive calls rotate over POOLS_32K copies of the 537 MB
    K/V pool (1.6 GB in all, beyond the 256 MB MALL), so every call reads
    HBM. Swept over 4/8/16/32/64 splits per sequence and the library's
    default split size."""
    import torch

    from mini_llm_runtime_amd import workloads
    from mini_llm_runtime_amd.kernels import paged_attention as kpa

    wl = workloads.bf16_decode_qwen7b_32k()
    pools = [(wl.k_cache.to(device), wl.v_cache.to(device)) for _ in range(POOLS_32K)]
    q, bt, ctx = wl.q.to(device), wl.block_tables.to(device), wl.context_lens.to(device)
    slots, new_k, new_v = (t.to(device) for t in (wl.slot_mapping, wl.new_k, wl.new_v))
    out = torch.empty_like(q)
    stream = torch.cuda.Stream(device)
    nbytes = wl.algorithmic_bytes() + wl.write_bytes()
    sweep = {}
    for splits in SPLITS_32K:
        ts = 0 if splits == 0 else 32768 // splits
        ws = torch.zeros(kpa.decode_workspace_bytes(8, 28, 128, bt.shape[1] * 16,
                                                    torch.bfloat16, ts),
                         dtype=torch.uint8, device=device)

        def step(i):
            kc, vc = pools[i % POOLS_32K]
            kpa.paged_decode_launch(q, kc, vc, bt, ctx, out, tokens_per_split=ts,
                                    workspace=ws, new_k=new_k, new_v=new_v,
                                    slot_mapping=slots)

        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(stream):
            for i in range(POOLS_32K):
                step(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(calls_per_graph):
                step(i)
        warm_graph(g, stream)
        us = timed_graph(g, reps, stream) / (reps * calls_per_graph) * 1e6
        check_decode_outputs(kpa, ws, out, stream, f"{wl.name} ({splits} splits)")
        sweep["default" if splits == 0 else str(splits)] = round(us, 2)
    best = min(sweep, key=sweep.get)
    best_us = sweep[best]

    # Read floor of the same step: a read-only pass over the same K/V rows
    # through the same block tables and rotated pools, 512-token items (the
    # floor kernel's best item size at this length).
    floor_items = 512
    floor_out = torch.empty(8 * -(-bt.shape[1] * 16 // floor_items), dtype=torch.int32,
                            device=device)

    def floor_step(i):
        kc, vc = pools[i % POOLS_32K]
        kpa.paged_kv_read_floor(kc, vc, bt, ctx, tokens_per_item=floor_items, out=floor_out)

    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for i in range(POOLS_32K):
            floor_step(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(calls_per_graph):
            floor_step(i)
    warm_graph(g, stream)
    floor_us = timed_graph(g, reps, stream) / (reps * calls_per_graph) * 1e6
    kv_bytes = wl.algorithmic_bytes()
    return {"workload": wl.name, "step_bytes": nbytes, "pools_rotated": POOLS_32K,
            "us_by_splits": sweep, "best": best,
            "read_floor": {"tokens_per_item": floor_items, "us": round(floor_us, 2),
                           "GBps": round(kv_bytes / floor_us / 1e3, 1),
                           "frac_of_hbm_peak": round(kv_bytes / floor_us / 1e3 / HBM_PEAK_GBS, 4),
                           "step_over_floor": round(sweep["default"] / floor_us, 3)},
            "GBps_default": round(nbytes / sweep["default"] / 1e3, 1),
            "frac_of_hbm_peak_default": round(nbytes / sweep["default"] / 1e3 / HBM_PEAK_GBS, 4),
            "GBps_best": round(nbytes / best_us / 1e3, 1),
            "frac_of_hbm_peak_best": round(nbytes / best_us / 1e3 / HBM_PEAK_GBS, 4)}


# The reference's published split-KV decode latencies (one request, Triton,
# fp16, RTX 5070 Ti Laptop GPU): benchmarks/results/paged_attention/
# seq_scaling.csv:2-7, split_kernel_ms.
REFERENCE_SPLIT_KV_US = {512: 18.21, 1024: 22.30, 2048: 31.94, 4096: 48.80, 8192: 83.30,
                         16384: 169.70}


def bench_reference_shapes(device, reps=3):
    """The reference's own decode benchmark shape
    (benchmarks/benchmark_paged_attention.py:206-210: one request, 32 q / 8 KV
    heads, head_dim 128, block 16) at the sequence lengths it publishes, on
    this library's decode (mlr_paged_decode, default split), in bf16 and in
    fp16 (the reference's default dtype), both on the matrix-core kernel. Each call reads one of enough copies of the K/V pool to exceed
    the 256 MB MALL, so every call reads HBM, as the reference's do_bench
    flushes its cache between calls."""
    import math

    import torch

    from mini_llm_runtime_amd.kernels import paged_attention as kpa

    hq, hkv, d, bs = 32, 8, 128, 16
    stream = torch.cuda.Stream(device)
    out = {}
    for dtype, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        by_len = {}
        for seq in REFERENCE_SPLIT_KV_US:
            nb = seq // bs
            gen = torch.Generator().manual_seed(seq)
            pool_bytes = 2 * nb * bs * hkv * d * 2
            copies = min(256, max(2, math.ceil(600e6 / pool_bytes)))
            k = torch.randn(nb, bs, hkv, d, generator=gen).to(device=device, dtype=dtype)
            v = torch.randn(nb, bs, hkv, d, generator=gen).to(device=device, dtype=dtype)
            pools = [(k.clone(), v.clone()) for _ in range(copies)]
            del k, v
            q = torch.randn(1, hq, d, generator=gen).to(device=device, dtype=dtype)
            bt = torch.randperm(nb, generator=gen).view(1, nb).to(device)
            ctx = torch.tensor([seq], device=device)
            res = torch.empty_like(q)
            ws = torch.zeros(kpa.decode_workspace_bytes(1, hq, d, seq, dtype),
                             dtype=torch.uint8, device=device)

            def call(i):
                kc, vc = pools[i % copies]
                kpa.paged_decode_launch(q, kc, vc, bt, ctx, res, workspace=ws)

            stream.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(stream):
                for i in range(copies):
                    call(i)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(copies):
                    call(i)
            warm_graph(g, stream, seconds=0.1)
            us = timed_graph(g, reps, stream) / (reps * copies) * 1e6
            check_decode_outputs(kpa, ws, res, stream, f"reference shape {name} {seq}")
            kv_bytes = 2 * seq * hkv * d * 2
            by_len[str(seq)] = {"us": round(us, 2), "GBps": round(kv_bytes / us / 1e3, 1),
                                "pools_rotated": copies}
            del pools, g
            torch.cuda.empty_cache()
        out[name] = by_len
    return {
        "shape": "one request, 32 q / 8 KV heads, head_dim 128, block 16 (the reference's "
                 "benchmark_paged_attention.py defaults)",
        "kernels": {"bf16": "matrix-core split-KV decode, merged in one launch",
                    "fp16": "matrix-core split-KV decode, merged in one launch"},
        "us_by_seq_len": out,
        "reference_published_us": {str(k): v for k, v in REFERENCE_SPLIT_KV_US.items()},
        "reference_published_on": "RTX 5070 Ti Laptop GPU, Triton split-KV kernel, fp16 "
                                  "(seq_scaling.csv split_kernel_ms; its merge pass is extra)",
    }


# The reference's published batched decode steps of the whole model
# (benchmarks/benchmark_decode_runtime.py, Qwen2.5-0.5B, block 16, median of
# 50 synchronised wall-clock samples after 10 warm-up calls, RTX 5070 Ti
# Laptop GPU): (dtype, batch, context, ragged) -> ms per step.
# benchmarks/results/decode_runtime_qwen25_bf16_b8_s512_ragged_reduced_default.csv:3,
# decode_runtime_qwen25_bf16_b16_s128_reduced_default.csv:3,
# decode_runtime_qwen25_bf16_s32_128_512.csv:21 (its JSON: dtype float32).
REFERENCE_DECODE_RUNTIME_MS = {("bf16", 8, 512, True): 41.98, ("bf16", 16, 128, False): 40.32,
                               ("fp32", 16, 128, False): 45.30}


def bench_decode_runtime(device, warmup=10, samples=50):
    """One batched decode step of the whole 24-layer model
    (TinyQwen2ForCausalLM.forward_decode_batch_with_cache: embedding, every
    layer's QKV GEMM, rotation, KV write and paged decode, MLP, final norm and
    LM head) at the reference's decode-benchmark cases, timed as it times
    them: host wall clock with a device synchronisation on both sides, median
    of `samples` calls after `warmup`. Ragged lengths follow the reference's
    formula, max(2, L/2 + (L - L/2)(i + 1)/B) for request i
    (benchmark_decode_runtime.py:202-203). Each request's prompt (context - 1
    random token ids) is prefilled through the model first; the timed step
    writes the next token of every request at position context - 1, the same
    slots on every call. Random-init weights (no checkpoint here); the step's
    time does not depend on their values. Each case is timed twice: the eager
    forward (as the reference runs it) and the same step replayed from a HIP
    graph (runtime/step_graphs.py: the metadata checks with one host sync,
    the input copies and the replay, inside the timed call). Every timed
    call's logits must be finite."""
    import math

    import torch

    from mini_llm_runtime_amd.model.qwen2 import TinyQwen2Config, TinyQwen2ForCausalLM
    from mini_llm_runtime_amd.runtime.step_graphs import DecodeGraphs
    from mini_llm_runtime_amd.runtime.paged_kv_cache import PagedKVCache
    from mini_llm_runtime_amd.workloads import QWEN05B_CONFIG

    cfg = TinyQwen2Config(**QWEN05B_CONFIG)
    bs = 16
    out = {}
    models = {}
    with torch.no_grad():
        for (name, batch, ctx, ragged), ref_ms in REFERENCE_DECODE_RUNTIME_MS.items():
            dtype = torch.bfloat16 if name == "bf16" else torch.float32
            if name not in models:
                models.clear()
                torch.manual_seed(0)
                models[name] = TinyQwen2ForCausalLM(cfg).to(device=device, dtype=dtype).eval()
            model = models[name]
            lengths = ([max(2, ctx // 2 + (ctx - ctx // 2) * (i + 1) // batch)
                        for i in range(batch)] if ragged else [ctx] * batch)
            cache = PagedKVCache(cfg.num_hidden_layers, sum(math.ceil(n / bs) for n in lengths),
                                 bs, cfg.num_key_value_heads, cfg.head_dim, dtype=dtype,
                                 device=device)
            gen = torch.Generator().manual_seed(1000 * batch + ctx)
            pending = []
            for i, n in enumerate(lengths):
                cache.add_sequence(i)
                assert cache.reserve_tokens(i, n)
                table = cache.block_tables[i]
                ids = torch.randint(10, 1000, (1, n - 1), generator=gen).to(device)
                pos = torch.arange(n - 1, device=device)
                slots = torch.tensor([table[t // bs] * bs + t % bs for t in range(n - 1)],
                                     device=device)
                logits = model.forward_prefill_with_cache(ids, pos[None, :], cache, slots)
                pending.append(int(logits[0, -1].argmax()))
            tables = [cache.block_tables[i] for i in range(batch)]
            width = max(map(len, tables))
            block_tables = torch.tensor([t + [-1] * (width - len(t)) for t in tables],
                                        device=device)
            contexts = torch.tensor(lengths, device=device)
            positions = (contexts - 1)[:, None]
            ids = torch.tensor(pending, device=device)[:, None]
            slots = torch.tensor([tables[i][(n - 1) // bs] * bs + (n - 1) % bs
                                  for i, n in enumerate(lengths)], device=device)

            graphs = DecodeGraphs(model, cache, max_blocks_per_seq=width)

            def eager():
                return model.forward_decode_batch_with_cache(ids, positions, cache, slots,
                                                             block_tables, contexts)[:, 0]

            def replayed():
                return graphs(ids, positions, slots, block_tables, contexts)[:, 0]

            row = {"contexts": f"{min(lengths)}..{max(lengths)}",
                   "reference_published_ms": ref_ms}
            for mode, step in (("eager", eager), ("graph", replayed)):
                for _ in range(warmup):
                    step()
                times, finite = [], []
                for _ in range(samples):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    logits = step()
                    torch.cuda.synchronize()
                    times.append((time.perf_counter() - t0) * 1e3)
                    finite.append(torch.isfinite(logits).all())
                if not bool(torch.stack(finite).all()):
                    raise RuntimeError(f"decode runtime {name} B={batch} {mode}: "
                                       "non-finite logits")
                med = statistics.median(times)
                row[mode] = {"median_ms": round(med, 3),
                             "p95_ms": round(sorted(times)[int(0.95 * (len(times) - 1))], 3),
                             "tokens_per_s": round(batch / med * 1e3, 1),
                             "reference_over_this": round(ref_ms / med, 2)}
            out[f"{name}_b{batch}_ctx{ctx}" + ("_ragged" if ragged else "")] = row
            del graphs, cache
    return {
        "what": ("TinyQwen2ForCausalLM.forward_decode_batch_with_cache, Qwen2.5-0.5B "
                 "architecture (random-init weights), block 16, one batched decode step; "
                 "eager, and replayed from a HIP graph (DecodeGraphs)"),
        "timing": (f"host wall clock with device synchronisation on both sides, median of "
                   f"{samples} calls after {warmup} warm-up calls (the reference's method)"),
        "reference_published_on": ("RTX 5070 Ti Laptop GPU, Qwen2.5-0.5B checkpoint "
                                   "(benchmarks/results/decode_runtime_qwen25_*.csv)"),
        "cases": out,
    }


def bench_accumulator(device, batch=1024, reps=4, calls_per_graph=100):
    """The CUDA accumulator extension's contract (p [B, 64], v [B, 64, 256],
    FP32) on mlr_pa_accumulate at the reference test's largest batch."""
    import torch

    from mini_llm_runtime_amd.kernels.accumulator import paged_attention_accumulator_cuda

    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    p = torch.randn(batch, 64, device=device, generator=gen)
    v = torch.randn(batch, 64, 256, device=device, generator=gen)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        paged_attention_accumulator_cuda(p, v)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(calls_per_graph):
            paged_attention_accumulator_cuda(p, v)
    warm_graph(g, stream)
    us = timed_graph(g, reps, stream) / (reps * calls_per_graph) * 1e6
    nbytes = batch * (64 * 256 + 64 + 256) * 4
    return {"workload": f"accumulator_b{batch}_n64_d256_fp32", "us": round(us, 3),
            "bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1),
            "frac_of_hbm_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


def cpu_model() -> str | None:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _median_runs(fn, budget, min_runs=5, max_runs=50):
    """One warm-up call, then at least min_runs timed calls (more while the
    budget in seconds lasts); returns (median seconds, runs)."""
    fn()
    times, spent = [], 0.0
    while len(times) < min_runs or (spent < budget and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        times.append(dt)
        spent += dt
        if spent > 3 * budget and len(times) >= min_runs:
            break
    return statistics.median(times), len(times)


def _cpu_threads():
    import torch
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return torch.get_num_threads()


def cpu_baseline_decode(wl, budget):
    """The reference's CPU path for the decode step (write_slots +
    paged_attention_decode_batch_parallel, restated by the oracle) on the
    same inputs."""
    import torch

    import oracle.paged_attention as opa
    from oracle.paged_kv_cache import OracleKVCache

    threads = _cpu_threads()
    cache = OracleKVCache(1, wl.k_cache.shape[0], 16, 2, 64, dtype=torch.bfloat16)
    cache.k_cache[0].copy_(wl.k_cache)
    cache.v_cache[0].copy_(wl.v_cache)

    def step():
        cache.write_slots(wl.slot_mapping, wl.new_k, wl.new_v, 0)
        k_layer, v_layer = cache.get_layer_cache(0)
        opa.decode_batch_parallel(wl.q, k_layer, v_layer, wl.block_tables,
                                  wl.context_lens, 16)

    med, runs = _median_runs(step, budget)
    return {
        "value": (wl.algorithmic_bytes() + wl.write_bytes()) / med / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"full bf16_decode_qwen05b_b64 step (64-token write_slots + "
                   f"decode_batch_parallel, oracle restatement in PyTorch CPU), "
                   f"median of {runs} runs after 1 warm-up, {med * 1e3:.1f} ms/step"),
    }


def bench_fp32_decode_b4(device, budget):
    """fp32_decode_b4 (FP32, batch 4, contexts {17, 64, 130, 255}, the new
    tokens written first): the HIP decode step (mlr_paged_decode_append)
    against the reference's CPU path (write_slots +
    paged_attention_decode_batch_parallel, restated by the oracle)."""
    import torch

    import oracle.paged_attention as opa
    from mini_llm_runtime_amd import workloads
    from mini_llm_runtime_amd.kernels import paged_attention as kpa
    from oracle.paged_kv_cache import OracleKVCache

    wl = workloads.fp32_decode_b4()
    nbytes = wl.algorithmic_bytes() + wl.write_bytes()
    kc, vc = wl.k_cache.to(device), wl.v_cache.to(device)
    q, bt, ctx = wl.q.to(device), wl.block_tables.to(device), wl.context_lens.to(device)
    slots, nk, nv = (t.to(device) for t in (wl.slot_mapping, wl.new_k, wl.new_v))
    out = torch.empty_like(q)
    ws = torch.zeros(kpa.decode_workspace_bytes(4, 14, 64, bt.shape[1] * 16, torch.float32),
                     dtype=torch.uint8, device=device)

    def call():
        kpa.paged_decode_launch(q, kc, vc, bt, ctx, out, workspace=ws, new_k=nk, new_v=nv,
                                slot_mapping=slots)

    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(10):
            call()
    warm_graph(g, stream, seconds=0.1)
    gpu_us = timed_graph(g, 10, stream) / 100 * 1e6
    check_decode_outputs(kpa, ws, out, stream, wl.name)

    threads = _cpu_threads()
    cache = OracleKVCache(1, wl.k_cache.shape[0], 16, 2, 64, dtype=torch.float32)
    cache.k_cache[0].copy_(wl.k_cache)
    cache.v_cache[0].copy_(wl.v_cache)

    def cpu_step():
        cache.write_slots(wl.slot_mapping, wl.new_k, wl.new_v, 0)
        k_layer, v_layer = cache.get_layer_cache(0)
        opa.decode_batch_parallel(wl.q, k_layer, v_layer, wl.block_tables, wl.context_lens, 16)

    med, runs = _median_runs(cpu_step, budget, min_runs=20, max_runs=2000)
    return {
        "workload": wl.name,
        "bytes_per_step": nbytes,
        "gpu_us_per_step": round(gpu_us, 3),
        "gpu_GBps": round(nbytes / gpu_us / 1e3, 2),
        "note": "latency-bound: 0.5 MB per step",
        "cpu_baseline": {
            "value": nbytes / med / 1e9,
            "unit": "GB/s",
            "us_per_step": round(med * 1e6, 1),
            "cores": threads,
            "cpu_model": cpu_model(),
            "kind": "port",
            "sample": (f"full fp32_decode_b4 step (write_slots + decode_batch_parallel, "
                       f"oracle restatement in PyTorch CPU), median of {runs} runs after "
                       f"1 warm-up"),
        },
    }


def cpu_baseline_prefill(wl, budget):
    """The reference's CPU chunk prefill (paged_attention_prefill_chunk_tiled,
    tile 64, restated by the oracle) over all 8 sequences of the workload,
    median of at least 5 passes after one warm-up pass."""
    import oracle.paged_attention as opa

    threads = _cpu_threads()
    kc, vc = wl.k_cache.clone(), wl.v_cache.clone()
    kc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.chunk_k)
    vc.view(-1, 2, 64).index_copy_(0, wl.slot_mapping, wl.chunk_v)

    def all_sequences():
        for s in range(len(wl.prefix_lens)):
            lo, hi = int(wl.query_start_loc[s]), int(wl.query_start_loc[s + 1])
            p = wl.prefix_lens[s]
            opa.prefill_chunk_tiled(wl.q[lo:hi], kc, vc, wl.tables[s], p, p + hi - lo, 16, 64)

    med, runs = _median_runs(all_sequences, budget, min_runs=5, max_runs=20)
    return {
        "value": wl.causal_flops() / med / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"all 8 sequences of bf16_prefill_chunk512_x8 (prefill_chunk_tiled, "
                   f"tile 64), median of {runs} passes after 1 warm-up pass, "
                   f"{med:.2f} s per pass"),
    }


def bench_serving(device, steps=None, graphs=False):
    """End-to-end continuous-batching steps at Qwen2.5-0.5B shape in BF16
    (workloads.qwen05b_serving): schedule, pack, 24-layer forward on the HIP
    attention kernels with PyTorch GEMMs, sample, update. After the warm-up
    (all 48 initial prompts admitted), each step is timed on the host with a
    device synchronisation on both sides. Every timed step's logits must be
    finite (checked after the loop; the merge-failure flag is checked inside
    each step). graphs: each step's decodes replay the batched decode forward
    from a HIP graph per batch size (runtime/step_graphs.py: DecodeGraphs),
    block tables padded to the workload's longest request, and packed
    prefills whose shape repeats replay theirs (PrefillGraphs: recorded the
    third time a shape is met, the eight most recent kept); the decode graphs
    of every batch size up to the scheduler's max_num_seqs are recorded before
    the warm-up (their recording time is reported, outside the steps)."""
    import torch

    from mini_llm_runtime_amd import workloads
    from mini_llm_runtime_amd.runtime.model_runner import run_generation_step

    w = workloads.qwen05b_serving()
    steps = steps or w.steps
    _, model, cache, scheduler, _ = workloads.build_serving(w, device, torch.bfloat16)
    dgraphs = pgraphs = None
    if graphs:
        from mini_llm_runtime_amd.runtime.step_graphs import DecodeGraphs, PrefillGraphs

        longest = max(len(p) + m for p, m in w.initial + w.arrivals)
        dgraphs = DecodeGraphs(model, cache, max_blocks_per_seq=-(-longest // w.block_size))
        pgraphs = PrefillGraphs(model, cache)
        t0 = time.perf_counter()
        with torch.no_grad():
            dgraphs.record(range(1, w.max_num_seqs + 1))
        torch.cuda.synchronize()
        record_s = time.perf_counter() - t0
    times, decode_tokens, prefill_tokens, finished = [], 0, 0, 0
    with torch.no_grad():
        warm = workloads.serving_warm_up(model, scheduler, len(w.initial),
                                         decode_graphs=dgraphs, prefill_graphs=pgraphs)
        finite = []  # per step, read after the timed loop
        for _ in range(steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            result = run_generation_step(model, scheduler, decode_graphs=dgraphs,
                                         prefill_graphs=pgraphs)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
            finite.append(torch.isfinite(result.packed_logits).all())
            out = result.scheduler_output
            decode_tokens += len(out.decode_requests)
            prefill_tokens += sum(out.num_scheduled_tokens[r.request_id]
                                  for r in out.prefill_requests)
            finished += len(result.finished_requests)
        bad = [i for i, ok in enumerate(torch.stack(finite).tolist()) if not ok]
        if bad:
            raise RuntimeError(f"{w.name}: non-finite logits at timed steps {bad[:8]}")
        # Host metadata of one step: the device path build_model_batch uses
        # (per-request host work + mlr_build_step_metadata) against the
        # reference-style per-token host construction.
        from mini_llm_runtime_amd.runtime.model_runner import build_model_batch
        probe = scheduler.schedule()
        meta = {}
        for name, dev in (("device", device), ("host", torch.device("cpu"))):
            build_model_batch(probe, w.block_size, dev)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(20):
                batch = build_model_batch(probe, w.block_size, dev)
                if dev.type == "cpu":  # the host lists still have to reach the GPU
                    for field in ("input_token_ids", "positions", "query_start_loc",
                                  "context_lens", "block_tables", "slot_mapping"):
                        getattr(batch, field).to(device)
            torch.cuda.synchronize()
            meta[f"build_{name}_ms"] = round((time.perf_counter() - t0) / 20 * 1e3, 3)
        meta["tokens"] = sum(probe.num_scheduled_tokens.values())
        meta["requests"] = len(probe.scheduled_requests)
    total = sum(times)
    return {
        "workload": w.name,
        "warmup_steps": warm,
        "step_metadata": meta,
        "steps": steps,
        "ms_per_step": round(1e3 * total / steps, 3),
        "ms_per_step_median": round(1e3 * statistics.median(times), 3),
        "decode_tokens_per_step": round(decode_tokens / steps, 2),
        "prefill_tokens_per_step": round(prefill_tokens / steps, 2),
        "tokens_per_s": round((decode_tokens + prefill_tokens) / total, 1),
        "decode_tokens_per_s": round(decode_tokens / total, 1),
        "requests_finished": finished,
        "decode_graphs": (None if dgraphs is None else
                          {"recorded": dgraphs.captures, "record_s": round(record_s, 2),
                           "replays": dgraphs.replays, "eager_calls": dgraphs.eager_calls,
                           "max_blocks_per_seq": dgraphs.width}),
        "prefill_graphs": (None if pgraphs is None else
                           {"recorded": pgraphs.captures, "replays": pgraphs.replays,
                            "eager_calls": pgraphs.eager_calls}),
    }


def kernel_sources_hash():
    """sha256 (first 16 hex digits) over the kernel sources and the ABI header:
    what a counter profile of the kernels depends on."""
    import glob
    import hashlib

    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(REPO, "mini-llm-runtime_amd", "csrc", "*")) +
                   glob.glob(os.path.join(REPO, "include", "*.h")))
    for path in files:
        h.update(os.path.relpath(path, REPO).encode())
        with open(path, "rb") as f:
            h.update(hashlib.sha256(f.read()).digest())
    return h.hexdigest()[:16]


def measured_traffic():
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (profiles/traffic.json), measured outside this run (counters need
    their own rocprofv3 passes). Used only when it was measured on these kernel
    sources: the file records their hash, and a profile of other sources is
    stale, so the line then carries traffic null and says why."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            traffic = json.load(f)
    except (OSError, ValueError):
        return None, "profiles/traffic.json is absent"
    if traffic.get("kernel_sources_sha256_16") != kernel_sources_hash():
        return None, ("profiles/traffic.json was measured on other kernel sources "
                      f"({traffic.get('kernel_sources_sha256_16')}; now {kernel_sources_hash()})")
    return traffic, traffic["source"]


def provenance():
    """What produced this line: the git HEAD when a checkout is present, the
    sha256 of every kernel source, the ABI header, this script and the built
    library, and the software and hardware versions."""
    import glob
    import hashlib
    import subprocess

    import torch

    def sha(path):
        h = hashlib.sha256()
        with open(path, "rb") as f:
            for chunk in iter(lambda: f.read(1 << 20), b""):
                h.update(chunk)
        return h.hexdigest()

    pkg = os.path.join(REPO, "mini-llm-runtime_amd")
    files = sorted(glob.glob(os.path.join(pkg, "csrc", "*")) +
                   glob.glob(os.path.join(REPO, "include", "*.h")) +
                   [os.path.join(REPO, "bench.py"),
                    os.path.join(pkg, "mini_llm_runtime_amd", "libmlr_attn.so")])
    hashes = {os.path.relpath(f, REPO): sha(f)[:16] for f in files if os.path.isfile(f)}
    combined = hashlib.sha256("".join(f"{k}={v};" for k, v in sorted(hashes.items()))
                              .encode()).hexdigest()[:16]
    head = None
    if os.path.isdir(os.path.join(REPO, ".git")):
        try:
            head = subprocess.run(["git", "-C", REPO, "rev-parse", "HEAD"], capture_output=True,
                                  text=True, timeout=10).stdout.strip() or None
        except (OSError, subprocess.SubprocessError):
            head = None
    props = torch.cuda.get_device_properties(0)
    return {
        "git_head": head,
        "sources_sha256_16": combined,
        "files_sha256_16": hashes,
        "torch": torch.__version__,
        "hip": getattr(torch.version, "hip", None),
        "gpu": props.name,
        "gpu_arch": getattr(props, "gcnArchName", None),
        "cpu_model": cpu_model(),
    }


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the paged attention kernels run one GPU's "
              "share of the work and have no cross-GPU step; run it with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    device = torch.device("cuda", 0)
    if args.profile:
        profile_run(args, device)
        return
    if args.serving:
        print(json.dumps({"metric": "serving step (qwen05b_serving, bf16)",
                          **bench_serving(device, graphs=args.graphs)}),
              flush=True)
        return
    dec = bench_decode(args, device)
    pre = None if args.no_prefill else bench_prefill(device)
    cpu = None
    cpu_pre = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_decode(dec["wl"], args.cpu_budget)
        if pre is not None:
            cpu_pre = cpu_baseline_prefill(pre["wl"], args.cpu_budget / 2)
    traffic, traffic_source = measured_traffic()
    line = {
        "metric": METRIC,
        "value": round(dec["value_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": dec["warmup"],
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "bf16_decode_qwen05b_b64",
            "batch": 64, "num_q_heads": 14, "num_kv_heads": 2, "head_dim": 64,
            "block_size": 16, "context": "U[128,4096]", "num_blocks": 24576,
            "kv_write_tokens": 64, "layers_rotated": LAYERS,
            "step": ("mlr_paged_decode_append: 64-token KV write fused into the "
                     "split-KV decode, splits merged in the same launch; one layer"),
            "step_bytes": dec["step_bytes"],
            "hbm_pct_of_peak": round(100 * dec["value_gbs"] / HBM_PEAK_GBS, 2),
            "us_per_step_10_replays": round(dec["us_per_step_10_replays"], 3),
            "decode_only_us": round(dec["decode_us"], 3),
            "served_step_us": round(dec["served1_us"], 3),
            "served_step": ("what Qwen2Attention.forward_decode_batch_with_cache runs after "
                            "its QKV GEMM: mlr_paged_decode_qkv (rotary embedding of q and "
                            "the new K, KV write and decode in one launch)"),
            "served_two_launch_us": round(dec["served_us"], 3),
            "served_two_launch": ("the same step as mlr_qkv_rope_write then mlr_paged_decode "
                                  "(the path for shapes the one-launch kernel lacks)"),
            "read_floor": dec["read_floor"],
            "sclk_mhz": dec["sclk"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": ("mlr_paged_decode_append (decode_mfma<64,4,false,true,true,2,false>: "
                       "320-token splits, a pair of KV heads per workgroup, KV write folded "
                       "in, splits merged in the same launch)"),
            "achieved": round(dec["value_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["value_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic["decode_step_bytes"] if traffic else None,
            "traffic_source": traffic_source,
            "algorithmic_bytes_per_launch": dec["step_bytes"],
            "avg_launch_us": round(dec["ms_per_step"] * 1e3, 3),
        },
        "cpu_baseline": cpu,
        "provenance": provenance(),
    }
    if pre is not None:
        line["prefill"] = {
            "workload": pre["workload"],
            "value": round(pre["tflops"], 3),
            "unit": "TFLOP/s",
            "roofline": {"bound": "mfma", "achieved": round(pre["tflops"], 3),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pre["tflops"] / BF16_PEAK_TFLOPS, 5),
                         "traffic": traffic["prefill_call_bytes"] if traffic else None,
                         "traffic_source": traffic_source},
            "flops_per_call": pre["flops_per_call"],
            "us_per_call": pre["us_per_call"],
            "us_per_call_min_max": pre["us_per_call_min_max"],
            "kv_tile": ("the call passes the reference's tile_size 64, which orders the FP32 "
                        "accumulation only; the kernel steps by its own 64-key tile for "
                        "any tile_size, so there is one timing, not a tile sweep (a "
                        "128-key instantiation, one workgroup per CU, measured 89.5 us "
                        "against 53.6 us on one box and was not kept)"),
            "sclk_mhz": pre["sclk"],
            "cpu_baseline": cpu_pre,
        }
        pre16 = bench_prefill(device, dtype=torch.float16)
        line["prefill"]["fp16"] = {
            "what": "the same call with q and the cache in fp16 (fp16 matrix-core operands)",
            "us_per_call": pre16["us_per_call"],
            "tflops": round(pre16["tflops"], 3),
            "frac_of_fp16_peak": round(pre16["tflops"] / BF16_PEAK_TFLOPS, 5)}
        pre32 = bench_prefill(device, dtype=torch.float32)
        line["prefill"]["fp32"] = {
            "what": ("the same call in FP32 (v_mfma_f32_16x16x4_f32), against the 157.3 "
                     "TFLOP/s FP32 matrix-core peak"),
            "us_per_call": pre32["us_per_call"],
            "tflops": round(pre32["tflops"], 3),
            "frac_of_fp32_peak": round(pre32["tflops"] / F32_PEAK_TFLOPS, 5)}
    line["fp32_decode_b4"] = bench_fp32_decode_b4(
        device, 0 if args.no_cpu_baseline else args.cpu_budget / 4)
    if not args.no_pre_attention:
        line["pre_attention"] = bench_pre_attention(device)
        line["pre_attention"]["roofline"]["traffic"] = (
            traffic.get("pre_attention_call_bytes") if traffic else None)
    line["kv_write"] = bench_kv_write(device)
    line["decode_32k"] = bench_decode_32k(device)
    line["decode_32k"]["traffic"] = traffic.get("decode_32k_bytes") if traffic else None
    line["accumulator"] = bench_accumulator(device)
    line["reference_shapes"] = bench_reference_shapes(device)
    line["decode_runtime"] = bench_decode_runtime(device)
    if not args.no_serving:
        line["serving"] = bench_serving(device)
        line["serving_graphs"] = bench_serving(device, graphs=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
