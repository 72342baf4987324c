#!/usr/bin/env python3
"""Benchmark of the paged-KV hot path on one MI355X.

Headline (BASELINE.json metric): paged decode attention at the Qwen2.5-7B shape
(28 query / 4 KV heads, head_dim 128, bf16 cache, 16-token pages), batch 64,
every row at context 1920. One "step" is one forward's worth of decode
attention: a hipGraph that replays the call once per decoder layer (28), each
layer on its own KV pool (251.7 MB each, 7 GB in all, far above the 256 MB
Infinity Cache), exactly the reference's method (benchmarks/bench_decode_attn.py:45-82).

  value    = KV bytes read per step (28 · B · ctx · Hkv · D · 2 · 2) / step time, GB/s
  roofline = the decode kernel's algorithmic bytes per launch / its mean launch
             time (HIP events on the replay stream), against 8 TB/s
  traffic  = HBM bytes per launch from the committed rocprofv3 counter summary
             (profiles/decode_b64_ctx1920_traffic.txt), null if absent
  cpu_baseline = the oracle's restatement of the reference's torch decode path
             (gather + SDPA, fp32) timed on this host on the same workload

Secondary lines (same method), each with its binding roof and the oracle's
restatement of the reference's torch CPU path timed on this host beside it:
BASELINE config 1 (the 0.5B-shape single-layer step: RoPE + append + decode),
decode B8/ctx1920, B1/ctx32768, B64/ctx2048 (the reference's published H100
point), RoPE + KV append (decode 64 tokens, prefill 8192 tokens), the four
varlen prefill configurations (TFLOP/s; fraction of the binding roof, MFMA or
HBM), the decode step's other kernels (greedy argmax over 64 x 152,064 logits,
residual add + RMSNorm and SiLU*mul at 64 and 8192 rows) in GB/s, and the
end-to-end generate of config 5. The host CPU (lscpu model, sockets, cores,
threads) is recorded once in `cpu_host`.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
                       [--only NAME] [--calib-copy] [--tune KNOB=VALUE ...]
(--tune sets a library tuning knob, bvllm_set_tuning, before measuring: for A/B
runs and the profiles of the alternative kernels.)
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "baby-vllm_amd"))
sys.path.insert(0, REPO)

import torch  # noqa: E402

METRIC = "decode-attn HBM GB/s (% of peak) at 7B-shape B64/ctx1920; prefill-attn TFLOP/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
LAYERS = 28
H, HKV, D, BS = 28, 4, 128, 16
TRAFFIC_FILE = os.path.join(REPO, "profiles", "decode_b64_ctx1920_traffic.txt")


def cdiv(a, b):
    return -(-a // b)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ----------------------------------------------------------------- builders

def build_decode(batch, ctx, layers, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    blocks = cdiv(ctx, BS)
    width = blocks + 1
    total = batch * blocks
    caches, tables = [], []
    for _ in range(layers):
        caches.append(torch.randn(2, total, BS, HKV, D, device="cuda", dtype=torch.bfloat16, generator=g))
        bt = torch.zeros(batch, width, dtype=torch.int32, device="cuda")
        bt[:, :blocks] = torch.randperm(total, device="cuda", generator=g).view(batch, blocks).to(torch.int32)
        tables.append(bt)
    # N(0,1) q, one per layer; the 1/sqrt(128) enters as the softmax scale, as Attention passes it.
    qs = [torch.randn(batch, H, D, device="cuda", dtype=torch.bfloat16, generator=g) for _ in range(layers)]
    seq_lens = torch.full((batch,), ctx, dtype=torch.int32, device="cuda")
    return qs, caches, tables, seq_lens


def time_graph(fn, warmup, iters):
    """Capture fn once in a hipGraph; return (median ms, list of ms) over replays timed with events."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    times = []
    for _ in range(iters):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end))
    del graph
    return statistics.median(times), times


# ------------------------------------------------------------ measurements

def bench_decode(batch, ctx, warmup, iters, layers=LAYERS):
    from babyvllm.kernels.decode_split import decode_split_plan
    from babyvllm.kernels.paged_attn import _num_sms, paged_decode_attention

    qs, caches, tables, seq_lens = build_decode(batch, ctx, layers, seed=batch + ctx)
    scale = D ** -0.5
    outs = []  # every layer's output stays allocated in the graph's pool (no reuse across layers)

    def fwd():
        outs[:] = [paged_decode_attention(qs[i], caches[i], tables[i], seq_lens, scale, max_seq_len=ctx)
                   for i in range(layers)]

    ms, _ = time_graph(fwd, warmup, iters)
    kv_bytes = batch * ctx * HKV * D * 2 * 2
    per_launch_us = ms * 1e3 / layers
    plan = decode_split_plan(batch, HKV, BS, tables[0].shape[1], ctx, _num_sms(0))
    del qs, caches, tables, seq_lens, outs
    torch.cuda.empty_cache()
    return {
        "batch": batch, "context": ctx, "plan": list(plan),
        "us_per_layer": per_launch_us,
        "gb_s": kv_bytes / (per_launch_us * 1e-6) / 1e9,
        "frac_of_hbm_peak": kv_bytes / (per_launch_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "kv_bytes_per_layer": kv_bytes,
        "step_ms": ms,
        "roofline": hbm_roof(kv_bytes, per_launch_us * 1e-6),
    }


def bench_append(tokens_per_seq, seqs, warmup, iters, layers=LAYERS):
    """RoPE + KV append at the 7B shape; algorithmic bytes 19,976 per token."""
    from babyvllm.kernels.rope import fused_rope_and_cache
    from babyvllm.layers.rotary import RotaryEmbedding

    T = tokens_per_seq * seqs
    nb = 8192
    g = torch.Generator(device="cuda").manual_seed(T)
    qkvs = [torch.randn(T, (H + 2 * HKV) * D, device="cuda", dtype=torch.bfloat16, generator=g)
            for _ in range(layers)]
    caches = [torch.zeros(2, nb, BS, HKV, D, device="cuda", dtype=torch.bfloat16) for _ in range(layers)]
    rope = RotaryEmbedding(D, 4097, base=1e6).cuda()
    if tokens_per_seq == 1:
        pos = torch.randint(128, 4097, (T,), device="cuda", generator=g)
    else:
        pos = torch.arange(tokens_per_seq, device="cuda").repeat(seqs)
    cos, sin = rope(pos, torch.bfloat16)
    perm = torch.randperm(nb, device="cuda", generator=g)
    if tokens_per_seq == 1:
        # One token per sequence: the page holding each token's position is a
        # distinct random page of the pool.
        slots = (perm[:T] * BS + pos % BS).to(torch.int64)
    else:
        per_seq = cdiv(tokens_per_seq, BS)
        tables = perm[: seqs * per_seq].view(seqs, per_seq)
        seq_idx = torch.arange(seqs, device="cuda").repeat_interleave(tokens_per_seq)
        slots = (tables[seq_idx, pos // BS] * BS + pos % BS).to(torch.int64)
    views = []
    for qkv in qkvs:
        views.append((qkv[:, : H * D].view(T, H, D), qkv[:, H * D:(H + HKV) * D].view(T, HKV, D),
                      qkv[:, (H + HKV) * D:].view(T, HKV, D)))

    def fwd():
        for i in range(layers):
            q, k, v = views[i]
            fused_rope_and_cache(q, k, v, cos, sin, caches[i], slots)

    ms, _ = time_graph(fwd, warmup, iters)
    per_us = ms * 1e3 / layers
    nbytes = T * 19976
    del qkvs, caches, views
    torch.cuda.empty_cache()
    return {"tokens": T, "us_per_layer": per_us, "gb_s": nbytes / (per_us * 1e-6) / 1e9,
            "frac_of_hbm_peak": nbytes / (per_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "algorithmic_bytes": nbytes, "roofline": hbm_roof(nbytes, per_us * 1e-6)}


PREFILL_SHAPES = {
    "64x128_fresh": [(0, 128)] * 64,
    "8x(1024+128)": [(1024, 128)] * 8,
    "1x(2048+4096)": [(2048, 4096)],
    "1x512+63x(1000+1)": [(0, 512)] + [(1000, 1)] * 63,
}


def prefill_flops(specs):
    return 512 * H * sum(sum(c + i + 1 for i in range(n)) for c, n in specs)


def prefill_bytes(specs):
    """Algorithmic HBM bytes: q read and output written once, each sequence's K/V read once per KV head."""
    tokens = sum(n for _, n in specs)
    return 2 * tokens * H * D * 2 + sum(c + n for c, n in specs) * HKV * D * 2 * 2


def hbm_roof(nbytes, seconds):
    ach = nbytes / seconds / 1e9
    return {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "algorithmic_bytes": nbytes}


def binding_roof(flops, nbytes, seconds):
    """The roof that binds at peak (the longer of flops / bf16 MFMA peak and bytes / HBM peak)."""
    t_mfma = flops / (BF16_PEAK_TFLOPS * 1e12)
    t_hbm = nbytes / (HBM_PEAK_GBS * 1e9)
    if t_mfma >= t_hbm:
        ach = flops / seconds / 1e12
        out = {"bound": "mfma", "achieved": round(ach, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
               "frac": round(t_mfma / seconds, 4)}
    else:
        out = hbm_roof(nbytes, seconds)
    out.update({"roof_us": round(max(t_mfma, t_hbm) * 1e6, 2), "flop": flops, "algorithmic_bytes": nbytes})
    return out


def bench_prefill(name, warmup, iters, layers=LAYERS):
    from babyvllm.kernels.paged_prefill import paged_prefill_attention
    from babyvllm.worker.context import AttentionMetadata

    specs = PREFILL_SHAPES[name]
    g = torch.Generator(device="cuda").manual_seed(len(specs))
    seq_lens = [c + n for c, n in specs]
    q_lens = [n for _, n in specs]
    blocks = [cdiv(s, BS) for s in seq_lens]
    total = sum(blocks)
    caches, mds = [], []
    qsl = [0]
    for n in q_lens:
        qsl.append(qsl[-1] + n)
    for _ in range(layers):
        caches.append(torch.randn(2, total, BS, HKV, D, device="cuda", dtype=torch.bfloat16, generator=g))
        perm = torch.randperm(total, generator=torch.Generator().manual_seed(len(mds))).tolist()
        tables, i = [], 0
        for nblk in blocks:
            tables.append(perm[i:i + nblk] + [0] * (max(blocks) - nblk))
            i += nblk
        mds.append(AttentionMetadata(
            slot_mapping=torch.zeros(sum(q_lens), dtype=torch.int64, device="cuda"),
            block_tables=torch.tensor(tables, dtype=torch.int32, device="cuda"),
            query_start_loc=torch.tensor(qsl, dtype=torch.int32, device="cuda"),
            seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device="cuda"),
            context_lens=torch.tensor([c for c, _ in specs], dtype=torch.int32, device="cuda"),
            query_start_loc_cpu=qsl, seq_lens_cpu=seq_lens, context_lens_cpu=[c for c, _ in specs],
            max_query_len=max(q_lens), max_seq_len=max(seq_lens)))
    # Every layer reads its own q and writes its own output, and all 28 outputs
    # stay allocated in the graph's pool, so no layer finds its q or output
    # lines in the 256 MB Infinity Cache from the previous layer.
    qs = [torch.randn(sum(q_lens), H, D, device="cuda", dtype=torch.bfloat16, generator=g) for _ in range(layers)]
    outs = []

    def fwd():
        outs[:] = [paged_prefill_attention(qs[i], caches[i], mds[i], D ** -0.5) for i in range(layers)]

    ms, _ = time_graph(fwd, warmup, iters)
    per_us = ms * 1e3 / layers
    flops = prefill_flops(specs)
    del caches, mds, qs, outs
    torch.cuda.empty_cache()
    return {"us_per_layer": per_us, "tflop_s": flops / (per_us * 1e-6) / 1e12, "flop": flops,
            "roofline": binding_roof(flops, prefill_bytes(specs), per_us * 1e-6)}


# the 0.5B-shape single-layer decode step.
C1_H, C1_HKV, C1_D, C1_B, C1_POOL, C1_WIDTH, C1_BUCKET = 14, 2, 64, 8, 512, 32, 512


def config1_inputs(seed, device, lens=None):
    """Lengths U[100, 512] (or the given ones), a 512-block pool whose rows are a
    seeded permutation (width 32), q/k/v ~ N(0, 1); the step's token sits at
    position seq_len - 1."""
    g = torch.Generator().manual_seed(seed)
    drawn = torch.randint(100, 513, (C1_B,), generator=g)
    lens = drawn if lens is None else lens
    cache = torch.randn(2, C1_POOL, BS, C1_HKV, C1_D, generator=g)
    bt = torch.randperm(C1_POOL, generator=g)[: C1_B * C1_WIDTH].view(C1_B, C1_WIDTH).int()
    qkv = torch.randn(C1_B, (C1_H + 2 * C1_HKV) * C1_D, generator=g)
    pos = lens - 1
    slots = bt[torch.arange(C1_B), pos // BS].long() * BS + pos % BS
    dt = torch.bfloat16 if device != "cpu" else torch.float32
    return (lens.to(device), cache.to(device, dt), bt.to(device), qkv.to(device, dt), pos.to(device),
            slots.to(device))


def config1_bytes(lens):
    """Append 5,128 B per token (q, k, v, cos, sin, slot read; q, k, cache rows written) + KV read."""
    return C1_B * 5128 + int(lens.sum()) * C1_HKV * C1_D * 2 * 2


def bench_config1(warmup, iters, layers=24):
    """One 'step' = the config-1 step for each of the 0.5B model's 24 layers, each
    layer on its own 512-block pool, table and q/k/v: RoPE (theta 1e6) + append
    through slot_mapping, then paged decode with max_seq_len = 512. As in the
    model, every layer of the step sees the same lengths and positions (seed
    100's); each layer's slots follow from those positions and its own table."""
    from babyvllm.kernels.paged_attn import paged_decode_attention
    from babyvllm.kernels.rope import fused_rope_and_cache
    from babyvllm.layers.rotary import RotaryEmbedding

    lens = config1_inputs(100, "cpu")[0]
    per_layer = [config1_inputs(100 + i, "cuda", lens=lens) for i in range(layers)]
    pos = per_layer[0][4]
    seq_lens = lens.int().cuda()
    for _, _, bt, _, p, slots in per_layer:
        bt, p = bt.cpu(), p.cpu()
        assert torch.equal(p, pos.cpu())
        assert torch.equal(slots.cpu(), bt[torch.arange(C1_B), p // BS].long() * BS + p % BS)
    rope = RotaryEmbedding(C1_D, 4096, base=1e6).cuda()
    views = []
    for _, cache, bt, qkv, _, slots in per_layer:
        q = qkv[:, : C1_H * C1_D].view(C1_B, C1_H, C1_D)
        k = qkv[:, C1_H * C1_D:(C1_H + C1_HKV) * C1_D].view(C1_B, C1_HKV, C1_D)
        v = qkv[:, (C1_H + C1_HKV) * C1_D:].view(C1_B, C1_HKV, C1_D)
        views.append((q, k, v, cache, bt, slots))

    def fwd():
        cos, sin = rope(pos, torch.bfloat16)
        for q, k, v, cache, bt, slots in views:
            fused_rope_and_cache(q, k, v, cos, sin, cache, slots)
            paged_decode_attention(q, cache, bt, seq_lens, C1_D ** -0.5, max_seq_len=C1_BUCKET)

    ms, _ = time_graph(fwd, warmup, iters)
    per_us = ms * 1e3 / layers
    nbytes = config1_bytes(lens)
    del per_layer, views
    torch.cuda.empty_cache()
    return {"us_per_layer": per_us, "gb_s": nbytes / (per_us * 1e-6) / 1e9, "algorithmic_bytes": nbytes,
            "roofline": hbm_roof(nbytes, per_us * 1e-6),
            "note": "latency-bound: 1.3 MB per step, 0.16 us at the HBM roof"}


def bench_step_kernels(warmup, iters):
    """The decode step's other kernels at the 7B shape, each over enough distinct
    buffers per replay that the inputs come from HBM (argmax, prefill-size rows)
    or as the decode step meets them (decode-size rows are cache-resident)."""
    from babyvllm.kernels.activation import fused_silu_mul
    from babyvllm.kernels.argmax import greedy_argmax
    from babyvllm.kernels.layernorm import fused_add_rms_norm

    hidden, inter, vocab = 3584, 18944, 152064
    out = {}

    def line(name, per_us, nbytes, reps):
        out[name] = {"us_per_call": per_us, "gb_s": nbytes / (per_us * 1e-6) / 1e9,
                     "frac_of_hbm_peak": nbytes / (per_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                     "algorithmic_bytes": nbytes, "calls_per_replay": reps,
                     "roofline": hbm_roof(nbytes, per_us * 1e-6)}

    g = torch.Generator(device="cuda").manual_seed(11)
    reps = 16
    logits = [torch.randn(64, vocab, device="cuda", dtype=torch.bfloat16, generator=g) for _ in range(reps)]
    tok = torch.empty(64, dtype=torch.int64, device="cuda")
    ms, _ = time_graph(lambda: [greedy_argmax(x, tok) for x in logits], warmup, iters)
    line("argmax_64x152064_bf16", ms * 1e3 / reps, 64 * vocab * 2, reps)
    del logits

    w = torch.rand(hidden, device="cuda", generator=g).to(torch.bfloat16)
    for rows, reps in ((64, 56), (8192, 8)):
        xs = [torch.randn(rows, hidden, device="cuda", generator=g).to(torch.bfloat16) for _ in range(reps)]
        rs = [torch.randn(rows, hidden, device="cuda", generator=g).to(torch.bfloat16) for _ in range(reps)]
        ms, _ = time_graph(lambda: [fused_add_rms_norm(x, r, w, 1e-6) for x, r in zip(xs, rs)], warmup, iters)
        line(f"add_rms_norm_{rows}x{hidden}", ms * 1e3 / reps, rows * hidden * 2 * 4 + hidden * 2, reps)
        del xs, rs

    for rows, reps in ((64, 28), (8192, 2)):
        gus = [torch.randn(rows, 2 * inter, device="cuda", generator=g).to(torch.bfloat16) for _ in range(reps)]
        ms, _ = time_graph(lambda: [fused_silu_mul(x) for x in gus], warmup, iters)
        line(f"silu_mul_{rows}x{inter}", ms * 1e3 / reps, rows * inter * 2 * 3, reps)
        del gus
    torch.cuda.empty_cache()
    return out


def bench_generate(n_prompts=64, prompt_len=1920, shared_len=1536, new_tokens=64, seed=0, caching=True):
    """continuous-batching greedy generate on a random-init
    Qwen2.5-7B-architecture model through LLM.generate's engine, prefix caching
    on. One untimed pass captures the decode graphs; the timed pass starts from
    an empty KV pool. Reports new tokens/s (prefill included), mean / max time
    to first token, decode steps/s and the peak number of KV pages in use."""
    from babyvllm.config import CacheConfig, SchedulerConfig, qwen2_5_7b
    from babyvllm.llm import LLM
    from babyvllm.sequence import SamplingParams

    cfg = qwen2_5_7b()
    g = torch.Generator().manual_seed(seed)
    shared = torch.randint(0, cfg.vocab_size, (shared_len,), generator=g).tolist()
    prompts = [shared + torch.randint(0, cfg.vocab_size, (prompt_len - shared_len,), generator=g).tolist()
               for _ in range(n_prompts)]
    t0 = time.perf_counter()
    llm = LLM(cfg, cache_config=CacheConfig(num_gpu_blocks=9000, enable_prefix_caching=caching),
              scheduler_config=SchedulerConfig(max_num_seqs=64, max_num_batched_tokens=8192), seed=seed)
    build_s = time.perf_counter() - t0
    params = SamplingParams(temperature=0.0, max_tokens=new_tokens, ignore_eos=True)
    engine = llm.engine

    def run():
        engine.reset()
        torch.cuda.synchronize()
        start = time.perf_counter()
        for p in prompts:
            engine.add_request(p, params)
        first, steps, decode_steps, peak_pages, n_tokens = {}, 0, 0, 0, 0
        while engine.has_unfinished_requests():
            sched_running = len(engine.scheduler.running)
            outs = engine.step()
            now = time.perf_counter() - start
            steps += 1
            peak_pages = max(peak_pages, engine.kv_cache_manager.num_used_blocks)
            for o in outs:
                n_tokens += len(o.new_token_ids)
                if o.new_token_ids and o.seq_id not in first:
                    first[o.seq_id] = now
            if sched_running == len(engine.scheduler.running) and len(outs) == sched_running:
                decode_steps += 1
        torch.cuda.synchronize()
        wall = time.perf_counter() - start
        return wall, first, steps, peak_pages, n_tokens, engine.kv_cache_manager.num_hit_tokens

    log("  e2e warm-up pass (graph capture) ...")
    run()
    wall, first, steps, peak_pages, n_tokens, hits = run()
    ttft = sorted(first.values())
    return {
        "metric": "end-to-end greedy generate, new tokens/s (prefill included)",
        "tokens_per_s": n_tokens / wall, "wall_s": wall, "new_tokens": n_tokens, "engine_steps": steps,
        "ttft_mean_ms": 1e3 * sum(ttft) / len(ttft), "ttft_max_ms": 1e3 * ttft[-1],
        "kv_blocks_peak": peak_pages,
        # Pages if all prompts ran at once: the shared prefix once, each private tail once.
        "kv_blocks_closed_form_all_at_once": (shared_len // 16 + n_prompts * (-(-(prompt_len + new_tokens) // 16)
                                                                      - shared_len // 16)),
        "prefix_hit_tokens": hits, "model_build_s": build_s,
        "config": {"model": "Qwen2.5-7B architecture, random init N(0, 0.02), bf16", "prompts": n_prompts,
                   "prompt_len": prompt_len, "shared_prefix": shared_len, "new_tokens": new_tokens,
                   "max_num_seqs": 64, "max_num_batched_tokens": 8192, "prefix_caching": caching},
    }


# ------------------------------------------------------------ CPU baseline
#
# The reference's torch CPU path, restated by the oracle (gather + SDPA decode,
# per-sequence SDPA prefill loop, apply_rope + index_copy_ store), in fp32 (the
# reference's CPU dtype), on the same shapes as the GPU lines, on this host's
# cores. Median of at least 5 runs after one warm-up, within a time budget.

def cpu_threads():
    """CPUs this process may use (its affinity mask, capped by OMP_NUM_THREADS when set)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_host():
    """lscpu model, sockets, cores and threads of this host, and the threads the baseline uses."""
    info = {"threads_used": cpu_threads(), "os_cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        fields = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                fields[k.strip()] = v.strip()
        info.update({"model": fields.get("Model name"), "sockets": fields.get("Socket(s)"),
                     "cores_per_socket": fields.get("Core(s) per socket"),
                     "threads_per_core": fields.get("Thread(s) per core"), "cpus": fields.get("CPU(s)")})
        try:
            info["physical_cores"] = int(fields["Socket(s)"]) * int(fields["Core(s) per socket"])
        except (KeyError, ValueError):
            pass
    except (OSError, subprocess.SubprocessError):
        info["model"] = None
    return info


def cpu_time(fn, budget_s=10.0, min_runs=5, max_runs=50):
    torch.set_num_threads(cpu_threads())
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def _cpu_line(value, unit, sec, runs, sample):
    return {"value": round(value, 4), "unit": unit, "cores": cpu_threads(), "kind": "port",
            "ms": round(sec * 1e3, 3), "runs": runs, "sample": sample}


# What the compact secondary entries of the JSON line mean (stated once).
LEGEND = {
    "us": "time per call: median replay of a hipGraph of 28 calls (24 for config 1), each call on its own "
          "cache pool, q and output, divided by the calls",
    "ach/unit": "algorithmic work per call / us; work = bytes for bound hbm, flop for bound mfma",
    "frac": "ach / the bound's peak (hbm 8000 GB/s, mfma 2500 TFLOP/s dense bf16)",
    "cpu": "the oracle's fp32 restatement of the reference's torch CPU path on one call of the same shape "
           "(gather + SDPA decode, per-sequence SDPA prefill loop, apply_rope + index_copy_ append, torch "
           "argmax / add + RMSNorm / SiLU*mul), median of >= 5 runs after a warm-up on cpu_host.threads_used "
           "threads: [ms, value in the line's unit]",
}


def compact(r):
    """A secondary line as it goes into the JSON line (full figures go to stderr)."""
    roof = r.get("roofline") or {}
    us = r.get("us_per_layer", r.get("us_per_call"))
    out = {"us": round(us, 2), "ach": roof.get("achieved"), "unit": roof.get("unit"), "frac": roof.get("frac"),
           "bound": roof.get("bound"),
           "work": roof.get("flop") if roof.get("bound") == "mfma" else roof.get("algorithmic_bytes")}
    if "plan" in r:
        out["plan"] = r["plan"]
    if "roof_us" in roof:
        out["roof_us"] = roof["roof_us"]
    cpu = r.get("cpu_baseline")
    if cpu and cpu.get("value") is not None:
        out["cpu"] = [cpu["ms"], cpu["value"]]
    return out


def compact_generate(r):
    return {"tok_s": round(r["tokens_per_s"], 1), "wall_s": round(r["wall_s"], 3),
            "ttft_ms": [round(r["ttft_mean_ms"], 1), round(r["ttft_max_ms"], 1)],
            "kv_peak": r["kv_blocks_peak"], "kv_closed_form": r["kv_blocks_closed_form_all_at_once"],
            "hit_tokens": r["prefix_hit_tokens"], "steps": r["engine_steps"], "cpu": None}


def summary_table(head, secondary, host):
    """The per-config figures as the last lines of stderr."""
    rows = [("decode_b64_ctx1920 (headline)", compact(head))]
    rows += [(k, compact(v)) for k, v in secondary.items() if "roofline" in v]
    log("")
    log(f"{'config':<36} {'us':>9} {'achieved':>10} {'unit':>8} {'frac':>7} {'bound':>5} {'cpu ms':>10} "
        f"{'cpu value':>10}")
    for name, c in rows:
        cpu = c.get("cpu") or ["-", "-"]
        log(f"{name:<36} {c['us']:>9} {c['ach']:>10} {c['unit']:>8} {c['frac']:>7} {c['bound']:>5} "
            f"{cpu[0]:>10} {cpu[1]:>10}")
    for k, v in secondary.items():
        if k.startswith("generate"):
            g = compact_generate(v)
            log(f"{k:<36} {g['tok_s']} new tok/s, wall {g['wall_s']} s, TTFT mean/max {g['ttft_ms']} ms, "
                f"KV peak {g['kv_peak']} pages (closed form {g['kv_closed_form']}), {g['hit_tokens']} hit tokens")
    if host:
        log(f"cpu baseline host: {host.get('model')}, {host.get('physical_cores')} cores, "
            f"{host['threads_used']} threads used")


def cpu_decode(batch, ctx, budget_s=10.0):
    """Oracle static_decode_attention (gather + SDPA, fp32) on one layer of the workload."""
    from oracle import attention as oa

    g = torch.Generator().manual_seed(0)
    blocks = cdiv(ctx, BS)
    cache = torch.randn(2, batch * blocks, BS, HKV, D, generator=g)
    bt = torch.randperm(batch * blocks, generator=g).view(batch, blocks).int()
    q = torch.randn(batch, H, D, generator=g)
    lens = torch.full((batch,), ctx, dtype=torch.int32)
    sec, runs = cpu_time(lambda: oa.static_decode_attention(q, cache, bt, lens, ctx, D ** -0.5), budget_s)
    kv_bytes = batch * ctx * HKV * D * 2 * 2
    return _cpu_line(kv_bytes / sec / 1e9, "GB/s", sec, runs,
                     f"oracle static_decode_attention (gather + SDPA, fp32), one layer of B{batch} x ctx {ctx} "
                     f"(7B shape), median of {runs} runs; GB/s of the same bf16 KV bytes as the GPU line")


def cpu_append(tokens_per_seq, seqs, budget_s=5.0):
    """Oracle apply_rope + store_kvcache (index_copy_) in fp32 on the same token count."""
    from oracle import rope as orope

    T = tokens_per_seq * seqs
    g = torch.Generator().manual_seed(T)
    q = torch.randn(T, H, D, generator=g)
    k = torch.randn(T, HKV, D, generator=g)
    v = torch.randn(T, HKV, D, generator=g)
    ct, st = orope.rope_tables(D, 4097, 1e6)
    pos = (torch.randint(128, 4097, (T,), generator=g) if tokens_per_seq == 1
           else torch.arange(tokens_per_seq).repeat(seqs))
    cos, sin = ct[pos], st[pos]
    cache = torch.zeros(2, 8192, BS, HKV, D)
    slots = torch.randperm(8192 * BS, generator=g)[:T]

    def run():
        qr, kr = orope.apply_rope(q, k, cos, sin)
        orope.store_kvcache(kr, v, cache, slots)

    sec, runs = cpu_time(run, budget_s)
    return _cpu_line(T * 19976 / sec / 1e9, "GB/s", sec, runs,
                     f"oracle apply_rope + store_kvcache (fp32), {T} tokens at the 7B shape, median of {runs} "
                     f"runs; GB/s of the same bf16 algorithmic bytes as the GPU line")


def cpu_prefill(name, budget_s=10.0):
    """Oracle paged_attention_torch (per-sequence SDPA loop, fp32) on the same shape."""
    from oracle import attention as oa
    from babyvllm.worker.context import AttentionMetadata

    specs = PREFILL_SHAPES[name]
    g = torch.Generator().manual_seed(len(specs))
    seq_lens = [c + n for c, n in specs]
    blocks = [cdiv(s_, BS) for s_ in seq_lens]
    total = sum(blocks)
    cache = torch.randn(2, total, BS, HKV, D, generator=g)
    perm = torch.randperm(total, generator=g).tolist()
    tables, i = [], 0
    for nblk in blocks:
        tables.append(perm[i:i + nblk] + [0] * (max(blocks) - nblk))
        i += nblk
    qsl = [0]
    for _, n in specs:
        qsl.append(qsl[-1] + n)
    ctx = [c for c, _ in specs]
    md = AttentionMetadata(torch.zeros(qsl[-1], dtype=torch.int64), torch.tensor(tables, dtype=torch.int32),
                           torch.tensor(qsl, dtype=torch.int32), torch.tensor(seq_lens, dtype=torch.int32),
                           torch.tensor(ctx, dtype=torch.int32), qsl, seq_lens, ctx, max(n for _, n in specs),
                           max(seq_lens))
    q = torch.randn(qsl[-1], H, D, generator=g)
    sec, runs = cpu_time(lambda: oa.paged_attention_torch(q, cache, md, D ** -0.5, H // HKV), budget_s)
    return _cpu_line(prefill_flops(specs) / sec / 1e12, "TFLOP/s", sec, runs,
                     f"oracle paged_attention_torch (per-sequence SDPA loop, fp32), {name} at the 7B shape, "
                     f"median of {runs} runs; TFLOP/s of the same visible-pair flops as the GPU line")


def cpu_step_kernel(name, budget_s=2.0):
    """The reference's torch path of a decode-step kernel (fp32) on the same shape:
    torch.argmax over the logits (the greedy sampler), the oracle's add + RMSNorm
    (babyvllm/layers/layernorm.py:27-37) and SiLU*mul."""
    from oracle import decode_step as ods

    hidden, inter, vocab = 3584, 18944, 152064
    g = torch.Generator().manual_seed(11)
    if name.startswith("argmax"):
        x = torch.randn(64, vocab, generator=g)
        fn, nbytes = (lambda: torch.argmax(x, dim=-1)), 64 * vocab * 2
    elif name.startswith("add_rms_norm"):
        rows = int(name.split("_")[3].split("x")[0])
        x = torch.randn(rows, hidden, generator=g)
        r = torch.randn(rows, hidden, generator=g)
        w = torch.rand(hidden, generator=g)
        fn, nbytes = (lambda: ods.fused_add_rms_norm(x, r, w, 1e-6)), rows * hidden * 2 * 4 + hidden * 2
    else:
        rows = int(name.split("_")[2].split("x")[0])
        gu = torch.randn(rows, 2 * inter, generator=g)
        fn, nbytes = (lambda: ods.silu_mul(gu)), rows * inter * 2 * 3
    sec, runs = cpu_time(fn, budget_s)
    return _cpu_line(nbytes / sec / 1e9, "GB/s", sec, runs,
                     f"torch / oracle path of {name} in fp32, median of {runs} runs; GB/s of the same bf16 "
                     f"algorithmic bytes as the GPU line")


def cpu_config1(budget_s=5.0):
    """Oracle step: apply_rope + store_kvcache + static_decode_attention (fp32), config 1."""
    from oracle import attention as oa
    from oracle import rope as orope

    lens, cache, bt, qkv, pos, slots = config1_inputs(100, "cpu")
    ct, st = orope.rope_tables(C1_D, 4096, 1e6)
    q = qkv[:, : C1_H * C1_D].view(C1_B, C1_H, C1_D)
    k = qkv[:, C1_H * C1_D:(C1_H + C1_HKV) * C1_D].view(C1_B, C1_HKV, C1_D)
    v = qkv[:, (C1_H + C1_HKV) * C1_D:].view(C1_B, C1_HKV, C1_D)
    seq_lens = lens.int()

    def run():
        qr, kr = orope.apply_rope(q, k, ct[pos], st[pos])
        orope.store_kvcache(kr, v, cache, slots)
        oa.static_decode_attention(qr, cache, bt, seq_lens, C1_BUCKET, C1_D ** -0.5)

    sec, runs = cpu_time(run, budget_s)
    return _cpu_line(config1_bytes(lens) / sec / 1e9, "GB/s", sec, runs,
                     f"oracle apply_rope + store_kvcache + static_decode_attention (fp32), the config-1 step "
                     f"(0.5B shape, B8, lengths U[100,512]), median of {runs} runs")


def read_traffic():
    if not os.path.exists(TRAFFIC_FILE):
        return None
    vals = {}
    with open(TRAFFIC_FILE) as f:
        for line in f:
            if ":" in line and not line.startswith("#"):
                k, v = line.split(":", 1)
                try:
                    vals[k.strip()] = float(v.split()[0])
                except (ValueError, IndexError):
                    pass
    return vals.get("hbm_bytes_per_launch")


def calib_copy(iters=20):
    """A plain device-to-device copy of known size, for scaling the FETCH/WRITE counters."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes": n, "iters": iters}), flush=True)


# -------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="headline only, no secondary lines")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default=None,
                    help="config1 | decode_b64 | decode_b8 | decode_b1 | append | prefill | prefill:<shape> | "
                         "step | e2e | cpu")
    ap.add_argument("--calib-copy", action="store_true")
    ap.add_argument("--tune", action="append", default=[], metavar="KNOB=VALUE",
                    help="set a library tuning knob (bvllm_set_tuning) before measuring; repeatable")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the paged-KV kernels would shard by KV head or by sequence, with no "
              "exchange inside attention). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    if args.calib_copy:
        calib_copy()
        return

    from babyvllm.kernels import _lib
    _lib.lib()  # fail loudly now if the HIP library is missing
    for kv in args.tune:
        knob, value = (int(x) for x in kv.split("="))
        if _lib.set_tuning(knob, value) < 0:
            raise SystemExit(f"unknown tuning knob {knob}")

    if args.only == "config1":
        r = bench_config1(args.warmup, args.steps)
        if not args.no_cpu:
            r["cpu_baseline"] = cpu_config1()
        print(json.dumps(r), flush=True)
        return
    if args.only == "cpu":
        print(json.dumps({"host": cpu_host(), "decode_b64": cpu_decode(64, 1920),
                          "prefill_1x(2048+4096)": cpu_prefill("1x(2048+4096)")}), flush=True)
        return
    if args.only == "decode_b64":
        r = bench_decode(64, 1920, args.warmup, args.steps)
        print(json.dumps(r), flush=True)
        return
    if args.only == "decode_b8":
        print(json.dumps(bench_decode(8, 1920, args.warmup, args.steps)), flush=True)
        return
    if args.only == "decode_b1":
        print(json.dumps(bench_decode(1, 32768, args.warmup, args.steps)), flush=True)
        return
    if args.only == "append":
        print(json.dumps({"decode64": bench_append(1, 64, args.warmup, args.steps),
                          "prefill8192": bench_append(128, 64, args.warmup, args.steps)}), flush=True)
        return
    if args.only == "prefill":
        print(json.dumps({n: bench_prefill(n, args.warmup, args.steps) for n in PREFILL_SHAPES}),
              flush=True)
        return
    if args.only == "e2e":
        print(json.dumps({"shared_prefix_caching_on": bench_generate(),
                          "distinct_caching_off": bench_generate(shared_len=0, caching=False)}), flush=True)
        return
    if args.only == "step":
        print(json.dumps(bench_step_kernels(args.warmup, args.steps)), flush=True)
        return
    if args.only and args.only.startswith("prefill:"):
        name = args.only.split(":", 1)[1]
        print(json.dumps({name: bench_prefill(name, args.warmup, args.steps)}), flush=True)
        return

    log("headline: decode B64 ctx1920 ...")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    head = bench_decode(64, 1920, args.warmup, args.steps)
    torch.cuda.synchronize()
    log(f"  {head['us_per_layer']:.2f} us/layer, {head['gb_s']:.0f} GB/s ({time.perf_counter() - t0:.1f} s)")

    secondary = {}
    cpu_jobs = {}  # line name -> CPU baseline of the same workload, run after the GPU lines
    if not args.quick:
        log("config 1: 0.5B-shape single-layer step ...")
        secondary["config1_step_0.5b_b8"] = bench_config1(args.warmup, args.steps)
        cpu_jobs["config1_step_0.5b_b8"] = lambda: cpu_config1()
        for b, c in ((8, 1920), (1, 32768), (64, 2048)):
            log(f"decode B{b} ctx{c} ...")
            key = f"decode_b{b}_ctx{c}"
            secondary[key] = bench_decode(b, c, args.warmup, args.steps)
            cpu_jobs[key] = (lambda b=b, c=c: cpu_decode(b, c, budget_s=3.0))
        log("append ...")
        secondary["append_decode_64tok"] = bench_append(1, 64, args.warmup, args.steps)
        cpu_jobs["append_decode_64tok"] = lambda: cpu_append(1, 64, budget_s=2.0)
        secondary["append_prefill_8192tok"] = bench_append(128, 64, args.warmup, args.steps)
        cpu_jobs["append_prefill_8192tok"] = lambda: cpu_append(128, 64, budget_s=3.0)
        for name in PREFILL_SHAPES:
            log(f"prefill {name} ...")
            key = f"prefill_{name}"
            secondary[key] = bench_prefill(name, args.warmup, max(5, args.steps // 5))
            cpu_jobs[key] = (lambda name=name: cpu_prefill(name, budget_s=3.0))
        log("decode-step kernels (argmax, add + RMSNorm, SiLU*mul) ...")
        step_lines = bench_step_kernels(args.warmup, max(5, args.steps // 5))
        secondary.update(step_lines)
        for key in step_lines:
            cpu_jobs[key] = (lambda key=key: cpu_step_kernel(key))
        log("end-to-end generate (config 5) ...")
        secondary["generate_shared_prefix_caching_on"] = bench_generate()
        secondary["generate_distinct_caching_off"] = bench_generate(shared_len=0, caching=False)
        for key in ("generate_shared_prefix_caching_on", "generate_distinct_caching_off"):
            secondary[key]["cpu_baseline"] = {
                "value": None, "note": "not timed: the reference's torch path on the CPU would take minutes per "
                                       "generated token of the 28-layer 7B model at 64 x 1920"}

    cpu = None
    host = None
    if not args.no_cpu:
        host = cpu_host()
        log(f"cpu baselines on {host.get('model')} ({host['threads_used']} threads) ...")
        cpu = cpu_decode(64, 1920, budget_s=15.0)
        for key, job in cpu_jobs.items():
            log(f"  cpu {key} ...")
            secondary[key]["cpu_baseline"] = job()

    kv_bytes = head["kv_bytes_per_layer"]
    ach = head["gb_s"]
    line = {
        "metric": METRIC,
        "value": round(kv_bytes * LAYERS / (head["step_ms"] * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) bf16 q/K/V, seeded random-permutation block tables, 28 distinct KV pools",
        "config": {
            "workload": "paged_decode_attention_b64_ctx1920_qwen2.5-7b_shape",
            "batch": 64, "context": 1920, "num_heads": H, "num_kv_heads": HKV, "head_dim": D,
            "block_size": BS, "calls_per_step": LAYERS, "split_plan": head["plan"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(ach, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(),
            "algorithmic_bytes_per_launch": kv_bytes,
            "launch_us": round(head["us_per_layer"], 3),
        },
        "cpu_baseline": cpu,
        "cpu_host": None if host is None else {k: host.get(k) for k in ("model", "physical_cores",
                                                                         "threads_used")},
    }
    if secondary:
        line["secondary"] = {k: (compact_generate(v) if k.startswith("generate") else compact(v))
                             for k, v in secondary.items()}
        line["legend"] = LEGEND
        line["reference_h100"] = {"decode_b64_ctx2048_gb_s": 2514.9, "prefill_1x(2048+4096)_ms": 1.2615,
                                  "generate_b64_distinct_tok_s": 1135.96}
    log("full secondary figures: " + json.dumps(secondary))
    summary_table(head, secondary, host)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
