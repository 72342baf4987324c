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

Secondary lines (same method): decode B8/ctx1920, B1/ctx32768, B64/ctx2048 (the
reference's published H100 point), RoPE + KV append (decode 64 tokens, prefill
8192 tokens), the four varlen prefill configurations in TFLOP/s, and the decode
step's other kernels (greedy argmax over 64 x 152,064 logits, residual add +
RMSNorm and SiLU*mul at 64 and 8192 rows) in GB/s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
                       [--only NAME] [--calib-copy]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
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
    # N(0,1) q; the 1/sqrt(128) enters as the softmax scale, as Attention passes it.
    q = torch.randn(batch, H, D, device="cuda", dtype=torch.bfloat16, generator=g)
    seq_lens = torch.full((batch,), ctx, dtype=torch.int32, device="cuda")
    return q, caches, tables, seq_lens


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

    q, caches, tables, seq_lens = build_decode(batch, ctx, layers, seed=batch + ctx)
    scale = D ** -0.5

    def fwd():
        for i in range(layers):
            paged_decode_attention(q, caches[i], tables[i], seq_lens, scale, max_seq_len=ctx)

    ms, _ = time_graph(fwd, warmup, iters)
    kv_bytes = batch * ctx * HKV * D * 2 * 2
    per_launch_us = ms * 1e3 / layers
    plan = decode_split_plan(batch, HKV, BS, tables[0].shape[1], ctx, _num_sms(0))
    del q, caches, tables, seq_lens
    torch.cuda.empty_cache()
    return {
        "batch": batch, "context": ctx, "plan": list(plan),
        "us_per_layer": per_launch_us,
        "gb_s": kv_bytes / (per_launch_us * 1e-6) / 1e9,
        "frac_of_hbm_peak": kv_bytes / (per_launch_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "kv_bytes_per_layer": kv_bytes,
        "step_ms": ms,
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
            "algorithmic_bytes": nbytes}


PREFILL_SHAPES = {
    "64x128_fresh": [(0, 128)] * 64,
    "8x(1024+128)": [(1024, 128)] * 8,
    "1x(2048+4096)": [(2048, 4096)],
    "1x512+63x(1000+1)": [(0, 512)] + [(1000, 1)] * 63,
}


def prefill_flops(specs):
    return 512 * H * sum(sum(c + i + 1 for i in range(n)) for c, n in specs)


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
    q = torch.randn(sum(q_lens), H, D, device="cuda", dtype=torch.bfloat16, generator=g)

    def fwd():
        for i in range(layers):
            paged_prefill_attention(q, caches[i], mds[i], D ** -0.5)

    ms, _ = time_graph(fwd, warmup, iters)
    per_us = ms * 1e3 / layers
    flops = prefill_flops(specs)
    del caches, mds, q
    torch.cuda.empty_cache()
    return {"us_per_layer": per_us, "tflop_s": flops / (per_us * 1e-6) / 1e12,
            "frac_of_bf16_peak": flops / (per_us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, "flop": flops}


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
                     "algorithmic_bytes": nbytes, "calls_per_replay": reps}

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
            peak_pages = max(peak_pages, len(engine.kv_cache_manager.used_block_ids))
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

def cpu_baseline(batch, ctx, budget_s=15.0):
    """Oracle restatement of the reference's torch decode (gather + SDPA, fp32) on this host."""
    from oracle import attention as oa

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    blocks = cdiv(ctx, BS)
    cache = torch.randn(2, batch * blocks, BS, HKV, D, generator=g)
    bt = torch.randperm(batch * blocks, generator=g).view(batch, blocks).int()
    q = torch.randn(batch, H, D, generator=g)
    lens = torch.full((batch,), ctx, dtype=torch.int32)
    oa.static_decode_attention(q, cache, bt, lens, ctx, D ** -0.5)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        oa.static_decode_attention(q, cache, bt, lens, ctx, D ** -0.5)
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    kv_bytes = batch * ctx * HKV * D * 2 * 2
    return {
        "value": kv_bytes / sec / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle static_decode_attention (gather + SDPA, fp32) on one layer of the "
                   f"same workload (B{batch}, ctx {ctx}, 7B shape), median of {len(times)} runs, "
                   f"{sec * 1e3:.1f} ms per layer"),
    }


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
                    help="decode_b64 | decode_b8 | decode_b1 | append | prefill | prefill:<shape> | step | e2e")
    ap.add_argument("--calib-copy", action="store_true")
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
    if not args.quick:
        for b, c in ((8, 1920), (1, 32768), (64, 2048)):
            log(f"decode B{b} ctx{c} ...")
            secondary[f"decode_b{b}_ctx{c}"] = bench_decode(b, c, args.warmup, args.steps)
        log("append ...")
        secondary["append_decode_64tok"] = bench_append(1, 64, args.warmup, args.steps)
        secondary["append_prefill_8192tok"] = bench_append(128, 64, args.warmup, args.steps)
        for name in PREFILL_SHAPES:
            log(f"prefill {name} ...")
            secondary[f"prefill_{name}"] = bench_prefill(name, args.warmup, max(5, args.steps // 5))
        log("decode-step kernels (argmax, add + RMSNorm, SiLU*mul) ...")
        secondary.update(bench_step_kernels(args.warmup, max(5, args.steps // 5)))
        log("end-to-end generate (config 5) ...")
        secondary["generate_shared_prefix_caching_on"] = bench_generate()
        secondary["generate_distinct_caching_off"] = bench_generate(shared_len=0, caching=False)
        secondary["reference_h100_published"] = {
            "decode_b64_ctx2048_gb_s": 2514.9, "prefill_1x(2048+4096)_ms": 1.2615,
            "generate_b64_distinct_caching_off_tok_s": 1135.96, "generate_ttft_ms": 2902.94,
            "source": "results_28Oct2026_H100_flash_decode/decode_attn_bench.json:1200-1208; "
                      "results_28Oct2026_H100_flash_decode/comparison_baby_partition_auto.json:705-707; "
                      "results_26Oct2026_H100/prefill_attn_bench_torch2.13.json:43-46",
        }

    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline(64, 1920)

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
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
