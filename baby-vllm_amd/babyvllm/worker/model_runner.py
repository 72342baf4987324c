"""Runs scheduled steps on the model: eager prefill / mixed steps and captured decode steps
(babyvllm/worker/model_runner.py:90-542).

* ``allocate_kv_cache()`` gives every Attention layer a zeroed ``[2, NB + 1,
  16, Hkv, D]`` bf16 pool (the extra last page is the dummy page that padded
  rows of a captured batch write to) and returns NB. NB is
  ``cache_config.num_gpu_blocks``, or what ``gpu_memory_fraction`` of the free
  device memory holds.
* A step in which every sequence computes exactly one token, with the batch
  and context inside BATCH_BUCKETS × CTX_BUCKETS, replays a hipGraph captured
  once per (batch bucket, context bucket): the whole forward, the LM head into
  a static logits buffer and the greedy argmax kernel into a static token
  buffer. Its inputs come from ``DecodeInputs`` staging (one pinned buffer
  edited in place) by a single non-blocking copy into a device buffer of the
  same layout, which every captured graph reads; the attention kernels see
  ``max_seq_len`` = the context bucket, so the captured grid fits every replay.
* Any other step runs eagerly with metadata built from the scheduler output,
  then takes each sequence's last row of hidden states to the LM head.
Greedy requests (temperature 0) are sampled with the HIP argmax kernel;
others with torch softmax / top-p / multinomial on the host side of the path.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from babyvllm.kernels.argmax import greedy_argmax
from babyvllm.layers.attention import Attention
from babyvllm.models.qwen2 import Qwen2ForCausalLM
from babyvllm.worker.context import AttentionMetadata, set_forward_context
from babyvllm.worker.decode_inputs import DecodeInputs

BATCH_BUCKETS = [1, 2, 4, 8, 16, 32, 64]
CTX_BUCKETS = [256, 2048]


def ceil_to_bucket(value: int, buckets: list[int]) -> int | None:
    for b in buckets:
        if value <= b:
            return b
    return None


@dataclass
class StaticBuffers:
    input_ids: torch.Tensor
    position_ids: torch.Tensor
    block_tables: torch.Tensor
    seq_lens: torch.Tensor
    context_lens: torch.Tensor
    slot_mapping: torch.Tensor
    query_start_loc: torch.Tensor
    logits: torch.Tensor
    tokens: torch.Tensor


class ModelRunner:
    def __init__(self, model_config, cache_config=None, scheduler_config=None, device=None,
                 use_cuda_graphs: bool | None = None, seed: int = 0, init_std: float = 0.02):
        self.model_config = model_config
        self.cache_config = cache_config
        self.scheduler_config = scheduler_config
        self.block_size = cache_config.block_size if cache_config else model_config.block_size
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.dtype = torch.bfloat16
        self.use_cuda_graphs = (self.device.type == "cuda") if use_cuda_graphs is None else (
            bool(use_cuda_graphs) and self.device.type == "cuda")
        saved = torch.get_default_dtype()
        torch.set_default_dtype(self.dtype)
        try:
            with torch.device(self.device):
                self.model = Qwen2ForCausalLM(model_config)
        finally:
            torch.set_default_dtype(saved)
        self.model.eval()
        self.model.init_random(seed, std=init_std)
        self.num_blocks: int | None = None
        self._dummy_block = 0
        self._static: dict[tuple[int, int], StaticBuffers] = {}
        self._graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}
        self._pool = None
        self._decode_inputs: DecodeInputs | None = None
        self._dev_packed: torch.Tensor | None = None
        self._dev_inputs: dict[str, torch.Tensor] | None = None
        # Observability for tests and benchmarks: decode steps served by a graph
        # replay, and an optional callable(seqs, logits) shown every step's
        # logits rows (row i belongs to seqs[i]) before sampling.
        self.graph_replays = 0
        self.logits_observer = None
        self.max_blocks_per_seq = -(-max(CTX_BUCKETS) // self.block_size) + 1

    # ------------------------------------------------------------- KV cache

    def _attention_layers(self):
        return [m for m in self.model.modules() if isinstance(m, Attention)]

    def determine_num_blocks(self) -> int:
        cc = self.cache_config
        if cc is not None and cc.num_gpu_blocks:
            return int(cc.num_gpu_blocks)
        frac = cc.gpu_memory_fraction if cc is not None else 0.5
        free, _ = torch.cuda.mem_get_info(self.device)
        per_block = self.model_config.kv_bytes_per_token * self.block_size
        return max(1, int(free * frac) // per_block - 1)

    def allocate_kv_cache(self) -> int:
        if self.num_blocks is not None:
            return self.num_blocks
        usable = self.determine_num_blocks()
        cfg = self.model_config
        for layer in self._attention_layers():
            layer.kv_cache = torch.zeros(2, usable + 1, self.block_size, cfg.num_key_value_heads, cfg.head_dim,
                                         dtype=self.dtype, device=self.device)
        self._dummy_block = usable
        self.num_blocks = usable
        return usable

    # ----------------------------------------------------------- eager steps

    def prepare_inputs(self, scheduler_output):
        ids, positions, slots, tables = [], [], [], []
        qsl, seq_lens, ctx_lens = [0], [], []
        for seq in scheduler_output.scheduled_sequences:
            n = scheduler_output.num_scheduled_tokens[seq.seq_id]
            ctx = seq.num_computed_tokens
            ids.extend(seq.token_ids[ctx:ctx + n])
            positions.extend(range(ctx, ctx + n))
            slots.extend(scheduler_output.slot_mappings[seq.seq_id])
            tables.append(scheduler_output.block_tables[seq.seq_id])
            qsl.append(qsl[-1] + n)
            seq_lens.append(ctx + n)
            ctx_lens.append(ctx)
        width = max(len(t) for t in tables)
        dev = self.device
        md = AttentionMetadata(
            slot_mapping=torch.tensor(slots, dtype=torch.int64, device=dev),
            block_tables=torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.int32,
                                      device=dev),
            query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=dev),
            seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=dev),
            context_lens=torch.tensor(ctx_lens, dtype=torch.int32, device=dev),
            query_start_loc_cpu=qsl, seq_lens_cpu=seq_lens, context_lens_cpu=ctx_lens,
            max_query_len=max(qsl[i + 1] - qsl[i] for i in range(len(tables))),
            max_seq_len=max(seq_lens),
        )
        return (torch.tensor(ids, dtype=torch.int64, device=dev),
                torch.tensor(positions, dtype=torch.int64, device=dev), md)

    def _sample(self, logits, seqs) -> dict[int, int]:
        tokens = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
        greedy = all(s.sampling_params.temperature == 0.0 for s in seqs)
        greedy_argmax(logits, tokens)
        if not greedy:
            for i, s in enumerate(seqs):
                p = s.sampling_params
                if p.temperature == 0.0:
                    continue
                probs = F.softmax(logits[i].float() / p.temperature, dim=-1)
                if p.top_p < 1.0:
                    sp, si = torch.sort(probs, descending=True)
                    drop = torch.cumsum(sp, dim=-1) - sp > p.top_p
                    probs[si[drop]] = 0.0
                    probs = probs / probs.sum()
                tokens[i] = torch.multinomial(probs, 1)[0]
        out = tokens.cpu().tolist()
        return {s.seq_id: t for s, t in zip(seqs, out)}

    @torch.inference_mode()
    def _execute_eager(self, scheduler_output) -> dict[int, int]:
        input_ids, positions, md = self.prepare_inputs(scheduler_output)
        with set_forward_context(md):
            hidden = self.model(input_ids, positions)
        last = torch.tensor([e - 1 for e in md.query_start_loc_cpu[1:]], device=self.device)
        logits = self.model.compute_logits(hidden[last])
        if self.logits_observer is not None:
            self.logits_observer(scheduler_output.scheduled_sequences, logits)
        return self._sample(logits, scheduler_output.scheduled_sequences)

    # ---------------------------------------------------------- graph steps

    def _can_graph_decode(self, scheduler_output) -> bool:
        seqs = scheduler_output.scheduled_sequences
        if not self.use_cuda_graphs or not seqs or self.num_blocks is None:
            return False
        if any(scheduler_output.num_scheduled_tokens[s.seq_id] != 1 for s in seqs):
            return False
        if ceil_to_bucket(len(seqs), BATCH_BUCKETS) is None:
            return False
        return ceil_to_bucket(max(s.num_computed_tokens for s in seqs) + 1, CTX_BUCKETS) is not None

    def _ensure_static_buffers(self, batch_bucket: int, ctx_bucket: int) -> StaticBuffers:
        key = (batch_bucket, ctx_bucket)
        if key not in self._static:
            B, dev = batch_bucket, self.device
            host = self._host_inputs()
            if self._dev_inputs is None:
                # One device buffer with the host staging's packed layout: a step's
                # inputs arrive by a single copy, and every graph reads its rows.
                self._dev_packed = torch.zeros(host.packed.numel(), dtype=torch.uint8, device=dev)
                self._dev_inputs = host.device_views(self._dev_packed)
            v = self._dev_inputs
            self._static[key] = StaticBuffers(
                input_ids=v["input_ids"][:B], position_ids=v["positions"][:B],
                block_tables=v["block_tables"][:B], seq_lens=v["seq_lens"][:B],
                context_lens=v["context_lens"][:B], slot_mapping=v["slot_mapping"][:B],
                query_start_loc=torch.arange(B + 1, dtype=torch.int32, device=dev),
                logits=torch.zeros(B, self.model_config.vocab_size, dtype=self.dtype, device=dev),
                tokens=torch.zeros(B, dtype=torch.int64, device=dev),
            )
        return self._static[key]

    def _host_inputs(self) -> DecodeInputs:
        if self._decode_inputs is None:
            self._decode_inputs = DecodeInputs(max(BATCH_BUCKETS), self.max_blocks_per_seq, self.block_size,
                                               self._dummy_block, pin=self.device.type == "cuda")
        return self._decode_inputs

    def prepare_decode_inputs(self, seqs, block_tables, batch_bucket: int, ctx_bucket: int) -> StaticBuffers:
        buf = self._ensure_static_buffers(batch_bucket, ctx_bucket)
        host = self._host_inputs()
        host.update(seqs, block_tables, batch_bucket)
        self._dev_packed.copy_(host.packed, non_blocking=True)
        return buf

    @torch.inference_mode()
    def _forward_static(self, buf: StaticBuffers, batch_bucket: int, ctx_bucket: int) -> None:
        B = batch_bucket
        md = AttentionMetadata(
            slot_mapping=buf.slot_mapping, block_tables=buf.block_tables, query_start_loc=buf.query_start_loc,
            seq_lens=buf.seq_lens, context_lens=buf.context_lens,
            query_start_loc_cpu=list(range(B + 1)), seq_lens_cpu=[ctx_bucket] * B,
            context_lens_cpu=[ctx_bucket - 1] * B, max_query_len=1, max_seq_len=ctx_bucket)
        with set_forward_context(md):
            hidden = self.model(buf.input_ids, buf.position_ids)
        self.model.compute_logits(hidden, out=buf.logits)
        greedy_argmax(buf.logits, buf.tokens)

    def capture_one(self, batch_bucket: int, ctx_bucket: int, warmup_steps: int = 2):
        key = (batch_bucket, ctx_bucket)
        if key in self._graphs:
            return self._graphs[key]
        buf = self._ensure_static_buffers(batch_bucket, ctx_bucket)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(warmup_steps):
                self._forward_static(buf, batch_bucket, ctx_bucket)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self._pool):
            self._forward_static(buf, batch_bucket, ctx_bucket)
        if self._pool is None:
            self._pool = graph.pool()
        self._graphs[key] = graph
        return graph

    def _execute_decode_graph(self, scheduler_output) -> dict[int, int]:
        seqs = scheduler_output.scheduled_sequences
        n = len(seqs)
        bb = ceil_to_bucket(n, BATCH_BUCKETS)
        cb = ceil_to_bucket(max(s.num_computed_tokens for s in seqs) + 1, CTX_BUCKETS)
        # Stage first: a first capture's warm-up runs then compute this step's
        # own tokens (the replay rewrites the same K/V values).
        buf = self.prepare_decode_inputs(seqs, scheduler_output.block_tables, bb, cb)
        graph = self.capture_one(bb, cb)
        graph.replay()
        self.graph_replays += 1
        if self.logits_observer is not None:
            self.logits_observer(seqs, buf.logits[:n])
        if all(s.sampling_params.temperature == 0.0 for s in seqs):
            host = self._decode_inputs
            host.token_buffer[:bb].copy_(buf.tokens, non_blocking=True)
            torch.cuda.current_stream(self.device).synchronize()
            return {s.seq_id: int(t) for s, t in zip(seqs, host.tokens[:n])}
        return self._sample(buf.logits[:n], seqs)

    @torch.inference_mode()
    def execute_model(self, scheduler_output) -> dict[int, int]:
        if self._can_graph_decode(scheduler_output):
            return self._execute_decode_graph(scheduler_output)
        return self._execute_eager(scheduler_output)
