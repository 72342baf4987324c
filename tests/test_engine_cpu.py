"""The KV-cache manager, scheduler, engine loop and decode-input staging on the CPU
(ports tests/test_scheduler.py, test_prefix_caching.py, test_decode_inputs.py,
test_cuda_graphs.py and test_static_buffers.py of the reference)."""

import itertools
import random

import numpy as np
import pytest
import torch

from babyvllm.engine import LLMEngine
from babyvllm.kv_cache_manager import KVCacheManager
from babyvllm.scheduler import Scheduler
from babyvllm.sequence import SamplingParams, Sequence, SequenceFinishReason
from babyvllm.worker.decode_inputs import DecodeInputs
from babyvllm.worker.model_runner import BATCH_BUCKETS, CTX_BUCKETS, ceil_to_bucket


# ------------------------------------------------------------------ runners

class TokenRunner:
    """Fake model: the next token is a function of the sequence; EOS at length 15."""

    def __init__(self, block_size=16, num_blocks=100):
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.eos_id = 999

    def allocate_kv_cache(self):
        return self.num_blocks

    def execute_model(self, sched):
        return {s.seq_id: self.eos_id if len(s) >= 15 else (s.seq_id + len(s)) % 1000
                for s in sched.scheduled_sequences}


class KVCheckingRunner:
    """Writes token ids into a fake pool through the slot mapping and reads every
    sequence's context back through its block table; the sampled token depends
    on what was read, so a wrong table or an overwritten shared page shows."""

    def __init__(self, block_size, num_blocks):
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.pool = [None] * (num_blocks * block_size)

    def allocate_kv_cache(self):
        return self.num_blocks

    def execute_model(self, sched):
        bs = self.block_size
        for s in sched.scheduled_sequences:
            start, n = s.num_computed_tokens, sched.num_scheduled_tokens[s.seq_id]
            for slot, tok in zip(sched.slot_mappings[s.seq_id], s.token_ids[start:start + n]):
                self.pool[slot] = tok
        out = {}
        for s in sched.scheduled_sequences:
            length = s.num_computed_tokens + sched.num_scheduled_tokens[s.seq_id]
            table = sched.block_tables[s.seq_id]
            ctx = [self.pool[table[p // bs] * bs + p % bs] for p in range(length)]
            assert ctx == s.token_ids[:length], f"seq {s.seq_id} read back the wrong context"
            out[s.seq_id] = (sum(ctx) * 31 + length) % 1000
        return out


# --------------------------------------------------------------- scheduler

def test_preempted_sequence_is_not_scheduled_twice():
    kv = KVCacheManager(num_blocks=2, block_size=1)
    sch = Scheduler(kv, max_num_batched_tokens=32, max_num_seqs=2)
    a, b = Sequence([1]), Sequence([2])
    sch.add_seq(a)
    sch.add_seq(b)
    first = sch.schedule()
    assert len(first.scheduled_sequences) == 2 and len(sch.running) == 2
    sch.update_from_output(first, {a.seq_id: 3, b.seq_id: 4})
    second = sch.schedule()
    sch.update_from_output(second, {a.seq_id: 5})
    assert len(second.scheduled_sequences) == 1
    assert len(second.preempted_seqs) == 1


def _stress(num_blocks):
    Sequence._counter = itertools.count()
    runner = TokenRunner(block_size=4, num_blocks=num_blocks)
    engine = LLMEngine(runner, max_num_batched_tokens=32, max_num_seqs=8)
    rng = random.Random(42)
    for _ in range(20):
        prompt = [rng.randint(0, 100) for _ in range(rng.randint(1, 10))]
        engine.add_request(prompt, SamplingParams(max_tokens=rng.randint(5, 20), ignore_eos=True))
    outputs = {}
    while engine.has_unfinished_requests():
        sched_out = None
        for out in engine.step():
            outputs.setdefault(out.seq_id, []).extend(out.new_token_ids)
        kv = engine.kv_cache_manager
        assert kv.num_free_blocks + len(kv.used_block_ids) == num_blocks
        assert all(s.num_computed_tokens <= len(s) for s in engine.scheduler.running)
        del sched_out
    return [outputs[k] for k in sorted(outputs)]


def test_outputs_do_not_depend_on_preemption():
    large, small = _stress(1000), _stress(10)
    assert len(large) == 20 and large == small


def test_stop_token_finishes_without_being_emitted():
    runner = TokenRunner(block_size=4)
    engine = LLMEngine(runner, max_num_batched_tokens=32, max_num_seqs=8)
    engine.add_request([1, 2, 3], SamplingParams(max_tokens=50, stop_tokens={runner.eos_id}))
    out = list(engine.run().values())[0]
    assert out.finish_reason == SequenceFinishReason.STOP
    assert runner.eos_id not in out.new_token_ids


def test_too_long_prompt_finishes_with_length():
    engine = LLMEngine(TokenRunner(block_size=4, num_blocks=100), max_num_batched_tokens=8, max_num_seqs=4)
    sid = engine.add_request(list(range(20)), SamplingParams(max_tokens=5))
    out = engine.run()
    assert out[sid].finish_reason == SequenceFinishReason.LENGTH and out[sid].new_token_ids == []


# ----------------------------------------------------------- prefix caching

def _admit(kv, seq):
    hits = kv.get_computed_blocks(seq)
    kv.allocate_slots(seq, len(seq) - len(hits) * kv.block_size, hits)
    seq.advance_computed(len(seq))
    return hits


def test_same_prefix_shares_full_blocks():
    kv = KVCacheManager(16, 4, enable_prefix_caching=True)
    prefix = [1, 2, 3, 4, 5, 6, 7, 8]
    a, b = Sequence(prefix + [9, 10]), Sequence(prefix + [11, 12])
    assert _admit(kv, a) == []
    ta = kv.get_block_table(a)
    assert _admit(kv, b) == ta[:2]
    tb = kv.get_block_table(b)
    assert tb[:2] == ta[:2] and tb[2] != ta[2]
    assert [kv.ref_counts[x] for x in ta] == [2, 2, 1]
    assert (kv.num_hit_tokens, kv.num_queried_tokens) == (8, 20)
    kv._check_invariants()
    kv.free(a)
    assert [kv.ref_counts[x] for x in tb] == [1, 1, 1]
    kv._check_invariants()


def test_partial_block_is_not_shared():
    kv = KVCacheManager(16, 4, enable_prefix_caching=True)
    a = Sequence([1, 2, 3, 4, 5, 6])
    _admit(kv, a)
    assert kv.block_keys[kv.get_block_table(a)[1]] is None
    assert _admit(kv, Sequence([1, 2, 3, 4, 5, 6, 7])) == kv.get_block_table(a)[:1]
    kv._check_invariants()


def test_identical_prompt_recomputes_its_last_block_privately():
    kv = KVCacheManager(16, 4, enable_prefix_caching=True)
    prompt = [1, 2, 3, 4, 5, 6, 7, 8]
    a, b = Sequence(prompt), Sequence(prompt)
    _admit(kv, a)
    hits = kv.get_computed_blocks(b)
    assert len(hits) == 1
    kv.allocate_slots(b, len(b) - 4, hits)
    b.advance_computed(4)
    ta, tb = kv.get_block_table(a), kv.get_block_table(b)
    assert tb[0] == ta[0] and tb[1] != ta[1]
    assert kv.get_slot_mapping(b, 4)[0] == tb[1] * 4
    assert kv.block_keys[tb[1]] is None
    kv._check_invariants()


def test_freed_blocks_stay_cached_until_evicted():
    kv = KVCacheManager(4, 4, enable_prefix_caching=True)
    prefix = [1, 2, 3, 4, 5, 6, 7, 8]
    a = Sequence(prefix + [9])
    _admit(kv, a)
    ta = list(kv.get_block_table(a))
    kv.free(a)
    assert kv.num_free_blocks == 4
    c = Sequence(prefix + [50])
    assert _admit(kv, c) == ta[:2]
    kv.free(c)
    d = Sequence(list(range(100, 116)))
    _admit(kv, d)
    kv.free(d)
    kv._check_invariants()
    assert kv.get_computed_blocks(Sequence(prefix + [60])) == []


def test_can_allocate_counts_revived_blocks():
    kv = KVCacheManager(3, 4, enable_prefix_caching=True)
    prefix = [1, 2, 3, 4, 5, 6, 7, 8]
    a = Sequence(prefix + [9])
    _admit(kv, a)
    kv.free(a)
    y = Sequence([77])
    _admit(kv, y)
    assert kv.num_free_blocks == 2
    b = Sequence(prefix + [42])
    hits = kv.get_computed_blocks(b)
    assert len(hits) == 2
    assert not kv.can_allocate(b, 1, hits)
    kv.free(y)
    assert kv.can_allocate(b, 1, hits)
    kv.allocate_slots(b, 1, hits)
    assert kv.num_free_blocks == 0
    kv._check_invariants()


def test_disabled_prefix_caching_never_shares():
    kv = KVCacheManager(16, 4)
    prefix = [1, 2, 3, 4, 5, 6, 7, 8]
    a, b = Sequence(prefix + [9]), Sequence(prefix + [10])
    _admit(kv, a)
    assert _admit(kv, b) == []
    assert not set(kv.get_block_table(a)) & set(kv.get_block_table(b))
    assert kv.cached_blocks == {}


def _shared_prefix_requests(seed, n):
    rng = random.Random(seed)
    systems = [[rng.randint(0, 100) for _ in range(rng.randint(6, 13))] for _ in range(3)]
    return [(rng.choice(systems) + [rng.randint(0, 100) for _ in range(rng.randint(1, 5))], rng.randint(3, 12))
            for _ in range(n)]


def _run_checked(requests, num_blocks, caching, stagger):
    Sequence._counter = itertools.count()
    engine = LLMEngine(KVCheckingRunner(4, num_blocks), max_num_batched_tokens=64, max_num_seqs=8,
                       enable_prefix_caching=caching)
    first = requests[: len(requests) // 2] if stagger else requests
    rest = requests[len(first):]
    for prompt, mt in first:
        engine.add_request(prompt, SamplingParams(max_tokens=mt, ignore_eos=True))
    outputs, steps = {}, 0
    while engine.has_unfinished_requests() or rest:
        if rest and steps == 3:
            for prompt, mt in rest:
                engine.add_request(prompt, SamplingParams(max_tokens=mt, ignore_eos=True))
            rest = []
        for out in engine.step():
            outputs.setdefault(out.seq_id, []).extend(out.new_token_ids)
        engine.kv_cache_manager._check_invariants()
        steps += 1
        assert steps < 10_000
    return outputs, engine.kv_cache_manager


@pytest.mark.parametrize("num_blocks", [200, 12])
@pytest.mark.parametrize("stagger", [False, True])
def test_engine_outputs_match_with_and_without_caching(num_blocks, stagger):
    requests = _shared_prefix_requests(0, 24)
    off, _ = _run_checked(requests, num_blocks, False, stagger)
    on, kv = _run_checked(requests, num_blocks, True, stagger)
    assert len(on) == len(requests) and on == off
    assert kv.num_hit_tokens > 0
    assert kv.num_free_blocks == num_blocks


# ------------------------------------------------------------ decode staging

BS, MB, DUMMY = 16, 32, 9999


def _rebuilt(seqs, out, bucket):
    ids = np.zeros(bucket, np.int64)
    pos = np.zeros(bucket, np.int64)
    lens = np.zeros(bucket, np.int32)
    ctx = np.zeros(bucket, np.int32)
    slots = np.full(bucket, DUMMY * BS, np.int64)
    tables = np.full((bucket, MB), DUMMY, np.int32)
    for i, s in enumerate(seqs):
        p = s.num_computed_tokens
        ids[i], pos[i], lens[i], ctx[i] = s.token_ids[p], p, p + 1, p
        slots[i] = out.slot_mappings[s.seq_id][0]
        t = out.block_tables[s.seq_id]
        tables[i, :len(t)] = t
    return ids, pos, lens, ctx, slots, tables


def _check(host, seqs, out):
    bucket = ceil_to_bucket(len(seqs), BATCH_BUCKETS)
    host.update(seqs, out.block_tables, bucket)
    for got, want in zip((host.input_ids, host.positions, host.seq_lens, host.context_lens, host.slot_mapping,
                          host.block_tables), _rebuilt(seqs, out, bucket)):
        assert np.array_equal(got[:bucket], want)


def _run_staging(seed, num_blocks, caching, n_requests, max_num_seqs):
    rng = random.Random(seed)
    kv = KVCacheManager(num_blocks, BS, enable_prefix_caching=caching)
    sch = Scheduler(kv, max_num_batched_tokens=512, max_num_seqs=max_num_seqs)
    host = DecodeInputs(64, MB, BS, DUMMY, pin=False)
    shared = [rng.randrange(10, 900) for _ in range(2 * BS)]
    for _ in range(n_requests):
        if rng.random() < 0.6:
            prompt = shared + [rng.randrange(10, 900) for _ in range(rng.randrange(1, 40))]
        else:
            prompt = [rng.randrange(10, 900) for _ in range(rng.randrange(5, 120))]
        sch.add_seq(Sequence(prompt, SamplingParams(temperature=0.0, max_tokens=rng.randrange(1, 70),
                                                    ignore_eos=True)))
    decode_steps = preempted = 0
    for _ in range(3000):
        if not sch.has_unfinished():
            break
        out = sch.schedule()
        preempted += len(out.preempted_seqs)
        seqs = out.scheduled_sequences
        if seqs and all(out.num_scheduled_tokens[s.seq_id] == 1 for s in seqs):
            _check(host, seqs, out)
            decode_steps += 1
        sch.update_from_output(out, {s.seq_id: 10 + (s.seq_id * 7 + len(s)) % 800 for s in seqs})
        sch.pop_finished()
    assert not sch.has_unfinished()
    return decode_steps, preempted


@pytest.mark.parametrize("caching", [False, True])
def test_incremental_staging_matches_a_full_rebuild(caching):
    steps, _ = _run_staging(1, 2000, caching, 40, 64)
    assert steps > 50


@pytest.mark.parametrize("caching", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_incremental_staging_matches_a_full_rebuild_under_preemption(seed, caching):
    steps, preempted = _run_staging(seed, 26, caching, 30, 12)
    assert steps > 20 and preempted > 0


def test_shrinking_batch_clears_dropped_rows():
    host = DecodeInputs(8, MB, BS, DUMMY, pin=False)
    sch = Scheduler(KVCacheManager(200, BS), max_num_batched_tokens=512, max_num_seqs=8)
    for i in range(4):
        sch.add_seq(Sequence([10 + i] * 20, SamplingParams(temperature=0.0, max_tokens=3 + 5 * i, ignore_eos=True)))
    out = sch.schedule()
    sch.update_from_output(out, {s.seq_id: 11 for s in out.scheduled_sequences})
    sizes = []
    while sch.has_unfinished():
        out = sch.schedule()
        _check(host, out.scheduled_sequences, out)
        sizes.append(len(out.scheduled_sequences))
        sch.update_from_output(out, {s.seq_id: 11 for s in out.scheduled_sequences})
        sch.pop_finished()
    assert sizes[0] == 4 and sizes[-1] == 1


def test_decode_slot_equals_the_table_formula():
    kv = KVCacheManager(50, BS)
    seq = Sequence(list(range(10, 60)))
    kv.allocate_slots(seq, 50)
    seq.advance_computed(50)
    seq.append_token(5)
    kv.allocate_slots(seq, 1)
    table = kv.get_block_table(seq)
    assert kv.get_slot_mapping(seq, 1) == [table[50 // BS] * BS + 50 % BS]


def test_recomputed_sequence_rewrites_its_row():
    host = DecodeInputs(4, MB, BS, DUMMY, pin=False)
    assert isinstance(host.t_block_tables, torch.Tensor) and host.block_tables.shape == (4, MB)
    seq = Sequence(list(range(10, 30)))
    seq.advance_computed(20)
    seq.append_token(7)
    host.update([seq], {seq.seq_id: [1, 2]}, 1)
    assert list(host.block_tables[0, :3]) == [1, 2, DUMMY]
    before = (seq.seq_id, seq.num_preemptions)
    seq.reset_for_recompute()
    assert (seq.seq_id, seq.num_preemptions) != before
    seq.advance_computed(20)
    host.update([seq], {seq.seq_id: [5, 6]}, 1)
    assert list(host.block_tables[0, :3]) == [5, 6, DUMMY]
    assert host.slot_mapping[0] == 6 * BS + 4


def test_buckets():
    assert [ceil_to_bucket(v, BATCH_BUCKETS) for v in (1, 3, 64, 65)] == [1, 4, 64, None]
    assert [ceil_to_bucket(v, CTX_BUCKETS) for v in (128, 256, 257, 2049)] == [256, 256, 2048, None]


def test_static_buffers_on_cpu():
    from babyvllm.config import CacheConfig, ModelConfig
    from babyvllm.worker.model_runner import ModelRunner

    cfg = ModelConfig(vocab_size=100, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=4, rms_norm_eps=1e-6,
                      max_position_embeddings=2048, rope_theta=10000.0, tie_word_embeddings=False)
    runner = ModelRunner(cfg, cache_config=CacheConfig(), device="cpu")
    buf = runner._ensure_static_buffers(batch_bucket=4, ctx_bucket=256)
    assert buf.block_tables.shape == (4, 2048 // 16 + 1) and buf.logits.shape == (4, 100)
