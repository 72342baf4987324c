"""The serving slice on the CPU: KV-page bookkeeping, scheduling, the engine
loop and the staging of a captured decode step's inputs.

The behaviours are those the reference's own CPU tests pin
(tests/test_prefix_caching.py, test_scheduler.py, test_decode_inputs.py,
test_cuda_graphs.py, test_static_buffers.py). Their inputs and known answers
are kept below as data tables; the checks are written for this build:

* ``PoolModel`` states the page pool's rules as naively as possible (a free
  list, whole-prefix tuples as page identities, linear scans) and runs in
  lock step with ``KVCacheManager`` through scripted scenarios and seeded
  random workloads; every observable (tables, reference counts, free count,
  hits, indexed pages, admission verdicts) must agree after every operation.
* Every scheduler step of random workloads is audited (no request scheduled
  twice or both scheduled and preempted, slots for exactly the scheduled
  tokens, budgets respected), and generation must not depend on how often the
  pool forced preemptions.
* ``DecodeInputs`` is driven by synthetic decode batches (arrivals,
  departures, recomputes, reorderings, page growth) and by a real scheduler,
  and compared field by field with the row contract rebuilt from scratch.
"""

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


# ================================================================ page pool

class PoolModel:
    """The page pool's rules, stated directly.

    Pages are taken from the front of ``free`` (least recently freed) and
    released tail first onto its back. A full page's identity is the tuple of
    every token up to its end; the first page to carry an identity keeps it,
    a page loses it when it is taken again, and a freed page keeps it until
    then. A new request reuses the leading pages whose identities match its
    prompt, but never the page of its last prompt token.
    """

    def __init__(self, pages, page_size, caching):
        self.bs = page_size
        self.caching = caching
        self.free = list(range(pages))
        self.refs = [0] * pages
        self.identity = [None] * pages
        self.tables = {}
        self.tokens = {}
        self.offered = {}
        self.hit_tokens = self.queried_tokens = 0

    def _page_with(self, ident):
        for p, x in enumerate(self.identity):
            if x == ident:
                return p
        return None

    def lookup(self, tokens):
        if not self.caching:
            return []
        hits = []
        for i in range((len(tokens) - 1) // self.bs):
            p = self._page_with(tuple(tokens[: (i + 1) * self.bs]))
            if p is None:
                break
            hits.append(p)
        return hits

    def _take(self):
        p = self.free.pop(0)
        self.identity[p] = None
        self.refs[p] = 1
        return p

    def _offer(self, name):
        toks, table = self.tokens[name], self.tables[name]
        full = len(toks) // self.bs
        for i in range(self.offered.get(name, 0), full):
            ident = tuple(toks[: (i + 1) * self.bs])
            if self.caching and self.identity[table[i]] is None and self._page_with(ident) is None:
                self.identity[table[i]] = ident
        self.offered[name] = max(self.offered.get(name, 0), full)

    def admits(self, tokens):
        hits = self.lookup(tokens)
        fresh = -(-len(tokens) // self.bs) - len(hits)
        revived = sum(self.refs[p] == 0 for p in hits)
        return fresh + revived <= len(self.free)

    def admit(self, name, tokens):
        hits = self.lookup(tokens)
        for p in hits:
            if self.refs[p] == 0:
                self.free.remove(p)
            self.refs[p] += 1
        fresh = -(-len(tokens) // self.bs) - len(hits)
        self.tables[name] = hits + [self._take() for _ in range(fresh)]
        self.tokens[name] = list(tokens)
        if self.caching:
            self.queried_tokens += len(tokens)
            self.hit_tokens += len(hits) * self.bs
        self._offer(name)
        return hits

    def grows(self, name):
        """True if one more token of ``name`` fits (a new page when it starts one)."""
        needs_page = len(self.tokens[name]) % self.bs == 0
        return not needs_page or len(self.free) > 0

    def append(self, name, token):
        if len(self.tokens[name]) % self.bs == 0:
            self.tables[name].append(self._take())
        self.tokens[name].append(token)
        self._offer(name)

    def release(self, name):
        for p in reversed(self.tables.pop(name)):
            self.refs[p] -= 1
            if self.refs[p] == 0:
                self.free.append(p)
        self.tokens.pop(name)
        self.offered.pop(name, None)


class PoolPair:
    """A KVCacheManager and a PoolModel driven together by request name."""

    def __init__(self, pages, page_size, caching):
        self.kv = KVCacheManager(pages, page_size, enable_prefix_caching=caching)
        self.model = PoolModel(pages, page_size, caching)
        self.seqs = {}
        self.last_table = {}

    def agree(self):
        kv, m = self.kv, self.model
        kv._check_invariants()
        assert kv.ref_counts == m.refs
        assert kv.num_free_blocks == len(m.free)
        assert [k is not None for k in kv.block_keys] == [x is not None for x in m.identity]
        for name, seq in self.seqs.items():
            assert kv.get_block_table(seq) == m.tables[name], name
        if m.caching:
            assert (kv.num_hit_tokens, kv.num_queried_tokens) == (m.hit_tokens, m.queried_tokens)

    def fits(self, tokens):
        seq = Sequence(tokens)
        hits = self.kv.get_computed_blocks(seq)
        verdict = self.kv.can_allocate(seq, len(seq) - len(hits) * self.kv.block_size, hits)
        assert verdict == self.model.admits(tokens)
        return verdict

    def admit(self, name, tokens):
        """Admits a request as the scheduler does and marks its prompt computed;
        returns the number of reused pages."""
        seq = Sequence(tokens)
        hits = self.kv.get_computed_blocks(seq)
        assert hits == self.model.lookup(tokens)
        n_new = len(seq) - len(hits) * self.kv.block_size
        self.kv.allocate_slots(seq, n_new, hits)
        self.model.admit(name, tokens)
        seq.advance_computed(len(hits) * self.kv.block_size)
        # The first computed token lands at offset 0 of the first fresh page.
        table = self.kv.get_block_table(seq)
        assert self.kv.get_slot_mapping(seq, n_new)[0] == table[len(hits)] * self.kv.block_size
        seq.advance_computed(n_new)
        self.seqs[name] = seq
        self.agree()
        return len(hits)

    def decode(self, name, token):
        """One more token for ``name``; releases it instead if the pool is full."""
        seq = self.seqs[name]
        seq.append_token(token)
        ok = self.kv.can_allocate(seq, 1)
        assert ok == self.model.grows(name)
        if ok:
            self.kv.allocate_slots(seq, 1)
            self.model.append(name, token)
            pos, bs = len(seq) - 1, self.kv.block_size
            assert self.kv.get_slot_mapping(seq, 1) == [self.model.tables[name][pos // bs] * bs + pos % bs]
            seq.advance_computed(1)
        else:
            self.release(name)
        self.agree()
        return ok

    def release(self, name):
        seq = self.seqs.pop(name)
        self.last_table[name] = list(self.kv.get_block_table(seq))
        self.kv.free(seq)
        self.model.release(name)
        self.agree()

    def table(self, name):
        if name in self.seqs:
            return self.kv.get_block_table(self.seqs[name])
        return self.last_table[name]


# Scenarios and known answers of the reference's prefix-caching tests
# (tests/test_prefix_caching.py:19-135): pool pages, page size, caching, script.
#   admit NAME TOKENS HITS      reused leading pages
#   refs NAME COUNTS            reference counts of NAME's pages
#   same X Y K                  the first K pages of X and Y are equal, the rest differ
#   tokens HIT QUERIED          prefix-cache token counters
#   free NAME / free_pages N / unkeyed NAME I (page I of NAME has no identity)
#   probe TOKENS HITS           lookup without admitting
#   fits TOKENS BOOL            admission verdict
#   disjoint X Y / index_empty
P8 = [1, 2, 3, 4, 5, 6, 7, 8]
SCENARIOS = {
    "same prefix shares full pages": (16, 4, True, [
        ("admit", "a", P8 + [9, 10], 0), ("admit", "b", P8 + [11, 12], 2), ("same", "a", "b", 2),
        ("refs", "a", [2, 2, 1]), ("tokens", 8, 20), ("free", "a"), ("refs", "b", [1, 1, 1])]),
    "partial page is not shared": (16, 4, True, [
        ("admit", "a", [1, 2, 3, 4, 5, 6], 0), ("unkeyed", "a", 1),
        ("admit", "b", [1, 2, 3, 4, 5, 6, 7], 1), ("same", "a", "b", 1)]),
    "identical prompt recomputes its last page privately": (16, 4, True, [
        ("admit", "a", P8, 0), ("admit", "b", P8, 1), ("same", "a", "b", 1), ("unkeyed", "b", 1)]),
    "freed pages stay cached until taken": (4, 4, True, [
        ("admit", "a", P8 + [9], 0), ("free", "a"), ("free_pages", 4),
        ("admit", "c", P8 + [50], 2), ("same", "a", "c", 2), ("free", "c"),
        ("admit", "d", list(range(100, 116)), 0), ("free", "d"), ("probe", P8 + [60], 0)]),
    "admission counts revived pages": (3, 4, True, [
        ("admit", "a", P8 + [9], 0), ("free", "a"), ("admit", "y", [77], 0), ("free_pages", 2),
        ("probe", P8 + [42], 2), ("fits", P8 + [42], False), ("free", "y"), ("fits", P8 + [42], True),
        ("admit", "b", P8 + [42], 2), ("free_pages", 0)]),
    "caching off never shares": (16, 4, False, [
        ("admit", "a", P8 + [9], 0), ("admit", "b", P8 + [10], 0), ("disjoint", "a", "b"), ("index_empty",)]),
}


@pytest.mark.parametrize("name", list(SCENARIOS))
def test_pool_scenarios(name):
    pages, size, caching, script = SCENARIOS[name]
    pair = PoolPair(pages, size, caching)
    for op, *args in script:
        if op == "admit":
            assert pair.admit(args[0], args[1]) == args[2], (op, args)
        elif op == "free":
            pair.release(args[0])
        elif op == "refs":
            assert [pair.kv.ref_counts[p] for p in pair.table(args[0])] == args[1]
        elif op == "same":
            x, y, k = pair.table(args[0]), pair.table(args[1]), args[2]
            assert x[:k] == y[:k] and all(a != b for a, b in zip(x[k:], y[k:]))
        elif op == "tokens":
            assert (pair.kv.num_hit_tokens, pair.kv.num_queried_tokens) == (args[0], args[1])
        elif op == "free_pages":
            assert pair.kv.num_free_blocks == args[0]
        elif op == "unkeyed":
            assert pair.kv.block_keys[pair.table(args[0])[args[1]]] is None
        elif op == "probe":
            assert len(pair.kv.get_computed_blocks(Sequence(args[0]))) == args[1]
        elif op == "fits":
            assert pair.fits(args[0]) == args[1]
        elif op == "disjoint":
            assert not set(pair.table(args[0])) & set(pair.table(args[1]))
        elif op == "index_empty":
            assert pair.kv.cached_blocks == {}
        else:
            raise AssertionError(op)


@pytest.mark.parametrize("caching", [True, False])
@pytest.mark.parametrize("seed,pages,size", [(0, 24, 4), (1, 9, 4), (2, 40, 3), (3, 14, 2), (4, 64, 16)])
def test_pool_agrees_with_the_model_on_random_workloads(seed, pages, size, caching):
    rng = random.Random(seed)
    systems = [[rng.randrange(50) for _ in range(rng.randrange(size, 4 * size))] for _ in range(3)]
    pair = PoolPair(pages, size, caching)
    names = itertools.count()
    for _ in range(400):
        r = rng.random()
        live = list(pair.seqs)
        if r < 0.35 or not live:
            tokens = rng.choice(systems)[: rng.randrange(1, 4 * size)] + \
                [rng.randrange(50) for _ in range(rng.randrange(0, 2 * size))]
            if not tokens:
                tokens = [rng.randrange(50)]
            if rng.random() < 0.15 and live:  # an exact copy of a live prompt
                tokens = list(pair.model.tokens[rng.choice(live)])
            if pair.fits(tokens):
                pair.admit(f"r{next(names)}", tokens)
        elif r < 0.85:
            pair.decode(rng.choice(live), rng.randrange(50))
        else:
            pair.release(rng.choice(live))
    for name in list(pair.seqs):
        pair.release(name)
    assert pair.kv.num_free_blocks == pages


# ================================================================ scheduler

def _audit(sch, out):
    """Properties every step must have, whatever the workload."""
    ids = [s.seq_id for s in out.scheduled_sequences]
    assert len(ids) == len(set(ids)), "a request was scheduled twice"
    assert not set(ids) & {s.seq_id for s in out.preempted_seqs}, "a request was both scheduled and preempted"
    assert sum(out.num_scheduled_tokens.values()) <= sch.max_num_batched_tokens
    assert len(ids) <= sch.max_num_seqs
    bs = sch.kv_cache_manager.block_size
    for s in out.scheduled_sequences:
        n = out.num_scheduled_tokens[s.seq_id]
        table = out.block_tables[s.seq_id]
        assert len(out.slot_mappings[s.seq_id]) == n
        assert len(table) * bs >= s.num_computed_tokens + n
        want = [table[p // bs] * bs + p % bs for p in range(s.num_computed_tokens, s.num_computed_tokens + n)]
        assert out.slot_mappings[s.seq_id] == want
    for s in out.preempted_seqs:
        assert s.num_computed_tokens == 0 and s in sch.waiting


class ContentModel:
    """Fake model whose next token is a function of the request's tokens only,
    so a recomputed request continues exactly as before; EOS when a request
    reaches 15 tokens."""

    eos_id = 999

    def __init__(self, block_size=4, num_blocks=100, sch=None):
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.sch = sch

    def allocate_kv_cache(self):
        return self.num_blocks

    def execute_model(self, out):
        if self.sch is not None:
            _audit(self.sch, out)
        return {s.seq_id: self.eos_id if len(s) >= 15 else (sum(s.token_ids) * 7 + len(s)) % 997
                for s in out.scheduled_sequences}


# Known answer of tests/test_scheduler.py:6-30: two one-token prompts in a pool
# of two one-token pages. Step 1 runs both; in step 2 each needs a second page,
# so the newer request is preempted and only the older one runs.
TWO_PAGE_POOL = {"pages": 2, "page_size": 1, "prompts": [[1], [2]], "scheduled": [2, 1], "preempted": [0, 1]}


def test_preemption_in_a_two_page_pool():
    case = TWO_PAGE_POOL
    sch = Scheduler(KVCacheManager(case["pages"], case["page_size"]), max_num_batched_tokens=32, max_num_seqs=2)
    seqs = [Sequence(p) for p in case["prompts"]]
    for s in seqs:
        sch.add_seq(s)
    for want_sched, want_pre in zip(case["scheduled"], case["preempted"]):
        out = sch.schedule()
        _audit(sch, out)
        assert (len(out.scheduled_sequences), len(out.preempted_seqs)) == (want_sched, want_pre)
        # Only the scheduled requests get tokens; updating must accept that.
        sch.update_from_output(out, {s.seq_id: 3 + s.seq_id for s in out.scheduled_sequences})
    assert [s.seq_id for s in sch.running] == [seqs[0].seq_id]
    assert list(sch.waiting) == [seqs[1]]


def _generate(num_blocks, seed=42, n=20):
    Sequence._counter = itertools.count()
    runner = ContentModel(block_size=4, num_blocks=num_blocks)
    engine = LLMEngine(runner, max_num_batched_tokens=32, max_num_seqs=8)
    runner.sch = engine.scheduler
    rng = random.Random(seed)
    for _ in range(n):
        prompt = [rng.randrange(101) for _ in range(rng.randrange(1, 11))]
        engine.add_request(prompt, SamplingParams(max_tokens=rng.randrange(5, 21), ignore_eos=True))
    tokens, preempted = {}, 0
    while engine.has_unfinished_requests():
        for o in engine.step():
            tokens.setdefault(o.seq_id, []).extend(o.new_token_ids)
        kv = engine.kv_cache_manager
        assert kv.num_free_blocks + len(kv.used_block_ids) == num_blocks
        assert all(s.num_computed_tokens <= len(s) for s in engine.scheduler.running)
        preempted += sum(s.num_preemptions for s in engine.scheduler.running)
    return [tokens[k] for k in sorted(tokens)], preempted


def test_generation_does_not_depend_on_preemption():
    roomy, none = _generate(1000)
    assert none == 0 and len(roomy) == 20
    for pool in (10, 8):
        tight, forced = _generate(pool)
        assert forced > 0, f"a pool of {pool} pages should force preemptions"
        assert tight == roomy


def test_stop_token_finishes_without_being_emitted():
    runner = ContentModel(block_size=4)
    engine = LLMEngine(runner, max_num_batched_tokens=32, max_num_seqs=8)
    engine.add_request([1, 2, 3], SamplingParams(max_tokens=50, stop_tokens={runner.eos_id}))
    (out,) = engine.run().values()
    assert out.finish_reason == SequenceFinishReason.STOP
    assert runner.eos_id not in out.new_token_ids and len(out.new_token_ids) == 12


def test_prompt_over_the_token_budget_finishes_with_length():
    engine = LLMEngine(ContentModel(block_size=4), max_num_batched_tokens=8, max_num_seqs=4)
    rid = engine.add_request(list(range(20)), SamplingParams(max_tokens=5))
    out = engine.run()[rid]
    assert out.finish_reason == SequenceFinishReason.LENGTH and out.new_token_ids == []


class PoolEchoModel:
    """Writes each scheduled token into a fake pool through its slot, reads every
    request's whole context back through its table, and samples from what it
    read: a wrong table, slot or an overwritten shared page changes the output."""

    def __init__(self, block_size, num_blocks, sch_ref):
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.pool = np.full(num_blocks * block_size, -1, dtype=np.int64)
        self.sch_ref = sch_ref

    def allocate_kv_cache(self):
        return self.num_blocks

    def execute_model(self, out):
        _audit(self.sch_ref[0], out)
        bs = self.block_size
        for s in out.scheduled_sequences:
            c, n = s.num_computed_tokens, out.num_scheduled_tokens[s.seq_id]
            self.pool[out.slot_mappings[s.seq_id]] = s.token_ids[c:c + n]
        sampled = {}
        for s in out.scheduled_sequences:
            length = s.num_computed_tokens + out.num_scheduled_tokens[s.seq_id]
            table = np.asarray(out.block_tables[s.seq_id], dtype=np.int64)
            pos = np.arange(length)
            seen = self.pool[table[pos // bs] * bs + pos % bs]
            assert seen.tolist() == s.token_ids[:length], f"request {s.seq_id} read a wrong context"
            sampled[s.seq_id] = int((seen.sum() * 31 + length) % 1000)
        return sampled


def _echo_run(requests, num_blocks, caching, late_half):
    Sequence._counter = itertools.count()
    sch_ref = []
    engine = LLMEngine(PoolEchoModel(4, num_blocks, sch_ref), max_num_batched_tokens=64, max_num_seqs=8,
                       enable_prefix_caching=caching)
    sch_ref.append(engine.scheduler)
    now, later = (requests[: len(requests) // 2], requests[len(requests) // 2:]) if late_half else (requests, [])
    for prompt, n in now:
        engine.add_request(prompt, SamplingParams(max_tokens=n, ignore_eos=True))
    got, step = {}, 0
    while engine.has_unfinished_requests() or later:
        if later and step == 3:
            for prompt, n in later:
                engine.add_request(prompt, SamplingParams(max_tokens=n, ignore_eos=True))
            later = []
        for o in engine.step():
            got.setdefault(o.seq_id, []).extend(o.new_token_ids)
        engine.kv_cache_manager._check_invariants()
        step += 1
        assert step < 10_000
    return got, engine.kv_cache_manager


def _prefix_heavy_requests(seed, n):
    rng = random.Random(seed)
    heads = [[rng.randrange(101) for _ in range(rng.randrange(6, 14))] for _ in range(3)]
    return [(rng.choice(heads) + [rng.randrange(101) for _ in range(rng.randrange(1, 6))], rng.randrange(3, 13))
            for _ in range(n)]


@pytest.mark.parametrize("num_blocks", [200, 12])
@pytest.mark.parametrize("late_half", [False, True])
def test_prefix_caching_changes_no_output(num_blocks, late_half):
    requests = _prefix_heavy_requests(0, 24)
    off, _ = _echo_run(requests, num_blocks, False, late_half)
    on, kv = _echo_run(requests, num_blocks, True, late_half)
    assert len(on) == len(requests) and on == off
    assert kv.num_hit_tokens > 0 and kv.num_free_blocks == num_blocks


# =========================================================== decode staging

PAGE, WIDTH, DUMMY = 16, 32, 9999


def _contract(seqs, tables, bucket, max_batch):
    """The staged rows, rebuilt from scratch: row i is the token at seqs[i]'s
    num_computed_tokens; rows past the batch are padding (token 0, lengths 0,
    the dummy page's slot and table)."""
    want = {
        "input_ids": np.zeros(bucket, np.int64), "positions": np.zeros(bucket, np.int64),
        "seq_lens": np.zeros(bucket, np.int32), "context_lens": np.zeros(bucket, np.int32),
        "slot_mapping": np.full(bucket, DUMMY * PAGE, np.int64),
        "block_tables": np.full((max_batch, WIDTH), DUMMY, np.int32),
    }
    for i, s in enumerate(seqs):
        p = s.num_computed_tokens
        t = tables[s.seq_id]
        want["input_ids"][i] = s.token_ids[p]
        want["positions"][i] = p
        want["context_lens"][i] = p
        want["seq_lens"][i] = p + 1
        want["slot_mapping"][i] = t[p // PAGE] * PAGE + p % PAGE
        want["block_tables"][i, :len(t)] = t
    return want


def _assert_staged(host, seqs, tables, bucket):
    want = _contract(seqs, tables, bucket, host.max_batch)
    for name, arr in want.items():
        got = getattr(host, name)
        got = got if name == "block_tables" else got[:bucket]
        assert np.array_equal(got, arr), name


def _bucket(n):
    return ceil_to_bucket(n, BATCH_BUCKETS)


class SyntheticBatches:
    """Decode batches that change the way a serving loop changes them:
    requests arrive and leave, are recomputed into new pages, keep or change
    their row, and gain a page every PAGE tokens."""

    def __init__(self, seed, max_batch):
        self.rng = random.Random(seed)
        self.max_batch = max_batch
        self.live = []
        self.tables = {}
        self.next_page = 0

    def _pages(self, n):
        pages = [(self.next_page + k * 7) % (DUMMY - 1) for k in range(n)]
        self.next_page += 13 * n + 1
        return pages

    def _new(self):
        length = self.rng.randrange(1, 9 * PAGE)
        s = Sequence([self.rng.randrange(10, 900) for _ in range(length)])
        s.advance_computed(length - 1)
        self.tables[s.seq_id] = self._pages(-(-length // PAGE))
        return s

    def step(self):
        rng = self.rng
        if self.live and rng.random() < 0.3:
            for s in rng.sample(self.live, rng.randrange(1, len(self.live) + 1) if rng.random() < 0.2 else 1):
                self.live.remove(s)
        while len(self.live) < self.max_batch and (not self.live or rng.random() < 0.3):
            self.live.append(self._new())
        if self.live and rng.random() < 0.2:  # recompute into fresh pages
            s = rng.choice(self.live)
            s.reset_for_recompute()
            s.advance_computed(len(s) - 1)
            self.tables[s.seq_id] = self._pages(-(-len(s) // PAGE))
        if rng.random() < 0.15:
            rng.shuffle(self.live)
        return list(self.live)

    def advance(self, seqs):
        """Every request of the step samples a token."""
        for s in seqs:
            s.append_token(self.rng.randrange(10, 900))
            s.advance_computed(1)
            if s.num_computed_tokens // PAGE >= len(self.tables[s.seq_id]):
                self.tables[s.seq_id].extend(self._pages(1))


@pytest.mark.parametrize("seed,max_batch", [(0, 8), (1, 64), (2, 3), (3, 64)])
def test_staging_follows_synthetic_batches(seed, max_batch):
    gen = SyntheticBatches(seed, max_batch)
    host = DecodeInputs(64, WIDTH, PAGE, DUMMY, pin=False)
    sizes = set()
    for _ in range(300):
        seqs = gen.step()
        if any(-(-(s.num_computed_tokens + 1) // PAGE) > WIDTH for s in seqs):
            break
        bucket = _bucket(len(seqs))
        assert host.update(seqs, gen.tables, bucket) == len(seqs)
        _assert_staged(host, seqs, gen.tables, bucket)
        sizes.add(len(seqs))
        gen.advance(seqs)
    assert len(sizes) > 2


def _scheduled_decode_run(seed, num_blocks, caching, n_requests, max_num_seqs):
    rng = random.Random(seed)
    sch = Scheduler(KVCacheManager(num_blocks, PAGE, enable_prefix_caching=caching),
                    max_num_batched_tokens=512, max_num_seqs=max_num_seqs)
    host = DecodeInputs(64, WIDTH, PAGE, DUMMY, pin=False)
    shared = [rng.randrange(10, 900) for _ in range(2 * PAGE)]
    for _ in range(n_requests):
        own = [rng.randrange(10, 900) for _ in range(rng.randrange(1, 40) if rng.random() < 0.6 else 0)]
        prompt = shared + own if own else [rng.randrange(10, 900) for _ in range(rng.randrange(5, 120))]
        sch.add_seq(Sequence(prompt, SamplingParams(temperature=0.0, max_tokens=rng.randrange(1, 70),
                                                    ignore_eos=True)))
    decode_steps = preemptions = 0
    for _ in range(3000):
        if not sch.has_unfinished():
            break
        out = sch.schedule()
        _audit(sch, out)
        preemptions += len(out.preempted_seqs)
        seqs = out.scheduled_sequences
        if seqs and all(out.num_scheduled_tokens[s.seq_id] == 1 for s in seqs):
            bucket = _bucket(len(seqs))
            host.update(seqs, out.block_tables, bucket)
            _assert_staged(host, seqs, out.block_tables, bucket)
            decode_steps += 1
        sch.update_from_output(out, {s.seq_id: 10 + (s.seq_id * 7 + len(s)) % 800 for s in seqs})
        sch.pop_finished()
    assert not sch.has_unfinished()
    return decode_steps, preemptions


# (seed, pool pages, requests, seats, minimum decode steps, preemption expected)
SCHEDULED_STAGING = [(1, 2000, 40, 64, 50, False), (0, 26, 30, 12, 20, True), (1, 26, 30, 12, 20, True),
                     (2, 26, 30, 12, 20, True)]


@pytest.mark.parametrize("caching", [False, True])
@pytest.mark.parametrize("case", SCHEDULED_STAGING)
def test_staging_follows_the_scheduler(case, caching):
    seed, pages, n, seats, min_steps, preempts = case
    steps, preempted = _scheduled_decode_run(seed, pages, caching, n, seats)
    assert steps > min_steps
    if preempts:
        assert preempted > 0, "this pool is meant to force preemptions"


def test_rows_released_by_a_shrinking_batch_return_to_padding():
    gen = SyntheticBatches(5, 8)
    host = DecodeInputs(8, WIDTH, PAGE, DUMMY, pin=False)
    seqs = [gen._new() for _ in range(6)]
    for n in (6, 5, 3, 1):
        batch = seqs[:n]
        host.update(batch, gen.tables, _bucket(n))
        _assert_staged(host, batch, gen.tables, _bucket(n))
        assert (host.block_tables[n:] == DUMMY).all()
        gen.advance(batch)


# Known answers of tests/test_decode_inputs.py:113-150.
SLOT_CASE = {"prompt_len": 50, "pool": 50, "pos": 50}
RECOMPUTE_CASE = {"prompt_len": 20, "table_before": [1, 2], "table_after": [5, 6], "slot_after": 6 * PAGE + 4}


def test_decode_slot_is_the_table_formula():
    kv = KVCacheManager(SLOT_CASE["pool"], PAGE)
    seq = Sequence(list(range(10, 10 + SLOT_CASE["prompt_len"])))
    kv.allocate_slots(seq, len(seq))
    seq.advance_computed(len(seq))
    seq.append_token(5)
    kv.allocate_slots(seq, 1)
    table, pos = kv.get_block_table(seq), SLOT_CASE["pos"]
    assert kv.get_slot_mapping(seq, 1) == [table[pos // PAGE] * PAGE + pos % PAGE]


def test_recompute_with_a_table_of_the_same_length_rewrites_the_row():
    case = RECOMPUTE_CASE
    host = DecodeInputs(4, WIDTH, PAGE, DUMMY, pin=False)
    assert isinstance(host.t_block_tables, torch.Tensor) and host.block_tables.shape == (4, WIDTH)
    seq = Sequence(list(range(10, 10 + case["prompt_len"])))
    seq.advance_computed(case["prompt_len"])
    seq.append_token(7)
    host.update([seq], {seq.seq_id: case["table_before"]}, 1)
    assert host.block_tables[0, :3].tolist() == case["table_before"] + [DUMMY]
    key = (seq.seq_id, seq.num_preemptions)
    seq.reset_for_recompute()
    assert (seq.seq_id, seq.num_preemptions) != key
    seq.advance_computed(case["prompt_len"])
    host.update([seq], {seq.seq_id: case["table_after"]}, 1)
    assert host.block_tables[0, :3].tolist() == case["table_after"] + [DUMMY]
    assert host.slot_mapping[0] == case["slot_after"]


# Bucket known answers (tests/test_cuda_graphs.py:4-12): value -> bucket.
BATCH_BUCKET_CASES = {1: 1, 3: 4, 64: 64, 65: None}
CTX_BUCKET_CASES = {128: 256, 256: 256, 257: 2048, 2049: None}


def test_graph_buckets():
    assert {v: ceil_to_bucket(v, BATCH_BUCKETS) for v in BATCH_BUCKET_CASES} == BATCH_BUCKET_CASES
    assert {v: ceil_to_bucket(v, CTX_BUCKETS) for v in CTX_BUCKET_CASES} == CTX_BUCKET_CASES


def test_static_decode_buffers_on_cpu():
    from babyvllm.config import CacheConfig, ModelConfig
    from babyvllm.worker.model_runner import ModelRunner

    cfg = ModelConfig(vocab_size=100, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=4, rms_norm_eps=1e-6,
                      max_position_embeddings=2048, rope_theta=10000.0, tie_word_embeddings=False)
    runner = ModelRunner(cfg, cache_config=CacheConfig(), device="cpu")
    buf = runner._ensure_static_buffers(batch_bucket=4, ctx_bucket=256)
    assert buf.block_tables.shape == (4, 2048 // 16 + 1) and buf.logits.shape == (4, 100)
