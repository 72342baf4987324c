"""Pages of the KV pool: reference counts, an LRU free list and a prefix index.

Producer of the path's inputs: it decides which page every token's K/V goes to
(``get_slot_mapping``, slot = page · block_size + offset) and which pages a
sequence reads (``get_block_table``). Public names, attributes and behaviour
follow the reference's KVCacheManager (babyvllm/kv_cache_manager.py:11-199),
whose tests pin them:

* pages are handed out least-recently-freed first; a freed page keeps its
  prefix key until it is handed out again, so a later request can revive it;
* with prefix caching, a full page is keyed by (hash of the previous page's
  key, its own token ids); a new sequence reuses the longest run of keyed
  pages at its start, but never its last prompt token's page (at least one
  prompt token is computed so that it yields logits);
* pages are registered when allocated, before the forward pass writes them:
  a sequence that hits them in the same step reads them after the same
  layer's store, which runs before attention for every token;
* a sequence is freed tail first, so its own suffix is evicted before a
  prefix that other requests may share.
"""

from __future__ import annotations

from collections import OrderedDict

from babyvllm.sequence import Sequence

# (hash of the previous page's key or None, the page's token ids)
BlockKey = tuple


class KVCacheManager:
    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = False):
        if num_blocks <= 0 or block_size <= 0:
            raise AssertionError("num_blocks and block_size must be > 0")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.enable_prefix_caching = enable_prefix_caching
        self.reset()

    # ------------------------------------------------------------------ state

    def reset(self) -> None:
        self.free_block_ids: OrderedDict[int, None] = OrderedDict((b, None) for b in range(self.num_blocks))
        self.used_block_ids: set[int] = set()
        self.ref_counts = [0] * self.num_blocks
        self.block_keys: list[BlockKey | None] = [None] * self.num_blocks
        self.cached_blocks: dict[BlockKey, int] = {}
        self.request_blocks: dict[int, list[int]] = {}
        self.num_registered_blocks: dict[int, int] = {}
        self.num_queried_tokens = 0
        self.num_hit_tokens = 0

    @property
    def num_free_blocks(self) -> int:
        return len(self.free_block_ids)

    @property
    def num_used_blocks(self) -> int:
        return self.num_blocks - len(self.free_block_ids)

    @property
    def prefix_cache_hit_rate(self) -> float:
        return self.num_hit_tokens / self.num_queried_tokens if self.num_queried_tokens else 0.0

    def _check_invariants(self) -> None:
        assert self.num_free_blocks + len(self.used_block_ids) == self.num_blocks
        held = [0] * self.num_blocks
        for table in self.request_blocks.values():
            for b in table:
                held[b] += 1
        assert held == self.ref_counts, "reference counts disagree with the block tables"
        for b in range(self.num_blocks):
            assert (self.ref_counts[b] == 0) == (b in self.free_block_ids), f"block {b}: free list vs refs"
            if self.block_keys[b] is not None:
                assert self.cached_blocks.get(self.block_keys[b]) == b, f"block {b}: key not indexed"
        for key, b in self.cached_blocks.items():
            assert self.block_keys[b] == key, f"index maps a key to block {b} holding another key"

    # ---------------------------------------------------------------- lookups

    def get_block_table(self, seq: Sequence) -> list[int]:
        return self.request_blocks.get(seq.seq_id, [])

    def get_slot_mapping(self, seq: Sequence, num_new_tokens: int) -> list[int]:
        """Cache slots of the next ``num_new_tokens`` tokens of ``seq``."""
        table = self.request_blocks.get(seq.seq_id, [])
        bs = self.block_size
        first = seq.num_computed_tokens
        last_page = (first + num_new_tokens - 1) // bs
        assert last_page < len(table), f"seq {seq.seq_id} position {first + num_new_tokens - 1} has no block"
        return [table[p // bs] * bs + p % bs for p in range(first, first + num_new_tokens)]

    def _key(self, seq: Sequence, page: int) -> BlockKey:
        parent = seq.block_hashes[page - 1] if page else None
        return (parent, tuple(seq.token_ids[page * self.block_size:(page + 1) * self.block_size]))

    def _hash_pages(self, seq: Sequence, num_tokens: int) -> None:
        """Extend seq.block_hashes over the full pages of its first num_tokens tokens."""
        full = min(num_tokens, len(seq)) // self.block_size
        while len(seq.block_hashes) < full:
            seq.block_hashes.append(hash(self._key(seq, len(seq.block_hashes))))

    def get_computed_blocks(self, seq: Sequence) -> list[int]:
        """Keyed pages covering the start of a new sequence (read-only)."""
        if not self.enable_prefix_caching or seq.seq_id in self.request_blocks:
            return []
        limit = (len(seq) - 1) // self.block_size
        self._hash_pages(seq, limit * self.block_size)
        hits: list[int] = []
        for page in range(limit):
            b = self.cached_blocks.get(self._key(seq, page))
            if b is None:
                break
            hits.append(b)
        return hits

    # ------------------------------------------------------------- allocation

    def num_blocks_needed(self, seq: Sequence, num_new_tokens: int, computed_blocks: list[int] = ()) -> int:
        tokens = seq.num_computed_tokens + len(computed_blocks) * self.block_size + num_new_tokens
        pages = -(-tokens // self.block_size)
        held = len(self.request_blocks.get(seq.seq_id, [])) + len(computed_blocks)
        return max(0, pages - held)

    def _revived(self, computed_blocks) -> int:
        """Hits that sit on the free list (reference count 0) and leave it when reused."""
        return sum(1 for b in computed_blocks if self.ref_counts[b] == 0)

    def can_allocate(self, seq: Sequence, num_new_tokens: int, computed_blocks: list[int] = ()) -> bool:
        need = self.num_blocks_needed(seq, num_new_tokens, computed_blocks) + self._revived(computed_blocks)
        return self.num_free_blocks >= need

    def _take_free(self) -> int:
        """Least recently freed page; it loses its prefix key."""
        b, _ = self.free_block_ids.popitem(last=False)
        key = self.block_keys[b]
        if key is not None:
            del self.cached_blocks[key]
            self.block_keys[b] = None
        return b

    def _hold(self, b: int) -> None:
        if self.ref_counts[b] == 0:
            del self.free_block_ids[b]
            self.used_block_ids.add(b)
        self.ref_counts[b] += 1

    def allocate_slots(self, seq: Sequence, num_new_tokens: int, computed_blocks: list[int] = ()) -> None:
        """Give seq pages for num_new_tokens more tokens (after computed_blocks, for a new seq).

        The caller then advances ``num_computed_tokens`` past the hit pages
        before building the slot mapping.
        """
        fresh = self.num_blocks_needed(seq, num_new_tokens, computed_blocks)
        assert self.num_free_blocks >= fresh + self._revived(computed_blocks), (
            f"OOM: cannot allocate for seq {seq.seq_id}. Free: {self.num_free_blocks}, needed: {fresh}")
        table = self.request_blocks.setdefault(seq.seq_id, [])
        if computed_blocks:
            assert not table and seq.num_computed_tokens == 0, f"seq {seq.seq_id} already has blocks"
            for b in computed_blocks:
                self._hold(b)
                table.append(b)
        for _ in range(fresh):
            b = self._take_free()
            self.ref_counts[b] = 1
            self.used_block_ids.add(b)
            table.append(b)
        if self.enable_prefix_caching:
            hit = len(computed_blocks) * self.block_size
            if seq.num_computed_tokens == 0:
                self.num_queried_tokens += hit + num_new_tokens
                self.num_hit_tokens += hit
            self.cache_full_blocks(seq, seq.num_computed_tokens + hit + num_new_tokens)

    def cache_full_blocks(self, seq: Sequence, num_tokens: int) -> None:
        """Key the full pages of seq's first num_tokens tokens (first holder of a content wins)."""
        table = self.request_blocks[seq.seq_id]
        full = num_tokens // self.block_size
        self._hash_pages(seq, full * self.block_size)
        done = self.num_registered_blocks.get(seq.seq_id, 0)
        for page in range(done, full):
            b = table[page]
            if self.block_keys[b] is not None:
                continue
            key = self._key(seq, page)
            if key not in self.cached_blocks:
                self.cached_blocks[key] = b
                self.block_keys[b] = key
        self.num_registered_blocks[seq.seq_id] = max(done, full)

    def free(self, seq: Sequence) -> None:
        assert seq.seq_id in self.request_blocks, (
            f"free() called on seq {seq.seq_id} with no allocated blocks. Double-free or free-without-allocate.")
        for b in reversed(self.request_blocks.pop(seq.seq_id)):
            self.ref_counts[b] -= 1
            if self.ref_counts[b] == 0:
                self.used_block_ids.discard(b)
                self.free_block_ids[b] = None
        self.num_registered_blocks.pop(seq.seq_id, None)

    def free_if_allocated(self, seq: Sequence) -> None:
        if seq.seq_id in self.request_blocks:
            self.free(seq)
