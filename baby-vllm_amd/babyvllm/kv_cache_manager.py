"""The paged KV pool's bookkeeping: which pages a request holds, which are free, and which can be shared.

Producer of the hot path's inputs: it decides the cache slot of every new
token (``get_slot_mapping``: slot = page · block_size + offset) and the pages
a request attends to (``get_block_table``). Public surface and behaviour of
the reference's KVCacheManager (babyvllm/kv_cache_manager.py:11-199), which
its tests pin:

* a free page is taken least-recently-freed first, and a freed page keeps its
  prefix identity until it is taken again, so a later request can revive it;
* with prefix caching on, a new request reuses the longest run of indexed full
  pages at the start of its prompt, but never the page of its last prompt
  token (at least one token is computed, to produce logits);
* pages are indexed when they are allocated, before the forward pass writes
  them: a request admitted later in the same step may read them, since each
  layer stores every token's K/V before its attention runs;
* a request's pages are released tail first, so its private suffix is reused
  before a prefix other requests may share.

Design of this build:

* Page state is struct-of-arrays: a numpy reference count per page and an
  intrusive doubly linked ring of the free pages (``_prev`` / ``_next``, one
  slot per page plus a sentinel at index ``num_blocks``), ordered from least
  to most recently freed. Taking a page, freeing one and reviving a cached
  free page are O(1) index updates.
* A full page's prefix identity is a 16-byte BLAKE2b digest chained over the
  prompt: digest(page i) = BLAKE2b(digest(page i−1) ‖ token ids of page i as
  little-endian int64). It names the whole prefix up to the page, so one
  dictionary lookup per page finds a shared prefix; equal digests are taken
  as equal prefixes (a 128-bit collision). Digests are cached on the sequence
  (``Sequence.page_digests``) and extended as pages fill.
* ``ref_counts``, ``block_keys``, ``cached_blocks`` and ``used_block_ids`` are
  read-only views of that state under the reference's names, for its tests.
"""

from __future__ import annotations

import hashlib

import numpy as np

from babyvllm.sequence import Sequence


def _chain_digest(parent: bytes | None, tokens) -> bytes:
    h = hashlib.blake2b(digest_size=16)
    if parent is not None:
        h.update(parent)
    h.update(np.asarray(tokens, dtype="<i8").tobytes())
    return h.digest()


class KVCacheManager:
    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = False):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError(f"a KV pool needs pages and a page size, got {num_blocks} x {block_size}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.enable_prefix_caching = enable_prefix_caching
        self.reset()

    def reset(self) -> None:
        n = self.num_blocks
        self._refs = np.zeros(n, dtype=np.int32)
        # Free ring: pages 0 .. n-1 in order, sentinel n.
        self._next = np.empty(n + 1, dtype=np.int64)
        self._prev = np.empty(n + 1, dtype=np.int64)
        order = np.arange(n + 1)
        self._next[:] = np.roll(order, -1)
        self._prev[:] = np.roll(order, 1)
        self._n_free = n
        self._digest_of_page: list[bytes | None] = [None] * n
        self._page_of_digest: dict[bytes, int] = {}
        self._tables: dict[int, list[int]] = {}
        self._indexed: dict[int, int] = {}  # seq_id -> leading pages already offered to the index
        self.num_queried_tokens = 0
        self.num_hit_tokens = 0

    # ------------------------------------------------------ the free ring

    def _ring_unlink(self, page: int) -> None:
        nxt, prv = self._next[page], self._prev[page]
        self._next[prv] = nxt
        self._prev[nxt] = prv
        self._n_free -= 1

    def _ring_push(self, page: int) -> None:
        """Appends a page at the most-recently-freed end."""
        tail = self._prev[self.num_blocks]
        self._next[tail] = page
        self._prev[page] = tail
        self._next[page] = self.num_blocks
        self._prev[self.num_blocks] = page
        self._n_free += 1

    def _take_oldest_free(self) -> int:
        """The least recently freed page; it loses its prefix identity."""
        page = int(self._next[self.num_blocks])
        self._ring_unlink(page)
        digest = self._digest_of_page[page]
        if digest is not None:
            del self._page_of_digest[digest]
            self._digest_of_page[page] = None
        self._refs[page] = 1
        return page

    def _share(self, page: int) -> None:
        if self._refs[page] == 0:
            self._ring_unlink(page)
        self._refs[page] += 1

    # ------------------------------------------------------------- counts

    @property
    def num_free_blocks(self) -> int:
        return self._n_free

    @property
    def num_used_blocks(self) -> int:
        return self.num_blocks - self._n_free

    @property
    def prefix_cache_hit_rate(self) -> float:
        return self.num_hit_tokens / self.num_queried_tokens if self.num_queried_tokens else 0.0

    # Read-only views under the reference's names (its tests read them).
    @property
    def ref_counts(self) -> list[int]:
        return self._refs.tolist()

    @property
    def block_keys(self) -> list[bytes | None]:
        return list(self._digest_of_page)

    @property
    def cached_blocks(self) -> dict[bytes, int]:
        return dict(self._page_of_digest)

    @property
    def used_block_ids(self) -> set[int]:
        return set(np.flatnonzero(self._refs).tolist())

    def _check_invariants(self) -> None:
        held = np.zeros(self.num_blocks, dtype=np.int64)
        for table in self._tables.values():
            np.add.at(held, np.asarray(table, dtype=np.int64), 1)
        assert np.array_equal(held, self._refs), "reference counts differ from the pages the tables hold"
        ring, page = [], int(self._next[self.num_blocks])
        while page != self.num_blocks:
            ring.append(page)
            page = int(self._next[page])
            assert len(ring) <= self.num_blocks, "free ring does not close"
        assert len(ring) == self._n_free, "free ring length differs from the free count"
        assert sorted(ring) == np.flatnonzero(self._refs == 0).tolist(), "free ring differs from unreferenced pages"
        for p, d in enumerate(self._digest_of_page):
            if d is not None:
                assert self._page_of_digest.get(d) == p, f"page {p}: digest not indexed"
        for d, p in self._page_of_digest.items():
            assert self._digest_of_page[p] == d, f"index maps a digest to page {p}, which holds another"

    # ----------------------------------------------------------- lookups

    def get_block_table(self, seq: Sequence) -> list[int]:
        return self._tables.get(seq.seq_id, [])

    def get_slot_mapping(self, seq: Sequence, num_new_tokens: int) -> list[int]:
        """Cache slots of the ``num_new_tokens`` tokens from ``seq.num_computed_tokens`` on."""
        table = self._tables.get(seq.seq_id, [])
        bs = self.block_size
        first = seq.num_computed_tokens
        last = first + num_new_tokens - 1
        if last // bs >= len(table):
            raise RuntimeError(f"sequence {seq.seq_id}: token {last} lies past its {len(table)} pages")
        if num_new_tokens == 1:
            return [table[first // bs] * bs + first % bs]
        pos = np.arange(first, first + num_new_tokens)
        return (np.asarray(table, dtype=np.int64)[pos // bs] * bs + pos % bs).tolist()

    def _digests(self, seq: Sequence, n_pages: int) -> list[bytes]:
        """The sequence's chained page digests, extended to its first n_pages full pages."""
        bs = self.block_size
        d = seq.page_digests
        while len(d) < n_pages:
            i = len(d)
            d.append(_chain_digest(d[i - 1] if i else None, seq.token_ids[i * bs:(i + 1) * bs]))
        return d

    def get_computed_blocks(self, seq: Sequence) -> list[int]:
        """Indexed pages that cover the start of a request not yet holding pages (read-only)."""
        if not self.enable_prefix_caching or seq.seq_id in self._tables:
            return []
        reusable = (len(seq) - 1) // self.block_size  # never the last prompt token's page
        hits = []
        for digest in self._digests(seq, reusable):
            page = self._page_of_digest.get(digest)
            if page is None:
                break
            hits.append(page)
        return hits

    # -------------------------------------------------------- allocation

    def num_blocks_needed(self, seq: Sequence, num_new_tokens: int, computed_blocks=()) -> int:
        """Fresh pages ``seq`` needs for ``num_new_tokens`` more tokens past ``computed_blocks``."""
        upto = seq.num_computed_tokens + len(computed_blocks) * self.block_size + num_new_tokens
        have = len(self._tables.get(seq.seq_id, ())) + len(computed_blocks)
        return max(0, -(-upto // self.block_size) - have)

    def _free_pages_taken(self, seq: Sequence, num_new_tokens: int, computed_blocks) -> int:
        # Hit pages nobody holds sit on the free ring, and reusing them takes them off it.
        revived = int(np.count_nonzero(self._refs[np.asarray(computed_blocks, dtype=np.int64)] == 0)) \
            if len(computed_blocks) else 0
        return self.num_blocks_needed(seq, num_new_tokens, computed_blocks) + revived

    def can_allocate(self, seq: Sequence, num_new_tokens: int, computed_blocks=()) -> bool:
        return self._free_pages_taken(seq, num_new_tokens, computed_blocks) <= self._n_free

    def allocate_slots(self, seq: Sequence, num_new_tokens: int, computed_blocks=()) -> None:
        """Gives ``seq`` pages for ``num_new_tokens`` more tokens, after the hit pages
        ``computed_blocks`` for a request that holds none yet. The caller then
        advances ``num_computed_tokens`` past the hits before asking for slots."""
        fresh = self.num_blocks_needed(seq, num_new_tokens, computed_blocks)
        taken = self._free_pages_taken(seq, num_new_tokens, computed_blocks)
        if taken > self._n_free:
            raise RuntimeError(f"KV pool exhausted: sequence {seq.seq_id} takes {taken} free pages, "
                               f"{self._n_free} are free")
        table = self._tables.setdefault(seq.seq_id, [])
        if len(computed_blocks):
            if table or seq.num_computed_tokens:
                raise RuntimeError(f"sequence {seq.seq_id} already holds pages; hits apply to new requests")
            for page in computed_blocks:
                self._share(page)
            table.extend(computed_blocks)
        table.extend(self._take_oldest_free() for _ in range(fresh))
        if self.enable_prefix_caching:
            hit_tokens = len(computed_blocks) * self.block_size
            if seq.num_computed_tokens == 0:
                self.num_queried_tokens += hit_tokens + num_new_tokens
                self.num_hit_tokens += hit_tokens
            self.cache_full_blocks(seq, seq.num_computed_tokens + hit_tokens + num_new_tokens)

    def cache_full_blocks(self, seq: Sequence, num_tokens: int) -> None:
        """Offers the full pages among seq's first ``num_tokens`` tokens to the index;
        the first page to carry a given prefix keeps it, later copies stay private."""
        table = self._tables[seq.seq_id]
        full = num_tokens // self.block_size
        digests = self._digests(seq, full)
        start = self._indexed.get(seq.seq_id, 0)
        for i in range(start, full):
            page = table[i]
            if self._digest_of_page[page] is None and digests[i] not in self._page_of_digest:
                self._page_of_digest[digests[i]] = page
                self._digest_of_page[page] = digests[i]
        self._indexed[seq.seq_id] = max(start, full)

    def free(self, seq: Sequence) -> None:
        table = self._tables.pop(seq.seq_id, None)
        if table is None:
            raise RuntimeError(f"sequence {seq.seq_id} holds no pages (released twice, or never allocated)")
        for page in reversed(table):
            self._refs[page] -= 1
            if self._refs[page] == 0:
                self._ring_push(page)
        self._indexed.pop(seq.seq_id, None)

    def free_if_allocated(self, seq: Sequence) -> None:
        if seq.seq_id in self._tables:
            self.free(seq)
