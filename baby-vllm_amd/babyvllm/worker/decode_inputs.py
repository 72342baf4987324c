"""Host staging of a captured decode step's inputs, edited in place (babyvllm/worker/decode_inputs.py:25-112).

The decode graph reads fixed device buffers; every step the host puts each
sequence's next token, position, lengths, slot and block table into pinned
staging arrays and queues one non-blocking copy per buffer. Between steps
almost nothing changes: positions move by one and a table grows by one page
every block_size tokens. So a row's table is rewritten only when the row now
holds another sequence or another lifetime of the same one (the row key is
(seq_id, num_preemptions)); otherwise only the pages appended since the last
step are written. The slot of a one-token step comes from the table row:
slot = table[pos // block_size] · block_size + pos % block_size.
Rows past the batch are padding: token 0, lengths 0 (the decode kernel returns
zeros for them) and the dummy page's slot, so their K/V writes land in a page
no sequence owns.
"""

from __future__ import annotations

import numpy as np
import torch


class DecodeInputs:
    def __init__(self, max_batch: int, max_blocks: int, block_size: int, dummy_block: int, pin: bool):
        self.max_batch = max_batch
        self.max_blocks = max_blocks
        self.block_size = block_size
        self.dummy_block = dummy_block
        self.dummy_slot = dummy_block * block_size

        def staging(shape, dtype, fill):
            t = torch.full(shape, fill, dtype=dtype, pin_memory=pin)
            return t, t.numpy()

        self.t_input_ids, self.input_ids = staging((max_batch,), torch.int64, 0)
        self.t_positions, self.positions = staging((max_batch,), torch.int64, 0)
        self.t_seq_lens, self.seq_lens = staging((max_batch,), torch.int32, 0)
        self.t_context_lens, self.context_lens = staging((max_batch,), torch.int32, 0)
        self.t_slot_mapping, self.slot_mapping = staging((max_batch,), torch.int64, self.dummy_slot)
        self.t_block_tables, self.block_tables = staging((max_batch, max_blocks), torch.int32, dummy_block)
        # Sampled tokens come back through this one.
        self.t_tokens, self.tokens = staging((max_batch,), torch.int64, 0)
        self._owner: list[tuple[int, int] | None] = [None] * max_batch
        self._written = [0] * max_batch
        self._live = 0
        self._row_index = np.arange(max_batch)

    def update(self, seqs, block_tables: dict[int, list[int]], bucket: int) -> int:
        """Stage this step's decode batch (each sequence computes its token at num_computed_tokens)."""
        n = len(seqs)
        if n > bucket or bucket > self.max_batch:
            raise ValueError(f"batch {n} does not fit bucket {bucket} (max {self.max_batch})")
        bs = self.block_size
        pos = [s.num_computed_tokens for s in seqs]
        self.positions[:n] = pos
        self.input_ids[:n] = [s.token_ids[p] for s, p in zip(seqs, pos)]
        self.context_lens[:n] = pos
        self.seq_lens[:n] = self.context_lens[:n] + 1

        for row in range(n, self._live):  # rows that held a sequence and are padding now
            self._owner[row] = None
            self._written[row] = 0
            self.block_tables[row].fill(self.dummy_block)
        for row, s in enumerate(seqs):
            table = block_tables[s.seq_id]
            owner = (s.seq_id, s.num_preemptions)
            have = self._written[row] if self._owner[row] == owner else 0
            if have == 0:
                self.block_tables[row].fill(self.dummy_block)
                self._owner[row] = owner
            if have < len(table):
                self.block_tables[row, have:len(table)] = table[have:]
                self._written[row] = len(table)
        self._live = n

        p = self.positions[:n]
        pages = self.block_tables[self._row_index[:n], p // bs].astype(np.int64)
        self.slot_mapping[:n] = pages * bs + p % bs
        if n < bucket:
            self.input_ids[n:bucket] = 0
            self.positions[n:bucket] = 0
            self.seq_lens[n:bucket] = 0
            self.context_lens[n:bucket] = 0
            self.slot_mapping[n:bucket] = self.dummy_slot
        return n
