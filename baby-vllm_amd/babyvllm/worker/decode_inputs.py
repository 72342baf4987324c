"""Host staging of a captured decode step's inputs: one packed pinned buffer, edited in place.

Contract of the reference's DecodeInputs (babyvllm/worker/decode_inputs.py:25-112),
which its tests pin: ``DecodeInputs(max_batch, max_blocks, block_size,
dummy_block, pin)``; ``update(seqs, block_tables, bucket)`` stages row i for
the i-th sequence (the token at ``num_computed_tokens``, its position, context
and sequence length, its slot ``table[pos // 16] · 16 + pos % 16`` and its
block table), and rows ``len(seqs) .. bucket`` as padding (token 0, lengths 0,
the dummy page's slot and table, so a padded row's K/V lands in a page no
request owns and its attention output is zero); ``input_ids``,
``positions``, ``seq_lens``, ``context_lens``, ``slot_mapping`` and
``block_tables`` are numpy views of the staged values, ``t_block_tables`` the
tensor under the tables.

Design of this build:

* Every field lives in ONE pinned byte buffer (``packed``) with a fixed layout
  (``layout``: the int64 fields, then the int32 fields, then the tables), so a
  step's whole input reaches the device by a single non-blocking copy into a
  device buffer of the same layout (``device_views``), where the graph
  reads it. Sampled tokens come back through a second small buffer
  (``tokens`` / ``token_buffer``).
* Between steps only positions move and tables grow by a page every
  block_size tokens, so rows are edited, not rebuilt: a row remembers its
  owner as one int64 key (seq_id and preemption count; a recompute gives the
  request a new table) and how many table entries it holds. Rows whose owner
  changed are refilled; rows whose table grew get only the new entries.
  Owner comparison and the slot formula run as numpy array operations.
"""

from __future__ import annotations

import numpy as np
import torch

_I64_FIELDS = ("input_ids", "positions", "slot_mapping")
_I32_FIELDS = ("seq_lens", "context_lens")


def _layout(max_batch: int, max_blocks: int) -> dict[str, tuple[int, tuple[int, ...], np.dtype]]:
    """Byte offset, shape and dtype of every field in the packed buffer (8-byte aligned)."""
    out, off = {}, 0
    for name in _I64_FIELDS:
        out[name] = (off, (max_batch,), np.dtype(np.int64))
        off += 8 * max_batch
    for name in _I32_FIELDS:
        out[name] = (off, (max_batch,), np.dtype(np.int32))
        off += 4 * max_batch
    off = (off + 7) // 8 * 8
    out["block_tables"] = (off, (max_batch, max_blocks), np.dtype(np.int32))
    off += 4 * max_batch * max_blocks
    out["_bytes"] = ((off + 7) // 8 * 8, (), np.dtype(np.uint8))
    return out


_TORCH = {np.dtype(np.int64): torch.int64, np.dtype(np.int32): torch.int32}


class DecodeInputs:
    def __init__(self, max_batch: int, max_blocks: int, block_size: int, dummy_block: int, pin: bool):
        self.max_batch = max_batch
        self.max_blocks = max_blocks
        self.block_size = block_size
        self.dummy_block = dummy_block
        self.dummy_slot = dummy_block * block_size
        self.layout = _layout(max_batch, max_blocks)
        nbytes = self.layout["_bytes"][0]
        self.packed = torch.zeros(nbytes, dtype=torch.uint8, pin_memory=pin)
        raw = self.packed.numpy()
        for name, (off, shape, dt) in self.layout.items():
            if name != "_bytes":
                setattr(self, name, raw[off:off + dt.itemsize * int(np.prod(shape))].view(dt).reshape(shape))
        self.token_buffer = torch.zeros(max_batch, dtype=torch.int64, pin_memory=pin)
        self.tokens = self.token_buffer.numpy()
        self.block_tables.fill(dummy_block)
        self.slot_mapping.fill(self.dummy_slot)
        self._owner = np.full(max_batch, -1, dtype=np.int64)  # (seq_id << 20) | preemptions; -1 = padding
        self._held = np.zeros(max_batch, dtype=np.int64)      # table entries staged in the row
        self._rows_in_use = 0

    @property
    def t_block_tables(self) -> torch.Tensor:
        off, shape, _ = self.layout["block_tables"]
        return self.packed[off:off + 4 * shape[0] * shape[1]].view(torch.int32).view(shape)

    def device_views(self, buffer: torch.Tensor) -> dict[str, torch.Tensor]:
        """Typed views of a byte tensor with the packed layout (the device copy's fields)."""
        views = {}
        for name, (off, shape, dt) in self.layout.items():
            if name != "_bytes":
                n = dt.itemsize * int(np.prod(shape))
                views[name] = buffer[off:off + n].view(_TORCH[dt]).view(shape)
        return views

    @staticmethod
    def _key(seq) -> int:
        return (seq.seq_id << 20) | seq.num_preemptions

    def update(self, seqs, block_tables: dict[int, list[int]], bucket: int) -> int:
        """Stages a decode step of ``seqs`` (each computing the token at its
        ``num_computed_tokens``) padded to ``bucket`` rows; returns len(seqs)."""
        n = len(seqs)
        if not n <= bucket <= self.max_batch:
            raise ValueError(f"{n} sequences do not fit a bucket of {bucket} rows (staging holds {self.max_batch})")
        pos = np.fromiter((s.num_computed_tokens for s in seqs), dtype=np.int64, count=n)
        self.positions[:n] = pos
        self.input_ids[:n] = [s.token_ids[p] for s, p in zip(seqs, pos.tolist())]
        self.context_lens[:n] = pos
        self.seq_lens[:n] = pos + 1

        # Rows that held a request last step and are padding now.
        stale = slice(n, self._rows_in_use)
        self._owner[stale] = -1
        self._held[stale] = 0
        self.block_tables[stale] = self.dummy_block
        # Rows whose owner changed are refilled; the rest get their new pages.
        keys = np.fromiter((self._key(s) for s in seqs), dtype=np.int64, count=n)
        moved = np.flatnonzero(self._owner[:n] != keys)
        self._owner[:n] = keys
        self._held[moved] = 0
        self.block_tables[moved] = self.dummy_block
        for row, s in enumerate(seqs):
            table = block_tables[s.seq_id]
            have = int(self._held[row])
            if len(table) > have:
                self.block_tables[row, have:len(table)] = table[have:]
                self._held[row] = len(table)
        self._rows_in_use = n

        bs = self.block_size
        pages = self.block_tables[np.arange(n), pos // bs].astype(np.int64)
        self.slot_mapping[:n] = pages * bs + pos % bs
        if n < bucket:
            pad = slice(n, bucket)
            self.input_ids[pad] = 0
            self.positions[pad] = 0
            self.seq_lens[pad] = 0
            self.context_lens[pad] = 0
            self.slot_mapping[pad] = self.dummy_slot
        return n
