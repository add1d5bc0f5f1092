"""Packed prefill metadata: the tensors the KV scatter and paged prefill read.

Restates the contract of the reference's ``PrefillBatch.from_sequences``
(mini_engine/engine/batch.py:66-137):

* request r's queries sit at absolute positions start_r .. start_r+len_r-1;
* slot = table[pos // block_size] * block_size + pos % block_size;
* context_len = start + len, cu_seqlens_q = cumulative query offsets;
* block tables are padded with -1 to the widest table;
* no slot is written twice, and no page written by one request may appear in
  another request's table (shared prefix pages are read-only).

All validation happens on host values before any device tensor is built, so
the scatter/prefill kernels can run with ``validate=False``.
"""

from __future__ import annotations

from dataclasses import dataclass
from numbers import Integral

import torch

_INT64_MIN, _INT64_LIMIT = -(1 << 63), 1 << 63


def _int_tuple(values, name):
    if isinstance(values, torch.Tensor):
        if values.ndim != 1 or values.dtype != torch.int64:
            raise ValueError(f"{name} must be a 1D int64 tensor")
        values = values.detach().cpu().tolist()
    try:
        items = tuple(values)
    except TypeError as error:
        raise ValueError(f"{name} must be a sequence of integers") from error
    for item in items:
        if isinstance(item, bool) or not isinstance(item, Integral):
            raise ValueError(f"{name} must contain integers")
        if not _INT64_MIN <= item < _INT64_LIMIT:
            raise ValueError(f"{name} values must fit int64")
    return tuple(int(item) for item in items)


@dataclass(frozen=True)
class PrefillBatch:
    input_ids: torch.Tensor
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    cu_seqlens_q: torch.Tensor
    query_starts: torch.Tensor
    context_lens: torch.Tensor
    block_tables: torch.Tensor
    query_lengths: tuple
    query_offsets: tuple
    starts: tuple
    block_ids: tuple
    block_size: int
    num_blocks: int

    @property
    def batch_size(self):
        return len(self.query_lengths)

    @property
    def num_tokens(self):
        return self.query_offsets[-1]

    @classmethod
    def from_sequences(cls, token_sequences, block_tables, query_starts, *,
                       block_size, num_blocks, device):
        for name, value in (("block_size", block_size), ("num_blocks", num_blocks)):
            if isinstance(value, bool) or not isinstance(value, Integral) or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        block_size, num_blocks = int(block_size), int(num_blocks)
        try:
            sequences = [_int_tuple(seq, "token sequence") for seq in token_sequences]
        except TypeError as error:
            raise ValueError("token_sequences must contain query sequences") from error
        if not sequences or any(len(seq) == 0 for seq in sequences):
            raise ValueError("prefill batch requires nonempty query sequences")
        starts = _int_tuple(query_starts, "query_starts")
        if isinstance(block_tables, torch.Tensor):
            if block_tables.ndim != 2 or block_tables.dtype != torch.int64:
                raise ValueError("block_tables must be a 2D int64 tensor")
            block_tables = block_tables.detach().cpu().tolist()
        tables = [_int_tuple(row, "block table") for row in block_tables]
        if not len(starts) == len(tables) == len(sequences):
            raise ValueError("queries, query_starts and block_tables must have equal batch size")

        ids, positions, slots, contexts, offsets, clean = [], [], [], [], [0], []
        written = set()
        readers: dict[int, set] = {}
        writers: dict[int, set] = {}
        for request, (tokens, table, start) in enumerate(zip(sequences, tables, starts)):
            if start < 0:
                raise ValueError("query_starts must be nonnegative")
            if min(tokens) < 0:
                raise ValueError("token IDs must be nonnegative")
            active = len(table)
            for index, page in enumerate(table):
                if page == -1:
                    active = index
                    break
            if any(page != -1 for page in table[active:]):
                raise ValueError("block table padding -1 must be trailing")
            table = table[:active]
            if any(not 0 <= page < num_blocks for page in table):
                raise ValueError("physical block ID out of range")
            if len(set(table)) != len(table):
                raise ValueError("a request block table cannot contain duplicate physical pages")
            end = start + len(tokens)
            if end > len(table) * block_size:
                raise ValueError("query range exceeds supplied block table capacity")
            for page in table:
                readers.setdefault(page, set()).add(request)
            for pos in range(start, end):
                page = table[pos // block_size]
                slot = page * block_size + pos % block_size
                if slot in written:
                    raise ValueError("prefill batch contains duplicate writable KV slots")
                written.add(slot)
                writers.setdefault(page, set()).add(request)
                positions.append(pos)
                slots.append(slot)
            ids.extend(tokens)
            contexts.append(end)
            offsets.append(offsets[-1] + len(tokens))
            clean.append(table)
        for page, who in writers.items():
            if len(readers[page] | who) > 1:
                raise ValueError("prefill cannot write a physical page shared by requests")

        width = max(len(table) for table in clean)
        padded = [list(table) + [-1] * (width - len(table)) for table in clean]

        def tensor(values):
            return torch.tensor(values, dtype=torch.int64, device=device)

        return cls(tensor(ids), tensor(positions), tensor(slots), tensor(offsets), tensor(list(starts)),
                   tensor(contexts), tensor(padded), tuple(len(seq) for seq in sequences), tuple(offsets),
                   starts, tuple(clean), block_size, num_blocks)
