"""Packed prefill metadata: the tensors the KV scatter and paged prefill read.

Keeps the contract of the reference's ``PrefillBatch.from_sequences``
(mini_engine/engine/batch.py:66-137) — the same fields, rules and error
messages — but derives everything with whole-batch tensor operations on the
host instead of walking positions one by one:

* request r's queries sit at absolute positions start_r .. start_r+len_r-1;
* slot = table[pos // block_size] * block_size + pos % block_size;
* context_len = start + len, cu_seqlens_q = cumulative query offsets;
* block tables are padded with -1 to the widest table;
* no slot is written twice, and no page written by one request may appear in
  another request's table (shared prefix pages are read-only).

``validate`` re-checks the batch at the model's execution boundary, as the
reference's ``PrefillBatch.validate`` does (batch.py:139-162): the cache
geometry, the tensors' type, device and layout, a fingerprint of every
tensor taken at construction (storage pointer, version counter, shape,
strides, dtype, device -- an in-place edit or a swapped tensor is refused
without reading the device), the model's context limit and vocabulary.

The checks run in three stages — argument types, the per-request layout
(each rule over the whole batch at once), then the rules that relate
requests (duplicate slots, written pages that another request reads) — and
all of them finish before any device tensor exists, so the scatter and
prefill kernels can run with ``validate=False``.  With several faults in one
batch the first failing stage names the error (the reference reports the
first faulty request instead); each single fault raises the reference's
message.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from numbers import Integral

import torch

_INT64 = (-(1 << 63), (1 << 63) - 1)


def _ints(values, name) -> list[int]:
    """Plain Python ints from a list/tuple or a 1D int64 tensor."""
    if isinstance(values, torch.Tensor):
        if values.ndim != 1 or values.dtype != torch.int64:
            raise ValueError(f"{name} must be a 1D int64 tensor")
        return values.detach().cpu().tolist()
    try:
        items = list(values)
    except TypeError as error:
        raise ValueError(f"{name} must be a sequence of integers") from error
    if not all(isinstance(v, Integral) and not isinstance(v, bool) for v in items):
        raise ValueError(f"{name} must contain integers")
    if items and not (_INT64[0] <= min(items) and max(items) <= _INT64[1]):
        raise ValueError(f"{name} values must fit int64")
    return [int(v) for v in items]


def _positive(value, name) -> int:
    if isinstance(value, bool) or not isinstance(value, Integral) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    return int(value)


def _padded_tables(rows) -> torch.Tensor:
    """[B, widest] int64, short rows filled with -1 (the padding marker)."""
    widest = max(len(row) for row in rows)
    table = torch.full((len(rows), max(widest, 1)), -1, dtype=torch.int64)
    for r, row in enumerate(rows):
        if row:
            table[r, :len(row)] = torch.tensor(row, dtype=torch.int64)
    return table


def _table_pages(table: torch.Tensor, num_blocks: int) -> torch.Tensor:
    """Validate the page part of every table; return each row's page count."""
    pad = table == -1
    # Once a row is padded it must stay padded.
    if bool((pad.cummax(dim=1).values & ~pad).any()):
        raise ValueError("block table padding -1 must be trailing")
    if bool((~pad & ((table < 0) | (table >= num_blocks))).any()):
        raise ValueError("physical block ID out of range")
    ordered = table.sort(dim=1).values
    if bool(((ordered[:, 1:] == ordered[:, :-1]) & (ordered[:, 1:] != -1)).any()):
        raise ValueError("a request block table cannot contain duplicate physical pages")
    return (~pad).sum(dim=1)


def _check_shared_writes(table: torch.Tensor, pages_per_row: torch.Tensor, slots: torch.Tensor,
                         block_size: int) -> None:
    """A page that receives new rows may be listed by one request only."""
    rows = torch.arange(table.shape[0]).repeat_interleave(pages_per_row)
    listed = table[table != -1]  # row-major, so it lines up with `rows`
    written = torch.unique(slots // block_size)
    hit = torch.isin(listed, written)
    if not bool(hit.any()):
        return
    # Distinct (page, request) pairs among the written pages; a page with more
    # than one is written by one request and read (or written) by another.
    pairs = torch.unique(listed[hit] * table.shape[0] + rows[hit])
    _, per_page = torch.unique(pairs // table.shape[0], return_counts=True)
    if bool((per_page > 1).any()):
        raise ValueError("prefill cannot write a physical page shared by requests")


def _fingerprint(tensor: torch.Tensor) -> tuple:
    """What an in-place edit or a swapped tensor changes, read on the host."""
    return (tensor.data_ptr(), tensor._version, tuple(tensor.shape), tuple(tensor.stride()), tensor.dtype,
            tensor.device)


_TENSOR_FIELDS = ("input_ids", "positions", "slot_mapping", "cu_seqlens_q", "query_starts", "context_lens",
                  "block_tables")


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
    # Host copies taken at construction: the largest token id, and one
    # fingerprint per tensor (empty when the batch was built by hand).
    max_token_id: int = field(default=-1, repr=False)
    fingerprints: tuple = field(default=(), repr=False, compare=False)

    @property
    def batch_size(self):
        return len(self.query_lengths)

    @property
    def num_tokens(self):
        return self.query_offsets[-1]

    @classmethod
    def from_sequences(cls, token_sequences, block_tables, query_starts, *, block_size, num_blocks, device):
        block_size = _positive(block_size, "block_size")
        num_blocks = _positive(num_blocks, "num_blocks")
        # Stage 1: argument types.
        try:
            sequences = [_ints(seq, "token sequence") for seq in token_sequences]
        except TypeError as error:
            raise ValueError("token_sequences must contain query sequences") from error
        if not sequences or not all(sequences):
            raise ValueError("prefill batch requires nonempty query sequences")
        starts = _ints(query_starts, "query_starts")
        if isinstance(block_tables, torch.Tensor):
            if block_tables.ndim != 2 or block_tables.dtype != torch.int64:
                raise ValueError("block_tables must be a 2D int64 tensor")
            block_tables = block_tables.detach().cpu().tolist()
        rows = [_ints(row, "block table") for row in block_tables]
        if not len(sequences) == len(starts) == len(rows):
            raise ValueError("queries, query_starts and block_tables must have equal batch size")

        # Stage 2: each request's own layout, checked for all requests at once.
        lengths = torch.tensor([len(seq) for seq in sequences], dtype=torch.int64)
        start = torch.tensor(starts, dtype=torch.int64)
        token_ids = torch.tensor([t for seq in sequences for t in seq], dtype=torch.int64)
        if bool((start < 0).any()):
            raise ValueError("query_starts must be nonnegative")
        if bool((token_ids < 0).any()):
            raise ValueError("token IDs must be nonnegative")
        table = _padded_tables(rows)
        pages_per_row = _table_pages(table, num_blocks)
        # Python ints: a start near 2^63 or a huge block_size must not wrap
        # around in int64 and slip past the capacity rule.
        if any(s + len(seq) > pages * block_size
               for s, seq, pages in zip(starts, sequences, pages_per_row.tolist())):
            raise ValueError("query range exceeds supplied block table capacity")
        if num_blocks * block_size > _INT64[1]:
            raise ValueError("KV slots (num_blocks * block_size) must fit int64")
        ends = start + lengths

        # Positions and slots of every packed token.
        owner = torch.arange(len(sequences)).repeat_interleave(lengths)
        offsets = torch.cat([torch.zeros(1, dtype=torch.int64), lengths.cumsum(0)])
        positions = start[owner] + torch.arange(token_ids.numel()) - offsets[owner]
        pages = table[owner, positions // block_size]
        slots = pages * block_size + positions % block_size

        # Stage 3: rules between requests.
        if torch.unique(slots).numel() != slots.numel():
            raise ValueError("prefill batch contains duplicate writable KV slots")
        _check_shared_writes(table, pages_per_row, slots, block_size)

        width = int(pages_per_row.max())
        clean = tuple(tuple(row[:int(n)]) for row, n in zip(rows, pages_per_row))
        # Outside inference mode the device tensors keep version counters, so
        # validate() can see in-place edits without a device-to-host copy.
        with torch.inference_mode(False):
            on_device = [t.to(device).clone() for t in (token_ids, positions, slots, offsets, start, ends,
                                                        table[:, :width].contiguous())]
        return cls(*on_device, tuple(lengths.tolist()), tuple(offsets.tolist()), tuple(starts), clean,
                   block_size, num_blocks, int(token_ids.max()), tuple(_fingerprint(t) for t in on_device))

    def validate(self, *, block_size, num_blocks, device, max_position_embeddings, vocab_size):
        """The execution-boundary checks of the reference (batch.py:139-162):
        after them the scatter and prefill kernels may run with
        validate=False.  Reads host state only."""
        if self.block_size != block_size or self.num_blocks != num_blocks:
            raise ValueError("prefill metadata does not match KV cache geometry")
        tensors = [getattr(self, name) for name in _TENSOR_FIELDS]
        if len(self.fingerprints) != len(tensors):
            raise ValueError("construct prefill metadata with PrefillBatch.from_sequences")
        device = torch.device(device)
        if not all(isinstance(t, torch.Tensor) and t.dtype == torch.int64 and t.device == device
                   and t.is_contiguous() for t in tensors):
            raise ValueError("prefill metadata must be contiguous int64 tensors on the cache device")
        if tuple(_fingerprint(t) for t in tensors) != self.fingerprints:
            raise ValueError("prefill metadata was modified; rebuild it with from_sequences")
        if max(s + n for s, n in zip(self.starts, self.query_lengths)) > max_position_embeddings:
            raise ValueError("prefill query range exceeds model context limit")
        if self.max_token_id >= vocab_size:
            raise ValueError("prefill token ID exceeds model vocabulary")
