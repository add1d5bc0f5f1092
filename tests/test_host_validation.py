"""Host-side contract checks of the hip backend entry points (CPU only).

These mirror the reference's pre-dispatch validation tests
(tests/test_ragged_kernels.py:48-99, tests/test_ragged_model.py:42-73): the
same ValueError messages fire before any kernel could run, and CPU tensors
are refused by the hip backend instead of being computed on the CPU.
"""

import dataclasses

import pytest
import torch

from mini_engine_hip.cache.page_pool import PagePool
from mini_engine_hip.engine.batch import PrefillBatch
from mini_engine_hip.kernels.data import write_kv_cache, write_kv_cache_batch, write_kv_cache_slots
from mini_engine_hip.kernels.paged import paged_attention
from mini_engine_hip.kernels.prefill import paged_prefill_attention, prefill_attention
from oracle import paged_oracle


def inputs(dtype=torch.float16, dim=16):
    gen = torch.Generator().manual_seed(631)
    key = torch.randn(8, 4, 2, dim, generator=gen).to(dtype)
    value = torch.randn(8, 4, 2, dim, generator=gen).to(dtype)
    q = torch.randn(8, 4, dim, generator=gen).to(dtype)
    meta = [torch.tensor(x, dtype=torch.int64) for x in ([0, 3, 8], [5, 1], [[5, 1, -1], [2, 7, -1]], [8, 6])]
    return [q, key, value, *meta]


def test_only_the_hip_backend_is_served():
    q, key, value, *_ = inputs()
    with pytest.raises(ValueError, match="hip"):
        paged_attention(q[:2], key, value, torch.zeros(2, 1, dtype=torch.long), torch.ones(2, dtype=torch.long), 4,
                        backend="torch")
    with pytest.raises(ValueError, match="hip"):
        write_kv_cache_slots(key, value, torch.tensor([0]), key[0, :1], value[0, :1], backend="cuda")
    with pytest.raises(ValueError, match="hip"):
        paged_prefill_attention(*inputs(), 4, backend="torch")


def test_cpu_tensors_are_refused_not_computed():
    q, key, value, *_ = inputs()
    with pytest.raises(ValueError, match="FP16/BF16"):
        paged_attention(q.float()[:2], key, value, torch.zeros(2, 1, dtype=torch.long),
                        torch.ones(2, dtype=torch.long), 4)
    with pytest.raises(RuntimeError, match="query must be CUDA"):
        paged_attention(q[:2], key, value, torch.zeros(2, 1, dtype=torch.long), torch.ones(2, dtype=torch.long), 4)
    with pytest.raises(ValueError, match="HIP packed KV"):
        write_kv_cache_slots(key, value, torch.tensor([3]), torch.ones(1, 2, 16).half(), torch.ones(1, 2, 16).half())
    with pytest.raises(ValueError, match="HIP paged prefill"):
        paged_prefill_attention(*inputs(), 4)


def test_dense_prefill_contract_on_cpu():
    """The reference's checks of prefill_attention (prefill.py:15-29) with its
    messages, then the HIP requirements (prefill.py:35-40 for "cuda"); no
    case reaches the library."""
    gen = torch.Generator().manual_seed(71)
    q = torch.randn(1, 4, 3, 16, generator=gen).half()
    k = torch.randn(1, 2, 11, 16, generator=gen).half()
    v = torch.randn(1, 2, 11, 16, generator=gen).half()
    with pytest.raises(ValueError, match="unknown prefill backend"):
        prefill_attention(q, k, v, "math", query_start=8)
    with pytest.raises(ValueError, match="divisible GQA heads"):
        prefill_attention(q[:, :3], k, v, query_start=8)
    with pytest.raises(ValueError, match="divisible GQA heads"):
        prefill_attention(q, k, v[:, :, :10], query_start=8)
    with pytest.raises(ValueError, match="divisible GQA heads"):
        prefill_attention(q[0], k, v, query_start=8)
    with pytest.raises(ValueError, match="share batch, head_dim, dtype and device"):
        prefill_attention(q, k.float(), v.float(), query_start=8)
    with pytest.raises(ValueError, match="share batch, head_dim, dtype and device"):
        prefill_attention(q[..., :8], k, v, query_start=8)
    for start in (9, -1, True, 8.0):
        with pytest.raises(ValueError, match="must fit the KV sequence"):
            prefill_attention(q, k, v, query_start=start)
    with pytest.raises(ValueError, match="must fit the KV sequence"):
        prefill_attention(q[:, :, :0], k, v, query_start=8)
    with pytest.raises(ValueError, match="HIP FP16/BF16"):
        prefill_attention(q, k, v, query_start=8)
    with pytest.raises(ValueError, match="HIP FP16/BF16"):
        prefill_attention(q.float(), k.float(), v.float(), query_start=8)


def test_dense_prefill_output_must_not_overlap_itself():
    """A caller's output for prefill_attention is written through its
    strides, so its elements must be distinct: the rule the wrapper and
    mvme_prefill_attention apply (by increasing stride, each dimension of
    more than one element steps past everything the smaller ones reach)."""
    from mini_engine_hip.kernels.prefill import _dense_disjoint

    assert _dense_disjoint(torch.empty(2, 4, 8, 16))
    assert _dense_disjoint(torch.empty(2, 8, 4, 16).transpose(1, 2))  # token-major
    assert _dense_disjoint(torch.empty(1, 1, 1, 16))
    assert _dense_disjoint(torch.empty(3, 64, 4, 16)[:, ::2].transpose(1, 2))  # gaps are fine
    assert not _dense_disjoint(torch.empty(2, 1, 8, 16).expand(2, 4, 8, 16))
    assert not _dense_disjoint(torch.empty(4096).as_strided((1, 4, 8, 16), (512, 8, 64, 1)))
    assert not _dense_disjoint(torch.empty(4096).as_strided((1, 4, 8, 16), (512, 16, 32, 1)))
    assert not _dense_disjoint(torch.empty(2, 4, 8, 32)[..., ::2])


def test_slot_scatter_rejects_races_before_mutation():
    """test_ragged_kernels.py:48-65: duplicate slots, overlap, capacity."""
    _, key, value, *_ = inputs()
    before = key.clone()
    source = torch.randn(8, 2, 16).half()
    with pytest.raises(ValueError, match="duplicate"):
        write_kv_cache_slots(key, value, torch.zeros(8, dtype=torch.int64), source, source)
    slots = torch.tensor([5, 6, 7, 9, 10, 11, 28, 29], dtype=torch.int64)
    with pytest.raises(ValueError, match="overlap"):
        write_kv_cache_slots(key, value, slots, key.view(-1, 2, 16)[:8], source)
    with pytest.raises(ValueError, match="overlap"):
        write_kv_cache_slots(key, key, slots, source, source)
    for slot in (-1, 32):
        with pytest.raises(ValueError, match="capacity"):
            write_kv_cache_slots(key, value, torch.tensor([slot]), torch.ones(1, 2, 16).half(),
                                 torch.ones(1, 2, 16).half())
    with pytest.raises(ValueError, match="int64"):
        write_kv_cache_slots(key, value, slots.int(), source, source)
    assert torch.equal(key, before)


@pytest.mark.parametrize("change,message", [
    (lambda a: a[3].fill_(0), "offset"),
    (lambda a: a[4].fill_(-1), "context"),
    (lambda a: a[6].fill_(99), "capacity"),
    (lambda a: a[5].fill_(-1), "physical"),
    (lambda a: a[5].fill_(8), "physical"),
    (lambda a: a.__setitem__(3, a[3].to(torch.int32)), "int64"),
])
def test_invalid_paged_metadata_rejected_before_dispatch(change, message):
    """test_ragged_kernels.py:68-80 for the hip backend."""
    args = inputs()
    change(args)
    with pytest.raises(ValueError, match=message):
        paged_prefill_attention(*args, 4, backend="hip")


def test_range_and_batch_write_contracts():
    _, key, value, *_ = inputs()
    with pytest.raises(ValueError, match="capacity"):
        write_kv_cache(key, value, torch.tensor([1, 2]), 6, torch.ones(3, 2, 16).half(), torch.ones(3, 2, 16).half(), 4)
    with pytest.raises(ValueError, match="shape mismatch"):
        write_kv_cache_batch(key, value, torch.zeros(3, 2, dtype=torch.long), torch.zeros(2, dtype=torch.long),
                             torch.ones(2, 2, 16).half(), torch.ones(2, 2, 16).half(), 4)
    with pytest.raises(RuntimeError, match="CUDA"):
        write_kv_cache(key, value, torch.tensor([1, 2]), 0, torch.ones(3, 2, 16).half(), torch.ones(3, 2, 16).half(), 4)


# ---------------------------------------------------------------------------
# PrefillBatch: the reference's KAT and rejection table (test_ragged_model.py:42-73)
# ---------------------------------------------------------------------------

def metadata(sequences, tables, starts, num_blocks=16):
    return PrefillBatch.from_sequences(sequences, tables, starts, block_size=4, num_blocks=num_blocks, device="cpu")


def test_prefill_metadata_positions_slots_and_readonly_prefix_sharing():
    batch = metadata([[5, 6, 7], [8, 9]], [[3, 1, -1], [3, 2]], [4, 4])
    assert batch.query_lengths == (3, 2) and batch.query_offsets == (0, 3, 5)
    assert batch.starts == (4, 4) and batch.block_ids == ((3, 1), (3, 2))
    assert batch.block_size == 4 and batch.batch_size == 2 and batch.num_tokens == 5
    assert batch.input_ids.tolist() == [5, 6, 7, 8, 9]
    assert batch.positions.tolist() == [4, 5, 6, 4, 5]
    assert batch.slot_mapping.tolist() == [4, 5, 6, 8, 9]
    assert batch.cu_seqlens_q.tolist() == [0, 3, 5]
    assert batch.context_lens.tolist() == [7, 6]
    assert batch.block_tables.tolist() == [[3, 1], [3, 2]]
    # Agrees with the oracle's restatement of the same rules.
    ref = paged_oracle.prefill_metadata([[5, 6, 7], [8, 9]], [[3, 1, -1], [3, 2]], [4, 4], 4)
    assert batch.slot_mapping.tolist() == ref["slot_mapping"] and batch.positions.tolist() == ref["positions"]


@pytest.mark.parametrize("sequences,tables,starts,error", [
    ([[]], [[0]], [0], "nonempty"),
    ([[1]], [[0]], [-1], "nonnegative"),
    ([[1]], [[0]], [True], "integers"),
    ([[1]], [[0]], [], "equal batch"),
    ([[-1]], [[0]], [0], "nonnegative"),
    ([[1]], [[16]], [0], "out of range"),
    ([[1]], [[0, 0]], [0], "duplicate physical"),
    ([[1]], [[0, -1, 2]], [0], "trailing"),
    ([[1, 2]], [[0]], [3], "capacity"),
    ([[1], [2]], [[0], [0]], [0, 0], "duplicate writable"),
    ([[1], [2]], [[0], [0]], [0, 1], "shared by requests"),
    ([torch.tensor([1.0])], [[0]], [0], "int64"),
    ([[1 << 64]], [[0]], [0], "int64"),
])
def test_prefill_metadata_rejects_invalid_layout(sequences, tables, starts, error):
    with pytest.raises(ValueError, match=error):
        metadata(sequences, tables, starts)


def test_prefill_metadata_validate_at_the_execution_boundary():
    """PrefillBatch.validate (reference batch.py:139-162): geometry, tensor
    type and device, in-place edits and swapped tensors, the context limit and
    the vocabulary, each with the reference's message."""
    batch = metadata([[5, 6, 7], [8, 9]], [[3, 1, -1], [3, 2]], [4, 4])
    ok = dict(block_size=4, num_blocks=16, device="cpu", max_position_embeddings=7, vocab_size=10)
    batch.validate(**ok)  # context 7 and token 9 are the largest allowed
    for change, message in [
        (dict(block_size=8), "geometry"), (dict(num_blocks=17), "geometry"),
        (dict(max_position_embeddings=6), "context limit"), (dict(vocab_size=9), "vocabulary"),
    ]:
        with pytest.raises(ValueError, match=message):
            batch.validate(**{**ok, **change})
    # A tensor edited in place after construction (its version counter moves).
    edited = metadata([[5, 6, 7], [8, 9]], [[3, 1, -1], [3, 2]], [4, 4])
    edited.slot_mapping.add_(0)
    with pytest.raises(ValueError, match="was modified"):
        edited.validate(**ok)
    # A tensor swapped for another with the same values.
    swapped = dataclasses.replace(batch, context_lens=batch.context_lens.clone())
    with pytest.raises(ValueError, match="was modified"):
        swapped.validate(**ok)
    # Wrong dtype or layout of a metadata tensor.
    as_int32 = dataclasses.replace(batch, positions=batch.positions.int())
    with pytest.raises(ValueError, match="contiguous int64"):
        as_int32.validate(**ok)
    # Built by hand rather than by from_sequences: no fingerprints.
    fields = {f.name: getattr(batch, f.name) for f in dataclasses.fields(batch)
              if f.name not in ("max_token_id", "fingerprints")}
    with pytest.raises(ValueError, match="from_sequences"):
        PrefillBatch(**fields).validate(**ok)
    # Construction under inference mode still keeps version counters.
    with torch.inference_mode():
        inferred = metadata([[5, 6, 7], [8, 9]], [[3, 1, -1], [3, 2]], [4, 4])
    inferred.validate(**ok)


@pytest.mark.parametrize("starts,block_size,error", [
    ([(1 << 63) - 1], 4, "capacity"),        # start + length wraps around in int64
    ([(1 << 63) - 2], 1 << 62, "fit int64"),  # inside the capacity, but slots cannot be int64
    ([0], 1 << 64, "fit int64"),             # block_size beyond int64
])
def test_prefill_metadata_rejects_int64_wraparound(starts, block_size, error):
    """Range rules are checked on Python integers: values near 2^63 raise the
    reference's ValueError instead of wrapping around (or an IndexError)."""
    with pytest.raises(ValueError, match=error):
        PrefillBatch.from_sequences([[1, 2]], [[0, 1]], starts, block_size=block_size, num_blocks=16,
                                    device="cpu")


@pytest.mark.parametrize("seed", range(6))
def test_prefill_metadata_matches_oracle_on_random_batches(seed):
    """Ragged batches whose requests share read-only prefix pages: every field
    equals the oracle's per-position restatement of the rules."""
    gen = torch.Generator().manual_seed(seed)
    bs, shared = 4, [40, 41]  # two prefix pages, read by every request
    order = torch.randperm(32, generator=gen).tolist()
    sequences, tables, starts = [], [], []
    for r in range(int(torch.randint(1, 6, (1,), generator=gen))):
        count = int(torch.randint(1, 9, (1,), generator=gen))
        start = 8 + int(torch.randint(0, 5, (1,), generator=gen))  # past the shared 8 tokens
        private = -(-(start + count) // bs) - 2
        table = shared + order[:private]
        order = order[private:]
        tables.append(table + [-1] * int(torch.randint(0, 3, (1,), generator=gen)))
        sequences.append(torch.randint(0, 1000, (count,), generator=gen).tolist())
        starts.append(start)
    batch = metadata(sequences, tables, starts, num_blocks=64)
    ref = paged_oracle.prefill_metadata(sequences, tables, starts, bs)
    assert batch.positions.tolist() == ref["positions"]
    assert batch.slot_mapping.tolist() == ref["slot_mapping"]
    assert batch.cu_seqlens_q.tolist() == ref["cu_seqlens_q"]
    assert batch.context_lens.tolist() == ref["context_lens"]
    assert batch.block_tables.tolist() == ref["block_tables"]
    assert batch.input_ids.tolist() == [t for s in sequences for t in s]
    assert batch.query_starts.tolist() == starts
    # Writing into a shared page is refused once another request reads it.
    starts_low = list(starts)
    starts_low[-1] = 7
    if len(starts) > 1:
        with pytest.raises(ValueError, match="shared by requests"):
            metadata(sequences, tables, starts_low, num_blocks=64)
    else:
        assert metadata(sequences, tables, starts_low, num_blocks=64).slot_mapping[0].item() == 41 * bs + 3


def test_page_pool_shared_prefix_refcounts():
    """block_manager.py:55-105 semantics: a cached prefix attached to several requests."""
    pool = PagePool(12, 4, order=[5, 3, 11, 0, 1, 2, 4, 6, 7, 8, 9, 10])
    prefix = pool.allocate("prefix", 8)
    assert prefix == [5, 3] and pool.refcount(5) == 1
    a = pool.allocate_with_prefix("a", 10, prefix)
    b = pool.allocate_with_prefix("b", 9, prefix)
    assert a[:2] == prefix == b[:2] and len(a) == 3 and len(b) == 3 and a[2] != b[2]
    assert pool.refcount(5) == 3 and pool.refcount(a[2]) == 1
    pool.free("a")
    assert pool.refcount(5) == 2
    with pytest.raises(ValueError, match="more blocks"):
        pool.allocate_with_prefix("c", 4, prefix)
    with pytest.raises(MemoryError):
        pool.allocate("d", 4 * 20)
    with pytest.raises(ValueError, match="unallocated"):
        pool.allocate_with_prefix("e", 12, [a[2]])


def test_page_pool_attach_retained_pages():
    """block_manager.py:83-97: a request whose whole table is retained pages
    (a prefix-cache hit covering the prompt) takes no free page, and its
    release leaves the pages with their other holders."""
    pool = PagePool(8, 4)
    prefix = pool.allocate("prefix", 8)
    pool.pin(prefix)
    free = pool.free_blocks
    assert pool.attach("hit", prefix) == prefix
    assert pool.free_blocks == free and pool.table("hit") == prefix
    assert [pool.refcount(p) for p in prefix] == [3, 3]
    with pytest.raises(ValueError, match="already owns"):
        pool.attach("hit", prefix)
    with pytest.raises(ValueError, match="attached pages must be distinct"):
        pool.attach("dup", [prefix[0], prefix[0]])
    with pytest.raises(ValueError, match="cannot attach unallocated block: 7"):
        pool.attach("dead", [prefix[0], 7])
    assert pool.refcount(prefix[0]) == 3  # a refused attach takes no reference
    pool.free("prefix")
    pool.free("hit")
    assert [pool.refcount(p) for p in prefix] == [1, 1] and pool.free_blocks == free
    pool.unpin(prefix)
    assert pool.free_blocks == 8
    with pytest.raises(ValueError, match="cannot attach unallocated block"):
        pool.attach("late", prefix)


def test_fused_norm_rope_write_checks_before_any_launch():
    from mini_engine_hip.kernels.rope import qk_norm_rope_write_kv
    q, key, value, *_ = inputs()
    k = v = torch.randn(8, 2, 16).half()
    cos = sin = torch.ones(8, 8).half()
    w = torch.ones(16).half()
    slots = torch.arange(8, dtype=torch.int64)
    with pytest.raises(ValueError, match="backend must be hip"):
        qk_norm_rope_write_kv(q, k, v, w, w, cos, sin, key, value, slot_mapping=slots, backend="torch")
    with pytest.raises(ValueError, match="either slot_mapping or block_tables"):
        qk_norm_rope_write_kv(q, k, v, w, w, cos, sin, key, value)
    with pytest.raises(ValueError, match="q and k must be"):
        qk_norm_rope_write_kv(q, k[:, :, :8], v, w, w, cos, sin, key, value, slot_mapping=slots)
    with pytest.raises(ValueError, match="FP16/BF16"):
        qk_norm_rope_write_kv(q.float(), k.float(), v, w, w, cos, sin, key, value, slot_mapping=slots)
    # CPU tensors are refused, never computed on the CPU.
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        qk_norm_rope_write_kv(q, k, v, w, w, cos, sin, key, value, slot_mapping=slots)


def test_greedy_sampling_contract_on_cpu():
    from mini_engine_hip.sampling import sample_next_token
    x = torch.randn(2, 9)
    with pytest.raises(ValueError, match="sampling backend must be hip"):
        sample_next_token(x, backend="torch")
    with pytest.raises(ValueError, match="greedy temperature=0"):
        sample_next_token(x, temperature=0.7)
    with pytest.raises(ValueError, match="logits must have shape"):
        sample_next_token(x[0])
    with pytest.raises(RuntimeError, match="contiguous CUDA"):
        sample_next_token(x)


def test_hip_linear_contract_on_cpu():
    """tests/test_prefill_linear_chat.py:22-29 for HipLinear: CPU input is refused."""
    from mini_engine_hip.kernels.linear import HipLinear, linear_rows

    x = torch.randn(2, 3, 7)
    with pytest.raises(ValueError, match="CUDA"):
        HipLinear(7, 5)(x)
    with pytest.raises(ValueError, match="CUDA"):
        linear_rows(torch.randn(2, 64), torch.randn(16, 64))


def test_row_stride_passes_only_dense_rows():
    """The scatter and fused-RoPE kernels read each token's [heads, dim] block
    as one dense run; any other view is copied first, also for one token."""
    from mini_engine_hip.kernels.data import _row_stride

    fused = torch.randn(5, 3 * 64).view(5, 3, 4, 16)[:, 1]  # one slice of a fused projection
    stride, same = _row_stride(fused)
    assert stride == 3 * 64 and same.data_ptr() == fused.data_ptr()
    for tokens in (1, 3):
        transposed = torch.randn(tokens, 64, 4).transpose(1, 2)  # [T, 4, 64], not dense per row
        assert not transposed.is_contiguous()
        stride, fixed = _row_stride(transposed)
        assert stride == 4 * 64 and fixed.is_contiguous() and torch.equal(fixed, transposed)
    one = torch.randn(1, 4, 16)
    assert _row_stride(one) == (64, one)
    single_head = torch.randn(6, 1, 16)[:, :, :]
    assert _row_stride(single_head)[0] == 16
