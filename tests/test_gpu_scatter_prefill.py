"""GPU parity of the HIP KV scatter/gather and paged prefill against the oracle.

Restates the reference's GPU tests for these paths
(tests/test_ragged_kernels.py:102-136, tests/test_data_kernels.py:40-57,
tests/test_kv_cache.py:6-23) for backend="hip".  KV writes and gathers must
be bit-exact; prefill outputs must sit within the north-star gate of the
fp32 oracle (max abs 2e-3 fp16, 1.6e-2 bf16) and within the reference's own
tolerance (test_ragged_kernels.py:120).
"""

import random

import pytest
import torch

from gpu_cases import prefill_inputs
from mini_engine_hip.cache.kv_cache import KVCachePool
from mini_engine_hip.kernels.data import write_kv_cache, write_kv_cache_batch, write_kv_cache_slots
from mini_engine_hip.kernels.prefill import paged_prefill_attention
from mini_engine_hip import workloads
from oracle import c_oracle, paged_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
GATE = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def max_err(actual, expected):
    return (actual.float().cpu() - expected.float().cpu()).abs().max().item()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim", [16, 128])
def test_packed_attention_and_slot_scatter_on_nondefault_stream(dtype, dim):
    q, key, value, offsets, starts, tables, lengths = prefill_inputs(dtype, head_dim=dim)
    slots = torch.tensor([5, 6, 7, 9, 10, 11, 28, 29], dtype=torch.int64)
    gen = torch.Generator().manual_seed(5)
    source_k = torch.randn(8, 2, dim, generator=gen).to(dtype)
    source_v = torch.randn(8, 2, dim, generator=gen).to(dtype)
    expected_k, expected_v = key.clone(), value.clone()
    paged_oracle.write_kv_cache_slots(expected_k, expected_v, slots, source_k, source_v)
    expected = paged_oracle.paged_prefill_attention(q, expected_k, expected_v, offsets, starts, tables,
                                                    lengths, 4, cast=False)
    dk, dv = key.to(DEV), value.to(DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        write_kv_cache_slots(dk, dv, slots.to(DEV), source_k.to(DEV), source_v.to(DEV), backend="hip")
        result = paged_prefill_attention(q.to(DEV), dk, dv, offsets.to(DEV), starts.to(DEV), tables.to(DEV),
                                         lengths.to(DEV), 4, backend="hip")
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), expected_k) and torch.equal(dv.cpu(), expected_v)
    assert max_err(result, expected) <= GATE[dtype]
    tolerance = 0.02 if dtype == torch.bfloat16 else 0.003
    torch.testing.assert_close(result.cpu(), expected.to(dtype), atol=tolerance, rtol=tolerance)


def test_slot_scatter_strided_sources_and_untouched_rows():
    """Split projection views (non-contiguous token stride) scatter bit-exactly."""
    dtype = torch.bfloat16
    gen = torch.Generator().manual_seed(11)
    cache_k = torch.randn(32, 16, 8, 128, generator=gen).to(dtype)
    cache_v = torch.randn(32, 16, 8, 128, generator=gen).to(dtype)
    packed = torch.randn(40, 16, 128, generator=gen).to(dtype)   # [tokens, k heads | v heads, D]
    src_k, src_v = packed[:, :8], packed[:, 8:]
    slots = torch.randperm(32 * 16, generator=gen)[:40]
    want_k, want_v = c_oracle.scatter_slots(cache_k, cache_v, slots, src_k, src_v)
    dk, dv, dpacked = cache_k.to(DEV), cache_v.to(DEV), packed.to(DEV)
    write_kv_cache_slots(dk, dv, slots.to(DEV), dpacked[:, :8], dpacked[:, 8:], backend="hip")
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), want_k) and torch.equal(dv.cpu(), want_v)


@pytest.mark.parametrize("tokens", [1, 2])
def test_slot_scatter_transposed_sources_one_token(tokens):
    """A source whose [kv_heads, head_dim] rows are not dense (a transposed
    view) is copied before the kernel reads it, also for a single token."""
    dtype = torch.float16
    gen = torch.Generator().manual_seed(5 + tokens)
    cache_k = torch.randn(4, 16, 8, 64, generator=gen).to(dtype)
    cache_v = torch.randn(4, 16, 8, 64, generator=gen).to(dtype)
    raw_k = torch.randn(tokens, 64, 8, generator=gen).to(dtype)
    raw_v = torch.randn(tokens, 64, 8, generator=gen).to(dtype)
    slots = torch.tensor([37, 5][:tokens], dtype=torch.int64)
    want_k, want_v = cache_k.clone(), cache_v.clone()
    paged_oracle.write_kv_cache_slots(want_k, want_v, slots, raw_k.transpose(1, 2), raw_v.transpose(1, 2))
    dk, dv = cache_k.to(DEV), cache_v.to(DEV)
    src_k, src_v = raw_k.to(DEV).transpose(1, 2), raw_v.to(DEV).transpose(1, 2)
    assert not src_k.is_contiguous()
    write_kv_cache_slots(dk, dv, slots.to(DEV), src_k, src_v, backend="hip")
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), want_k) and torch.equal(dv.cpu(), want_v)


def test_slot_scatter_trusted_out_of_range_slots_are_skipped():
    dtype = torch.float16
    cache_k = torch.zeros(4, 4, 2, 16, dtype=dtype, device=DEV)
    cache_v = torch.zeros_like(cache_k)
    slots = torch.tensor([-1, 3, 16, 1 << 40], dtype=torch.int64, device=DEV)
    src = torch.ones(4, 2, 16, dtype=dtype, device=DEV)
    write_kv_cache_slots(cache_k, cache_v, slots, src, src, backend="hip", validate=False)
    torch.cuda.synchronize()
    rows = cache_k.view(-1, 2, 16)
    assert rows[3].eq(1).all() and rows.sum().item() == 32


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_kv_write_crosses_pages_and_uses_stream(dtype):
    gen = torch.Generator().manual_seed(63)
    block_size, blocks, kv_heads, dim = 4, 6, 2, 8
    key_cache = torch.zeros(blocks, block_size, kv_heads, dim, dtype=dtype)
    value_cache = torch.zeros_like(key_cache)
    ids = torch.tensor([4, 1, 5], dtype=torch.long)
    key = torch.randn(7, kv_heads, dim, generator=gen).to(dtype)
    value = torch.randn(7, kv_heads, dim, generator=gen).to(dtype)
    expected_k, expected_v = key_cache.clone(), value_cache.clone()
    paged_oracle.write_kv_cache(expected_k, expected_v, ids, 1, key, value, block_size)
    dk, dv = key_cache.to(DEV), value_cache.to(DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        write_kv_cache(dk, dv, ids.to(DEV), 1, key.to(DEV), value.to(DEV), block_size, backend="hip")
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), expected_k) and torch.equal(dv.cpu(), expected_v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_batch_write_matches_oracle(dtype):
    gen = torch.Generator().manual_seed(64)
    kc = torch.randn(20, 16, 8, 128, generator=gen).to(dtype)
    vc = torch.randn(20, 16, 8, 128, generator=gen).to(dtype)
    tables = torch.randperm(20, generator=gen)[:12].view(4, 3)
    offsets = torch.tensor([0, 15, 16, 47], dtype=torch.int64)
    key = torch.randn(4, 8, 128, generator=gen).to(dtype)
    value = torch.randn(4, 8, 128, generator=gen).to(dtype)
    want_k, want_v = kc.clone(), vc.clone()
    paged_oracle.write_kv_cache_batch(want_k, want_v, tables, offsets, key, value, 16)
    dk, dv = kc.to(DEV), vc.to(DEV)
    write_kv_cache_batch(dk, dv, tables.to(DEV), offsets.to(DEV), key.to(DEV), value.to(DEV), 16, backend="hip")
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), want_k) and torch.equal(dv.cpu(), want_v)


def test_kv_cache_pool_write_gather_and_clear():
    """tests/test_kv_cache.py:6-23 on the HIP pool: page-crossing write, gather, clear."""
    cache = KVCachePool(2, 3, 4, 2, 8, dtype=torch.float16, device=DEV)
    cache.clear()
    gen = torch.Generator().manual_seed(3)
    key = torch.randn(3, 2, 8, generator=gen).half().to(DEV)
    value = key + 100
    cache.write_hip(1, [2, 0], 3, key, value)
    got_key, got_value = cache.gather(1, [2, 0], 6)
    assert torch.equal(got_key[3:6], key) and torch.equal(got_value[3:6], value)
    want_k, want_v = paged_oracle.gather(cache.key[1].cpu(), cache.value[1].cpu(), [2, 0], 6)
    assert torch.equal(got_key.cpu(), want_k) and torch.equal(got_value.cpu(), want_v)
    assert cache.memory_bytes == 2 * 3 * 4 * 2 * 8 * 2 * 2
    cache.key.fill_(1)
    cache.value.fill_(1)
    cache.clear([1])
    assert torch.all(cache.key[:, 1] == 0) and torch.all(cache.value[:, 0] == 1)


def test_prefill_context_beyond_dense_limit():
    """8193-token context through 32-token pages (test_ragged_kernels.py:124-136)."""
    block, context = 32, 8193
    gen = torch.Generator().manual_seed(81)
    pages = (context + block - 1) // block
    key = torch.randn(pages, block, 1, 16, generator=gen).half()
    value = torch.randn(pages, block, 1, 16, generator=gen).half()
    q = torch.randn(1, 2, 16, generator=gen).half()
    tables = torch.randperm(pages, generator=gen).view(1, -1)
    offsets = torch.tensor([0, 1])
    starts, lengths = torch.tensor([context - 1]), torch.tensor([context])
    actual = paged_prefill_attention(q.to(DEV), key.to(DEV), value.to(DEV), offsets.to(DEV), starts.to(DEV),
                                     tables.to(DEV), lengths.to(DEV), block, backend="hip")
    expected = paged_oracle.paged_prefill_attention(q, key, value, offsets, starts, tables, lengths, block,
                                                    cast=False)
    assert max_err(actual, expected) <= GATE[torch.float16]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("priors,block_size", [
    ([0, 5, 64, 300], 16), ([1000, 0, 17, 255], 256), ([3, 1, 0, 129], 4),
])
def test_mfma_prefill_ragged_priors(dtype, priors, block_size):
    case = workloads.chunked_prefill_case(device=DEV, num_seqs=len(priors), new_tokens=37, block_size=block_size,
                                          dtype=dtype, priors=priors, seed=7)
    write_kv_cache_slots(case["key_cache"], case["value_cache"], case["slot_mapping"], case["new_key"],
                         case["new_value"], backend="hip")
    names = ("q", "key_cache", "value_cache", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
    args = [case[n] for n in names]
    actual = paged_prefill_attention(*args, block_size, backend="hip")
    cpu = [a.cpu() for a in args]
    expected = paged_oracle.paged_prefill_attention(*cpu, block_size, cast=False)
    assert max_err(actual, expected) <= GATE[dtype]
    # The float64 C restatement agrees too.
    assert max_err(actual, c_oracle.paged_prefill(*cpu, block_size)) <= GATE[dtype]


@pytest.mark.parametrize("block", [16, 64])  # per-row copies; whole-tile pages (the pipelined loop)
@pytest.mark.parametrize("group,heads", [(1, 8), (4, 16), (8, 16)])
def test_mfma_prefill_gqa_groups(group, heads, block):
    dtype = torch.bfloat16
    gen = torch.Generator().manual_seed(group)
    kv_heads = heads // group
    width = -(-140 // block)
    pages = 2 * width + 4
    kc = torch.randn(pages, block, kv_heads, 128, generator=gen).to(dtype)
    vc = torch.randn(pages, block, kv_heads, 128, generator=gen).to(dtype)
    tables = torch.randperm(pages, generator=gen)[:2 * width].view(2, width)
    cu = torch.tensor([0, 50, 71])
    starts = torch.tensor([90, 3])
    lens = starts + (cu[1:] - cu[:-1])
    q = torch.randn(71, heads, 128, generator=gen).to(dtype)
    args = [q, kc, vc, cu, starts, tables, lens]
    actual = paged_prefill_attention(*[a.to(DEV) for a in args], block, backend="hip")
    expected = paged_oracle.paged_prefill_attention(*args, block, cast=False)
    assert max_err(actual, expected) <= GATE[dtype]


@pytest.mark.parametrize("block", [16, 256])  # per-row copies; whole-tile pages (the pipelined loop)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("group,heads,chunk_tokens", [
    (3, 24, 0), (5, 40, 256), (7, 28, 0), (7, 28, 192), (6, 12, 320), (40, 40, 0), (100, 100, 256),
])
def test_mfma_prefill_groups_not_dividing_the_row_block(dtype, group, heads, chunk_tokens, block):
    """Groups that do not divide the 256 rows of a query block (Qwen-family
    layouts such as 28/4 and 40/8 heads): the block holds 256 // group tokens
    and its last 256 % group rows are idle.  Every head of every token is
    checked, so an idle row that wrote into the next kv head's output would
    fail, with and without a key split (the merge then reads the partials)."""
    gen = torch.Generator().manual_seed(1000 + group)
    kv_heads = heads // group
    width = -(-1440 // block)
    pages = 2 * width + 20
    kc = torch.randn(pages, block, kv_heads, 128, generator=gen).to(dtype)
    vc = torch.randn(pages, block, kv_heads, 128, generator=gen).to(dtype)
    tables = torch.randperm(pages, generator=gen)[:2 * width].view(2, width)
    cu = torch.tensor([0, 150, 227])
    starts = torch.tensor([1200, 41])
    lens = starts + (cu[1:] - cu[:-1])
    q = torch.randn(227, heads, 128, generator=gen).to(dtype)
    args = [q, kc, vc, cu, starts, tables, lens]
    print(f"prefill group={group} heads={heads} chunk={chunk_tokens} block={block} {dtype}", flush=True)
    actual = paged_prefill_attention(*[a.to(DEV) for a in args], block, backend="hip", chunk_tokens=chunk_tokens)
    expected = paged_oracle.paged_prefill_attention(*args, block, cast=False)
    assert max_err(actual, expected) <= GATE[dtype]


def _two_sequence_case(head_dim, heads, kv_heads, block, dtype, seed):
    """Two sequences: 150 new tokens after 1200 cached, 77 after 41."""
    gen = torch.Generator().manual_seed(seed)
    cu = torch.tensor([0, 150, 227])
    starts = torch.tensor([1200, 41])
    lens = starts + (cu[1:] - cu[:-1])
    width = -(-int(lens.max()) // block)
    pages = 2 * width + 3
    kc = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype)
    vc = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype)
    tables = torch.randperm(pages, generator=gen)[:2 * width].view(2, width)
    q = torch.randn(227, heads, head_dim, generator=gen).to(dtype)
    return [q, kc, vc, cu, starts, tables, lens]


@pytest.mark.parametrize("dtype,chunk_tokens,priors", [
    (torch.bfloat16, 8192, [6000, 4500]),  # one chunk per sequence: items of 96 and 73 tiles
    (torch.float16, 4160, [6000, 4500]),   # first chunks of 65 tiles, a second chunk each
    (torch.bfloat16, 4224, [4100, 130]),   # 66 tiles, the last one partial
])
def test_prefill_items_longer_than_a_page_window(dtype, chunk_tokens, priors):
    """Items of more than 64 key tiles: the tile loop moves to its next window
    of page offsets (64 tiles, loaded a window ahead) inside the item."""
    case = workloads.chunked_prefill_case(device=DEV, num_seqs=2, new_tokens=96, block_size=256, dtype=dtype,
                                          priors=priors, seed=chunk_tokens)
    write_kv_cache_slots(case["key_cache"], case["value_cache"], case["slot_mapping"], case["new_key"],
                         case["new_value"], backend="hip")
    names = ("q", "key_cache", "value_cache", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
    args = [case[n] for n in names]
    print(f"prefill long items {dtype} chunk={chunk_tokens} priors={priors}", flush=True)
    actual = paged_prefill_attention(*args, 256, backend="hip", chunk_tokens=chunk_tokens)
    cpu_args = [a.cpu() for a in args]
    assert max_err(actual, paged_oracle.paged_prefill_attention(*cpu_args, 256, cast=False)) <= GATE[dtype]
    assert max_err(actual, c_oracle.paged_prefill(*cpu_args, 256)) <= GATE[dtype]


@pytest.mark.parametrize("head_dim,block,chunk_tokens,dtype,heads,kv_heads", [
    (64, 256, 0, torch.bfloat16, 16, 8), (64, 256, 256, torch.float16, 16, 8), (8, 256, 0, torch.bfloat16, 8, 1),
    (16, 16, 0, torch.float16, 4, 4), (40, 5, 0, torch.bfloat16, 16, 4), (72, 64, 192, torch.float16, 9, 3),
    (96, 256, 192, torch.bfloat16, 28, 4), (120, 16, 320, torch.float16, 4, 2),
])
def test_mfma_prefill_narrow_heads(head_dim, block, chunk_tokens, dtype, heads, kv_heads):
    """head_dim a multiple of 8 below 128 runs the MFMA kernel with rows
    zero-padded to 128 in LDS: whole-tile copies (block 256, 64) skip the
    padded chunks, per-row copies (block 16, 5) read zeros for them; with a
    key split the partials are 128 wide and the merge writes head_dim."""
    args = _two_sequence_case(head_dim, heads, kv_heads, block, dtype, seed=head_dim + block)
    print(f"narrow prefill D={head_dim} block={block} chunk={chunk_tokens} {dtype} {heads}/{kv_heads}", flush=True)
    actual = paged_prefill_attention(*[a.to(DEV) for a in args], block, backend="hip", chunk_tokens=chunk_tokens)
    assert actual.shape == args[0].shape
    assert max_err(actual, paged_oracle.paged_prefill_attention(*args, block, cast=False)) <= GATE[dtype]
    assert max_err(actual, c_oracle.paged_prefill(*args, block)) <= GATE[dtype]


@pytest.mark.parametrize("block,chunk_tokens,dtype,heads,kv_heads", [
    (256, 0, torch.bfloat16, 16, 8), (256, 256, torch.float16, 16, 8), (32, 0, torch.bfloat16, 40, 8),
    (16, 0, torch.bfloat16, 8, 1), (5, 320, torch.float16, 28, 4), (64, 96, torch.bfloat16, 100, 100),
])
def test_mfma_prefill_head_dim_256(block, chunk_tokens, dtype, heads, kv_heads):
    """head_dim 256 runs the MFMA kernel with 16 query rows per wave and
    32-key tiles: whole-tile copies (blocks 256, 64, 32), per-row-pair copies
    (block 16), per-row copies (block 5), key splits with 256-wide partials,
    and GQA groups 2, 5, 8, 7 and 1."""
    args = _two_sequence_case(256, heads, kv_heads, block, dtype, seed=block + chunk_tokens)
    print(f"prefill D=256 block={block} chunk={chunk_tokens} {dtype} {heads}/{kv_heads}", flush=True)
    actual = paged_prefill_attention(*[a.to(DEV) for a in args], block, backend="hip", chunk_tokens=chunk_tokens)
    assert max_err(actual, paged_oracle.paged_prefill_attention(*args, block, cast=False)) <= GATE[dtype]
    assert max_err(actual, c_oracle.paged_prefill(*args, block)) <= GATE[dtype]


@pytest.mark.parametrize("head_dim,block,chunk_tokens,dtype", [
    (192, 256, 0, torch.float16), (136, 16, 256, torch.bfloat16), (248, 5, 0, torch.bfloat16),
    (160, 64, 128, torch.float16),
])
def test_mfma_prefill_heads_between_128_and_256(head_dim, block, chunk_tokens, dtype):
    """Multiples of 8 between 128 and 256 run the 256 tile shape with rows
    zero-padded to 256 (whole-tile and per-row copies, with key splits)."""
    args = _two_sequence_case(head_dim, 8, 4, block, dtype, seed=head_dim + block)
    print(f"prefill D={head_dim} block={block} chunk={chunk_tokens} {dtype}", flush=True)
    actual = paged_prefill_attention(*[a.to(DEV) for a in args], block, backend="hip", chunk_tokens=chunk_tokens)
    assert max_err(actual, paged_oracle.paged_prefill_attention(*args, block, cast=False)) <= GATE[dtype]
    assert max_err(actual, c_oracle.paged_prefill(*args, block)) <= GATE[dtype]


@pytest.mark.parametrize("head_dim,block,dtype", [(100, 16, torch.bfloat16), (12, 4, torch.float16),
                                                  (264, 16, torch.float16)])
def test_generic_prefill_other_head_dims(head_dim, block, dtype):
    """Head dims the MFMA kernel does not take (not a multiple of 8, or
    above 256) run the one-wave-per-row kernel."""
    args = _two_sequence_case(head_dim, 8, 4, block, dtype, seed=head_dim)
    print(f"generic prefill D={head_dim} block={block} {dtype}", flush=True)
    actual = paged_prefill_attention(*[a.to(DEV) for a in args], block, backend="hip")
    assert max_err(actual, paged_oracle.paged_prefill_attention(*args, block, cast=False)) <= GATE[dtype]


def test_c5_chunked_prefill_full_size():
    """8 sequences x 128 new tokens after U[0,3968] prior tokens, block 256, bf16."""
    case = workloads.chunked_prefill_case(device=DEV)
    write_kv_cache_slots(case["key_cache"], case["value_cache"], case["slot_mapping"], case["new_key"],
                         case["new_value"], backend="hip")
    names = ("q", "key_cache", "value_cache", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
    args = [case[n] for n in names]
    actual = paged_prefill_attention(*args, 256, backend="hip")
    expected = paged_oracle.paged_prefill_attention(*[a.cpu() for a in args], 256, cast=False)
    assert max_err(actual, expected) <= GATE[torch.bfloat16]
    # Scatter bit-exactness at full size: every new row sits in its slot.
    rows = case["key_cache"].view(-1, 8, 128)[case["slot_mapping"]]
    assert torch.equal(rows, case["new_key"])


@pytest.mark.parametrize("dtype,block_size,chunk_tokens", [
    (torch.bfloat16, 256, 0), (torch.float16, 16, 0), (torch.bfloat16, 256, 192),
])
def test_prefill_work_groups_walk_several_items(dtype, block_size, chunk_tokens):
    """Few query blocks over long contexts: the keys are split into more chunk
    items than there are CU slots, so each work-group walks several items and
    the merge combines up to 37 partials per row."""
    priors = [7000, 3000, 5000, 6100] * 4
    case = workloads.chunked_prefill_case(device=DEV, num_seqs=16, new_tokens=64, block_size=block_size,
                                          dtype=dtype, priors=priors, seed=11)
    write_kv_cache_slots(case["key_cache"], case["value_cache"], case["slot_mapping"], case["new_key"],
                         case["new_value"], backend="hip")
    names = ("q", "key_cache", "value_cache", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
    args = [case[n] for n in names]
    actual = paged_prefill_attention(*args, block_size, backend="hip", chunk_tokens=chunk_tokens)
    expected = paged_oracle.paged_prefill_attention(*[a.cpu() for a in args], block_size, cast=False)
    assert max_err(actual, expected) <= GATE[dtype]


@pytest.mark.parametrize("chunk_tokens", [0, 512])
def test_prefill_walk_over_more_than_64_sequences(chunk_tokens):
    """70 sequences of 8 new tokens (GQA group 8, so 32 tokens per query
    block) after 500..3000 prior tokens: the keys split, the work-groups walk
    several items each, and with more than 64 sequences the lookups take the
    general path; with chunk_tokens=0 the walk also picks its chunk from the
    lengths."""
    dtype, block, heads, kv_heads = torch.bfloat16, 16, 16, 2
    gen = torch.Generator().manual_seed(70)
    seqs, new = 70, 8
    priors = torch.randint(500, 3001, (seqs,), generator=gen)
    widths = (priors + new + block - 1) // block
    width = int(widths.max())
    pages = int(widths.sum()) + 3
    kc = torch.randn(pages, block, kv_heads, 128, generator=gen).to(dtype)
    vc = torch.randn(pages, block, kv_heads, 128, generator=gen).to(dtype)
    perm = torch.randperm(pages, generator=gen)
    tables = torch.full((seqs, width), -1, dtype=torch.int64)
    used = 0
    for s in range(seqs):
        w = int(widths[s])
        tables[s, :w] = perm[used:used + w]
        used += w
    cu = torch.arange(0, (seqs + 1) * new, new, dtype=torch.int64)
    starts = priors.to(torch.int64)
    lens = starts + new
    q = torch.randn(seqs * new, heads, 128, generator=gen).to(dtype)
    args = [q, kc, vc, cu, starts, tables, lens]
    actual = paged_prefill_attention(*[a.to(DEV) for a in args], block, backend="hip", chunk_tokens=chunk_tokens)
    expected = paged_oracle.paged_prefill_attention(*args, block, cast=False)
    assert max_err(actual, expected) <= GATE[dtype]


@pytest.mark.parametrize("block", [16, 64])
def test_trusted_mode_offsets_out_of_order_stay_in_bounds(block):
    """validate=False with query offsets that are not monotone or pass the
    packed rows: the kernel clamps them to the rows, so it neither writes
    past the output nor loops over absurd block counts; rows no sequence
    covers are unspecified, every value finite."""
    dtype = torch.bfloat16
    gen = torch.Generator().manual_seed(5)
    width = -(-192 // block)
    pages = 3 * width + 4
    kc = torch.randn(pages, block, 8, 128, generator=gen).to(dtype).to(DEV)
    vc = torch.randn(pages, block, 8, 128, generator=gen).to(dtype).to(DEV)
    tables = torch.randperm(pages, generator=gen)[:3 * width].view(3, width).to(DEV)
    q = torch.randn(71, 16, 128, generator=gen).to(dtype).to(DEV)
    starts = torch.tensor([90, 3, 10], device=DEV)
    lens = torch.tensor([140, 50, 100], device=DEV)
    for cu in ([0, 50, 30, 71], [0, 50, 1 << 40, 71], [-5, 20, 60, 1 << 33]):
        out = paged_prefill_attention(q, kc, vc, torch.tensor(cu, device=DEV), starts, tables, lens, block,
                                      backend="hip", validate=False)
        torch.cuda.synchronize()
        assert out.shape == q.shape


def random_prefill_case(case):
    """A seeded random ragged prefill: head dim (MFMA tile shapes, narrow and
    wide rows, the generic kernel), GQA group, page size, sequences with 0 to
    300 new tokens after 0 to 3000 cached ones, and the key-chunk request."""
    rng = random.Random(5000 + case)
    dim = rng.choice([8, 16, 40, 64, 96, 128, 128, 136, 200, 256, 12, 100])
    kv = rng.choice([1, 2, 4, 8])
    heads = kv * rng.choice([1, 2, 3, 4, 7, 8])
    block = rng.choice([5, 16, 64, 256])
    nseq = rng.choice([1, 2, 3, 6])
    new = [rng.choice([0, 1, 17, 64, 130, 300]) for _ in range(nseq)]
    if sum(new) == 0:
        new[0] = 33
    priors = [rng.choice([0, 5, 200, 1000, 3000]) for _ in range(nseq)]
    dtype = rng.choice([torch.float16, torch.bfloat16])
    chunk = rng.choice([0, 0, 256, 512])
    gen = torch.Generator().manual_seed(case)
    cu = torch.tensor([0] + torch.tensor(new).cumsum(0).tolist())
    starts = torch.tensor(priors)
    lens = starts + torch.tensor(new)
    width = max(1, -(-int(lens.max()) // block))
    pages = nseq * width + 3
    kc = torch.randn(pages, block, kv, dim, generator=gen).to(dtype)
    vc = torch.randn(pages, block, kv, dim, generator=gen).to(dtype)
    tables = torch.randperm(pages, generator=gen)[:nseq * width].view(nseq, width)
    q = torch.randn(int(cu[-1]), heads, dim, generator=gen).to(dtype)
    return [q, kc, vc, cu, starts, tables, lens], block, chunk, dtype


@pytest.mark.parametrize("case", range(16))
def test_random_prefill_shapes_match_oracle(case):
    args, block, chunk, dtype = random_prefill_case(case)
    print(f"random prefill {case}: D={args[0].shape[2]} {args[0].shape[1]}/{args[1].shape[2]} "
          f"new={(args[3][1:] - args[3][:-1]).tolist()} priors={args[4].tolist()} block={block} chunk={chunk} "
          f"{dtype}", flush=True)
    actual = paged_prefill_attention(*[a.to(DEV) for a in args], block, backend="hip", chunk_tokens=chunk)
    assert torch.isfinite(actual).all()
    assert max_err(actual, paged_oracle.paged_prefill_attention(*args, block, cast=False)) <= GATE[dtype]
