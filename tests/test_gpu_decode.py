"""GPU parity of HIP paged decode attention against the CPU oracle.

Restates the reference's kernel tests (tests/test_cuda_paged_attention.py)
for backend="hip": all supported head dims and both dtypes vs the fp32
oracle, block/partition boundaries, metadata rejection, non-default stream,
trusted-mode corrupt tables, graph capture with mutated inputs, and the
benchmark workloads.  Tolerances: the north-star gate (max abs error
<= 2e-3 fp16, <= 1.6e-2 bf16 vs the fp32 oracle) unless a tighter reference
tolerance applies.
"""

import random

import pytest
import torch

from gpu_cases import decode_inputs
from mini_engine_hip.kernels.paged import paged_attention, workspace_bytes
from oracle import c_oracle, paged_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
GATE = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def to_dev(args):
    return [a.to(DEV) if isinstance(a, torch.Tensor) else a for a in args]


def oracle(args):
    q, k, v, t, l, bs = args
    return paged_oracle.fp32_oracle(dict(zip(paged_oracle.TENSOR_NAMES, (q, k, v, t, l))), bs)


def max_err(actual, expected):
    return (actual.float().cpu() - expected.float()).abs().max().item()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim", [16, 32, 64, 80, 96, 128, 192, 256])
def test_hip_gqa_splitkv_matches_oracle(dtype, dim):
    args = decode_inputs(dtype, head_dim=dim)
    actual = paged_attention(*to_dev(args), backend="hip")
    expected = oracle(args)
    assert max_err(actual, expected) <= GATE[dtype]
    # Reference tolerance against fp32 SDPA (test_cuda_paged_attention.py:43-44).
    atol = 0.004 if dtype == torch.bfloat16 else 0.0006
    torch.testing.assert_close(actual.float().cpu(), expected, atol=atol, rtol=0.015)


@pytest.mark.parametrize("block_size,lengths,heads,kv_heads", [
    (4, (1,), 4, 4), (16, (256, 255), 8, 1),
    (32, (257, 1025, 9), 16, 8), (16, (4097,), 16, 8),
    (1, (3, 70), 6, 2), (7, (50, 13, 1), 12, 4), (256, (2048, 1, 700), 16, 8),
])
def test_hip_block_and_partition_boundaries(block_size, lengths, heads, kv_heads):
    args = decode_inputs(torch.bfloat16, block_size=block_size, lengths=lengths, heads=heads, kv_heads=kv_heads)
    actual = paged_attention(*to_dev(args), backend="hip")
    assert max_err(actual, oracle(args)) <= GATE[torch.bfloat16]


@pytest.mark.parametrize("batch", [2, 37, 64, 65, 203, 256])
def test_longest_first_unit_order_keeps_each_sequence_its_own_output(batch):
    """Whole-sequence mode hands units out longest context first; every
    sequence must still get its own result, with ties, a one-token context
    and lengths that change between calls on the same tables."""
    gen = torch.Generator().manual_seed(900 + batch)
    lengths = torch.randint(1, 700, (batch,), generator=gen)
    lengths[: batch // 3] = 333  # ties keep the index order
    lengths[-1] = 1
    args = decode_inputs(torch.float16, lengths=tuple(lengths.tolist()), block_size=16, seed=batch)
    dev = to_dev(args)
    actual = paged_attention(*dev, backend="hip")
    expected = oracle(args)
    assert max_err(actual, expected) <= GATE[torch.float16]
    for b in (0, batch // 2, batch - 1):  # each sequence alone gives the same rows
        alone = paged_attention(dev[0][b:b + 1], dev[1], dev[2], dev[3][b:b + 1], dev[4][b:b + 1], 16,
                                backend="hip")
        assert (alone.float() - actual[b:b + 1].float()).abs().max().item() <= 2e-3
    reversed_lens = dev[4].flip(0).contiguous()  # a permutation of the same lengths
    args2 = list(args)
    args2[4] = reversed_lens.cpu()
    again = paged_attention(dev[0], dev[1], dev[2], dev[3], reversed_lens, 16, backend="hip")
    assert max_err(again, oracle(args2)) <= GATE[torch.float16]


@pytest.mark.parametrize("batch,heads,kv_heads,high", [(37, 16, 8, 4096), (64, 16, 8, 4096), (200, 4, 2, 3000)])
def test_two_work_groups_per_cu_pair_long_with_short(batch, heads, kv_heads, high):
    """Units in (CUs, 2 CUs]: two 8-wave work-groups per CU hold every unit,
    and the second half of the unit groups takes the lengths shortest first
    (odd batch, batch 64, and the LDS ranking of more than 64 sequences):
    every sequence still gets its own result."""
    gen = torch.Generator().manual_seed(batch)
    lengths = torch.randint(1, high + 1, (batch,), generator=gen)
    lengths[0] = high
    lengths[1] = 1
    args = decode_inputs(torch.bfloat16, lengths=tuple(lengths.tolist()), block_size=16, heads=heads,
                         kv_heads=kv_heads, seed=batch)
    dev = to_dev(args)
    print(f"paired units B={batch} {heads}/{kv_heads}", flush=True)
    actual = paged_attention(*dev, backend="hip")
    assert max_err(actual, oracle(args)) <= GATE[torch.bfloat16]
    for b in (0, 1, batch // 2, batch - 1):
        alone = paged_attention(dev[0][b:b + 1], dev[1], dev[2], dev[3][b:b + 1], dev[4][b:b + 1], 16,
                                backend="hip")
        assert (alone.float() - actual[b:b + 1].float()).abs().max().item() <= GATE[torch.bfloat16]


@pytest.mark.parametrize("partition", [64, 128, 256, 512, 4096])
def test_split_count_does_not_change_result(partition):
    """Split-K invariant: any partition size gives the single-partition answer."""
    args = decode_inputs(torch.float16, lengths=(1, 63, 64, 65, 700, 2049), block_size=16)
    dev = to_dev(args)
    single = paged_attention(*dev, backend="hip", partition_tokens=1 << 20)
    split = paged_attention(*dev, backend="hip", partition_tokens=partition)
    assert (split.float() - single.float()).abs().max().item() <= 2e-3
    assert max_err(split, oracle(args)) <= GATE[torch.float16]


def test_split_merge_over_several_weight_windows():
    """2188 partitions of 64 tokens: the merge holds at most 2048 partition
    weights at a time, so it combines two windows."""
    args = decode_inputs(torch.float16, lengths=(140000,), block_size=256, heads=2, kv_heads=1, extra_pages=1)
    dev = to_dev(args)
    single = paged_attention(*dev, backend="hip", partition_tokens=1 << 20)
    split = paged_attention(*dev, backend="hip", partition_tokens=64)
    assert (split.float() - single.float()).abs().max().item() <= 2e-3
    assert max_err(split, oracle(args)) <= GATE[torch.float16]


def ragged_lengths(batch, high, seed):
    gen = torch.Generator().manual_seed(seed)
    lengths = torch.randint(1, high + 1, (batch,), generator=gen)
    lengths[0] = high  # one unit spans several shares
    lengths[-1] = 1
    return tuple(lengths.tolist())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim,heads,kv_heads,lengths,block_size,plan", [
    (128, 16, 8, ragged_lengths(32, 4096, 1), 16, True),   # the plan's pick: 256 long units
    (128, 16, 8, (1, 5), 16, False),                       # fewer chunks than work-groups: empty shares
    (64, 16, 4, ragged_lengths(256, 600, 2), 16, False),   # 256 sequences, 4-head tiles
    (256, 8, 8, (3000, 17, 1, 4096, 900), 32, True),       # group 1, head dim 256 (40 long units)
    (80, 12, 4, (100, 2000, 3), 7, False),                 # group 3, pages not a multiple of the wave tile
    (16, 32, 8, ragged_lengths(9, 5000, 3), 64, False),    # head dim 16: 128-token chunks
    (128, 16, 8, ragged_lengths(16, 8192, 4), 16, True),   # the plan's pick: 128 long units
    (128, 2, 1, (20000,), 16, True),                       # one unit over every share: 256 pieces
    (128, 2, 1, ragged_lengths(256, 5000, 5), 16, True),   # the plan's pick: 256 sequences, one kv head
])
def test_balanced_walk_matches_oracle(dtype, dim, heads, kv_heads, lengths, block_size, plan):
    """Balanced walk: units laid end to end and cut into equal shares per
    work-group; units cut by a share boundary are merged from their pieces.
    Forced with partition_tokens=-1; the plan takes it too for long units
    (2 MiB of K+V capacity or more) numbering at most one per CU."""
    args = decode_inputs(dtype, head_dim=dim, heads=heads, kv_heads=kv_heads, lengths=lengths,
                         block_size=block_size, seed=len(lengths) + dim)
    dev = to_dev(args)
    print(f"balanced walk {dtype} D={dim} {heads}/{kv_heads} B={len(lengths)} block={block_size}", flush=True)
    walk = paged_attention(*dev, backend="hip", partition_tokens=-1)
    expected = oracle(args)
    assert max_err(walk, expected) <= GATE[dtype]
    single = paged_attention(*dev, backend="hip", partition_tokens=1 << 20)
    assert (walk.float() - single.float()).abs().max().item() <= GATE[dtype]
    if plan:
        assert torch.equal(paged_attention(*dev, backend="hip"), walk)


def test_balanced_walk_trusted_empty_and_invalid_rows():
    """Trusted mode on the walk: contexts of 0 or beyond the capacity and
    all-absent pages give zeros; the other sequences are unaffected."""
    lengths = (700, 1, 2048, 300)
    args = decode_inputs(torch.bfloat16, lengths=lengths, block_size=16, seed=77)
    dev = to_dev(args)
    dev[4][1] = 0
    dev[4][3] = 10**6
    dev[3][2].fill_(-1)
    actual = paged_attention(*dev, backend="hip", validate=False, partition_tokens=-1)
    assert torch.isfinite(actual).all()
    assert not actual[1:4].any()
    alone = paged_attention(dev[0][:1], dev[1], dev[2], dev[3][:1], dev[4][:1], 16, backend="hip")
    assert (actual[0].float() - alone[0].float()).abs().max().item() <= GATE[torch.bfloat16]


@pytest.mark.parametrize("batch,block_size,low,high,partition", [
    (2, 256, 40000, 40001, 4096), (2, 256, 40000, 40001, 0), (40, 16, 1500, 2600, 0)])
def test_streaming_loads_match_oracle(batch, block_size, low, high, partition):
    """Calls with more than 64 MiB of K/V within the tables' capacity load
    rows with the non-temporal hint: split-K (forced) and the balanced walk
    (the plan's choice) for two long sequences, whole-sequence work-groups
    for forty ragged ones."""
    gen = torch.Generator().manual_seed(batch)
    lengths = tuple(torch.randint(low, high, (batch,), generator=gen).tolist())
    args = decode_inputs(torch.float16, lengths=lengths, block_size=block_size, seed=batch)
    width = args[3].shape[1]
    assert batch * width * block_size * 8 * 128 * 4 > 64 << 20
    actual = paged_attention(*to_dev(args), backend="hip", partition_tokens=partition)
    assert max_err(actual, oracle(args)) <= GATE[torch.float16]


def test_hip_rejects_bad_metadata_and_noncontiguous_query():
    args = to_dev(decode_inputs(torch.float16))
    args[4][0] = 0
    with pytest.raises(RuntimeError, match="context length"):
        paged_attention(*args, backend="hip")
    args[4][0] = 17
    args[3][0, 0] = -1
    with pytest.raises(RuntimeError, match="physical block"):
        paged_attention(*args, backend="hip")
    args[3][0, 0] = 0
    args[0] = args[0].transpose(0, 1).contiguous().transpose(0, 1)
    with pytest.raises(RuntimeError, match="contiguous"):
        paged_attention(*args, backend="hip")


def test_hip_current_stream_and_trusted_invalid_indices():
    args = decode_inputs(torch.bfloat16, lengths=(65,))
    dev = to_dev(args)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        actual = paged_attention(*dev, backend="hip", validate=False)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert max_err(actual, oracle(args)) <= GATE[torch.bfloat16]
    # Trusted mode never reads through a corrupt page id: all -1 -> zeros.
    dev[3].fill_(-1)
    actual = paged_attention(*dev, backend="hip", validate=False)
    assert torch.isfinite(actual).all() and not actual.any()
    # Lengths beyond the table capacity, or <= 0, give zeros as well.
    dev = to_dev(args)
    dev[4].fill_(10**6)
    assert not paged_attention(*dev, backend="hip", validate=False).any()


def test_single_token_context_returns_first_value_row():
    """Closed form: context length 1 -> output = v_0 (rounded to the dtype)."""
    args = decode_inputs(torch.float16, lengths=(1, 1, 1), block_size=16)
    q, k, v, t, l, bs = args
    actual = paged_attention(*to_dev(args), backend="hip").cpu()
    group = q.shape[1] // k.shape[2]
    for b in range(q.shape[0]):
        v0 = v[t[b, 0], 0].repeat_interleave(group, dim=0)
        assert torch.equal(actual[b], v0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("block_size", [4, 16, 64, 256])
def test_graph_replay_with_mutated_query_and_lengths(dtype, block_size):
    """Capture once, mutate q and context_lens in place, replay (cuda_graph.py:244-275 pattern)."""
    args = decode_inputs(dtype, block_size=block_size, lengths=(1, 17, 127, 256))
    dev = to_dev(args)
    originals = dev[1].clone(), dev[2].clone()
    paged_attention(*dev, backend="hip", validate=False)  # warm the allocator
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = paged_attention(*dev, backend="hip", validate=False)
    for replay in range(3):
        dev[4].copy_(torch.tensor([256, 128, 16, 1][replay:] + [256, 128, 16, 1][:replay], device=DEV))
        dev[0].mul_(0.75)
        graph.replay()
        torch.cuda.synchronize()
        eager = paged_attention(*dev, backend="hip", validate=False)
        expected = oracle([x.cpu() if isinstance(x, torch.Tensor) else x for x in dev])
        assert max_err(captured, expected) <= GATE[dtype]
        assert torch.equal(captured, eager)
    assert torch.equal(originals[0], dev[1]) and torch.equal(originals[1], dev[2])


def test_oracle_c_restatement_agrees_on_gpu_case():
    """The HIP output also sits within tolerance of the float64 C oracle."""
    args = decode_inputs(torch.bfloat16, lengths=(5, 300), block_size=32, seed=99)
    actual = paged_attention(*to_dev(args), backend="hip")
    expected = c_oracle.paged_decode(*args)
    assert max_err(actual, expected) <= GATE[torch.bfloat16]


# ---------------------------------------------------------------------------
# Benchmark workloads (seeded as in the benchmark).
# ---------------------------------------------------------------------------

def test_c1_make_case_b1_ctx128_fp16():
    tensors, _ = paged_oracle.make_case(1, 128)
    args = [tensors[n] for n in paged_oracle.TENSOR_NAMES] + [256]
    actual = paged_attention(*to_dev(args), backend="hip")
    result = paged_oracle.validate_output(actual.cpu(), paged_oracle.fp32_oracle(tensors, 256))
    assert result["passed"] and result["max_absolute_error"] <= 2e-3


def test_c3_make_case_b32_ctx2048_fp16():
    tensors, _ = paged_oracle.make_case(32, 2048)
    args = [tensors[n] for n in paged_oracle.TENSOR_NAMES] + [256]
    actual = paged_attention(*to_dev(args), backend="hip")
    result = paged_oracle.validate_output(actual.cpu(), paged_oracle.fp32_oracle(tensors, 256))
    assert result["passed"] and result["max_absolute_error"] <= 2e-3


def test_c4_ragged_shared_prefix_bf16():
    """Ragged lengths in [1, 4096], 16 sequences sharing one prefix's pages."""
    from mini_engine_hip.workloads import ragged_shared_prefix_case

    case = ragged_shared_prefix_case(device=DEV)
    args = [case[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lens")] + [16]
    actual = paged_attention(*args, backend="hip", validate=True)
    expected = oracle([a.cpu() if isinstance(a, torch.Tensor) else a for a in args])
    assert max_err(actual, expected) <= GATE[torch.bfloat16]
    # Shared prefix pages really are shared: 16 tables name the same first 64 pages.
    tables = case["block_tables"].cpu()
    assert all(torch.equal(tables[i, :64], tables[0, :64]) for i in range(16))


def test_ragged_b32_balanced_walk_workload_fp16():
    """The benchmark's ragged B32 workload (contexts U[1,4096], block 256):
    one long unit per CU, which the plan hands to the balanced walk."""
    from mini_engine_hip.workloads import ragged_decode_case

    case = ragged_decode_case(device=DEV)
    args = [case[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lens")] + [256]
    actual = paged_attention(*args, backend="hip", validate=True)
    expected = oracle([a.cpu() if isinstance(a, torch.Tensor) else a for a in args])
    assert max_err(actual, expected) <= GATE[torch.float16]
    assert torch.equal(paged_attention(*args, backend="hip", partition_tokens=-1), actual)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim", [16, 32, 80, 96, 128])
@pytest.mark.parametrize("partition", [64, 0])
def test_split_merge_with_strongly_negative_scores(dtype, dim, partition):
    """Every score far below -126 in log2 units (q = -c * |k|): the merge's
    reference maximum is negative, so a reduction that let absent lanes
    contribute 0 would underflow every partition weight and return zeros.
    Head dims below 64 or not a multiple of 64 run the merge in a partial wave."""
    q, k, v, t, l, bs = decode_inputs(dtype, head_dim=dim, lengths=(300, 1000, 2500), block_size=16, seed=dim)
    k = k.abs()
    q = torch.full_like(q, -256.0)
    args = (q, k, v, t, l, bs)
    # The largest score of the whole cache, in log2 units, is far below -126.
    assert -256.0 * k.float().sum(-1).min().item() / dim ** 0.5 * 1.4427 < -300
    print(f"negative-score merge {dtype} D={dim} partition={partition}", flush=True)
    actual = paged_attention(*to_dev(args), backend="hip", partition_tokens=partition)
    expected = oracle(args)
    assert actual.float().abs().amax().item() > 0.1
    assert max_err(actual, expected) <= GATE[dtype]


def test_c2_decode_b8_with_scatter_bf16():
    """The B8 / ctx 512 / block 16 / 2048-page workload exactly: the new token
    of each sequence is scattered to position 511 (slot table[b, 31]*16+15),
    rows bit-exact, then decode over the updated pages against the oracle."""
    from mini_engine_hip.kernels.data import write_kv_cache_slots
    from mini_engine_hip.workloads import decode_b8_with_scatter

    case = decode_b8_with_scatter(device=DEV)
    kc, vc = case["key_cache"], case["value_cache"]
    assert kc.shape == (2048, 16, 8, 128) and kc.dtype == torch.bfloat16
    want_k, want_v = kc.cpu(), vc.cpu()
    paged_oracle.write_kv_cache_slots(want_k, want_v, case["slot_mapping"].cpu(), case["new_key"].cpu(),
                                      case["new_value"].cpu())
    write_kv_cache_slots(kc, vc, case["slot_mapping"], case["new_key"], case["new_value"], backend="hip")
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), want_k) and torch.equal(vc.cpu(), want_v)
    assert case["context_lens"].tolist() == [512] * 8
    args = [case["query"], kc, vc, case["block_tables"], case["context_lens"], 16]
    actual = paged_attention(*args, backend="hip")
    expected = oracle([a.cpu() if isinstance(a, torch.Tensor) else a for a in args])
    assert max_err(actual, expected) <= GATE[torch.bfloat16]
    torch.testing.assert_close(actual.float().cpu(), expected, atol=0.004, rtol=0.015)


def random_decode_shape(case):
    """A seeded random decode shape: head dim, GQA group, batch, block size
    and ragged lengths (half the cases with one sequence at the maximum)."""
    rng = random.Random(1000 + case)
    dim = rng.choice([16, 32, 64, 80, 96, 128, 128, 192, 256])
    kv = rng.choice([1, 2, 4, 8])
    heads = kv * rng.choice([1, 2, 3, 4, 8])
    batch = rng.choice([1, 2, 3, 5, 8, 13, 16, 24, 40, 64])
    block = rng.choice([1, 7, 16, 32, 64, 256])
    high = rng.choice([100, 700, 2049, 4096, 5000, 9000])
    if block == 1:
        high = min(high, 700)
    lengths = tuple(rng.randint(1, high) for _ in range(batch))
    if rng.random() < 0.5:
        lengths = (high,) + lengths[1:]
    dtype = rng.choice([torch.float16, torch.bfloat16])
    return dim, heads, kv, block, lengths, dtype


@pytest.mark.parametrize("case", range(16))
def test_random_shapes_every_mode_matches_oracle(case):
    """The library's plan, the forced balanced walk and forced split-K on the
    same seeded random shape, each against the oracle."""
    dim, heads, kv, block, lengths, dtype = random_decode_shape(case)
    args = decode_inputs(dtype, head_dim=dim, block_size=block, lengths=lengths, heads=heads, kv_heads=kv,
                         seed=case)
    dev = to_dev(args)
    print(f"random decode {case}: D={dim} {heads}/{kv} B={len(lengths)} block={block} max={max(lengths)} {dtype}",
          flush=True)
    expected = oracle(args)
    for partition in (0, -1, 256):
        assert max_err(paged_attention(*dev, backend="hip", partition_tokens=partition), expected) <= GATE[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_graph_replay_of_the_balanced_walk_with_new_lengths(dtype):
    """The plan's balanced walk (long units, fewer than the CUs) captured once
    and replayed with new context lengths: every replay rewrites the shares'
    partial rows and merge descriptors from the lengths it finds."""
    lengths = [5000, 4097, 1, 3000, 700, 4500]
    args = decode_inputs(dtype, block_size=16, lengths=tuple(lengths), seed=88)
    dev = to_dev(args)
    ws = torch.empty(workspace_bytes(len(lengths), 16, 8, 128, 16, dev[3].shape[1]), dtype=torch.uint8, device=DEV)
    out = torch.empty_like(dev[0])
    paged_attention(*dev, backend="hip", validate=False, out=out, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_attention(*dev, backend="hip", validate=False, out=out, workspace=ws)
    for replay in range(3):
        dev[4].copy_(torch.tensor(lengths[replay + 1:] + lengths[:replay + 1], device=DEV))
        graph.replay()
        torch.cuda.synchronize()
        print(f"walk graph replay {replay} {dtype}", flush=True)
        expected = oracle([x.cpu() if isinstance(x, torch.Tensor) else x for x in dev])
        assert max_err(out, expected) <= GATE[dtype]
        assert torch.equal(out, paged_attention(*dev, backend="hip", validate=False, partition_tokens=-1))
