"""The decode step's KV write fused into paged attention, against the
two-launch sequences it replaces.

Attention.forward_decode_batch (mini_engine/model/native_qwen3.py:179-197)
writes each sequence's new K/V row at position len - 1
(write_kv_cache_batch, data.py:67-81 -- or, with the q/k RMSNorm and RoPE
before it, the fused qk_norm_rope_write_kv in decode mode) and then runs
paged_attention over len tokens.  paged_attention_decode_write does both in
one launch; its cache rows, rotated queries and outputs must equal the
two-launch results bit for bit (the same kernels' arithmetic), across the
whole-sequence and split-K modes, longest-first order, GQA tiles, head dims
and dtypes, and the attention must match the fp32 oracle.
"""

import random

import pytest
import torch

from mini_engine_hip.kernels.data import write_kv_cache_batch
from mini_engine_hip.kernels.paged import paged_attention, paged_attention_decode_write
from mini_engine_hip.kernels.rope import qk_norm_rope_write_kv
from oracle import paged_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
GATE = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def make_step(batch, q_heads, kv_heads, head_dim, block, lengths, dtype, seed, pool_extra=3, fused_qkv=False):
    gen = torch.Generator().manual_seed(seed)
    width = -(-max(lengths) // block)
    pages = batch * width + pool_extra
    kc = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype)
    vc = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype)
    perm = torch.randperm(pages, generator=gen)
    tables = torch.full((batch, width), -1, dtype=torch.int64)
    for b, n in enumerate(lengths):
        used = -(-n // block)
        tables[b, :used] = perm[b * width:b * width + used]
    lens = torch.tensor(lengths, dtype=torch.int64)
    if fused_qkv:
        # q, k, v as strided slices of one projection output [batch, (Hq + 2 Hkv) D].
        qkv = torch.randn(batch, (q_heads + 2 * kv_heads) * head_dim, generator=gen).to(dtype).to(DEV)
        q = qkv[:, :q_heads * head_dim].view(batch, q_heads, head_dim)
        k = qkv[:, q_heads * head_dim:(q_heads + kv_heads) * head_dim].view(batch, kv_heads, head_dim)
        v = qkv[:, (q_heads + kv_heads) * head_dim:].view(batch, kv_heads, head_dim)
    else:
        q = torch.randn(batch, q_heads, head_dim, generator=gen).to(dtype).to(DEV)
        k = torch.randn(batch, kv_heads, head_dim, generator=gen).to(dtype).to(DEV)
        v = torch.randn(batch, kv_heads, head_dim, generator=gen).to(dtype).to(DEV)
    angles = torch.randn(batch, head_dim // 2, generator=gen) * 3
    norm = dict(q_weight=(torch.rand(head_dim, generator=gen) + 0.5).to(dtype).to(DEV),
                k_weight=(torch.rand(head_dim, generator=gen) + 0.5).to(dtype).to(DEV),
                cos=angles.cos().to(dtype).to(DEV), sin=angles.sin().to(dtype).to(DEV))
    return dict(kc=kc.to(DEV), vc=vc.to(DEV), tables=tables.to(DEV), lens=lens.to(DEV), q=q, k=k, v=v, norm=norm)


def two_launches(step, block, rope, partition_tokens, validate=True):
    """The reference's order.  The writes run unvalidated: their checks
    reject the -1 padding past each sequence's pages (data.py:67-81), which
    the fused call's checks (those of paged_attention) accept."""
    kc, vc = step["kc"].clone(), step["vc"].clone()
    positions = step["lens"] - 1
    if rope:
        n = step["norm"]
        query = qk_norm_rope_write_kv(step["q"], step["k"], step["v"], n["q_weight"], n["k_weight"], n["cos"],
                                      n["sin"], kc, vc, block_tables=step["tables"], positions=positions,
                                      validate=False)
    else:
        write_kv_cache_batch(kc, vc, step["tables"], positions, step["k"].contiguous(), step["v"].contiguous(),
                             block, validate=False)
        query = step["q"]
    out = paged_attention(query, kc, vc, step["tables"], step["lens"], block, partition_tokens=partition_tokens,
                          validate=validate)
    return kc, vc, query, out


def one_launch(step, block, rope, partition_tokens, validate=True):
    kc, vc = step["kc"].clone(), step["vc"].clone()
    q_out = torch.empty(step["q"].shape, dtype=step["q"].dtype, device=DEV) if rope else None
    extra = dict(step["norm"], q_out=q_out) if rope else {}
    out = paged_attention_decode_write(step["q"], kc, vc, step["tables"], step["lens"], block, step["k"], step["v"],
                                       partition_tokens=partition_tokens, validate=validate, **extra)
    return kc, vc, q_out, out


def check_equal(step, block, rope, partition_tokens=0, oracle=True):
    want_k, want_v, want_q, want_out = two_launches(step, block, rope, partition_tokens)
    got_k, got_v, got_q, got_out = one_launch(step, block, rope, partition_tokens)
    torch.cuda.synchronize()
    assert torch.equal(got_v, want_v)
    assert torch.equal(got_k, want_k)
    if rope:
        assert torch.equal(got_q, want_q)
    assert torch.equal(got_out, want_out)
    # The written rows are really there (the two-launch path could be wrong too).
    b = 0
    pos = int(step["lens"][b]) - 1
    page = int(step["tables"][b, pos // block])
    assert torch.equal(got_v[page, pos % block], step["v"][b])
    if oracle:
        q = (got_q if rope else step["q"]).cpu()
        tensors = dict(zip(paged_oracle.TENSOR_NAMES, (q, got_k.cpu(), got_v.cpu(), step["tables"].cpu(),
                                                        step["lens"].cpu())))
        want = paged_oracle.fp32_oracle(tensors, block)
        assert (got_out.float().cpu() - want).abs().max().item() <= GATE[step["q"].dtype]


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_headline_shape_whole_sequence(rope, dtype):
    """B32, Hq16/Hkv8/D128, block 256, ragged lengths up to 2048: one 8-wave
    work-group per (sequence, kv head), longest sequences first."""
    gen = torch.Generator().manual_seed(3)
    lengths = torch.randint(1, 2049, (32,), generator=gen).tolist()
    step = make_step(32, 16, 8, 128, 256, lengths, dtype, seed=11)
    print(f"decode write headline rope={rope} {dtype}", flush=True)
    check_equal(step, 256, rope)


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("head_dim", [16, 32, 64, 128, 256])
def test_split_k_and_head_dims(rope, head_dim):
    """Few sequences over long contexts: split-K partitions; only the
    partition holding the new position writes it."""
    step = make_step(2, 8, 2, head_dim, 16, [1500, 777], torch.bfloat16, seed=head_dim)
    print(f"decode write split-K rope={rope} D={head_dim}", flush=True)
    check_equal(step, 16, rope, partition_tokens=256)
    check_equal(step, 16, rope, partition_tokens=0)


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_balanced_walk(rope, head_dim):
    """The balanced walk (units cut into equal shares per work-group): the
    share holding position len - 1 writes the row, the share that starts the
    unit writes the rotated query."""
    gen = torch.Generator().manual_seed(head_dim)
    lengths = torch.randint(1, 3001, (24,), generator=gen)
    lengths[0] = 3000
    step = make_step(24, 16, 8, head_dim, 16, lengths.tolist(), torch.bfloat16, seed=head_dim + 1)
    print(f"decode write balanced walk rope={rope} D={head_dim}", flush=True)
    check_equal(step, 16, rope, partition_tokens=-1)


@pytest.mark.parametrize("q_heads,kv_heads", [(8, 8), (32, 8), (64, 8), (28, 4)])
def test_gqa_tiles(q_heads, kv_heads):
    """Group 1, 4, 8 (two 4-head tiles, both writing the same rows) and 7."""
    step = make_step(6, q_heads, kv_heads, 128, 32, [5, 300, 64, 1, 129, 700], torch.float16, seed=q_heads)
    print(f"decode write GQA {q_heads}/{kv_heads}", flush=True)
    check_equal(step, 32, True)
    check_equal(step, 32, False)


def test_strided_fused_qkv_rows():
    """Raw q, k, v as slices of one projection output (rows not dense); the
    attention query of the write-only form is contiguous, as paged_attention
    requires."""
    step = make_step(8, 16, 8, 128, 16, [33, 17, 1, 250, 96, 7, 128, 64], torch.bfloat16, seed=5, fused_qkv=True)
    check_equal(step, 16, True)
    check_equal(dict(step, q=step["q"].contiguous()), 16, False)


def test_absent_page_is_not_written():
    """Trusted mode: a new position whose page entry is -1 or out of range
    writes nothing (the batch KV write skips it too); attention treats the
    page as absent."""
    step = make_step(4, 16, 8, 128, 16, [40, 40, 40, 40], torch.float16, seed=9)
    step["tables"][1, 2] = -1
    step["tables"][2, 2] = step["kc"].shape[0] + 5
    want_k, want_v, _, want_out = two_launches(step, 16, True, 0, validate=False)
    got_k, got_v, _, got_out = one_launch(step, 16, True, 0, validate=False)
    torch.cuda.synchronize()
    assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v) and torch.equal(got_out, want_out)
    changed = ~(got_v == step["vc"]).all(-1).all(-1)  # [page, row]
    assert int(changed.sum()) == 2  # sequences 0 and 3 wrote their row; 1 and 2 wrote nothing


def test_other_head_dims_run_two_launches():
    """head_dim 80 has no fused prologue: the call runs the write and the
    attention as two launches and gives the same results."""
    step = make_step(3, 8, 4, 80, 16, [20, 3, 57], torch.float16, seed=80)
    check_equal(step, 16, True)
    check_equal(step, 16, False)


def test_trusted_empty_context_and_no_q_out():
    """Trusted mode: a sequence with context length 0 writes nothing and
    returns zeros (as the two launches do); norm/RoPE mode without q_out."""
    step = make_step(3, 16, 8, 128, 16, [1, 5, 33], torch.bfloat16, seed=21)
    step["lens"][0] = 0
    want_k, want_v, _, want_out = two_launches(step, 16, True, 0, validate=False)
    kc, vc = step["kc"].clone(), step["vc"].clone()
    got = paged_attention_decode_write(step["q"], kc, vc, step["tables"], step["lens"], 16, step["k"], step["v"],
                                       validate=False, **step["norm"])
    torch.cuda.synchronize()
    assert torch.equal(kc, want_k) and torch.equal(vc, want_v) and torch.equal(got, want_out)
    assert not got[0].any()


def test_in_place_rotation_takes_two_launches():
    """q_out that is the query itself (an in-place rotation) runs the two
    launches, whose norm/RoPE kernel reads and writes each row in the same
    lanes; a q_out that overlaps the query any other way is refused (one
    launch reads the raw rows in every work-group while another writes
    q_out)."""
    step = make_step(4, 16, 8, 128, 16, [40, 9, 300, 77], torch.bfloat16, seed=31)
    want_k, want_v, want_q, want_out = two_launches(step, 16, True, 0)
    kc, vc = step["kc"].clone(), step["vc"].clone()
    q = step["q"].clone()
    got = paged_attention_decode_write(q, kc, vc, step["tables"], step["lens"], 16, step["k"], step["v"],
                                       q_out=q, **step["norm"])
    torch.cuda.synchronize()
    assert torch.equal(kc, want_k) and torch.equal(vc, want_v)
    assert torch.equal(q, want_q) and torch.equal(got, want_out)
    tensors = dict(zip(paged_oracle.TENSOR_NAMES, (q.cpu(), kc.cpu(), vc.cpu(), step["tables"].cpu(),
                                                    step["lens"].cpu())))
    want = paged_oracle.fp32_oracle(tensors, 16)
    assert (got.float().cpu() - want).abs().max().item() <= GATE[torch.bfloat16]
    # A q_out shifted by one query row overlaps the query without being it.
    storage = torch.empty(5 * 16 * 128, dtype=torch.bfloat16, device=DEV)
    raw = storage[:4 * 16 * 128].view(4, 16, 128).copy_(step["q"])
    shifted = storage[16 * 128:].view(4, 16, 128)
    with pytest.raises(ValueError, match="overlap"):
        paged_attention_decode_write(raw, step["kc"].clone(), step["vc"].clone(), step["tables"], step["lens"], 16,
                                     step["k"], step["v"], q_out=shifted, **step["norm"])


@pytest.mark.parametrize("case", range(12))
def test_random_steps_every_mode(case):
    """Seeded random decode steps (head dim, GQA group, batch, page size,
    ragged lengths, with or without the norm/RoPE prologue), each through the
    library's plan, the forced balanced walk and forced split-K: bit-equal to
    the two launches and within the oracle's gate."""
    rng = random.Random(7000 + case)
    head_dim = rng.choice([16, 32, 64, 128, 128, 256])
    kv_heads = rng.choice([1, 2, 4, 8])
    q_heads = kv_heads * rng.choice([1, 2, 4, 8])
    batch = rng.choice([1, 3, 8, 16, 40])
    block = rng.choice([16, 32, 256])
    high = rng.choice([300, 2049, 5000])
    lengths = [rng.randint(1, high) for _ in range(batch)]
    lengths[0] = high
    dtype = rng.choice([torch.float16, torch.bfloat16])
    rope = rng.random() < 0.5
    step = make_step(batch, q_heads, kv_heads, head_dim, block, lengths, dtype, seed=case)
    print(f"decode write random {case}: D={head_dim} {q_heads}/{kv_heads} B={batch} block={block} max={high} "
          f"rope={rope} {dtype}", flush=True)
    for partition_tokens in (0, -1, 256):
        check_equal(step, block, rope, partition_tokens=partition_tokens)
