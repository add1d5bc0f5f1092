"""GPU parity of the fused q/k RMSNorm + RoPE + KV write against the oracle.

Restates the reference's tests of the three steps it fuses for backend="hip":
RoPE with GQA (tests/test_data_kernels.py:26-37: atol 0.004 bf16 / 0.001
fp16, rtol 0.01), RMSNorm (tests/test_cuda_elementwise.py:80-81: atol 0.004,
rtol 0.008) and the KV writes (tests/test_data_kernels.py:40-57, bit-exact),
composed as Attention._forward_prefill_batch / forward_decode_batch run them
(mini_engine/model/native_qwen3.py:150-157, :179-191).

The kernel rounds at the same places as the oracle; only the fp32 sum of
squares (order) and the reciprocal square root may differ in the last fp32
bit, which can move a normalised value by one fp16/bf16 ulp.  So every element
must lie within the reference's tolerance or within two ulps of the operands
of its rotation, and at least 99% of the elements must be bit-identical to the
oracle (a dropped rounding step changes far more than 1%).
"""

import pytest
import torch

from gpu_cases import assert_rope_close
from mini_engine_hip.kernels.rope import qk_norm_rope_write_kv
from oracle import paged_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def fused_case(dtype, tokens, heads, kv_heads, dim, block, pages, seed, pad=0):
    """Rows of one fused QKV projection [T, (Hq + 2 Hkv) * D (+ pad)], as _project_qkv slices them."""
    gen = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(tokens, (heads + 2 * kv_heads) * dim + pad, generator=gen) * 3).to(dtype)
    angles = torch.randn(tokens, dim // 2, generator=gen) * 4
    cos, sin = angles.cos().to(dtype), angles.sin().to(dtype)
    wq = (torch.rand(dim, generator=gen) + 0.5).to(dtype)
    wk = (torch.rand(dim, generator=gen) + 0.5).to(dtype)
    kc = torch.randn(pages, block, kv_heads, dim, generator=gen).to(dtype)
    vc = torch.randn(pages, block, kv_heads, dim, generator=gen).to(dtype)
    return qkv, cos, sin, wq, wk, kc, vc


def split_qkv(qkv, heads, kv_heads, dim):
    t, off = qkv.shape[0], qkv.shape[1] - (heads + 2 * kv_heads) * dim   # leading pad columns
    q = qkv[:, off:off + heads * dim].view(t, heads, dim)
    k = qkv[:, off + heads * dim:off + (heads + kv_heads) * dim].view(t, kv_heads, dim)
    v = qkv[:, off + (heads + kv_heads) * dim:].view(t, kv_heads, dim)
    return q, k, v


def run_and_check(dtype, tokens, heads, kv_heads, dim, block, pages, seed, *, slots=None, tables=None,
                  positions=None, stream=None, pad=0):
    qkv, cos, sin, wq, wk, kc, vc = fused_case(dtype, tokens, heads, kv_heads, dim, block, pages, seed, pad)
    q, k, v = split_qkv(qkv, heads, kv_heads, dim)
    ke, ve = kc.clone(), vc.clone()
    expected_q = paged_oracle.qk_norm_rope_write_kv(q, k, v, wq, wk, cos, sin, ke, ve, slot_mapping=slots,
                                                    block_tables=tables, positions=positions)
    normed_q, normed_k = paged_oracle.rms_norm(q, wq), paged_oracle.rms_norm(k, wk)
    dq, dk, dv = split_qkv(qkv.to(DEV), heads, kv_heads, dim)
    kd, vd = kc.to(DEV), vc.to(DEV)
    meta = {}
    if slots is not None:
        meta["slot_mapping"] = slots.to(DEV)
    else:
        meta["block_tables"], meta["positions"] = tables.to(DEV), positions.to(DEV)
    args = (dq, dk, dv, wq.to(DEV), wk.to(DEV), cos.to(DEV), sin.to(DEV), kd, vd)
    print(f"fused norm/rope/write {dtype} T={tokens} Hq={heads} Hkv={kv_heads} D={dim} seed={seed}", flush=True)
    if stream is None:
        actual_q = qk_norm_rope_write_kv(*args, validate=False, **meta)
    else:
        with torch.cuda.stream(stream):
            actual_q = qk_norm_rope_write_kv(*args, validate=False, **meta)
        stream.synchronize()
    torch.cuda.synchronize()
    assert_rope_close(actual_q, expected_q, normed_q, dtype)
    # Written K rows within tolerance; every other cache row, and all of V, bit-exact.
    written = ~(ke == kc).all(-1).all(-1)   # [pages, block] rows the oracle changed
    kd, vd = kd.cpu(), vd.cpu()
    assert torch.equal(vd, ve)
    assert torch.equal(kd[~written], ke[~written])
    if slots is not None:
        rows = [t for t, s in enumerate(slots.tolist()) if 0 <= s < pages * block]
        flat = torch.tensor([slots[t] for t in rows], dtype=torch.long)
    else:
        rows, flat = [], []
        for t, pos in enumerate(positions.tolist()):
            if 0 <= pos < tables.shape[1] * block and 0 <= tables[t, pos // block] < pages:
                rows.append(t)
                flat.append(int(tables[t, pos // block]) * block + pos % block)
        flat = torch.tensor(flat, dtype=torch.long)
    got_k = kd.view(-1, kv_heads, dim)[flat]
    want_k = ke.view(-1, kv_heads, dim)[flat]
    _, want_rot = paged_oracle.apply_rope(normed_q[rows], normed_k[rows], cos[rows].unsqueeze(1),
                                          sin[rows].unsqueeze(1))
    assert torch.equal(want_rot, want_k)
    assert_rope_close(got_k, want_k, normed_k[rows], dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim,heads,kv_heads", [(16, 8, 2), (64, 4, 4), (128, 16, 8), (256, 8, 1)])
def test_prefill_slots_match_oracle(dtype, dim, heads, kv_heads):
    tokens, block, pages = 37, 16, 5
    gen = torch.Generator().manual_seed(dim)
    slots = torch.randperm(pages * block, generator=gen)[:tokens].to(torch.int64)
    slots[3] = -1                       # invalid slots are skipped, their q rows still written
    slots[11] = pages * block
    run_and_check(dtype, tokens, heads, kv_heads, dim, block, pages, seed=dim + heads, slots=slots)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim,pad", [(96, 0), (40, 0), (128, 3), (64, 8)])
def test_general_kernel_odd_dims_and_unaligned_rows(dtype, dim, pad):
    """head_dim not a power of two, or rows off 16-byte alignment (pad 3): the general kernel; pad 8 keeps
    the vector kernel with a token stride that is not the row width."""
    tokens, block, pages = 19, 8, 4
    gen = torch.Generator().manual_seed(dim + pad)
    slots = torch.randperm(pages * block, generator=gen)[:tokens].to(torch.int64)
    run_and_check(dtype, tokens, 6, 3, dim, block, pages, seed=dim * 3 + pad, slots=slots, pad=pad)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_tables_positions_on_nondefault_stream(dtype):
    batch, block, pages, width = 6, 4, 20, 3
    gen = torch.Generator().manual_seed(77)
    tables = torch.randperm(pages, generator=gen)[:batch * width].view(batch, width).to(torch.int64)
    tables[4, 1] = -1                   # page id out of range: skipped
    positions = torch.tensor([0, 5, 11, 3, 6, 12], dtype=torch.int64)   # 12 is beyond the table
    run_and_check(dtype, batch, 16, 8, 128, block, pages, seed=78, tables=tables, positions=positions,
                  stream=torch.cuda.Stream())


def test_full_prefill_batch_1024_tokens_bf16():
    """8 sequences x 128 tokens, Hq 16 / Hkv 8 / D 128, block 256: the benchmark's prefill batch."""
    tokens, block, pages = 1024, 256, 40
    gen = torch.Generator().manual_seed(5)
    slots = torch.randperm(pages * block, generator=gen)[:tokens].to(torch.int64)
    run_and_check(torch.bfloat16, tokens, 16, 8, 128, block, pages, seed=6, slots=slots)


def test_repeated_calls_are_bit_identical_and_validation_raises():
    dtype, tokens, heads, kv_heads, dim = torch.float16, 9, 4, 2, 32
    qkv, cos, sin, wq, wk, kc, vc = (t.to(DEV) for t in fused_case(dtype, tokens, heads, kv_heads, dim, 4, 6, 3))
    q, k, v = split_qkv(qkv, heads, kv_heads, dim)
    slots = torch.arange(tokens, dtype=torch.int64, device=DEV) * 2
    first = qk_norm_rope_write_kv(q, k, v, wq, wk, cos, sin, kc, vc, slot_mapping=slots)
    k1 = kc.clone()
    second = qk_norm_rope_write_kv(q, k, v, wq, wk, cos, sin, kc, vc, slot_mapping=slots)
    assert torch.equal(first, second) and torch.equal(kc, k1)
    with pytest.raises(ValueError, match="duplicate KV slots"):
        qk_norm_rope_write_kv(q, k, v, wq, wk, cos, sin, kc, vc, slot_mapping=torch.zeros_like(slots))
    with pytest.raises(RuntimeError, match="RoPE cos/sin shape mismatch"):
        qk_norm_rope_write_kv(q, k, v, wq, wk, cos[:-1], sin[:-1], kc, vc, slot_mapping=slots)
    with pytest.raises(RuntimeError, match="GQA head mismatch"):
        qk_norm_rope_write_kv(q[:, :3], k, v, wq, wk, cos, sin, kc, vc, slot_mapping=slots)
    with pytest.raises(RuntimeError, match="eps must be positive"):
        qk_norm_rope_write_kv(q, k, v, wq, wk, cos, sin, kc, vc, slot_mapping=slots, eps=0.0)
    empty = qk_norm_rope_write_kv(q[:0], k[:0], v[:0], wq, wk, cos[:0], sin[:0], kc, vc,
                                  slot_mapping=slots[:0])
    assert empty.shape == (0, heads, dim)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_single_token_transposed_sources(dtype):
    """Decode batch of one whose q/k/v are transposed views ([1, H, D] with
    non-dense rows): the wrapper copies them, so the results equal those of
    the contiguous tensors."""
    heads, kv_heads, dim, block, pages = 4, 2, 64, 16, 3
    qkv, cos, sin, wq, wk, kc, vc = fused_case(dtype, 1, heads, kv_heads, dim, block, pages, seed=31)
    q, k, v = split_qkv(qkv, heads, kv_heads, dim)
    tables = torch.tensor([[2, 0]], dtype=torch.int64)
    positions = torch.tensor([19], dtype=torch.int64)
    ke, ve = kc.clone(), vc.clone()
    expected_q = paged_oracle.qk_norm_rope_write_kv(q, k, v, wq, wk, cos, sin, ke, ve, block_tables=tables,
                                                    positions=positions)

    def transposed(x):  # same values, stored [1, D, H] and viewed as [1, H, D]
        return x.to(DEV).transpose(1, 2).contiguous().transpose(1, 2)

    dq, dk, dv = transposed(q), transposed(k), transposed(v)
    assert not (dq.is_contiguous() or dk.is_contiguous() or dv.is_contiguous())
    kd, vd = kc.to(DEV), vc.to(DEV)
    got_q = qk_norm_rope_write_kv(dq, dk, dv, wq.to(DEV), wk.to(DEV), cos.to(DEV), sin.to(DEV), kd, vd,
                                  block_tables=tables.to(DEV), positions=positions.to(DEV))
    ref_q = qk_norm_rope_write_kv(q.to(DEV).contiguous(), k.to(DEV).contiguous(), v.to(DEV).contiguous(),
                                  wq.to(DEV), wk.to(DEV), cos.to(DEV), sin.to(DEV), kc.to(DEV), vc.to(DEV),
                                  block_tables=tables.to(DEV), positions=positions.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(got_q, ref_q)
    assert_rope_close(got_q, expected_q, paged_oracle.rms_norm(q, wq), dtype)
    assert torch.equal(vd.cpu(), ve)
    written = ~(ke == kc).all(-1).all(-1)
    assert torch.equal(kd.cpu()[~written], ke[~written])
