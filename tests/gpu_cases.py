"""Seeded input builders shared by the GPU parity tests (CPU tensors).

Shapes follow the reference's own test inputs and the benchmark configs:
tests/test_cuda_paged_attention.py:17-26 (decode), test_ragged_kernels.py:17-24
(packed prefill), plus the five benchmark workloads at reduced or full size.
"""

from __future__ import annotations

import torch


def decode_inputs(dtype, *, head_dim=128, block_size=16, lengths=(17, 257, 521), heads=16, kv_heads=8,
                  seed=23, extra_pages=3):
    """Random non-contiguous pages; one table row per sequence."""
    gen = torch.Generator().manual_seed(seed)
    width = (max(lengths) + block_size - 1) // block_size
    blocks = len(lengths) * width + extra_pages
    key = torch.randn(blocks, block_size, kv_heads, head_dim, generator=gen).to(dtype)
    value = torch.randn(blocks, block_size, kv_heads, head_dim, generator=gen).to(dtype)
    table = torch.randperm(blocks, generator=gen)[:len(lengths) * width].view(len(lengths), width)
    lens = torch.tensor(lengths, dtype=torch.int64)
    query = torch.randn(len(lengths), heads, head_dim, generator=gen).to(dtype)
    return query, key, value, table, lens, block_size


def prefill_inputs(dtype, *, head_dim=16, seed=631):
    """The reference's packed-prefill case (test_ragged_kernels.py:17-24)."""
    gen = torch.Generator().manual_seed(seed)
    key = torch.randn(8, 4, 2, head_dim, generator=gen).to(dtype)
    value = torch.randn(8, 4, 2, head_dim, generator=gen).to(dtype)
    q = torch.randn(8, 4, head_dim, generator=gen).to(dtype)
    meta = [torch.tensor(x, dtype=torch.int64) for x in ([0, 3, 8], [5, 1], [[5, 1, -1], [2, 7, -1]], [8, 6])]
    return (q, key, value, *meta)


ROPE_ATOL = {torch.float16: 0.001, torch.bfloat16: 0.004}
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def assert_rope_close(actual, expected, normed, dtype):
    """Reference tolerance, or two ulps of the rotated pair, per element; >= 99% bit-exact."""
    actual, expected, normed = actual.cpu().float(), expected.float(), normed.float()
    half = normed.shape[-1] // 2
    pair = normed[..., :half].abs() + normed[..., half:].abs()
    bound = 2 * ULP[dtype] * torch.cat((pair, pair), -1) + 1e-6
    diff = (actual - expected).abs()
    reference_ok = diff <= ROPE_ATOL[dtype] + 0.01 * expected.abs()
    assert bool((reference_ok | (diff <= bound)).all()), f"max diff {diff.max().item()}"
    exact = (actual == expected).float().mean().item()
    assert exact >= 0.99, f"only {exact:.4f} of the elements are bit-identical"
