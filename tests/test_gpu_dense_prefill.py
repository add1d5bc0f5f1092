"""GPU parity of the dense causal suffix prefill (prefill_attention, backend
"hip") against the oracle's restatement of the reference's torch path
(mini_engine/kernels/prefill.py:42-60).

The reference's own GPU tests of this entry are restated first
(tests/test_prefill_linear_chat.py:9-19, tests/test_chunked_prefix.py:314-321),
then the model's call pattern (Attention.forward, native_qwen3.py:133-140:
transposed views of [tokens, heads, head_dim] tensors), batches, head dims
on both kernels, contexts past the reference kernel's 8192-token limit and a
caller-supplied output.  Gate: max abs error against the fp32 oracle 2e-3
(fp16) / 1.6e-2 (bf16).
"""

import pytest
import torch

from mini_engine_hip.kernels.prefill import prefill_attention
from oracle import paged_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
GATE = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
REFERENCE_ATOL = {torch.float16: 0.012, torch.bfloat16: 0.05}  # test_prefill_linear_chat.py:19


def check(out, q, k, v, query_start, dtype):
    want = paged_oracle.prefill_attention(q.cpu(), k.cpu(), v.cpu(), query_start=query_start, cast=False)
    err = (out.float().cpu() - want).abs().max().item()
    assert err <= GATE[dtype], err
    assert bool(torch.isfinite(out).all())


def randn(gen, *shape, dtype):
    return torch.randn(*shape, generator=gen).to(dtype).to(DEV)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_square_case(dtype):
    """test_prefill_linear_chat.py:9-19: [1, 4, 17, 16] queries, 2 kv heads."""
    gen = torch.Generator().manual_seed(71)
    q, k, v = randn(gen, 1, 4, 17, 16, dtype=dtype), randn(gen, 1, 2, 17, 16, dtype=dtype), \
        randn(gen, 1, 2, 17, 16, dtype=dtype)
    print(f"dense prefill square 17 {dtype}", flush=True)
    out = prefill_attention(q, k, v, "hip")
    torch.cuda.synchronize()
    check(out, q, k, v, 0, dtype)
    math_ref = paged_oracle.prefill_attention(q.cpu(), k.cpu(), v.cpu())
    torch.testing.assert_close(out.cpu(), math_ref, atol=REFERENCE_ATOL[dtype], rtol=0.03)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_suffix_case(dtype):
    """test_chunked_prefix.py:314-321: 3 queries after 8 keys of 11."""
    gen = torch.Generator().manual_seed(233)
    q, k, v = randn(gen, 1, 4, 3, 16, dtype=dtype), randn(gen, 1, 2, 11, 16, dtype=dtype), \
        randn(gen, 1, 2, 11, 16, dtype=dtype)
    print(f"dense prefill suffix 3 after 8 {dtype}", flush=True)
    out = prefill_attention(q, k, v, "hip", query_start=8)
    torch.cuda.synchronize()
    check(out, q, k, v, 8, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("query_start,tokens", [(0, 1000), (1700, 300), (5, 1)])
def test_model_call_pattern_reads_views(dtype, query_start, tokens):
    """Attention.forward's call (native_qwen3.py:137-140): q, k, v are
    [tokens, heads, head_dim] tensors passed as transpose(0, 1).unsqueeze(0)
    views; the result transposed back is contiguous (written token-major)."""
    gen = torch.Generator().manual_seed(tokens)
    context = query_start + tokens
    q_rows = randn(gen, tokens, 16, 128, dtype=dtype)
    k_rows, v_rows = randn(gen, context, 8, 128, dtype=dtype), randn(gen, context, 8, 128, dtype=dtype)
    q, k, v = (t.transpose(0, 1).unsqueeze(0) for t in (q_rows, k_rows, v_rows))
    assert tokens == 1 or not q.is_contiguous()
    print(f"dense prefill views start={query_start} tokens={tokens} {dtype}", flush=True)
    out = prefill_attention(q, k, v, "hip", query_start=query_start)
    torch.cuda.synchronize()
    assert out.shape == (1, 16, tokens, 128)
    assert out.squeeze(0).transpose(0, 1).is_contiguous()
    check(out, q, k, v, query_start, dtype)


@pytest.mark.parametrize("head_dim,q_heads,kv_heads", [(128, 16, 8), (64, 8, 8), (80, 12, 4), (96, 8, 2),
                                                       (256, 8, 4), (192, 4, 2), (16, 32, 4), (20, 4, 2),
                                                       (264, 4, 4)])
def test_batched_head_dims_both_kernels(head_dim, q_heads, kv_heads):
    """Contiguous [B, H, T, D] batches with keys past the last query's
    position; multiples of 8 up to 256 on MFMA tiles (zero-padded below the
    tile's width), 20 and 264 on the element-wise kernel."""
    dtype = torch.bfloat16
    gen = torch.Generator().manual_seed(head_dim)
    q = randn(gen, 3, q_heads, 129, head_dim, dtype=dtype)
    k, v = randn(gen, 3, kv_heads, 200, head_dim, dtype=dtype), randn(gen, 3, kv_heads, 200, head_dim, dtype=dtype)
    print(f"dense prefill batch D={head_dim} {q_heads}/{kv_heads}", flush=True)
    out = prefill_attention(q, k, v, "hip", query_start=37)
    torch.cuda.synchronize()
    check(out, q, k, v, 37, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_context_beyond_reference_limit_splits_keys(dtype):
    """64 queries after 9000 keys (the reference kernel stops at 8192): few
    query blocks, so the keys are split into chunks and merged."""
    gen = torch.Generator().manual_seed(9)
    q = randn(gen, 1, 16, 64, 128, dtype=dtype)
    k, v = randn(gen, 1, 8, 9064, 128, dtype=dtype), randn(gen, 1, 8, 9064, 128, dtype=dtype)
    print(f"dense prefill 64 after 9000 {dtype}", flush=True)
    out = prefill_attention(q, k, v, "hip", query_start=9000)
    torch.cuda.synchronize()
    check(out, q, k, v, 9000, dtype)


def test_caller_output_and_workspace_match_the_default():
    """A caller's contiguous output (and a reused workspace) get the same bits
    as the default token-major output."""
    dtype = torch.bfloat16
    gen = torch.Generator().manual_seed(4)
    q = randn(gen, 2, 16, 96, 128, dtype=dtype)
    k, v = randn(gen, 2, 8, 3000, 128, dtype=dtype), randn(gen, 2, 8, 3000, 128, dtype=dtype)
    print("dense prefill out= and workspace", flush=True)
    want = prefill_attention(q, k, v, "hip", query_start=2900)
    out = torch.empty_like(q)
    workspace = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)
    got = prefill_attention(q, k, v, "hip", query_start=2900, out=out, workspace=workspace)
    torch.cuda.synchronize()
    assert got is out and out.is_contiguous()
    assert torch.equal(out, want)
    check(out, q, k, v, 2900, dtype)


def test_sliced_views_differing_kv_strides_and_graph_replay():
    """Queries sliced out of a longer token range (a batch stride that is not
    a multiple of the tensor's own size), K and V with different layouts
    (the wrapper then copies both), and the call captured in a HIP graph and
    replayed with new query values."""
    dtype = torch.float16
    gen = torch.Generator().manual_seed(12)
    big_q = randn(gen, 2, 8, 300, 64, dtype=dtype)
    q = big_q[:, :, 40:140]                                   # [2, 8, 100, 64], token window of a longer range
    k = randn(gen, 2, 4, 400, 64, dtype=dtype)
    v = randn(gen, 2, 400, 4, 64, dtype=dtype).transpose(1, 2)  # same shape as k, other strides
    assert k.stride() != v.stride()
    print("dense prefill sliced views / differing strides", flush=True)
    out = prefill_attention(q, k, v, "hip", query_start=250)
    torch.cuda.synchronize()
    check(out, q, k, v, 250, dtype)
    static_out = torch.empty_like(q)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        prefill_attention(q, k, v, "hip", query_start=250, out=static_out)
    for step in range(3):
        big_q.copy_(randn(gen, 2, 8, 300, 64, dtype=dtype))
        graph.replay()
        torch.cuda.synchronize()
        eager = prefill_attention(q, k, v, "hip", query_start=250)
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), step
        check(static_out, q, k, v, 250, dtype)


def test_misaligned_contiguous_inputs_are_copied():
    """Contiguous q/k/v that start one element into their storage (so their
    rows are not 16-byte aligned) are served through aligned copies instead of
    being refused by the MFMA path."""
    gen = torch.Generator().manual_seed(919)
    dtype = torch.bfloat16

    def shifted(*shape):
        flat = randn(gen, 1 + torch.Size(shape).numel(), dtype=dtype)
        return flat[1:].view(*shape)

    q, k, v = shifted(1, 16, 40, 128), shifted(1, 8, 72, 128), shifted(1, 8, 72, 128)
    assert q.is_contiguous() and q.data_ptr() % 16 != 0
    print("dense prefill misaligned contiguous inputs", flush=True)
    out = prefill_attention(q, k, v, "hip", query_start=32)
    torch.cuda.synchronize()
    check(out, q, k, v, 32, dtype)
