"""GPU parity of greedy sampling (argmax) against the oracle, bit-exact indices.

Restates the reference's tests for backend="hip" (tests/test_cuda_sampling.py:
ties, NaN, +-inf and the tail of the row at vocab 1 / 257 / 4097 / 151936, graph
capture with replays on changed logits, and validation).
"""

import pytest
import torch

from mini_engine_hip.sampling import greedy_argmax, sample_next_token
from oracle import paged_oracle

pytestmark = pytest.mark.gpu


def special_rows(dtype, vocab, rows=6, seed=29):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, vocab, generator=gen).to(dtype)
    x[0].fill_(float("-inf"))
    x[1].fill_(1)
    x[2, -1] = float("inf")
    x[3, -1] = float("nan")
    x[3, 0] = float("nan")
    x[4, -1] = 99
    x[5].fill_(0)
    x[5, vocab // 2:] = -0.0
    return x


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("vocab", [1, 257, 4097, 151936, 151939])
def test_greedy_ties_nan_and_tail(dtype, vocab):
    x = special_rows(dtype, vocab)
    print(f"greedy argmax {dtype} vocab={vocab}", flush=True)
    got = sample_next_token(x.cuda(), backend="hip")
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), paged_oracle.greedy_argmax(x))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_greedy_random_batches_and_nondefault_stream(dtype):
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(64, 151936, generator=gen).to(dtype)
    stream = torch.cuda.Stream()
    xd = x.cuda()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        got = greedy_argmax(xd)
    stream.synchronize()
    assert torch.equal(got.cpu(), paged_oracle.greedy_argmax(x))


def test_greedy_graph_replay_and_validation():
    x = torch.randn(3, 8193, device="cuda", dtype=torch.float16)
    sample_next_token(x, backend="hip")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = sample_next_token(x, backend="hip")
    for index in [0, 8192, 4096]:
        x.fill_(0)
        x[:, index] = 2
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), paged_oracle.greedy_argmax(x.cpu()))
    with pytest.raises(ValueError, match="greedy"):
        sample_next_token(x, temperature=1, backend="hip")
    with pytest.raises(RuntimeError, match="contiguous CUDA"):
        sample_next_token(x.cpu(), backend="hip")
    with pytest.raises(RuntimeError, match="contiguous CUDA"):
        sample_next_token(x[:, ::2], backend="hip")
    with pytest.raises(RuntimeError, match="FP32/FP16/BF16"):
        sample_next_token(x.to(torch.float64), backend="hip")
    assert sample_next_token(x[:0], backend="hip").numel() == 0
