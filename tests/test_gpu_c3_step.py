"""The headline decode step as specified: 28 layers back to back, each with
its own 263-page KV pool, queries and random non-contiguous block table
(batch 32, every context 2048, Hq16/Hkv8/D128, fp16, block 256), captured in
ONE graph of 28 paged_attention calls and replayed.

Layers 0, 9, 18 and 27 are checked against the fp32 oracle
(benchmarks/compare_paged_backends.py:58-72 restated in the oracle) with the
fp16 gate 2e-3 after every replay, and every replay's outputs must equal
the eager call's bit for bit.  The pools are separate allocations, so no
layer reads another layer's pages.
"""

import pytest
import torch

from mini_engine_hip import workloads
from mini_engine_hip.kernels.paged import paged_attention
from oracle import paged_oracle

pytestmark = pytest.mark.gpu
LAYERS, BLOCK, GATE = 28, 256, 2e-3
CHECKED = (0, 9, 18, 27)
BASE_SEED = 20261026


def test_captured_28_layer_step_matches_the_oracle():
    dev = torch.device("cuda:0")
    layers = [workloads.decode_b32_layer(dev, seed=BASE_SEED + 2 + 1000 * layer) for layer in range(LAYERS)]
    assert len({c["key_cache"].data_ptr() for c in layers}) == LAYERS
    assert all(c["key_cache"].shape == (263, BLOCK, 8, 128) for c in layers)
    for c in layers:
        c["out"] = torch.empty_like(c["query"])

    def step():
        for c in layers:
            paged_attention(c["query"], c["key_cache"], c["value_cache"], c["block_tables"], c["context_lens"],
                            BLOCK, backend="hip", validate=False, out=c["out"])

    print("c3 step: eager 28 layers", flush=True)
    step()
    torch.cuda.synchronize()
    eager = [c["out"].clone() for c in layers]
    wants = {}
    for idx in CHECKED:
        c = layers[idx]
        tensors = {name: c[name].cpu() for name in paged_oracle.TENSOR_NAMES}
        wants[idx] = paged_oracle.fp32_oracle(tensors, BLOCK)
        err = (eager[idx].float().cpu() - wants[idx]).abs().max().item()
        assert err <= GATE, (idx, err)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for replay in range(3):
        for c in layers:
            c["out"].zero_()
        torch.cuda.synchronize()
        print(f"c3 step: graph replay {replay}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        for idx, c in enumerate(layers):
            assert torch.equal(c["out"], eager[idx]), (replay, idx)
        for idx in CHECKED:
            err = (layers[idx]["out"].float().cpu() - wants[idx]).abs().max().item()
            assert err <= GATE, (replay, idx, err)
