"""The allocation-free decode entry point against the workspace one.

mvme_paged_attention_noalloc runs the same kernels as mvme_paged_attention
with the split-K partials in the library's fixed per-device scratch array.
Called through the C ABI, two calls in a row (the second smaller, so it reuses
scratch that still holds the first call's partials) must give outputs
bit-identical to the workspace entry point's on the same inputs, and within
the oracle's gate.
"""

import pytest
import torch

from gpu_cases import decode_inputs
from mini_engine_hip.kernels import hip_extension as ext
from mini_engine_hip.kernels.paged import paged_attention
from oracle import paged_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
GATE = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def noalloc(q, k, v, tables, lens, block_size, partition=0):
    lib = ext.load_hip_extension()
    out = torch.full_like(q, float("nan"))
    batch, q_heads, head_dim = q.shape
    num_blocks, _, kv_heads, _ = k.shape
    with torch.cuda.device(q.device):
        lib.call("mvme_paged_attention_noalloc", out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                 tables.data_ptr(), lens.data_ptr(), batch, q_heads, kv_heads, head_dim, num_blocks, block_size,
                 tables.shape[1], partition, ext.dtype_code(q.dtype), ext.current_stream(q.device))
    return out


def check(args, partition=0):
    dev = [a.to(DEV) if isinstance(a, torch.Tensor) else a for a in args]
    q, k, v, t, l, bs = dev
    batch, q_heads, head_dim = q.shape
    need = ext.load_hip_extension().workspace_size(batch, q_heads, k.shape[2], head_dim, bs, t.shape[1], partition)
    got = noalloc(*dev, partition)
    want = paged_attention(*dev, backend="hip", partition_tokens=partition)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    expected = paged_oracle.fp32_oracle(dict(zip(paged_oracle.TENSOR_NAMES, args[:5])), bs)
    assert (got.float().cpu() - expected).abs().max().item() <= GATE[q.dtype]
    return need


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_noalloc_matches_workspace_entry_on_two_calls(dtype):
    print(f"no-alloc decode {dtype}: large split-K call, then a smaller one", flush=True)
    big = decode_inputs(dtype, lengths=(3000, 1800, 2999), block_size=16, seed=71)
    small = decode_inputs(dtype, lengths=(700,), block_size=32, seed=72)
    need_big = check(big)
    need_small = check(small)
    assert 0 < need_small < need_big <= 8 << 20
    # Explicit small partitions: more partials than the plan's, still within the scratch.
    assert check(big, partition=64) > need_big


def test_noalloc_whole_sequence_and_rejection():
    """Enough units for whole-sequence work-groups: no scratch used; a plan
    above 8 MiB of scratch is refused with nothing launched."""
    args = decode_inputs(torch.float16, lengths=tuple(range(100, 100 + 40 * 7, 7)), block_size=16, seed=73)
    assert check(args) == 0
    q, k, v, t, l, bs = [a.to(DEV) if isinstance(a, torch.Tensor) else a for a in args]
    out = torch.zeros_like(q)
    lib = ext.load_hip_extension()
    with pytest.raises(RuntimeError, match="no-alloc"):
        lib.call("mvme_paged_attention_noalloc", out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                 t.data_ptr(), l.data_ptr(), q.shape[0], q.shape[1], k.shape[2], q.shape[2], k.shape[0], bs,
                 4096, 16, ext.FP16, ext.current_stream(q.device))
    torch.cuda.synchronize()
    assert not out.any()


def test_noalloc_balanced_walk_two_calls():
    """The balanced walk in the scratch (partial rows and the per-share merge
    descriptors): the plan's pick for long units, then a smaller forced walk
    that rewrites every descriptor."""
    print("no-alloc decode: balanced walk, long units then a forced small call", flush=True)
    long_units = decode_inputs(torch.bfloat16, lengths=(5000, 17, 4100), block_size=16, seed=74)
    small = decode_inputs(torch.bfloat16, lengths=(700,), block_size=32, seed=72)
    assert check(long_units) > 0
    assert check(small, partition=-1) > 0
