"""Paged GQA decode attention, ``backend="hip"``.

Same call signature, argument meaning and error behaviour as the reference's
dispatcher ``paged_attention`` (mini_engine/kernels/paged.py:8-22) with its
native checks (mini_engine/kernels/csrc/bindings.cpp:152-184): dtype errors
are ``ValueError`` before dispatch, shape/metadata errors are ``RuntimeError``
with the native messages.  ``validate=False`` skips the host-synchronising
metadata checks so the call can be captured in a HIP graph; the kernels still
treat out-of-range pages and lengths as absent.

The output tensor is new (``torch.empty_like``); the split-K workspace comes
from torch's caching allocator, so nothing here allocates device memory
outside torch or synchronises when ``validate=False``.
"""

from __future__ import annotations

import torch

from . import hip_extension as ext

SUPPORTED_HEAD_DIMS = (16, 32, 64, 80, 96, 128, 192, 256)
MAX_TABLE_CAPACITY = 1048576


def _check(condition, message):
    if not condition:
        raise RuntimeError(message)


def _native_checks(query, key, value, tables, lengths, block_size, validate):
    """Restates the argument checks of bindings.cpp:152-184."""
    _check(query.is_cuda, "query must be CUDA")
    for t in (key, value, tables, lengths):
        _check(t.device == query.device, "all inputs must be on the same CUDA device")
        _check(t.is_contiguous(), "inputs must be contiguous")
    _check(query.is_contiguous(), "query must be contiguous")
    _check(query.dim() == 3 and key.dim() == 4 and value.shape == key.shape, "invalid query/cache shapes")
    _check(query.dtype in (torch.float16, torch.bfloat16), "FP16/BF16 required")
    _check(key.dtype == query.dtype and value.dtype == query.dtype, "cache dtype mismatch")
    _check(tables.dtype == torch.int64 and lengths.dtype == torch.int64, "metadata must be int64")
    _check(query.shape[0] > 0 and query.shape[1] > 0 and key.shape[0] > 0 and key.shape[2] > 0,
           "empty batch/heads/cache")
    _check(block_size > 0 and key.shape[1] == block_size, "block size mismatch")
    _check(query.shape[2] == key.shape[3] and query.shape[1] % key.shape[2] == 0,
           "head dimension or GQA mismatch")
    _check(query.shape[2] in SUPPORTED_HEAD_DIMS, "supported head_dim: 16,32,64,80,96,128,192,256")
    _check(tables.dim() == 2 and tables.shape[0] == query.shape[0] and tables.shape[1] > 0,
           "invalid block table")
    _check(lengths.dim() == 1 and lengths.shape[0] == query.shape[0], "invalid context lengths")
    _check(tables.shape[1] * block_size <= MAX_TABLE_CAPACITY, "maximum table capacity is 1M tokens")
    _check(query.shape[0] * query.shape[1] <= 2147483647, "batch/head product too large")
    if validate:
        # Host-synchronising metadata checks; the trusted path skips them.
        capacity = tables.shape[1] * block_size
        _check(not bool(((lengths <= 0) | (lengths > capacity)).any()), "invalid context length")
        positions = torch.arange(tables.shape[1], device=lengths.device, dtype=lengths.dtype) * block_size
        active = positions.unsqueeze(0) < lengths.unsqueeze(1)
        bad = ((tables < 0) | (tables >= key.shape[0])) & active
        _check(not bool(bad.any()), "physical block id out of range")


def workspace_bytes(batch, q_heads, kv_heads, head_dim, block_size, table_width, partition_tokens=0):
    """Split-K workspace the decode kernels need for these shapes."""
    return ext.load_hip_extension().workspace_size(batch, q_heads, kv_heads, head_dim, block_size,
                                                   table_width, partition_tokens)


def paged_attention(query, key_cache, value_cache, block_tables, context_lens, block_size,
                    *, backend="hip", validate=True, partition_tokens=0, out=None, workspace=None):
    """Decode attention over a paged KV cache.

    query [B, Hq, D]; key_cache/value_cache [num_blocks, block_size, Hkv, D];
    block_tables [B, W] int64 (-1 padding past the active pages);
    context_lens [B] int64.  Returns [B, Hq, D] in the query dtype.

    ``partition_tokens`` (0 = library default) sets the split-K partition;
    ``out`` / ``workspace`` let a caller supply preallocated buffers.
    """
    if backend != "hip":
        raise ValueError("decode backend must be hip")
    if query.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("HIP paged attention supports FP16/BF16")
    _native_checks(query, key_cache, value_cache, block_tables, context_lens, block_size, validate)
    lib = ext.load_hip_extension()
    batch, q_heads, head_dim = query.shape
    num_blocks, _, kv_heads, _ = key_cache.shape
    width = block_tables.shape[1]
    if out is None:
        out = torch.empty_like(query)
    else:
        _check(out.shape == query.shape and out.dtype == query.dtype and out.is_contiguous()
               and out.device == query.device, "output buffer must match the query")
    need = lib.workspace_size(batch, q_heads, kv_heads, head_dim, block_size, width, partition_tokens)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=query.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else 0
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    with torch.cuda.device(query.device):
        lib.call("mvme_paged_attention", out.data_ptr(), query.data_ptr(), key_cache.data_ptr(),
                 value_cache.data_ptr(), block_tables.data_ptr(), context_lens.data_ptr(),
                 batch, q_heads, kv_heads, head_dim, num_blocks, block_size, width,
                 partition_tokens, ext.dtype_code(query.dtype), ws_ptr, ws_bytes,
                 ext.current_stream(query.device))
    return out
