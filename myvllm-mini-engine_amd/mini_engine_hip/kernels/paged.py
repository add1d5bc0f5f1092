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

    ``partition_tokens`` (0 = library plan) sets the split-K partition, or
    with -1 forces the balanced walk (equal shares of tokens per work-group;
    batches above 256 take the plan);
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


FUSED_WRITE_HEAD_DIMS = (16, 32, 64, 128, 256)


def paged_attention_decode_write(query, key_cache, value_cache, block_tables, context_lens, block_size,
                                 new_key, new_value, *, q_weight=None, k_weight=None, cos=None, sin=None,
                                 eps=1e-6, q_out=None, backend="hip", validate=True, partition_tokens=0,
                                 out=None, workspace=None):
    """The decode step's KV write and paged attention in one launch.

    Writes each sequence's new token, at position ``context_lens[b] - 1``,
    into the paged cache, then attends over ``context_lens[b]`` tokens --
    what Attention.forward_decode_batch (mini_engine/model/native_qwen3.py:
    179-197) runs as separate launches:

    * without norm weights: ``write_kv_cache_batch(kc, vc, tables,
      context_lens - 1, new_key, new_value)`` then ``paged_attention(query,
      ...)``;
    * with ``q_weight``/``k_weight``/``cos``/``sin``: ``query`` holds the raw
      query rows; ``qk_norm_rope_write_kv(query, new_key, new_value, ...,
      block_tables=tables, positions=context_lens - 1, out=q_out)`` then
      ``paged_attention(q_out, ...)``.

    Outputs and cache rows equal those sequences bit for bit.  head_dim 16,
    32, 64, 128 and 256 with 16-byte aligned rows run one kernel; other
    shapes run the two launches above.  Returns the attention output
    ``[B, Hq, D]``.
    """
    from .data import _row_stride, write_kv_cache_batch
    from .rope import qk_norm_rope_write_kv

    if backend != "hip":
        raise ValueError("decode backend must be hip")
    if query.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("HIP paged attention supports FP16/BF16")
    rope = q_weight is not None
    if rope and (k_weight is None or cos is None or sin is None):
        raise ValueError("norm/RoPE needs q_weight, k_weight, cos and sin")
    if query.dim() != 3 or new_key.dim() != 3 or new_value.shape != new_key.shape:
        raise ValueError("query must be [batch, q_heads, head_dim] and new key/value [batch, kv_heads, head_dim]")
    batch, q_heads, head_dim = query.shape
    if new_key.shape[0] != batch or new_key.shape[1:] != key_cache.shape[2:]:
        raise ValueError("packed key/value must be [tokens, kv_heads, head_dim] matching the cache")
    for t in (new_key, new_value):
        _check(t.dtype == query.dtype and t.device == query.device, "new key/value must match the query")
    _check(query.is_cuda, "query must be CUDA")
    if out is None:
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    else:
        _check(out.shape == query.shape and out.dtype == query.dtype and out.is_contiguous()
               and out.device == query.device, "output buffer must match the query")
    # The attention-side checks of paged_attention; in norm/RoPE mode the raw
    # query may be a strided slice (a fused QKV projection), so the
    # contiguous output stands in for its shape.
    _native_checks(out if rope else query, key_cache, value_cache, block_tables, context_lens, block_size,
                   validate)
    if rope:
        _check(q_out is None or (q_out.shape == query.shape and q_out.dtype == query.dtype
                                 and q_out.is_contiguous() and q_out.device == query.device),
               "q_out must be a contiguous tensor shaped like the query")
    if validate:
        _check(not any(torch._C._overlaps(cache, src) for cache in (key_cache, value_cache)
                       for src in (query, new_key, new_value)),
               "KV destinations and source tensors must not overlap")
    # One launch reads the raw query rows in every work-group while the first
    # writes q_out, so an overlapping q_out takes the two launches; only an
    # exact in-place rotation (q_out is the contiguous query) is defined there.
    in_place = rope and q_out is not None and torch._C._overlaps(q_out, query)
    if in_place and not (q_out.data_ptr() == query.data_ptr() and query.is_contiguous()):
        raise ValueError("q_out must be the query itself or not overlap it")
    num_blocks, _, kv_heads, _ = key_cache.shape
    width = block_tables.shape[1]
    q_stride, q_src = _row_stride(query) if rope else (q_heads * head_dim, query)
    k_stride, k_src = _row_stride(new_key)
    v_stride, v_src = _row_stride(new_value)
    pointers = [q_src, key_cache, value_cache, k_src, v_src]
    if rope:
        for weight in (q_weight, k_weight):
            _check(weight.dtype == query.dtype and weight.dim() == 1 and weight.numel() == head_dim
                   and weight.is_contiguous() and weight.device == query.device,
                   "RMSNorm weight shape/dtype mismatch")
        _check(cos.dim() == 2 and sin.shape == cos.shape and cos.shape[0] == batch and cos.shape[1] * 2 == head_dim
               and cos.is_contiguous() and sin.is_contiguous() and cos.dtype == query.dtype
               and sin.dtype == query.dtype and cos.device == query.device and sin.device == query.device,
               "RoPE cos/sin shape mismatch")
        pointers += [q_weight, k_weight, cos, sin] + ([q_out] if q_out is not None else [])
    fused = (not in_place and head_dim in FUSED_WRITE_HEAD_DIMS
             and all(t.data_ptr() % 16 == 0 for t in pointers)
             and q_stride % 8 == 0 and k_stride % 8 == 0 and v_stride % 8 == 0)
    if not fused:
        positions = context_lens - 1
        if rope:
            q_rot = qk_norm_rope_write_kv(query, new_key, new_value, q_weight, k_weight, cos, sin, key_cache,
                                          value_cache, block_tables=block_tables, positions=positions, eps=eps,
                                          validate=False, out=q_out)
        else:
            write_kv_cache_batch(key_cache, value_cache, block_tables, positions, new_key.contiguous(),
                                 new_value.contiguous(), block_size, validate=False)
            q_rot = query
        return paged_attention(q_rot, key_cache, value_cache, block_tables, context_lens, block_size,
                               validate=False, partition_tokens=partition_tokens, out=out, workspace=workspace)
    lib = ext.load_hip_extension()
    need = lib.workspace_size(batch, q_heads, kv_heads, head_dim, block_size, width, partition_tokens)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=query.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else 0
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    ptr = (lambda t: t.data_ptr() if t is not None else None)
    with torch.cuda.device(query.device):
        lib.call("mvme_paged_attention_decode_write", out.data_ptr(), q_src.data_ptr(), key_cache.data_ptr(),
                 value_cache.data_ptr(), block_tables.data_ptr(), context_lens.data_ptr(), batch, q_heads,
                 kv_heads, head_dim, num_blocks, block_size, width, partition_tokens,
                 ext.dtype_code(query.dtype), k_src.data_ptr(), v_src.data_ptr(), k_stride, v_stride,
                 ptr(q_weight), ptr(k_weight), ptr(cos), ptr(sin), float(eps), q_stride, ptr(q_out),
                 ws_ptr, ws_bytes, ext.current_stream(query.device))
    return out
