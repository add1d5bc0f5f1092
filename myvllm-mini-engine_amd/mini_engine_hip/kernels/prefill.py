"""Prefill attention, ``backend="hip"``: ragged chunked paged prefill and
dense causal suffix prefill.

``paged_prefill_attention`` has the same signature, metadata contract and
validation messages as the reference's (mini_engine/kernels/prefill.py:61-131)
and its native op (mini_engine/kernels/csrc/prefill.cu:200-240): packed
queries read the paged KV cache directly.  ``prefill_attention`` is the
reference's dense entry (mini_engine/kernels/prefill.py:8-41, native op
prefill.cu:15-98) for [batch, heads, tokens, head_dim] tensors.  Head dims
that are multiples of 8 up to 256 run on bf16/fp16 MFMA tiles, other head
sizes (up to 1024) on a generic HIP kernel.
"""

from __future__ import annotations

import torch

from . import hip_extension as ext

MAX_HEAD_DIM = 1024


def paged_prefill_workspace_bytes(num_seqs, total_tokens, q_heads, kv_heads, head_dim, block_size, table_width,
                                  dtype, chunk_tokens=0):
    """Bytes of the key-chunk workspace paged_prefill_attention needs for
    these shapes (from shapes only: lengths stay on the device).  A layer
    loop sizes one buffer for its largest call and passes it to every call
    as ``workspace=``; 0 means the call never splits keys."""
    return ext.load_hip_extension().prefill_workspace_size(num_seqs, total_tokens, q_heads, kv_heads, head_dim,
                                                           block_size, table_width, chunk_tokens,
                                                           ext.dtype_code(dtype))


def paged_prefill_attention(q, key_cache, value_cache, cu_seqlens_q, query_starts,
                            block_tables, context_lens, block_size, *, backend="hip", validate=True,
                            chunk_tokens=0, workspace=None):
    """Packed causal queries read paged KV directly.

    Q is [total_queries, query_heads, head_dim].  Each request describes a
    suffix starting at its absolute query_start; context_len equals
    start + query_count.  Validation of metadata values synchronizes the
    device; trusted model batches can skip it.

    ``chunk_tokens`` (0 = library default) sets the key-chunk length used to
    split long contexts; ``workspace`` may supply the partial-result buffer.
    """
    if backend != "hip":
        raise ValueError("paged prefill backend must be hip")
    if (type(block_size) is not int or block_size <= 0 or key_cache.ndim != 4
            or value_cache.shape != key_cache.shape or key_cache.shape[1] != block_size
            or any(size <= 0 for size in key_cache.shape)
            or not key_cache.is_contiguous() or not value_cache.is_contiguous()):
        raise ValueError("paged prefill caches must be contiguous [pages, block_size, kv_heads, head_dim]")
    if (q.ndim != 3 or q.shape[1] <= 0 or q.shape[2] != key_cache.shape[3]
            or q.shape[1] % key_cache.shape[2]):
        raise ValueError("paged prefill Q must be [tokens, heads, head_dim] with divisible GQA heads")
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("paged prefill requires FP32/FP16/BF16")
    if key_cache.dtype != q.dtype or value_cache.dtype != q.dtype:
        raise ValueError("paged prefill Q/K/V must share dtype")
    metadata = (cu_seqlens_q, query_starts, block_tables, context_lens)
    if (cu_seqlens_q.ndim != 1 or query_starts.ndim != 1 or context_lens.ndim != 1
            or block_tables.ndim != 2 or query_starts.numel() != block_tables.shape[0]
            or context_lens.numel() != block_tables.shape[0]
            or cu_seqlens_q.numel() != block_tables.shape[0] + 1):
        raise ValueError("paged prefill metadata shapes do not match request count")
    if any(t.dtype != torch.int64 or not t.is_contiguous() for t in metadata):
        raise ValueError("paged prefill metadata must be contiguous int64 tensors")
    if any(t.device != q.device for t in (key_cache, value_cache, *metadata)):
        raise ValueError("paged prefill tensors must share device")
    if validate:
        offsets, starts, tables, lengths = (t.tolist() for t in metadata)
        if offsets[0] != 0 or offsets[-1] != q.shape[0] or any(b < a for a, b in zip(offsets, offsets[1:])):
            raise ValueError("query offsets must be monotone and cover all packed queries")
        for index, (start, length, table) in enumerate(zip(starts, lengths, tables)):
            count = offsets[index + 1] - offsets[index]
            if start < 0 or length != start + count or length > len(table) * block_size:
                raise ValueError("query start/context length exceeds block table capacity or query range")
            used = (length + block_size - 1) // block_size
            if any(page < 0 or page >= key_cache.shape[0] for page in table[:used]):
                raise ValueError("active block table contains an invalid physical page")
    if q.device.type != "cuda" or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("HIP paged prefill requires HIP FP16/BF16")
    if q.shape[2] > MAX_HEAD_DIM:
        raise ValueError("HIP paged prefill supports head_dim up to 1024")
    q = q.contiguous()
    output = torch.empty_like(q)
    if q.shape[0] == 0:
        return output
    lib = ext.load_hip_extension()
    num_blocks, _, kv_heads, head_dim = key_cache.shape
    num_seqs, width = query_starts.numel(), block_tables.shape[1]
    need = lib.prefill_workspace_size(num_seqs, q.shape[0], q.shape[1], kv_heads, head_dim, block_size, width,
                                      chunk_tokens, ext.dtype_code(q.dtype))
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else 0
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    with torch.cuda.device(q.device):
        lib.call("mvme_paged_prefill_attention", output.data_ptr(), q.data_ptr(), key_cache.data_ptr(),
                 value_cache.data_ptr(), cu_seqlens_q.data_ptr(), query_starts.data_ptr(),
                 block_tables.data_ptr(), context_lens.data_ptr(), num_seqs, q.shape[0],
                 q.shape[1], kv_heads, head_dim, num_blocks, block_size, width, chunk_tokens,
                 ext.dtype_code(q.dtype), ws_ptr, ws_bytes, ext.current_stream(q.device))
    return output


MAX_DENSE_CONTEXT = 1048576


def _mfma_head_dim(head_dim):
    return head_dim % 8 == 0 and head_dim <= 256


def _dense_strides(tensor):
    """(batch, head, token) strides in elements as the kernels read them:
    dimensions of size 1 never move, so their stride is passed as 0."""
    return tuple(st if size > 1 else 0 for size, st in zip(tensor.shape[:3], tensor.stride()[:3]))


def _dense_layout_ok(tensor, head_dim):
    """Innermost dim dense and, on the MFMA path, 16-byte rows: 16-byte
    aligned base and strides in multiples of 8 elements."""
    if head_dim > 1 and tensor.stride(3) != 1:
        return False
    if not _mfma_head_dim(head_dim):
        return True
    return tensor.data_ptr() % 16 == 0 and all(st % 8 == 0 for st in _dense_strides(tensor))


def _aligned_copy(tensor):
    """A new contiguous copy (the caching allocator's blocks are 16-byte
    aligned, so its rows meet the MFMA path's alignment)."""
    return torch.empty_like(tensor, memory_format=torch.contiguous_format).copy_(tensor)


def _dense_disjoint(tensor):
    """No two elements of a [batch, heads, tokens, head_dim] tensor share an
    address: taken by increasing stride, every dimension of more than one
    element steps past all the offsets the smaller ones reach (the kernels'
    rule for an output; expanded views break it)."""
    if tensor.shape[3] > 1 and tensor.stride(3) != 1:
        return False
    reach = tensor.shape[3]
    for size, stride in sorted(zip(tensor.shape[:3], tensor.stride()[:3]), key=lambda d: d[1]):
        if size <= 1:
            continue
        if stride < reach:
            return False
        reach += stride * (size - 1)
    return True


def prefill_attention(q, k, v, backend="hip", *, query_start=0, out=None, workspace=None):
    """Causal prefill attention over [batch, heads, tokens, head_dim] tensors.

    Query row t of q attends keys [0, query_start + t] of k / v (GQA: query
    head h reads kv head h // (q_heads // kv_heads)); the square case
    (query_start 0, equal lengths) is plain causal attention.  Views are
    read through their strides -- the transposes of [tokens, heads,
    head_dim] tensors the model passes cost no copy -- and the result is
    written token-major: without ``out`` the returned [batch, q_heads,
    tokens, head_dim] tensor is a view of [batch, tokens, q_heads, head_dim]
    storage, so the caller's transpose back to [tokens, heads, head_dim] is
    contiguous.  ``out`` may supply any [batch, q_heads, tokens, head_dim]
    tensor of q's dtype whose innermost dim is dense and whose elements are
    distinct (not an expanded view).
    """
    if backend != "hip":
        raise ValueError("unknown prefill backend")
    if (q.ndim != 4 or k.ndim != 4 or k.shape != v.shape or k.shape[1] == 0
            or q.shape[1] % k.shape[1]):
        raise ValueError("prefill expects [batch, heads, tokens, dim] and divisible GQA heads")
    if (q.shape[0] != k.shape[0] or q.shape[-1] != k.shape[-1]
            or q.dtype != k.dtype or q.dtype != v.dtype or q.device != k.device or q.device != v.device):
        raise ValueError("prefill tensors must share batch, head_dim, dtype and device")
    if (not isinstance(query_start, int) or isinstance(query_start, bool) or query_start < 0
            or q.shape[-2] <= 0 or query_start + q.shape[-2] > k.shape[-2]):
        raise ValueError("query_start and query length must fit the KV sequence")
    if q.device.type != "cuda" or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("HIP prefill requires HIP FP16/BF16 tensors")
    batch, q_heads, tokens, head_dim = q.shape
    kv_heads, kv_tokens = k.shape[1], k.shape[2]
    if head_dim > MAX_HEAD_DIM:
        raise ValueError("HIP prefill supports head_dim up to 1024")
    if query_start + tokens > MAX_DENSE_CONTEXT:
        raise ValueError("HIP prefill supports at most 1048576 context tokens")
    # A fresh copy, not .contiguous(): a tensor that is already contiguous but
    # starts at a misaligned storage offset would come back unchanged.
    if not _dense_layout_ok(q, head_dim):
        q = _aligned_copy(q)
    if k.stride() != v.stride() or not _dense_layout_ok(k, head_dim) or not _dense_layout_ok(v, head_dim):
        k, v = _aligned_copy(k), _aligned_copy(v)
    if out is None:
        result = torch.empty(batch, tokens, q_heads, head_dim, dtype=q.dtype, device=q.device).transpose(1, 2)
    else:
        if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
            raise ValueError("out must be a [batch, q_heads, tokens, head_dim] tensor of q's dtype and device")
        if not _dense_layout_ok(out, head_dim):
            raise ValueError("out must have a dense head_dim and 16-byte aligned rows")
        if not _dense_disjoint(out):
            raise ValueError("out must not overlap itself")
        result = out
    if min(batch, q_heads, head_dim) == 0:
        return result
    lib = ext.load_hip_extension()
    dtype = ext.dtype_code(q.dtype)
    need = lib.dense_prefill_workspace_size(batch, tokens, q_heads, kv_heads, head_dim, query_start, dtype)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else 0
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    with torch.cuda.device(q.device):
        lib.call("mvme_prefill_attention", result.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                 batch, q_heads, kv_heads, tokens, kv_tokens, head_dim, query_start,
                 *_dense_strides(q), *_dense_strides(k), *_dense_strides(result),
                 dtype, ws_ptr, ws_bytes, ext.current_stream(q.device))
    return result
