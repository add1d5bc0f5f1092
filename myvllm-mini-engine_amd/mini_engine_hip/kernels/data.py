"""KV-cache writes (scatter) with ``backend="hip"``.

Mirrors the KV entry points of the reference's data dispatch
(mini_engine/kernels/data.py:39-130) and their native checks
(mini_engine/kernels/csrc/bindings.cpp:98-150, csrc/data.cu:209-250):
Python-side contract violations raise ``ValueError`` before anything runs,
native-side ones ``RuntimeError``.  Every write is a bit-exact row copy done
by a HIP kernel on the current stream; nothing falls back to torch.
"""

from __future__ import annotations

import torch

from . import hip_extension as ext


def _backend(backend):
    if backend != "hip":
        raise ValueError("data backend must be hip")


def _check(condition, message):
    if not condition:
        raise RuntimeError(message)


def _native_kv_checks(key_cache, value_cache, tensors, key, value, label):
    for t in (key_cache, value_cache, *tensors, key, value):
        _check(t.is_cuda and t.is_contiguous(), f"{label} inputs must be contiguous CUDA tensors")
        _check(t.device == key_cache.device, f"{label} inputs must share a device")
    _check(key_cache.dim() == 4 and value_cache.shape == key_cache.shape, "cache shape mismatch")
    _check(key.dim() == 3 and value.shape == key.shape, "K/V shape mismatch")
    _check(key.shape[1] == key_cache.shape[2] and key.shape[2] == key_cache.shape[3],
           "K/V head shape mismatch")
    _check(key_cache.dtype in (torch.float16, torch.bfloat16), "KV cache requires FP16/BF16")
    _check(key.dtype == key_cache.dtype and value.dtype == key_cache.dtype, "KV dtype mismatch")


def write_kv_cache(key_cache, value_cache, block_ids, token_offset, key, value,
                   block_size, *, backend="hip", validate=True):
    """Write a contiguous token range [offset, offset+T) across ``block_ids``."""
    _backend(backend)
    if key.shape != value.shape or key.ndim != 3:
        raise ValueError("key and value must be [tokens, kv_heads, head_dim]")
    if key.device != key_cache.device or value.device != key_cache.device:
        raise ValueError("KV tensors must be on the cache device")
    if key.dtype != key_cache.dtype or value.dtype != key_cache.dtype:
        raise ValueError("KV tensors must match cache dtype")
    ids = block_ids.reshape(-1).to(device=key_cache.device, dtype=torch.long)
    if token_offset < 0 or token_offset + key.shape[0] > ids.numel() * block_size:
        raise ValueError("write exceeds supplied block table capacity")
    _native_kv_checks(key_cache, value_cache, (ids,), key, value, "KV write")
    _check(block_size > 0 and key_cache.shape[1] == block_size, "block size mismatch")
    if validate:
        _check(not bool(((ids < 0) | (ids >= key_cache.shape[0])).any()), "KV physical block id out of range")
    lib = ext.load_hip_extension()
    num_blocks, _, kv_heads, head_dim = key_cache.shape
    with torch.cuda.device(key_cache.device):
        lib.call("mvme_write_kv_cache", key_cache.data_ptr(), value_cache.data_ptr(), num_blocks,
                 block_size, kv_heads, head_dim, ids.data_ptr(), ids.numel(), int(token_offset),
                 key.data_ptr(), value.data_ptr(), key.shape[0], ext.dtype_code(key_cache.dtype),
                 ext.current_stream(key_cache.device))


def write_kv_cache_batch(key_cache, value_cache, block_tables, token_offsets, key, value,
                         block_size, *, backend="hip", validate=True):
    """Decode-step write: row b goes to position token_offsets[b] of sequence b."""
    _backend(backend)
    if key.shape != value.shape or key.ndim != 3:
        raise ValueError("batch key/value must be [batch, kv_heads, head_dim]")
    if (block_tables.ndim != 2 or token_offsets.ndim != 1 or block_tables.shape[0] != key.shape[0]
            or token_offsets.shape[0] != key.shape[0]):
        raise ValueError("batch block table or offset shape mismatch")
    tables = block_tables.to(device=key_cache.device, dtype=torch.long).contiguous()
    offsets = token_offsets.to(device=key_cache.device, dtype=torch.long).contiguous()
    _native_kv_checks(key_cache, value_cache, (tables, offsets), key, value, "batch KV write")
    _check(block_size > 0 and key_cache.shape[1] == block_size, "batch block size mismatch")
    if validate:
        # Host-synchronising checks of the native op (bindings.cpp:143-147,
        # data.cu:179): every table entry must name a page.
        capacity = tables.shape[1] * block_size
        _check(not bool(((offsets < 0) | (offsets >= capacity)).any()), "batch KV offset out of range")
        _check(not bool(((tables < 0) | (tables >= key_cache.shape[0])).any()),
               "KV batch physical block id out of range")
    lib = ext.load_hip_extension()
    num_blocks, _, kv_heads, head_dim = key_cache.shape
    with torch.cuda.device(key_cache.device):
        lib.call("mvme_write_kv_cache_batch", key_cache.data_ptr(), value_cache.data_ptr(), num_blocks,
                 block_size, kv_heads, head_dim, tables.data_ptr(), tables.shape[1], offsets.data_ptr(),
                 key.data_ptr(), value.data_ptr(), key.shape[0], ext.dtype_code(key_cache.dtype),
                 ext.current_stream(key_cache.device))


def _row_stride(tensor):
    """(token stride in elements, tensor) for a kernel that reads [T, H, D] rows.

    The kernels read each token's [heads, head_dim] block as one dense run
    of H*D elements starting at ``t * stride``.  A view whose rows are dense
    (a slice of a fused QKV projection) is passed as it is, with its token
    stride; any other layout — for one token as for many — is copied to a
    contiguous tensor first.  Strides of dimensions of size 1 never matter.
    """
    tokens, heads, dim = tensor.shape
    dense_rows = (dim == 1 or tensor.stride(2) == 1) and (heads == 1 or tensor.stride(1) == dim)
    if dense_rows and tokens <= 1:
        return heads * dim, tensor
    if dense_rows and tensor.stride(0) >= heads * dim:
        return tensor.stride(0), tensor
    tensor = tensor.contiguous()
    return heads * dim, tensor


def write_kv_cache_slots(key_cache, value_cache, slot_mapping, key, value,
                         *, backend="hip", validate=True):
    """Copy row t of ``key``/``value`` to cache slot ``slot_mapping[t]``.

    A slot numbers a token row of the whole pool, ``page * block_size +
    offset``.  With ``validate=True`` the slots are read on the host and must
    be in range and distinct, and no source may alias a cache; with
    ``validate=False`` (graph capture) only shapes, dtypes and devices are
    checked, and the kernel skips any slot outside the pool.  The sources
    may be strided views whose per-token [kv_heads, head_dim] rows are dense.
    """
    _backend(backend)
    if (key_cache.ndim != 4 or value_cache.shape != key_cache.shape
            or any(size <= 0 for size in key_cache.shape)
            or not key_cache.is_contiguous() or not value_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous [pages, block_size, kv_heads, head_dim]")
    if key.ndim != 3 or key.shape != value.shape or key.shape[1:] != key_cache.shape[2:]:
        raise ValueError("packed key/value must be [tokens, kv_heads, head_dim] matching the cache")
    if (slot_mapping.ndim != 1 or slot_mapping.numel() != key.shape[0]
            or slot_mapping.dtype != torch.int64 or not slot_mapping.is_contiguous()):
        raise ValueError("slot_mapping must be contiguous int64 [tokens]")
    for tensor in (value_cache, slot_mapping, key, value):
        if tensor.device != key_cache.device:
            raise ValueError("packed KV tensors and slots must share the cache device")
    if any(t.dtype != key_cache.dtype for t in (value_cache, key, value)):
        raise ValueError("packed KV tensors must share the cache dtype")
    if key_cache.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("packed KV requires FP32/FP16/BF16")
    if validate:
        slots = slot_mapping.tolist()
        capacity = key_cache.shape[0] * key_cache.shape[1]
        if any(slot < 0 or slot >= capacity for slot in slots):
            raise ValueError("KV slot is outside cache capacity")
        if len(set(slots)) != len(slots):
            raise ValueError("duplicate KV slots would race during scatter")
        if (torch._C._overlaps(key_cache, value_cache)
                or any(torch._C._overlaps(cache, source)
                       for cache in (key_cache, value_cache) for source in (key, value, slot_mapping))):
            raise ValueError("KV destinations and source tensors must not overlap")
    if key_cache.device.type != "cuda" or key_cache.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("HIP packed KV writes require HIP FP16/BF16")
    if key.shape[0] == 0:
        return
    key_stride, key = _row_stride(key)
    value_stride, value = _row_stride(value)
    lib = ext.load_hip_extension()
    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    with torch.cuda.device(key_cache.device):
        lib.call("mvme_write_kv_cache_slots", key_cache.data_ptr(), value_cache.data_ptr(), num_blocks,
                 block_size, kv_heads, head_dim, slot_mapping.data_ptr(), key.data_ptr(),
                 value.data_ptr(), key.shape[0], key_stride, value_stride,
                 ext.dtype_code(key_cache.dtype), ext.current_stream(key_cache.device))
