"""Fused q/k RMSNorm + RoPE + KV page write, ``backend="hip"``.

One HIP launch for the four steps the reference's attention layer runs before
paged attention (mini_engine/model/native_qwen3.py:150-157 for a prefill
batch, :179-191 for a decode batch):

    q, k = q_norm(q), k_norm(k)                  # elementwise.py:16-21 (RMSNorm over head_dim)
    q, k = apply_rope(q, k, cos, sin)            # data.py:27-36
    write_kv_cache_slots(kc, vc, slots, k, v)    # prefill (data.py:84-130), or
    write_kv_cache_batch(kc, vc, tables, positions, k, v, block_size)   # decode (data.py:67-81)

with the same fp16/bf16 rounding steps (fallback.py:8-20).  Validation keeps
the reference's messages: the Python-side shape/dtype checks raise
``ValueError`` (data.py:27-36), native-side checks ``RuntimeError``
(bindings.cpp:52-66, :96-108), slot contract violations ``ValueError``
(data.py:109-119).
"""

from __future__ import annotations

import math

import torch

from . import hip_extension as ext
from .data import _row_stride

MAX_HEAD_DIM = 512


def _check(condition, message):
    if not condition:
        raise RuntimeError(message)


def qk_norm_rope_write_kv(q, k, v, q_weight, k_weight, cos, sin, key_cache, value_cache, *,
                          slot_mapping=None, block_tables=None, positions=None, eps=1e-6,
                          backend="hip", validate=True, out=None):
    """Return rope(rmsnorm(q)) and write rope(rmsnorm(k)), v into their KV slots.

    q ``[T, Hq, D]``, k/v ``[T, Hkv, D]`` (rows may be strided slices of a
    fused QKV projection), weights ``[D]``, cos/sin ``[T, D/2]`` in the
    activation dtype.  Either ``slot_mapping`` ``[T]`` (prefill) or
    ``block_tables`` ``[T, W]`` with ``positions`` ``[T]`` (decode: token t is
    the new token of sequence t, written at ``positions[t]``).
    """
    if backend != "hip":
        raise ValueError("fused norm/RoPE/KV-write backend must be hip")
    if (slot_mapping is None) == (positions is None):
        raise ValueError("pass either slot_mapping or block_tables with positions")
    if q.ndim != 3 or k.ndim != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q and k must be [tokens, heads, head_dim] with matching token/head dimensions")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("HIP RoPE supports FP16/BF16")
    tensors = [q, k, v, q_weight, k_weight, cos, sin, key_cache, value_cache]
    for t in tensors:
        _check(t.is_cuda, "RoPE inputs must be contiguous CUDA tensors")
        _check(t.device == q.device, "RoPE inputs must share a device")
    _check(cos.is_contiguous() and sin.is_contiguous(), "RoPE inputs must be contiguous CUDA tensors")
    _check(cos.dim() == 2 and sin.shape == cos.shape and cos.size(0) == q.size(0) and cos.size(1) * 2 == q.size(2),
           "RoPE cos/sin shape mismatch")
    _check(all(t.dtype == q.dtype for t in (k, v, cos, sin)), "RoPE dtype mismatch")
    _check(k.size(1) > 0 and q.size(1) >= k.size(1) and q.size(1) % k.size(1) == 0, "RoPE GQA head mismatch")
    for weight in (q_weight, k_weight):
        _check(weight.dtype == q.dtype and weight.dim() == 1 and weight.numel() == q.size(2)
               and weight.is_contiguous(), "RMSNorm weight shape/dtype mismatch")
    _check(math.isfinite(eps) and eps > 0 and float(torch.tensor(eps, dtype=torch.float32)) > 0,
           "eps must be positive, finite and representable in FP32")
    _check(q.size(2) % 2 == 0 and q.size(2) <= MAX_HEAD_DIM, "RoPE cos/sin shape mismatch")
    if (key_cache.ndim != 4 or value_cache.shape != key_cache.shape or not key_cache.is_contiguous()
            or not value_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous [pages, block_size, kv_heads, head_dim]")
    if v.shape != k.shape or k.shape[1:] != key_cache.shape[2:]:
        raise ValueError("packed key/value must be [tokens, kv_heads, head_dim] matching the cache")
    if key_cache.dtype != q.dtype or value_cache.dtype != q.dtype:
        raise ValueError("packed KV tensors must share the cache dtype")
    tokens = q.size(0)
    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    if slot_mapping is not None:
        if (slot_mapping.ndim != 1 or slot_mapping.numel() != tokens or slot_mapping.dtype != torch.int64
                or not slot_mapping.is_contiguous() or slot_mapping.device != q.device):
            raise ValueError("slot_mapping must be contiguous int64 [tokens]")
        if validate:
            slots = slot_mapping.tolist()
            if any(slot < 0 or slot >= num_blocks * block_size for slot in slots):
                raise ValueError("KV slot is outside cache capacity")
            if len(set(slots)) != len(slots):
                raise ValueError("duplicate KV slots would race during scatter")
        tables_ptr, width, pos_ptr = None, 0, None
    else:
        if block_tables is None or block_tables.ndim != 2 or positions.ndim != 1 \
                or block_tables.shape[0] != tokens or positions.shape[0] != tokens:
            raise ValueError("batch block table or offset shape mismatch")
        _check(block_tables.dtype == torch.int64 and positions.dtype == torch.int64
               and block_tables.is_contiguous() and positions.is_contiguous()
               and block_tables.device == q.device and positions.device == q.device,
               "batch KV write inputs must be contiguous int64 CUDA tensors")
        if validate:
            capacity = block_tables.shape[1] * block_size
            _check(not bool(((positions < 0) | (positions >= capacity)).any()), "batch KV offset out of range")
            _check(not bool(((block_tables < 0) | (block_tables >= num_blocks)).any()),
                   "KV batch physical block id out of range")
        tables_ptr, width, pos_ptr = block_tables.data_ptr(), block_tables.shape[1], positions.data_ptr()
    if validate and any(torch._C._overlaps(cache, src) for cache in (key_cache, value_cache)
                        for src in (q, k, v)):
        raise ValueError("KV destinations and source tensors must not overlap")
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous() or out.device != q.device:
        raise ValueError("out must be a contiguous tensor shaped like q")
    if tokens == 0:
        return out
    q_stride, q = _row_stride(q)
    k_stride, k = _row_stride(k)
    v_stride, v = _row_stride(v)
    lib = ext.load_hip_extension()
    with torch.cuda.device(q.device):
        lib.call("mvme_qk_norm_rope_write_kv", out.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                 num_blocks, block_size, kv_heads, head_dim,
                 slot_mapping.data_ptr() if slot_mapping is not None else None, tables_ptr, width, pos_ptr,
                 q.data_ptr(), k.data_ptr(), v.data_ptr(), q_stride, k_stride, v_stride,
                 q_weight.data_ptr(), k_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(), tokens, q.shape[1],
                 float(eps), ext.dtype_code(q.dtype), ext.current_stream(q.device))
    return out
