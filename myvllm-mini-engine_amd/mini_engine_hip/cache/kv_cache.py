"""Paged KV-cache storage on the GPU.

Keeps the reference's layout contract, ``[layer, block, token, kv_head,
head_dim]`` with a contiguous per-layer view ``[num_blocks, block_size,
kv_heads, head_dim]`` (mini_engine/cache/kv_cache.py:25-60).  Writes and the
block-table gather run as HIP kernels (``write_hip``, ``gather``), bit-exact
with the reference's torch copies (kv_cache.py:82-166).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ..kernels import data as _data
from ..kernels import hip_extension as ext


@dataclass(frozen=True)
class KVCacheShape:
    num_layers: int
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int


class KVCachePool:
    """Preallocated key/value tensors indexed by physical block id."""

    def __init__(self, num_layers, num_blocks, block_size, num_kv_heads, head_dim, *,
                 dtype=torch.bfloat16, device="cuda"):
        values = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        if any(value <= 0 for value in values):
            raise ValueError("all KV cache dimensions must be positive")
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("HIP KV cache requires FP16/BF16")
        self.shape = KVCacheShape(*values)
        self.dtype = dtype
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("HIP KV cache must live on a GPU device")
        self.key = torch.empty(values, dtype=dtype, device=self.device)
        self.value = torch.empty_like(self.key)
        self.device = self.key.device  # resolved index, e.g. cuda -> cuda:0

    @property
    def numel(self) -> int:
        return self.key.numel() * 2

    @property
    def memory_bytes(self) -> int:
        return self.numel * self.key.element_size()

    def _block_ids(self, block_ids):
        ids = torch.as_tensor(block_ids, dtype=torch.long, device=self.device).flatten().contiguous()
        if ids.numel() and bool(((ids < 0) | (ids >= self.shape.num_blocks)).any()):
            raise IndexError("physical block id out of range")
        return ids

    def _layer(self, layer):
        if layer < 0 or layer >= self.shape.num_layers:
            raise IndexError("layer out of range")

    def clear(self, block_ids=None) -> None:
        """Zero all blocks or only blocks returned to the allocator."""
        if block_ids is None:
            self.key.zero_()
            self.value.zero_()
            return
        if not len(block_ids):
            return
        ids = self._block_ids(block_ids)
        self.key.index_fill_(1, ids, 0)
        self.value.index_fill_(1, ids, 0)

    def write_hip(self, layer, block_ids, token_offset, key, value, *, validate=True) -> None:
        """Write a contiguous token range across pages with the HIP scatter kernel."""
        if key.shape != value.shape or key.ndim != 3:
            raise ValueError("key and value must both have shape [tokens, kv_heads, head_dim]")
        self._layer(layer)
        ids = self._block_ids(block_ids)
        if token_offset < 0 or token_offset + key.shape[0] > ids.numel() * self.shape.block_size:
            raise ValueError("write exceeds supplied block table capacity")
        if key.device != self.device or value.device != self.device or key.dtype != self.dtype or value.dtype != self.dtype:
            raise ValueError("HIP KV write inputs must match cache device and dtype")
        _data.write_kv_cache(self.key[layer], self.value[layer], ids, token_offset, key.contiguous(),
                             value.contiguous(), self.shape.block_size, backend="hip", validate=validate)

    def gather(self, layer, block_ids, token_count):
        """Gather the logical prefix [0, token_count) of a block table (HIP kernel)."""
        if token_count < 0:
            raise ValueError("token_count cannot be negative")
        self._layer(layer)
        ids = self._block_ids(block_ids)
        if token_count > ids.numel() * self.shape.block_size:
            raise ValueError("token_count exceeds supplied block table capacity")
        shape = (token_count, self.shape.num_kv_heads, self.shape.head_dim)
        key = torch.empty(shape, dtype=self.dtype, device=self.device)
        value = torch.empty_like(key)
        if token_count == 0:
            return key, value
        lib = ext.load_hip_extension()
        s = self.shape
        with torch.cuda.device(self.device):
            lib.call("mvme_gather_kv_cache", key.data_ptr(), value.data_ptr(), self.key[layer].data_ptr(),
                     self.value[layer].data_ptr(), s.num_blocks, s.block_size, s.num_kv_heads, s.head_dim,
                     ids.data_ptr(), ids.numel(), token_count, ext.dtype_code(self.dtype),
                     ext.current_stream(self.device))
        return key, value
