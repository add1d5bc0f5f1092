"""Paged KV-cache storage on the GPU.

Layout contract of the reference's ``KVCachePool``
(mini_engine/cache/kv_cache.py:25-60): ``key`` and ``value`` are
``[layer, block, token, kv_head, head_dim]`` and every layer's slice
``[num_blocks, block_size, kv_heads, head_dim]`` is contiguous, so the paged
kernels take ``pool.key[layer]`` directly.

Here both planes live in ONE device allocation ``[2, layer, block, token,
kv_head, head_dim]`` (K plane, then V plane); ``key``/``value`` are its two
planes.  Page lists are validated once into a :class:`PageList` (a device
int64 tensor plus its token capacity) that the HIP write and gather kernels
read directly.  Writes and gathers are bit-exact with the reference's torch
copies (kv_cache.py:82-166); ``clear`` zeroes pages in place.
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

    @property
    def row_shape(self):
        """Shape of one token's K (or V) row: [kv_heads, head_dim]."""
        return (self.num_kv_heads, self.head_dim)


@dataclass(frozen=True)
class PageList:
    """Physical page ids of one request, checked against the pool, on device."""

    ids: torch.Tensor
    capacity: int  # tokens the pages hold

    @classmethod
    def of(cls, block_ids, shape: KVCacheShape, device) -> "PageList":
        ids = torch.as_tensor(block_ids, dtype=torch.long, device=device).reshape(-1).contiguous()
        if ids.numel():
            lo, hi = ids.aminmax()
            if int(lo) < 0 or int(hi) >= shape.num_blocks:
                raise IndexError("physical block id out of range")
        return cls(ids, ids.numel() * shape.block_size)


class KVCachePool:
    """K and V pages of every layer in one HIP allocation."""

    def __init__(self, num_layers, num_blocks, block_size, num_kv_heads, head_dim, *,
                 dtype=torch.bfloat16, device="cuda"):
        dims = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        if min(dims) <= 0:
            raise ValueError("all KV cache dimensions must be positive")
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("HIP KV cache requires FP16/BF16")
        if torch.device(device).type != "cuda":
            raise ValueError("HIP KV cache must live on a GPU device")
        self.shape = KVCacheShape(*dims)
        self.dtype = dtype
        self._planes = torch.empty((2, *dims), dtype=dtype, device=device)
        self.key, self.value = self._planes[0], self._planes[1]
        self.device = self._planes.device  # resolved index, e.g. cuda -> cuda:0

    @property
    def numel(self) -> int:
        return self._planes.numel()

    @property
    def memory_bytes(self) -> int:
        return self._planes.numel() * self._planes.element_size()

    def pages(self, block_ids) -> PageList:
        return PageList.of(block_ids, self.shape, self.device)

    def layer(self, layer):
        """(key, value) pages of one layer: contiguous [NB, BS, Hkv, D] each."""
        if not 0 <= layer < self.shape.num_layers:
            raise IndexError("layer out of range")
        return self.key[layer], self.value[layer]

    def clear(self, block_ids=None) -> None:
        """Zero every page, or only the listed pages (of every layer, K and V)."""
        if block_ids is None:
            self._planes.zero_()
        elif len(block_ids):
            self._planes.index_fill_(2, self.pages(block_ids).ids, 0)

    def write_hip(self, layer, block_ids, token_offset, key, value, *, validate=True) -> None:
        """Write rows for positions [token_offset, token_offset + T) of a page list."""
        if key.ndim != 3 or value.shape != key.shape:
            raise ValueError("key and value must both have shape [tokens, kv_heads, head_dim]")
        key_pages, value_pages = self.layer(layer)
        pages = self.pages(block_ids)
        if not 0 <= token_offset <= pages.capacity - key.shape[0]:
            raise ValueError("write exceeds supplied block table capacity")
        if any(t.device != self.device or t.dtype != self.dtype for t in (key, value)):
            raise ValueError("HIP KV write inputs must match cache device and dtype")
        _data.write_kv_cache(key_pages, value_pages, pages.ids, token_offset, key.contiguous(),
                             value.contiguous(), self.shape.block_size, backend="hip", validate=validate)

    def gather(self, layer, block_ids, token_count):
        """K and V rows of positions [0, token_count) of a page list, packed (HIP kernel)."""
        if token_count < 0:
            raise ValueError("token_count cannot be negative")
        key_pages, value_pages = self.layer(layer)
        pages = self.pages(block_ids)
        if token_count > pages.capacity:
            raise ValueError("token_count exceeds supplied block table capacity")
        packed = torch.empty((2, token_count, *self.shape.row_shape), dtype=self.dtype, device=self.device)
        if token_count:
            s = self.shape
            lib = ext.load_hip_extension()
            with torch.cuda.device(self.device):
                lib.call("mvme_gather_kv_cache", packed[0].data_ptr(), packed[1].data_ptr(),
                         key_pages.data_ptr(), value_pages.data_ptr(), s.num_blocks, s.block_size,
                         s.num_kv_heads, s.head_dim, pages.ids.data_ptr(), pages.ids.numel(), token_count,
                         ext.dtype_code(self.dtype), ext.current_stream(self.device))
        return packed[0], packed[1]
