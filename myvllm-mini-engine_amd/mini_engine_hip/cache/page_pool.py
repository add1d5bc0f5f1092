"""Refcounted physical pages, including shared read-only prefix pages.

Restates the ownership semantics of the reference's ``BlockManager``
(mini_engine/cache/block_manager.py:10-166) that decide which physical page
ids appear in the block tables the kernels read: private pages are
refcount 1, a cached prefix attached to several requests appears in each of
their tables (refcount = number of holders), and a request can be given
retained pages only (``attach``, block_manager.py:83-97 — the prefix cache's
whole-prompt hit, prefix_cache.py:45-48), so its table holds no private
page at all.  Host-side only.
"""

from __future__ import annotations


class PagePool:
    def __init__(self, num_blocks: int, block_size: int, order=None):
        """``order`` (optional) is the sequence in which free pages are handed out."""
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.num_blocks = num_blocks
        self.block_size = block_size
        order = list(range(num_blocks)) if order is None else [int(p) for p in order]
        if sorted(order) != list(range(num_blocks)):
            raise ValueError("order must be a permutation of the page ids")
        self._free = order[::-1]
        self._refs = [0] * num_blocks
        self._owned: dict[str, list[int]] = {}

    @property
    def free_blocks(self) -> int:
        return len(self._free)

    def blocks_required(self, token_count: int) -> int:
        if token_count < 0:
            raise ValueError("token_count cannot be negative")
        return -(-token_count // self.block_size)

    def refcount(self, block: int) -> int:
        return self._refs[block]

    def _take(self, count: int) -> list[int]:
        if count > len(self._free):
            raise MemoryError(f"need {count} blocks, only {len(self._free)} free")
        pages = [self._free.pop() for _ in range(count)]
        for page in pages:
            self._refs[page] = 1
        return pages

    def _check_live(self, pages, what="prefix") -> None:
        if len(set(pages)) != len(pages):
            raise ValueError(f"{what} pages must be distinct")
        for page in pages:
            if page < 0 or page >= self.num_blocks or self._refs[page] <= 0:
                raise ValueError(f"cannot attach unallocated block: {page}")

    def allocate(self, request_id: str, token_count: int) -> list[int]:
        return self.allocate_with_prefix(request_id, token_count, ())

    def allocate_with_prefix(self, request_id: str, token_count: int, prefix) -> list[int]:
        """Attach shared prefix pages, then allocate private pages for the rest."""
        if request_id in self._owned:
            raise ValueError(f"request already owns blocks: {request_id}")
        prefix = list(prefix)
        self._check_live(prefix)
        required = self.blocks_required(token_count)
        if len(prefix) > required:
            raise ValueError("prefix has more blocks than the request needs")
        suffix = self._take(required - len(prefix))
        for page in prefix:
            self._refs[page] += 1
        self._owned[request_id] = prefix + suffix
        return list(self._owned[request_id])

    def attach(self, request_id: str, pages) -> list[int]:
        """Give a request a table made only of pages other holders retain."""
        if request_id in self._owned:
            raise ValueError(f"request already owns blocks: {request_id}")
        pages = [int(p) for p in pages]
        self._check_live(pages, "attached")
        for page in pages:
            self._refs[page] += 1
        self._owned[request_id] = pages
        return list(pages)

    def pin(self, pages) -> None:
        """Hold one external reference (e.g. a prefix-cache entry)."""
        pages = list(pages)
        self._check_live(pages, "pinned")
        for page in pages:
            self._refs[page] += 1

    def unpin(self, pages) -> None:
        for page in pages:
            self._release(page)

    def free(self, request_id: str) -> None:
        for page in self._owned.pop(request_id):
            self._release(page)

    def _release(self, page: int) -> None:
        if self._refs[page] <= 0:
            raise ValueError(f"double free of block {page}")
        self._refs[page] -= 1
        if self._refs[page] == 0:
            self._free.append(page)

    def table(self, request_id: str) -> list[int]:
        return list(self._owned[request_id])
