"""Synthetic inputs of the paged-attention benchmark workloads.

q/K/V are N(0, 1) (fp32 randn cast to the dtype), physical pages come from a
seeded permutation so block tables are non-contiguous, scale is 1/sqrt(D).
Large tensors are drawn on the target device with a device generator; the
metadata (tables, lengths, slots) is drawn on the CPU so it is identical on
every device.

Workloads (Hq=16, Hkv=8, D=128 throughout):
  decode_b1     fp16, B=1,  ctx 128,  block 256, 64-page pool
  decode_b8     bf16, B=8,  ctx 512,  block 16, 2048-page pool, + KV scatter
  decode_b32    fp16, B=32, ctx 2048, block 256, one layer (263-page pool)
  ragged_b64    bf16, B=64, ctx U[1,4096], block 16, 16 sequences sharing a
                1024-token prefix's pages (refcounted, as BlockManager does)
  prefill_8x128 bf16, 8 sequences x 128 new queries after U[0,3968] prior
                tokens, block 256, chunk K/V scattered through a slot mapping
"""

from __future__ import annotations

import math

import torch

from .cache.page_pool import PagePool

HEADS, KV_HEADS, HEAD_DIM = 16, 8, 128
BASE_SEED = 20261026


def _randn(shape, dtype, device, gen):
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(dtype)


def _device_generator(device, seed):
    return torch.Generator(device=device).manual_seed(seed)


def uniform_decode_case(*, batch, context, block_size, dtype, pool_pages=None, seed, device):
    """Equal-length decode: random distinct pages for every sequence."""
    gen = torch.Generator().manual_seed(seed)
    width = math.ceil(context / block_size)
    pool_pages = pool_pages or batch * width + 7
    tables = torch.randperm(pool_pages, generator=gen)[:batch * width].view(batch, width).contiguous()
    lens = torch.full((batch,), context, dtype=torch.int64)
    dgen = _device_generator(device, seed)
    query = _randn((batch, HEADS, HEAD_DIM), dtype, device, dgen)
    key = _randn((pool_pages, block_size, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    value = _randn((pool_pages, block_size, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    return {"query": query, "key_cache": key, "value_cache": value, "block_tables": tables.to(device),
            "context_lens": lens.to(device), "block_size": block_size}


def decode_b1(device, seed=BASE_SEED + 0):
    return uniform_decode_case(batch=1, context=128, block_size=256, dtype=torch.float16, pool_pages=64,
                               seed=seed, device=device)


def decode_b8_with_scatter(device, seed=BASE_SEED + 1):
    """The new token at position 511 of every sequence is scattered first."""
    case = uniform_decode_case(batch=8, context=512, block_size=16, dtype=torch.bfloat16, pool_pages=2048,
                               seed=seed, device=device)
    tables = case["block_tables"].cpu()
    slots = tables[:, 31] * 16 + 15
    dgen = _device_generator(device, seed + 7)
    case["slot_mapping"] = slots.to(device)
    case["new_key"] = _randn((8, KV_HEADS, HEAD_DIM), torch.bfloat16, device, dgen)
    case["new_value"] = _randn((8, KV_HEADS, HEAD_DIM), torch.bfloat16, device, dgen)
    return case


def decode_b32_layer(device, seed):
    return uniform_decode_case(batch=32, context=2048, block_size=256, dtype=torch.float16, seed=seed,
                               device=device)


def ragged_decode_case(*, seed=BASE_SEED + 5, device, batch=32, max_len=4096, block_size=256,
                       dtype=torch.float16):
    """Ragged decode, contexts U[1, max_len] seeded, every sequence on its own
    random pages (-1 past its last page)."""
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, max_len + 1, (batch,), generator=gen)
    width = math.ceil(max_len / block_size)
    pool_pages = batch * width + 7
    order = torch.randperm(pool_pages, generator=gen)
    tables = torch.full((batch, width), -1, dtype=torch.int64)
    for b in range(batch):
        used = math.ceil(int(lens[b]) / block_size)
        tables[b, :used] = order[b * width:b * width + used]
    dgen = _device_generator(device, seed)
    query = _randn((batch, HEADS, HEAD_DIM), dtype, device, dgen)
    key = _randn((pool_pages, block_size, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    value = _randn((pool_pages, block_size, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    return {"query": query, "key_cache": key, "value_cache": value, "block_tables": tables.to(device),
            "context_lens": lens.to(torch.int64).to(device), "block_size": block_size}


def ragged_shared_prefix_case(*, seed=BASE_SEED + 3, device, batch=64, max_len=4096, block_size=16,
                              shared=16, prefix_tokens=1024, pool_pages=16384, dtype=torch.bfloat16):
    """Ragged decode where `shared` sequences map their first `prefix_tokens`
    tokens to the same physical pages (a refcounted prefix-cache hit)."""
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, max_len + 1, (batch,), generator=gen)
    lens[:shared] = lens[:shared].clamp(min=prefix_tokens + 1)
    pool = PagePool(pool_pages, block_size, order=torch.randperm(pool_pages, generator=gen).tolist())
    prefix = pool.allocate("prefix-cache", prefix_tokens)
    width = math.ceil(max_len / block_size)
    tables = torch.full((batch, width), -1, dtype=torch.int64)
    for b in range(batch):
        length = int(lens[b])
        pages = (pool.allocate_with_prefix(f"seq{b}", length, prefix) if b < shared
                 else pool.allocate(f"seq{b}", length))
        tables[b, :len(pages)] = torch.tensor(pages)
    dgen = _device_generator(device, seed)
    query = _randn((batch, HEADS, HEAD_DIM), dtype, device, dgen)
    key = _randn((pool_pages, block_size, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    value = _randn((pool_pages, block_size, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    unique_pages = len({int(p) for p in tables[tables >= 0].tolist()})
    unique_rows = 0
    seen = set()
    for b in range(batch):
        length = int(lens[b])
        for t in range(length):
            key_row = (int(tables[b, t // block_size]), t % block_size)
            if key_row not in seen:
                seen.add(key_row)
                unique_rows += 1
    return {"query": query, "key_cache": key, "value_cache": value, "block_tables": tables.to(device),
            "context_lens": lens.to(torch.int64).to(device), "block_size": block_size,
            "unique_pages": unique_pages, "unique_rows": unique_rows, "logical_rows": int(lens.sum())}


def chunked_prefill_case(*, seed=BASE_SEED + 4, device, num_seqs=8, new_tokens=128, max_prior=3968,
                         block_size=256, dtype=torch.bfloat16, priors=None):
    """Ragged chunked prefill inputs; the chunk K/V still has to be scattered."""
    gen = torch.Generator().manual_seed(seed)
    if priors is None:
        priors = torch.randint(0, max_prior + 1, (num_seqs,), generator=gen).tolist()
    counts = [new_tokens] * num_seqs
    widths = [math.ceil((p + c) / block_size) for p, c in zip(priors, counts)]
    pool_pages = sum(widths) + 7
    perm = torch.randperm(pool_pages, generator=gen)
    tables = torch.full((num_seqs, max(widths)), -1, dtype=torch.int64)
    used = 0
    for s, w in enumerate(widths):
        tables[s, :w] = perm[used:used + w]
        used += w
    slots = []
    for s in range(num_seqs):
        for pos in range(priors[s], priors[s] + counts[s]):
            slots.append(int(tables[s, pos // block_size]) * block_size + pos % block_size)
    total = sum(counts)
    cu = torch.tensor([0] + torch.tensor(counts).cumsum(0).tolist(), dtype=torch.int64)
    starts = torch.tensor(priors, dtype=torch.int64)
    dgen = _device_generator(device, seed)
    key = _randn((pool_pages, block_size, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    value = _randn((pool_pages, block_size, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    q = _randn((total, HEADS, HEAD_DIM), dtype, device, dgen)
    new_k = _randn((total, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    new_v = _randn((total, KV_HEADS, HEAD_DIM), dtype, device, dgen)
    return {"q": q, "key_cache": key, "value_cache": value, "cu_seqlens_q": cu.to(device),
            "query_starts": starts.to(device), "block_tables": tables.to(device),
            "context_lens": (starts + torch.tensor(counts)).to(device), "slot_mapping": torch.tensor(slots).to(device),
            "new_key": new_k, "new_value": new_v, "block_size": block_size, "priors": priors}


def prefill_flops(priors, new_tokens=128, heads=HEADS, head_dim=HEAD_DIM):
    """Unmasked (q, k) pairs x 4*D*Hq: sum_i sum_{t<n} (P_i + t + 1)."""
    pairs = sum(new_tokens * p + new_tokens * (new_tokens + 1) // 2 for p in priors)
    return 4 * head_dim * heads * pairs
