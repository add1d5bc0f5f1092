"""CPU oracle of the paged-attention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only to compute the outputs GPU results are
compared with, or as the timed CPU baseline.  The
HIP product path never calls it.

Every function restates, in this repository's own code, one CPU algorithm of
the reference (dandan20031031/myvllm-mini-engine) and cites the file:line it
follows.  The reference's torch paths are restated with the same torch
operations (gather -> repeat_interleave -> fp32 einsum/softmax -> cast), so
the same module doubles as "the reference's CPU torch path" for timing.

Pinning (see tests/test_oracle.py): every function here is checked against
an independent formulation -- torch SDPA on densely gathered K/V, the C
restatement in oracle/paged_ref.c (float64 accumulation), closed forms
(single token, equal keys, permutation invariance), the reference's own
known-answer metadata test and the published make_case SHA-256 manifest.
"""

from __future__ import annotations

import hashlib
import json
import math

import torch
from torch.nn import functional as F

TENSOR_NAMES = ("query", "key_cache", "value_cache", "block_tables", "context_lens")


def sha256_json(value) -> str:
    """benchmarks/common.py:19-21: canonical JSON -> SHA-256."""
    text = json.dumps(value, ensure_ascii=False, sort_keys=True, separators=(",", ":"))
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


def tensor_sha256(tensor: torch.Tensor) -> str:
    return hashlib.sha256(memoryview(tensor.contiguous().view(torch.uint8).numpy())).hexdigest()


def make_case(batch, context, *, heads=16, kv_heads=8, head_dim=128, block_size=256, seed=20261026):
    """Seeded decode inputs (benchmarks/compare_paged_backends.py:32-55).

    Private CPU generator seeded with seed + batch*1000003 + context; fp32
    randn cast to fp16 for q, K, V; block tables are the first batch*width
    entries of a randperm over batch*width + 7 pages.  Returns (tensors,
    manifest) where the manifest hashes the actual bytes.
    """
    if min(batch, context, heads, kv_heads, head_dim, block_size) <= 0 or heads % kv_heads:
        raise ValueError("positive dimensions and heads divisible by KV heads are required")
    width = math.ceil(context / block_size)
    blocks = batch * width + 7
    gen = torch.Generator(device="cpu").manual_seed(seed + batch * 1000003 + context)
    query = torch.randn(batch, heads, head_dim, generator=gen, dtype=torch.float32).half()
    key = torch.randn(blocks, block_size, kv_heads, head_dim, generator=gen, dtype=torch.float32).half()
    value = torch.randn(key.shape, generator=gen, dtype=torch.float32).half()
    table = torch.randperm(blocks, generator=gen)[:batch * width].reshape(batch, width)
    lengths = torch.full((batch,), context, dtype=torch.int64)
    tensors = dict(zip(TENSOR_NAMES, (query, key, value, table, lengths)))
    manifest = {name: {"shape": list(t.shape), "dtype": str(t.dtype), "sha256": tensor_sha256(t)}
                for name, t in tensors.items()}
    shape = {"batch": batch, "context": context, "heads": heads, "kv_heads": kv_heads,
             "head_dim": head_dim, "block_size": block_size, "seed": seed}
    return tensors, {"shape": shape, "tensors": manifest,
                     "case_sha256": sha256_json({"shape": shape, "tensors": manifest})}


def _pages(table_row, length, block_size):
    return table_row[: math.ceil(length / block_size)]


def fp32_oracle(tensors, block_size):
    """The repo's fp32 numerical reference (compare_paged_backends.py:58-72).

    Per sequence: gather pages, fp32 QK, scale 1/sqrt(D), softmax, fp32 PV.
    Returns fp32 [B, Hq, D] (no cast).
    """
    q, key, value, tables, lengths = (tensors[name] for name in TENSOR_NAMES)
    outputs = []
    for row, length in enumerate(lengths.cpu().tolist()):
        ids = _pages(tables[row], length, block_size)
        k = key[ids].reshape(-1, key.shape[2], key.shape[3])[:length].float()
        v = value[ids].reshape(-1, value.shape[2], value.shape[3])[:length].float()
        group = q.shape[1] // k.shape[1]
        scores = torch.einsum("hd,thd->ht", q[row].float(), k.repeat_interleave(group, dim=1))
        prob = (scores / math.sqrt(q.shape[-1])).softmax(-1)
        outputs.append(torch.einsum("ht,thd->hd", prob, v.repeat_interleave(group, dim=1)))
    return torch.stack(outputs)


def validate_output(actual, reference, *, atol=0.006, rtol=0.03):
    """Tolerance gate of compare_paged_backends.py:75-87."""
    if actual.shape != reference.shape:
        return {"passed": False, "reason": "shape mismatch", "atol": atol, "rtol": rtol}
    actual = actual.float()
    reference = reference.float()
    finite = bool(torch.isfinite(actual).all() and torch.isfinite(reference).all())
    error = (actual - reference).abs()
    passed = finite and bool(torch.allclose(actual, reference, atol=atol, rtol=rtol))
    return {"passed": passed, "finite": finite, "atol": atol, "rtol": rtol,
            "max_absolute_error": error.max().item() if finite and error.numel() else None,
            "rms_error": error.square().mean().sqrt().item() if finite and error.numel() else None,
            "outside_tolerance_fraction":
                (error > atol + rtol * reference.abs()).float().mean().item() if error.numel() else 0.0}


def paged_attention(query, key_cache, value_cache, block_tables, context_lens, block_size):
    """The reference's torch decode path (mini_engine/kernels/fallback.py:27-64).

    Per sequence: gather pages, repeat_interleave K/V over the GQA group,
    fp32 einsum QK * 1/sqrt(D), softmax, fp32 einsum PV, cast to q dtype.
    Raises ValueError on the same shape/length violations.
    """
    if query.ndim != 3 or key_cache.ndim != 4 or key_cache.shape != value_cache.shape:
        raise ValueError("invalid query or cache shape")
    if key_cache.shape[1] != block_size or query.shape[-1] != key_cache.shape[-1]:
        raise ValueError("block size or head dimension mismatch")
    if query.shape[1] % key_cache.shape[2]:
        raise ValueError("query heads must be divisible by KV heads")
    scale = 1.0 / math.sqrt(query.shape[-1])
    outputs = []
    for b in range(query.shape[0]):
        length = int(context_lens[b])
        if length <= 0 or length > block_tables.shape[1] * block_size:
            raise ValueError("invalid context length")
        ids = _pages(block_tables[b], length, block_size)
        keys = key_cache[ids].reshape(-1, key_cache.shape[2], key_cache.shape[3])[:length]
        values = value_cache[ids].reshape(-1, value_cache.shape[2], value_cache.shape[3])[:length]
        group = query.shape[1] // keys.shape[1]
        keys = keys.repeat_interleave(group, dim=1)
        values = values.repeat_interleave(group, dim=1)
        scores = torch.einsum("hd,thd->ht", query[b].float(), keys.float()) * scale
        probs = torch.softmax(scores, dim=-1)
        outputs.append(torch.einsum("ht,thd->hd", probs, values.float()).to(query.dtype))
    return torch.stack(outputs)


def write_kv_cache_slots(key_cache, value_cache, slot_mapping, key, value):
    """Slot scatter of the torch path (mini_engine/kernels/data.py:120-125)."""
    rows_k = key_cache.view(-1, *key_cache.shape[2:])
    rows_v = value_cache.view(-1, *value_cache.shape[2:])
    rows_k.index_copy_(0, slot_mapping, key)
    rows_v.index_copy_(0, slot_mapping, value)


def write_kv_cache(key_cache, value_cache, block_ids, token_offset, key, value, block_size):
    """Contiguous-range write across pages (mini_engine/kernels/data.py:51-62)."""
    ids = block_ids.reshape(-1).to(dtype=torch.long)
    if token_offset < 0 or token_offset + key.shape[0] > ids.numel() * block_size:
        raise ValueError("write exceeds supplied block table capacity")
    remaining, source, position = key.shape[0], 0, token_offset
    while remaining:
        block_index, in_block = divmod(position, block_size)
        count = min(remaining, block_size - in_block)
        page = ids[block_index]
        key_cache[page, in_block:in_block + count].copy_(key[source:source + count])
        value_cache[page, in_block:in_block + count].copy_(value[source:source + count])
        source += count
        position += count
        remaining -= count


def write_kv_cache_batch(key_cache, value_cache, block_tables, token_offsets, key, value, block_size):
    """One token per sequence (mini_engine/kernels/data.py:76-79)."""
    for b in range(key.shape[0]):
        write_kv_cache(key_cache, value_cache, block_tables[b], int(token_offsets[b]),
                       key[b].unsqueeze(0), value[b].unsqueeze(0), block_size)


def gather(key_layer, value_layer, block_ids, token_count):
    """Block-table gather (mini_engine/cache/kv_cache.py:147-166)."""
    ids = torch.as_tensor(block_ids, dtype=torch.long).flatten()
    shape = (-1, key_layer.shape[2], key_layer.shape[3])
    return (key_layer[ids].reshape(shape)[:token_count], value_layer[ids].reshape(shape)[:token_count])


def paged_prefill_attention(q, key_cache, value_cache, cu_seqlens_q, query_starts, block_tables,
                            context_lens, block_size, *, cast=True):
    """The torch paged-prefill path (mini_engine/kernels/prefill.py:114-131).

    Per request: gather the pages of the context, repeat over the GQA group,
    fp32 SDPA with the bool mask key <= start + i, cast to q dtype (unless
    cast=False, which keeps the fp32 result for tolerance checks).
    """
    output = torch.empty(q.shape, dtype=q.dtype if cast else torch.float32)
    offsets, starts, lengths = (t.tolist() for t in (cu_seqlens_q, query_starts, context_lens))
    for index, (start, length) in enumerate(zip(starts, lengths)):
        begin, end = offsets[index:index + 2]
        if begin == end:
            continue
        pages = block_tables[index, :(length + block_size - 1) // block_size]
        key = key_cache[pages].reshape(-1, *key_cache.shape[2:])[:length]
        value = value_cache[pages].reshape(-1, *value_cache.shape[2:])[:length]
        groups = q.shape[1] // key.shape[1]
        key = key.repeat_interleave(groups, dim=1).transpose(0, 1).float()
        value = value.repeat_interleave(groups, dim=1).transpose(0, 1).float()
        query = q[begin:end].transpose(0, 1).float()
        mask = torch.arange(length)[None, :] <= (start + torch.arange(end - begin)[:, None])
        rows = F.scaled_dot_product_attention(query, key, value, attn_mask=mask)
        output[begin:end] = rows.transpose(0, 1).to(output.dtype)
    return output


def prefill_attention(q, k, v, *, query_start=0, cast=True):
    """The torch dense prefill path (mini_engine/kernels/prefill.py:42-60).

    q [B, Hq, T, D], k / v [B, Hkv, S, D]: K/V repeated over the GQA group
    (repeat_interleave, :42-45), then SDPA -- with the bool mask
    key <= query_start + t for a suffix (query_start > 0 or T != S, :46-53),
    is_causal for the square case (:54-55).  Computed in fp32 (the reference
    runs SDPA in the input dtype); cast=False keeps the fp32 result.
    """
    groups = q.shape[1] // k.shape[1]
    key = k.repeat_interleave(groups, dim=1).float()
    value = v.repeat_interleave(groups, dim=1).float()
    query = q.float()
    if query_start != 0 or q.shape[-2] != k.shape[-2]:
        mask = torch.arange(k.shape[-2])[None, :] <= (query_start + torch.arange(q.shape[-2]))[:, None]
        out = F.scaled_dot_product_attention(query, key, value, attn_mask=mask)
    else:
        out = F.scaled_dot_product_attention(query, key, value, is_causal=True)
    return out.to(q.dtype) if cast else out


def prefill_metadata(token_sequences, block_tables, query_starts, block_size):
    """Slot/position/offset rules of PrefillBatch (mini_engine/engine/batch.py:88-129).

    Small pure-Python restatement used to pin the package's PrefillBatch;
    returns plain lists.
    """
    positions, slots, offsets, contexts, padded = [], [], [0], [], []
    width = 0
    clean = []
    for tokens, table, start in zip(token_sequences, block_tables, query_starts):
        table = list(table)
        while table and table[-1] == -1:
            table.pop()
        clean.append(table)
        width = max(width, len(table))
        for pos in range(start, start + len(tokens)):
            positions.append(pos)
            slots.append(table[pos // block_size] * block_size + pos % block_size)
        offsets.append(offsets[-1] + len(tokens))
        contexts.append(start + len(tokens))
    padded = [t + [-1] * (width - len(t)) for t in clean]
    return {"positions": positions, "slot_mapping": slots, "cu_seqlens_q": offsets,
            "context_lens": contexts, "block_tables": padded}


def rms_norm(x, weight, eps=1e-6):
    """Qwen3 RMSNorm of the torch path (mini_engine/kernels/fallback.py:8-10).

    fp32 mean of squares over the last dimension; the normalised value is cast
    to the input dtype before the (low-precision) weight multiply.
    """
    variance = x.float().pow(2).mean(dim=-1, keepdim=True)
    return (x.float() * torch.rsqrt(variance + eps)).to(x.dtype) * weight


def apply_rope(q, k, cos, sin):
    """Half-split rotary embedding of the torch path (mini_engine/kernels/fallback.py:13-20).

    cos/sin are [tokens, 1, head_dim/2] (the torch branch unsqueezes them,
    native_qwen3.py:153-154); every product is rounded to the tensor dtype
    before the add/subtract, as eager fp16/bf16 arithmetic does.
    """
    half = q.shape[-1] // 2
    q1, q2, k1, k2 = q[..., :half], q[..., half:], k[..., :half], k[..., half:]
    return (torch.cat((q1 * cos - q2 * sin, q1 * sin + q2 * cos), dim=-1),
            torch.cat((k1 * cos - k2 * sin, k1 * sin + k2 * cos), dim=-1))


def qk_norm_rope_write_kv(q, k, v, q_weight, k_weight, cos, sin, key_cache, value_cache, *,
                          slot_mapping=None, block_tables=None, positions=None, eps=1e-6):
    """The four steps before paged attention in one call (torch data backend).

    Attention._forward_prefill_batch (mini_engine/model/native_qwen3.py:150-157)
    with a slot mapping, forward_decode_batch (:179-191) with block tables and
    positions: q_norm/k_norm, apply_rope, then the KV write.  Writes the caches
    in place and returns the rotated q.  Slots outside the cache and positions
    outside the table are skipped (the HIP kernel's rule for metadata it does
    not trust; the reference validates them away before this point).
    """
    q, k = rms_norm(q, q_weight, eps), rms_norm(k, k_weight, eps)
    q, k = apply_rope(q, k, cos.unsqueeze(1), sin.unsqueeze(1))
    num_blocks, block_size = key_cache.shape[:2]
    if slot_mapping is not None:
        slots = slot_mapping.tolist()
    else:
        slots = []
        width = block_tables.shape[1]
        for t, pos in enumerate(positions.tolist()):
            page = int(block_tables[t, pos // block_size]) if 0 <= pos < width * block_size else -1
            slots.append(page * block_size + pos % block_size if 0 <= page < num_blocks else -1)
    keep = [t for t, slot in enumerate(slots) if 0 <= slot < num_blocks * block_size]
    if keep:
        index = torch.tensor(keep, dtype=torch.long)
        write_kv_cache_slots(key_cache, value_cache, torch.tensor([slots[t] for t in keep], dtype=torch.long),
                             k[index], v[index])
    return q


def greedy_argmax(logits):
    """Greedy sampler of the torch path (mini_engine/sampling.py:22-23): torch.argmax per row."""
    return logits.argmax(dim=-1)
