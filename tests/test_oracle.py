"""Pins of the CPU oracle (CPU only).

Each oracle function is checked against something it cannot share a mistake
with: torch SDPA on densely gathered K/V (the reference's own independent
formulation, tests/test_paged_comparison.py:29-39 and
tests/test_native_qwen3.py:13-21), the float64 C restatement, closed forms,
the reference's known-answer metadata test and the published make_case
manifest.  The planted-mistake tests at the end show that each check fails
for a plausible wrong oracle.
"""

import json
import math
from pathlib import Path

import pytest
import torch
from torch.nn import functional as F

from oracle import c_oracle, paged_oracle as po

GOLDEN = Path(__file__).resolve().parent / "golden"


def small_case(seed=0, batch=3, heads=8, kv_heads=2, dim=16, block=4, lengths=(7, 1, 13), dtype=torch.float16):
    gen = torch.Generator().manual_seed(seed)
    width = math.ceil(max(lengths) / block)
    pages = batch * width + 5
    q = torch.randn(batch, heads, dim, generator=gen).to(dtype)
    k = torch.randn(pages, block, kv_heads, dim, generator=gen).to(dtype)
    v = torch.randn(pages, block, kv_heads, dim, generator=gen).to(dtype)
    tables = torch.randperm(pages, generator=gen)[:batch * width].view(batch, width)
    lens = torch.tensor(lengths, dtype=torch.int64)
    return q, k, v, tables, lens, block


def sdpa_decode(q, k, v, tables, lens, block):
    """Independent formulation: dense gather + torch SDPA (fp32)."""
    out = []
    group = q.shape[1] // k.shape[2]
    for b, n in enumerate(lens.tolist()):
        ids = tables[b, :math.ceil(n / block)]
        kk = k[ids].reshape(-1, k.shape[2], k.shape[3])[:n].repeat_interleave(group, 1).float().transpose(0, 1)
        vv = v[ids].reshape(-1, v.shape[2], v.shape[3])[:n].repeat_interleave(group, 1).float().transpose(0, 1)
        out.append(F.scaled_dot_product_attention(q[b].float().unsqueeze(1), kk, vv).squeeze(1))
    return torch.stack(out)


# ---------------------------------------------------------------------------
# make_case: published SHA-256 manifest (reports/data/engine_comparison_20261026.json)
# ---------------------------------------------------------------------------

MANIFEST = json.loads((GOLDEN / "make_case_manifest.json").read_text())["cases"]


@pytest.mark.parametrize("case", MANIFEST, ids=lambda c: f"B{c['shape']['batch']}_ctx{c['shape']['context']}")
def test_make_case_reproduces_published_query_table_and_lengths(case):
    shape = case["shape"]
    _, manifest = po.make_case(shape["batch"], shape["context"], heads=shape["heads"], kv_heads=shape["kv_heads"],
                               head_dim=shape["head_dim"], block_size=shape["block_size"], seed=shape["seed"])
    for name in ("query", "block_tables", "context_lens"):
        assert manifest["tensors"][name] == case["tensors"][name], name
    for name in ("key_cache", "value_cache"):
        assert manifest["tensors"][name]["shape"] == case["tensors"][name]["shape"]
        assert manifest["tensors"][name]["dtype"] == case["tensors"][name]["dtype"]


@pytest.mark.xfail(strict=False, reason="torch CPU randn for large tensors differs between the reference's "
                   "Windows torch 2.9.1 build and this torch 2.10 build; query (2K values), tables and lengths "
                   "match byte-for-byte, the 2M+-value K/V caches do not")
def test_make_case_reproduces_published_kv_hashes():
    case = MANIFEST[0]
    _, manifest = po.make_case(1, 128)
    assert manifest["tensors"]["key_cache"]["sha256"] == case["tensors"]["key_cache"]["sha256"]


def test_make_case_is_deterministic_private_and_non_contiguous():
    """tests/test_paged_comparison.py:12-26 restated."""
    state = torch.random.get_rng_state().clone()
    first, a = po.make_case(3, 11, heads=4, kv_heads=2, head_dim=16, block_size=4)
    po.make_case(1, 3, heads=4, kv_heads=2, head_dim=16, block_size=4)
    second, b = po.make_case(3, 11, heads=4, kv_heads=2, head_dim=16, block_size=4)
    assert a == b and torch.equal(state, torch.random.get_rng_state())
    for name in po.TENSOR_NAMES:
        assert torch.equal(first[name], second[name])
    table = first["block_tables"]
    assert table.unique().numel() == table.numel()
    assert not torch.equal(table.flatten(), torch.arange(table.numel()))
    _, other = po.make_case(3, 11, heads=4, kv_heads=2, head_dim=16, block_size=4, seed=4)
    assert a["case_sha256"] != other["case_sha256"]


# ---------------------------------------------------------------------------
# Decode
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("seed", [0, 1, 2])
def test_fp32_oracle_matches_dense_sdpa(seed):
    args = small_case(seed)
    tensors = dict(zip(po.TENSOR_NAMES, args[:5]))
    torch.testing.assert_close(po.fp32_oracle(tensors, args[5]), sdpa_decode(*args), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_torch_decode_path_matches_c_float64(dtype):
    args = small_case(5, dtype=dtype, lengths=(9, 16, 3))
    torch_path = po.paged_attention(*args)
    c_path = c_oracle.paged_decode(*args)
    tol = 2e-3 if dtype == torch.float16 else 1.6e-2  # one rounding to the dtype
    assert (torch_path.double() - c_path).abs().max().item() <= tol
    fp32 = po.fp32_oracle(dict(zip(po.TENSOR_NAMES, args[:5])), args[5])
    assert (fp32.double() - c_path).abs().max().item() <= 1e-5


def test_single_token_context_is_first_value_row():
    q, k, v, tables, _, block = small_case(3, lengths=(1, 1, 1))
    lens = torch.ones(3, dtype=torch.int64)
    out = po.fp32_oracle(dict(zip(po.TENSOR_NAMES, (q, k, v, tables, lens))), block)
    for b in range(3):
        want = v[tables[b, 0], 0].float().repeat_interleave(q.shape[1] // k.shape[2], 0)
        assert torch.equal(out[b], want)


def test_equal_keys_give_mean_of_values():
    q, k, v, tables, lens, block = small_case(4)
    k = torch.ones_like(k)
    out = c_oracle.paged_decode(q, k, v, tables, lens, block)
    for b, n in enumerate(lens.tolist()):
        ids = tables[b, :math.ceil(n / block)]
        mean = v[ids].reshape(-1, v.shape[2], v.shape[3])[:n].double().mean(0)
        want = mean.repeat_interleave(q.shape[1] // k.shape[2], 0)
        assert torch.allclose(out[b], want, atol=1e-12)


def test_page_permutation_invariance():
    """Relabelling physical pages (and the tables with them) changes nothing."""
    q, k, v, tables, lens, block = small_case(6)
    perm = torch.randperm(k.shape[0], generator=torch.Generator().manual_seed(1))
    inverse = torch.empty_like(perm)
    inverse[perm] = torch.arange(perm.numel())
    k2, v2 = k[perm], v[perm]            # new page i holds old page perm[i]
    tables2 = inverse[tables]            # old page p now lives at inverse[p]
    a = po.fp32_oracle(dict(zip(po.TENSOR_NAMES, (q, k, v, tables, lens))), block)
    b = po.fp32_oracle(dict(zip(po.TENSOR_NAMES, (q, k2, v2, tables2, lens))), block)
    assert torch.equal(a, b)


def test_torch_path_rejects_bad_lengths_and_shapes():
    q, k, v, tables, lens, block = small_case(0)
    with pytest.raises(ValueError, match="context length"):
        po.paged_attention(q, k, v, tables, torch.zeros_like(lens), block)
    with pytest.raises(ValueError, match="divisible"):
        po.paged_attention(q[:, :7], k, v, tables, lens, block)


def test_validate_output_rejects_offset_and_nan():
    args = small_case(2)
    oracle = po.fp32_oracle(dict(zip(po.TENSOR_NAMES, args[:5])), args[5])
    assert po.validate_output(oracle.half(), oracle)["passed"]
    assert not po.validate_output(oracle + 1, oracle)["passed"]
    poisoned = oracle.clone()
    poisoned[0, 0, 0] = float("nan")
    assert not po.validate_output(poisoned, oracle)["passed"]


# ---------------------------------------------------------------------------
# Prefill
# ---------------------------------------------------------------------------

def prefill_case(seed=631, dim=16, dtype=torch.float32):
    """The reference's packed case (tests/test_ragged_kernels.py:17-24)."""
    gen = torch.Generator().manual_seed(seed)
    key = torch.randn(8, 4, 2, dim, generator=gen).to(dtype)
    value = torch.randn(8, 4, 2, dim, generator=gen).to(dtype)
    q = torch.randn(8, 4, dim, generator=gen).to(dtype)
    meta = [torch.tensor(x, dtype=torch.int64) for x in ([0, 3, 8], [5, 1], [[5, 1, -1], [2, 7, -1]], [8, 6])]
    return (q, key, value, *meta)


def per_token_einsum_oracle(q, kc, vc, offsets, starts, tables, lengths, block):
    """The reference test's explicit per-token oracle (test_ragged_kernels.py:27-38)."""
    result = []
    for request, (begin, end) in enumerate(zip(offsets.tolist(), offsets.tolist()[1:])):
        for token in range(begin, end):
            context = starts[request].item() + token - begin + 1
            logical = torch.arange(context)
            physical = tables[request, logical // block]
            key = kc[physical, logical % block].repeat_interleave(q.shape[1] // kc.shape[2], dim=1).float()
            value = vc[physical, logical % block].repeat_interleave(q.shape[1] // kc.shape[2], dim=1).float()
            score = torch.einsum("hd,thd->ht", q[token].float(), key) / q.shape[-1] ** 0.5
            result.append(torch.einsum("ht,thd->hd", score.softmax(-1), value))
    return torch.stack(result)


def test_prefill_oracle_matches_per_token_einsum_and_c():
    args = prefill_case()
    got = po.paged_prefill_attention(*args, 4, cast=False)
    torch.testing.assert_close(got, per_token_einsum_oracle(*args, 4), atol=1e-6, rtol=1e-5)
    assert (got.double() - c_oracle.paged_prefill(*args, 4)).abs().max().item() <= 1e-5


def test_prefill_from_zero_is_dense_causal_sdpa():
    gen = torch.Generator().manual_seed(9)
    block, n, heads, kv_heads, dim = 4, 11, 4, 2, 8
    k = torch.randn(6, block, kv_heads, dim, generator=gen)
    v = torch.randn(6, block, kv_heads, dim, generator=gen)
    q = torch.randn(n, heads, dim, generator=gen)
    tables = torch.tensor([[4, 0, 2]])
    out = po.paged_prefill_attention(q, k, v, torch.tensor([0, n]), torch.tensor([0]), tables, torch.tensor([n]),
                                      block, cast=False)
    kk = k[tables[0]].reshape(-1, kv_heads, dim)[:n].repeat_interleave(2, 1).transpose(0, 1)
    vv = v[tables[0]].reshape(-1, kv_heads, dim)[:n].repeat_interleave(2, 1).transpose(0, 1)
    dense = F.scaled_dot_product_attention(q.transpose(0, 1), kk, vv, is_causal=True).transpose(0, 1)
    torch.testing.assert_close(out, dense, atol=1e-6, rtol=1e-5)


def test_one_token_chunk_reduces_to_decode():
    q, k, v, tables, lens, block = small_case(8, dtype=torch.float32)
    b = q.shape[0]
    cu = torch.arange(b + 1, dtype=torch.int64)
    pre = po.paged_prefill_attention(q, k, v, cu, lens - 1, tables, lens, block, cast=False)
    dec = po.fp32_oracle(dict(zip(po.TENSOR_NAMES, (q, k, v, tables, lens))), block)
    torch.testing.assert_close(pre, dec, atol=1e-6, rtol=1e-5)


def dense_as_paged(q, k, v, query_start, block, seed=0):
    """The dense prefill's inputs laid out for the paged prefill: each batch
    entry a sequence whose keys sit in shuffled pages of `block` tokens."""
    batch, q_heads, tokens, dim = q.shape
    kv_heads, kv_tokens = k.shape[1], k.shape[2]
    context = query_start + tokens
    width = -(-context // block)
    pages = torch.randperm(batch * width + 3, generator=torch.Generator().manual_seed(seed))
    kc = torch.zeros(batch * width + 3, block, kv_heads, dim, dtype=k.dtype)
    vc = torch.zeros_like(kc)
    tables = pages[:batch * width].view(batch, width).clone()
    for b in range(batch):
        for t in range(context):
            kc[tables[b, t // block], t % block] = k[b, :, t]
            vc[tables[b, t // block], t % block] = v[b, :, t]
    packed = q.transpose(1, 2).reshape(batch * tokens, q_heads, dim)
    meta = [torch.arange(0, batch * tokens + 1, tokens), torch.full((batch,), query_start),
            tables, torch.full((batch,), context)]
    return packed, kc, vc, meta


def dense_case(seed, batch=2, q_heads=4, kv_heads=2, tokens=5, kv_tokens=13, dim=16):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(batch, q_heads, tokens, dim, generator=gen),
            torch.randn(batch, kv_heads, kv_tokens, dim, generator=gen),
            torch.randn(batch, kv_heads, kv_tokens, dim, generator=gen))


@pytest.mark.parametrize("query_start,tokens,kv_tokens", [(6, 5, 13), (8, 3, 11), (0, 9, 9), (0, 4, 10)])
def test_dense_prefill_oracle_matches_paged_c_float64(query_start, tokens, kv_tokens):
    """The dense path (prefill.py:42-60) equals the float64 C restatement of
    the paged path on the same rows, laid into shuffled pages: mask start,
    GQA mapping and the keys past query_start + T (never visible) agree."""
    q, k, v = dense_case(query_start * 31 + tokens, tokens=tokens, kv_tokens=kv_tokens)
    got = po.prefill_attention(q, k, v, query_start=query_start, cast=False)
    packed, kc, vc, meta = dense_as_paged(q, k, v, query_start, 4)
    want = c_oracle.paged_prefill(packed, kc, vc, *meta, 4)
    got_packed = got.transpose(1, 2).reshape(packed.shape).double()
    assert (got_packed - want).abs().max().item() <= 1e-5


def test_dense_prefill_square_is_row_by_row_softmax():
    """Brute force in float64: each query row's softmax over keys 0..t."""
    q, k, v = dense_case(5, batch=1, q_heads=2, kv_heads=1, tokens=4, kv_tokens=4, dim=8)
    got = po.prefill_attention(q, k, v, cast=False).double()
    qd, kd, vd = q.double(), k.double(), v.double()
    for h in range(2):
        for t in range(4):
            scores = [float(qd[0, h, t] @ kd[0, 0, j]) / math.sqrt(8) for j in range(t + 1)]
            top = max(scores)
            weights = [math.exp(x - top) for x in scores]
            row = sum(w * vd[0, 0, j] for j, w in enumerate(weights)) / sum(weights)
            assert (got[0, h, t] - row).abs().max().item() <= 1e-6


def test_planted_dense_gqa_mistake_is_caught():
    """Heads mapped by tiling (h % kv_heads) instead of h // group."""
    q, k, v = dense_case(7, tokens=5, kv_tokens=13)
    wrong = po.prefill_attention(q, k.repeat(1, 2, 1, 1), v.repeat(1, 2, 1, 1), query_start=6, cast=False)
    packed, kc, vc, meta = dense_as_paged(q, k, v, 6, 4)
    want = c_oracle.paged_prefill(packed, kc, vc, *meta, 4)
    assert (wrong.transpose(1, 2).reshape(packed.shape).double() - want).abs().max().item() > 1e-3


# ---------------------------------------------------------------------------
# KV writes / gather (bit-exact)
# ---------------------------------------------------------------------------

def test_slot_scatter_matches_index_put_and_c_and_keeps_other_rows():
    """tests/test_ragged_kernels.py:48-59 restated."""
    _, key, value, *_ = prefill_case(dtype=torch.float16)
    original_k, original_v = key.clone(), value.clone()
    slots = torch.tensor([5, 6, 7, 9, 10, 11, 28, 29], dtype=torch.int64)
    packed = torch.randn(8, 4, 16, generator=torch.Generator().manual_seed(1)).half()
    source_k, source_v = packed[:, :2].contiguous(), packed[:, 2:].contiguous()
    c_k, c_v = c_oracle.scatter_slots(key, value, slots, source_k, source_v)
    po.write_kv_cache_slots(key, value, slots, source_k, source_v)
    expected_k, expected_v = original_k.view(-1, 2, 16).clone(), original_v.view(-1, 2, 16).clone()
    expected_k[slots], expected_v[slots] = source_k, source_v
    assert torch.equal(key.view_as(expected_k), expected_k) and torch.equal(value.view_as(expected_v), expected_v)
    assert torch.equal(c_k, key) and torch.equal(c_v, value)
    untouched = torch.ones(32, dtype=torch.bool)
    untouched[slots] = False
    assert torch.equal(key.view(-1, 2, 16)[untouched], original_k.view(-1, 2, 16)[untouched])


def test_range_and_batch_writes_equal_slot_scatter():
    gen = torch.Generator().manual_seed(2)
    block, pages = 4, 6
    kc = torch.randn(pages, block, 2, 8, generator=gen).half()
    vc = torch.randn(pages, block, 2, 8, generator=gen).half()
    ids = torch.tensor([4, 1, 5])
    key = torch.randn(7, 2, 8, generator=gen).half()
    value = torch.randn(7, 2, 8, generator=gen).half()
    a_k, a_v = kc.clone(), vc.clone()
    po.write_kv_cache(a_k, a_v, ids, 1, key, value, block)
    positions = torch.arange(1, 8)
    slots = ids[positions // block] * block + positions % block
    b_k, b_v = c_oracle.scatter_slots(kc, vc, slots, key, value)
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)
    # Batch write: one token per sequence at its offset.
    tables = torch.tensor([[4, 1], [0, 3]])
    offsets = torch.tensor([5, 2])
    c_k, c_v = kc.clone(), vc.clone()
    po.write_kv_cache_batch(c_k, c_v, tables, offsets, key[:2], value[:2], block)
    slots = torch.stack([tables[i, offsets[i] // block] * block + offsets[i] % block for i in range(2)])
    d_k, d_v = c_oracle.scatter_slots(kc, vc, slots, key[:2], value[:2])
    assert torch.equal(c_k, d_k) and torch.equal(c_v, d_v)


def test_gather_matches_per_token_lookup():
    """tests/test_kv_cache.py:6-13 restated: page-crossing write then gather."""
    kc = torch.zeros(3, 4, 2, 2)
    vc = torch.zeros(3, 4, 2, 2)
    key = torch.arange(12, dtype=torch.float32).reshape(3, 2, 2)
    po.write_kv_cache(kc, vc, torch.tensor([2, 0]), 3, key, key + 100, 4)
    got_k, got_v = po.gather(kc, vc, [2, 0], 6)
    assert torch.equal(got_k[3:6], key) and torch.equal(got_v[3:6], key + 100)
    for t in range(6):
        page = [2, 0][t // 4]
        assert torch.equal(got_k[t], kc[page, t % 4])


# ---------------------------------------------------------------------------
# Element conversions of the C oracle (exhaustive)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_c_conversions_match_torch_for_every_bit_pattern(dtype):
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    values = bits.view(dtype)
    ours = c_oracle.to_float32(values)
    ref = values.float()
    same = (ours == ref) | (torch.isnan(ours) & torch.isnan(ref))
    assert bool(same.all())


# ---------------------------------------------------------------------------
# Prefill metadata: reference known-answer test (tests/test_ragged_model.py:42-53)
# ---------------------------------------------------------------------------

def test_prefill_metadata_known_answer():
    meta = po.prefill_metadata([[5, 6, 7], [8, 9]], [[3, 1, -1], [3, 2]], [4, 4], 4)
    assert meta["positions"] == [4, 5, 6, 4, 5]
    assert meta["slot_mapping"] == [4, 5, 6, 8, 9]
    assert meta["cu_seqlens_q"] == [0, 3, 5]
    assert meta["context_lens"] == [7, 6]
    slots = c_oracle.prefill_slots(torch.tensor([0, 3, 5]), torch.tensor([4, 4]),
                                   torch.tensor([[3, 1], [3, 2]]), 4)
    assert slots.tolist() == [4, 5, 6, 8, 9]


# ---------------------------------------------------------------------------
# Planted mistakes: each check above fails for a plausible wrong oracle.
# ---------------------------------------------------------------------------

def _mutant_decode(q, k, v, tables, lens, block, *, mistake):
    out = []
    group = q.shape[1] // k.shape[2]
    for b, n in enumerate(lens.tolist()):
        ids = tables[b, :math.ceil(n / block)]
        kk = k[ids].reshape(-1, k.shape[2], k.shape[3])[:n].float()
        vv = v[ids].reshape(-1, v.shape[2], v.shape[3])[:n].float()
        if mistake == "gqa_tile":      # heads mapped h % Hkv instead of h // G
            kk, vv = kk.repeat(1, group, 1), vv.repeat(1, group, 1)
        else:
            kk, vv = kk.repeat_interleave(group, 1), vv.repeat_interleave(group, 1)
        scale = 1 / q.shape[-1] if mistake == "scale" else 1 / math.sqrt(q.shape[-1])
        if mistake == "drop_last":     # off-by-one context
            kk, vv = kk[:-1] if n > 1 else kk, vv[:-1] if n > 1 else vv
        s = torch.einsum("hd,thd->ht", q[b].float(), kk) * scale
        out.append(torch.einsum("ht,thd->hd", s.softmax(-1), vv))
    return torch.stack(out)


@pytest.mark.parametrize("mistake", ["gqa_tile", "scale", "drop_last"])
def test_planted_decode_mistakes_are_caught(mistake):
    args = small_case(11)
    wrong = _mutant_decode(*args, mistake=mistake)
    assert (wrong.double() - c_oracle.paged_decode(*args)).abs().max().item() > 1e-3
    assert (wrong - sdpa_decode(*args)).abs().max().item() > 1e-3


def test_planted_prefill_mask_mistake_is_caught():
    q, kc, vc, offsets, starts, tables, lengths = prefill_case()
    # Strict mask (key < position) instead of key <= position.
    out = torch.empty(q.shape)
    for i, (start, length) in enumerate(zip(starts.tolist(), lengths.tolist())):
        begin, end = offsets[i].item(), offsets[i + 1].item()
        pages = tables[i, :(length + 3) // 4]
        key = kc[pages].reshape(-1, 2, 16)[:length].repeat_interleave(2, 1).transpose(0, 1)
        value = vc[pages].reshape(-1, 2, 16)[:length].repeat_interleave(2, 1).transpose(0, 1)
        mask = torch.arange(length)[None, :] < (start + torch.arange(end - begin)[:, None])
        mask[:, 0] = True
        out[begin:end] = F.scaled_dot_product_attention(q[begin:end].transpose(0, 1), key, value,
                                                        attn_mask=mask).transpose(0, 1)
    assert (out.double() - c_oracle.paged_prefill(q, kc, vc, offsets, starts, tables, lengths, 4)).abs().max() > 1e-3


# --- fused q/k RMSNorm + RoPE + KV write --------------------------------------------------------

def _f16_rope_loops(x, cos, sin):
    """Per-element numpy float16 scalar arithmetic: every product and sum rounded to fp16."""
    import numpy as np
    x, cos, sin = (t.numpy() for t in (x, cos, sin))
    half = x.shape[-1] // 2
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        for h in range(x.shape[1]):
            for p in range(half):
                a, b, c, s = x[t, h, p], x[t, h, p + half], cos[t, p], sin[t, p]
                out[t, h, p] = np.float16(a * c) - np.float16(b * s)
                out[t, h, p + half] = np.float16(a * s) + np.float16(b * c)
    return torch.from_numpy(out)


def _rope_case(seed=3, tokens=5, heads=4, kv_heads=2, dim=16, dtype=torch.float16):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(tokens, heads, dim, generator=gen).to(dtype)
    k = torch.randn(tokens, kv_heads, dim, generator=gen).to(dtype)
    angles = torch.randn(tokens, dim // 2, generator=gen) * 3
    return q, k, angles.cos().to(dtype), angles.sin().to(dtype)


def test_rope_identity_and_quarter_turn_closed_forms():
    q, k, cos, sin = _rope_case()
    ones, zeros = torch.ones_like(cos), torch.zeros_like(sin)
    rq, rk = po.apply_rope(q, k, ones.unsqueeze(1), zeros.unsqueeze(1))
    assert torch.equal(rq, q) and torch.equal(rk, k)
    # cos = 0, sin = 1 rotates each (x1, x2) pair by 90 degrees: (-x2, x1).
    rq, rk = po.apply_rope(q, k, zeros.unsqueeze(1), ones.unsqueeze(1))
    assert torch.equal(rq, torch.cat((-q[..., 8:], q[..., :8]), -1))
    assert torch.equal(rk, torch.cat((-k[..., 8:], k[..., :8]), -1))


def test_rope_rounding_matches_float16_scalar_arithmetic():
    q, k, cos, sin = _rope_case(seed=9)
    rq, rk = po.apply_rope(q, k, cos.unsqueeze(1), sin.unsqueeze(1))
    assert torch.equal(rq, _f16_rope_loops(q, cos, sin))
    assert torch.equal(rk, _f16_rope_loops(k, cos, sin))
    # Planted mistake: rounding only the finished sum (fp32 products) is not the reference's arithmetic.
    half = 8
    q1, q2 = q[..., :half].float(), q[..., half:].float()
    c, s = cos.float().unsqueeze(1), sin.float().unsqueeze(1)
    fused = torch.cat((q1 * c - q2 * s, q1 * s + q2 * c), -1).half()
    assert not torch.equal(fused, rq)


def test_rms_norm_constant_rows_and_float64():
    dim = 16
    weight = (torch.arange(dim, dtype=torch.float32) / 8 - 1).half()   # distinct per-element weights
    # A constant row c normalises to sign(c) / sqrt(1 + eps / c^2): with eps = 3, c = 1 that is 1/2.
    x = torch.ones(1, dim, dtype=torch.float16)
    assert torch.equal(po.rms_norm(x, weight, eps=3.0)[0], (weight.float() * 0.5).half())
    x = torch.full((1, dim), -2.0, dtype=torch.float16)
    assert torch.equal(po.rms_norm(x, weight, eps=1e-6)[0], -weight)
    # Random rows against a float64 restatement (mean, not sum; weight per element).
    gen = torch.Generator().manual_seed(4)
    x = (torch.randn(6, 3, dim, generator=gen) * 4).half()
    x64 = x.double()
    inv = 1 / torch.sqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6)
    expected = (x64 * inv).half().double() * weight.double()
    assert torch.allclose(po.rms_norm(x, weight).double(), expected, atol=2e-3, rtol=1e-3)
    # Planted mistake: sum instead of mean fails the constant-row closed form.
    wrong = (x[:1, 0].float() * torch.rsqrt(x[:1, 0].float().pow(2).sum(-1, keepdim=True) + 1e-6)).half() * weight
    assert not torch.allclose(wrong.double(), expected[:1, 0], atol=2e-3, rtol=1e-3)


def test_fused_oracle_writes_the_slots_of_the_batch_rules():
    gen = torch.Generator().manual_seed(12)
    tokens, heads, kv_heads, dim, block, pages = 4, 4, 2, 16, 4, 6
    q, k, cos, sin = _rope_case(seed=12, tokens=tokens, heads=heads, kv_heads=kv_heads, dim=dim)
    v = torch.randn(tokens, kv_heads, dim, generator=gen).half()
    wq, wk = torch.rand(dim, generator=gen).half() + 0.5, torch.rand(dim, generator=gen).half() + 0.5
    kc = torch.randn(pages, block, kv_heads, dim, generator=gen).half()
    vc = torch.randn(pages, block, kv_heads, dim, generator=gen).half()
    tables = torch.tensor([[3, 1], [0, 5], [2, 4], [-1, 1]], dtype=torch.int64)
    positions = torch.tensor([5, 0, 9, 2], dtype=torch.int64)   # token 2 beyond capacity, token 3 on page -1
    kd, vd = kc.clone(), vc.clone()
    qd = po.qk_norm_rope_write_kv(q, k, v, wq, wk, cos, sin, kd, vd, block_tables=tables, positions=positions)
    nq, nk = po.apply_rope(po.rms_norm(q, wq), po.rms_norm(k, wk), cos.unsqueeze(1), sin.unsqueeze(1))
    assert torch.equal(qd, nq)
    ke, ve = kc.clone(), vc.clone()
    po.write_kv_cache_batch(ke, ve, tables[:2], positions[:2], nk[:2], v[:2], block)
    assert torch.equal(kd, ke) and torch.equal(vd, ve)
    # Slot mode: the same two rows through explicit slots, the invalid ones marked -1 / out of range.
    ks, vs = kc.clone(), vc.clone()
    slots = torch.tensor([1 * block + 1, 0, -1, pages * block], dtype=torch.int64)
    qs = po.qk_norm_rope_write_kv(q, k, v, wq, wk, cos, sin, ks, vs, slot_mapping=slots)
    assert torch.equal(qs, qd) and torch.equal(ks, kd) and torch.equal(vs, vd)


# --- greedy sampling ------------------------------------------------------------------------------

def _argmax_loops(x):
    """First NaN of a row, else the first index of its maximum (-0.0 == +0.0)."""
    out = []
    for row in x.float().tolist():
        nan = [i for i, v in enumerate(row) if v != v]
        if nan:
            out.append(nan[0])
            continue
        best = max(row)
        out.append(next(i for i, v in enumerate(row) if v == best))
    return torch.tensor(out, dtype=torch.int64)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("vocab", [1, 257, 4097])
def test_greedy_oracle_ties_nan_inf_and_tail(dtype, vocab):
    """The reference's sampling cases (tests/test_cuda_sampling.py:16-25) against plain loops."""
    gen = torch.Generator().manual_seed(29)
    x = torch.randn(6, vocab, generator=gen).to(dtype)
    x[0].fill_(float("-inf"))
    x[1].fill_(1)
    x[2, -1] = float("inf")
    x[3, -1] = float("nan")
    x[3, 0] = float("nan")
    x[4, -1] = 99
    x[5].fill_(0)
    x[5, vocab // 2:] = -0.0
    assert torch.equal(po.greedy_argmax(x), _argmax_loops(x))
