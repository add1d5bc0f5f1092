"""The paged prefill walk's chunk choice on the device (choose_chunk in
paged_prefill.hip).

Every chunk length gives a correct result, so the outputs alone cannot show
which chunk the device took.  Two checks pin it:

* the chunk count that the first item of each query block records for every
  token of the block (an int per packed token, the workspace's last region)
  equals the count of the chunk that a host restatement of the cost model
  picks;
* the call gives the same bits as a call given that chunk explicitly.

The model (restated from the kernel), with K keys per tile (64 for head
dims up to 128, 32 above) and query blocks of 256 rows (128 above 128):
candidates are the host's chunk max(512, capacity/32 rounded up to K keys)
plus multiples of K*step keys, 128 of them (512 with fewer than 16 query
blocks) up to the capacity; each costs
max(ceil(items/W) * (F + chunk/K), (tiles + F * items) / W) in fp32 with
F = 5 * 64 / K tiles and W = 256 / kv_heads work-groups per kv head; the
cheapest wins, ties going to the smaller chunk.  The choice is made only when
the host's chunk gives more than one round of items.
"""

import numpy as np
import pytest
import torch

from mini_engine_hip import workloads
from mini_engine_hip.kernels import hip_extension as ext
from mini_engine_hip.kernels.prefill import paged_prefill_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"
CUS = 256
KEYS = 64
NAMES = ("q", "key_cache", "value_cache", "cu_seqlens_q", "query_starts", "block_tables", "context_lens")
PRIORS8 = [2220, 601, 877, 1126, 1381, 3550, 2532, 347]


def ceil_div(a, b):
    return -(-a // b)


def block_ends(priors, new_tokens, qb, cap):
    return [min(p + min(q0 + qb, new_tokens), cap) for p in priors for q0 in range(0, new_tokens, qb)]


def model_chunk(priors, new_tokens, block_size, table_width, q_heads, kv_heads, head_dim=128):
    keys = KEYS if head_dim <= 128 else KEYS // 2
    fixed = np.float32(5.0 * 64 / keys)
    qb = (256 if head_dim <= 128 else 128) // (q_heads // kv_heads)
    cap = table_width * block_size
    host = max(512, ceil_div(ceil_div(cap, 32), keys) * keys)
    cmax = ceil_div(cap, keys) * keys
    ends = block_ends(priors, new_tokens, qb, cap)
    cands = 512 if len(priors) <= 64 and len(ends) < 16 else 128
    step = max(1, ceil_div((cmax - host) // keys, cands))
    w = max(1, CUS // kv_heads)

    def items(c):
        return sum(ceil_div(e, c) if e > 0 else 1 for e in ends)

    if items(host) <= w:
        return host, False
    tiles = sum(ceil_div(e, keys) for e in ends)
    best = None
    for i in range(cands):
        c = host + keys * step * i
        if c > cmax:
            break
        n = items(c)
        rounds = np.float32(ceil_div(n, w))
        cost = max(rounds * (fixed + np.float32(c // keys)),
                   (np.float32(tiles) + fixed * np.float32(n)) / np.float32(w))
        if best is None or cost < best[0]:
            best = (cost, c)
    return best[1], True


@pytest.mark.parametrize("num_seqs,new_tokens,priors", [
    (1, 2048, [0]),
    (1, 4096, [0]),          # 832 and 1408 tie in the model: the smaller wins
    (2, 2048, [0, 1000]),
    (8, 512, PRIORS8),
    (16, 256, None),
    (1, 512, [16000]),       # 4 blocks: 512 candidates, one per 64 keys
    (4, 128, [8000, 12000, 3000, 30000]),  # 512 candidates take 1792 (128 would step by 256 keys: 1984)
    (2, 1024, [20000, 40000]),  # 16 blocks: 128 candidates stepping by 320 keys
])
def test_device_choice_matches_the_model(num_seqs, new_tokens, priors):
    c = workloads.chunked_prefill_case(device=torch.device(DEV), num_seqs=num_seqs, new_tokens=new_tokens,
                                       priors=priors)
    args = [c[n] for n in NAMES]
    q, kc = c["q"], c["key_cache"]
    priors = c["priors"]
    tokens, q_heads = q.shape[0], q.shape[1]
    _, block_size, kv_heads, head_dim = kc.shape
    width = c["block_tables"].shape[1]
    want, chose = model_chunk(priors, new_tokens, block_size, width, q_heads, kv_heads)
    print(f"chunk choice {num_seqs}x{new_tokens}: model {want} (choice made: {chose})", flush=True)
    assert chose, "shape must need more than one round of items at the host's chunk"

    check_choice(args, priors, new_tokens, want)


def check_choice(args, priors, new_tokens, want):
    """The device's chunk counts are those of `want`, and the call equals one given `want`."""
    q, kc, tables = args[0], args[1], args[5]
    tokens, q_heads = q.shape[0], q.shape[1]
    _, block_size, kv_heads, head_dim = kc.shape
    width = tables.shape[1]
    lib = ext.load_hip_extension()
    need = lib.prefill_workspace_size(len(priors), tokens, q_heads, kv_heads, head_dim, block_size, width, 0,
                                      ext.dtype_code(q.dtype))
    workspace = torch.zeros(need, dtype=torch.uint8, device=DEV)
    auto = paged_prefill_attention(*args, block_size, backend="hip", validate=False, workspace=workspace)
    explicit = paged_prefill_attention(*args, block_size, backend="hip", validate=False, chunk_tokens=want)
    torch.cuda.synchronize()

    tok_bytes = (tokens * 4 + 15) // 16 * 16
    counts = workspace[need - tok_bytes:need - tok_bytes + tokens * 4].cpu().view(torch.int32).tolist()
    qb = (256 if head_dim <= 128 else 128) // (q_heads // kv_heads)
    expected = []
    for p in priors:
        for t in range(new_tokens):
            end = min(p + min(t // qb * qb + qb, new_tokens), width * block_size)
            expected.append(ceil_div(end, want))
    assert counts == expected
    assert torch.equal(auto, explicit)


def test_head_dim_256_tiles_of_32_keys():
    """Head dim 256: 32-key tiles (an item's fixed cost is 10 of them) and
    query blocks of 128 rows (64 tokens at GQA 2).  One 2048-token prompt,
    Hq8/Hkv4: 80 items at the host's 512-key chunk against 64 work-groups
    per kv head, so the device chooses."""
    gen = torch.Generator().manual_seed(256)
    tokens, q_heads, kv_heads, head_dim, block = 2048, 8, 4, 256, 256
    pages = tokens // block
    perm = torch.randperm(pages + 3, generator=gen)[:pages]
    tables = perm.view(1, pages).to(torch.int64)
    kc = torch.randn(pages + 3, block, kv_heads, head_dim, generator=gen).to(torch.bfloat16)
    vc = torch.randn(pages + 3, block, kv_heads, head_dim, generator=gen).to(torch.bfloat16)
    q = torch.randn(tokens, q_heads, head_dim, generator=gen).to(torch.bfloat16)
    meta = (torch.tensor([0, tokens]), torch.tensor([0]), tables, torch.tensor([tokens]))
    args = [t.to(DEV) for t in (q, kc, vc, *meta)]
    want, chose = model_chunk([0], tokens, block, pages, q_heads, kv_heads, head_dim)
    print(f"chunk choice D=256 1x{tokens}: model {want} (choice made: {chose})", flush=True)
    assert chose
    check_choice(args, [0], tokens, want)


@pytest.mark.parametrize("batch", [1, 2])
def test_dense_prefill_chooses_like_the_paged_walk(batch):
    """prefill_attention's dense mode: each batch entry is a sequence whose
    keys are one page of the context rounded up to a power of two (2048
    here), and the walk chooses its chunk by the same model."""
    from mini_engine_hip.kernels.prefill import prefill_attention

    tokens, q_heads, kv_heads, head_dim = 2048, 16, 8, 128
    gen = torch.Generator().manual_seed(batch)
    q = torch.randn(batch, q_heads, tokens, head_dim, generator=gen).to(torch.bfloat16).to(DEV)
    k = torch.randn(batch, kv_heads, tokens, head_dim, generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn(batch, kv_heads, tokens, head_dim, generator=gen).to(torch.bfloat16).to(DEV)
    want, chose = model_chunk([0] * batch, tokens, tokens, 1, q_heads, kv_heads)
    print(f"dense chunk choice {batch}x{tokens}: model {want} (choice made: {chose})", flush=True)
    assert chose
    lib = ext.load_hip_extension()
    need = lib.dense_prefill_workspace_size(batch, tokens, q_heads, kv_heads, head_dim, 0, ext.dtype_code(q.dtype))
    workspace = torch.zeros(need, dtype=torch.uint8, device=DEV)
    prefill_attention(q, k, v, "hip", workspace=workspace)
    torch.cuda.synchronize()
    rows = batch * tokens
    tok_bytes = (rows * 4 + 15) // 16 * 16
    counts = workspace[need - tok_bytes:need - tok_bytes + rows * 4].cpu().view(torch.int32).tolist()
    qb = 256 // (q_heads // kv_heads)
    expected = [ceil_div(min(t // qb * qb + qb, tokens), want) for _ in range(batch) for t in range(tokens)]
    assert counts == expected
