"""A decode step captured as a graph bucket, replayed with new metadata.

Restates the capture/replay contract of the reference's decode graph bucket
(mini_engine/engine/cuda_graph.py:196-222 capture, :244-275 replay) for the
hip path, without the model around it: per layer the new token's K/V write
(``write_kv_cache_batch``, or the fused q/k RMSNorm + RoPE + KV write in
decode mode), then paged attention over ``positions + 1`` tokens — the order
of Attention.forward_decode_batch (mini_engine/model/native_qwen3.py:179-197)
— or all of it in one launch (``paged_attention_decode_write``).

The bucket has a fixed batch; rows past the active count are padding rows
that decode position 0 through a private reserved page (column 0 of their
table; the rest -1), as the reference's padding tables do (cuda_graph.py:66-87,
:188-195).  Capture runs on padding metadata only.  Each replay copies new
positions, tables, q/k/v (and cos/sin) into the captured buffers, then:

* the whole cache after the replay equals the oracle's writes bit for bit
  (scatter mode; K rows within the RoPE tolerance in fused mode), so padding
  rows touched nothing but their own reserved pages;
* active rows' attention matches the fp32 oracle, and padding rows return
  their single value row;
* the same step run eagerly from the same cache state gives bit-identical
  caches and outputs (replays interleaved with eager work and syncs).
"""

import pytest
import torch

from gpu_cases import assert_rope_close
from mini_engine_hip.cache.kv_cache import KVCachePool
from mini_engine_hip.kernels.data import write_kv_cache_batch
from mini_engine_hip.kernels.paged import paged_attention, paged_attention_decode_write
from mini_engine_hip.kernels.rope import qk_norm_rope_write_kv
from oracle import paged_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
BUCKET, LAYERS, BLOCK, HQ, HKV, D = 8, 2, 16, 16, 8, 128
GATE = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


class DecodeBucket:
    """Static buffers + a captured multi-layer decode step."""

    def __init__(self, mode, dtype, width, live_pages):
        self.mode, self.dtype, self.width = mode, dtype, width
        self.live_pages = live_pages
        self.cache = KVCachePool(LAYERS, live_pages + BUCKET, BLOCK, HKV, D, dtype=dtype, device=DEV)
        gen = torch.Generator().manual_seed(width)
        self.cache.key.copy_(torch.randn(self.cache.key.shape, generator=gen).to(dtype))
        self.cache.value.copy_(torch.randn(self.cache.value.shape, generator=gen).to(dtype))
        self.padding_pages = torch.arange(live_pages, live_pages + BUCKET)
        self.padding_tables = torch.full((BUCKET, width), -1, dtype=torch.int64)
        self.padding_tables[:, 0] = self.padding_pages
        self.positions = torch.zeros(BUCKET, dtype=torch.int64, device=DEV)
        self.tables = self.padding_tables.to(DEV)
        self.q = torch.zeros(LAYERS, BUCKET, HQ, D, dtype=dtype, device=DEV)
        self.k = torch.zeros(LAYERS, BUCKET, HKV, D, dtype=dtype, device=DEV)
        self.v = torch.zeros_like(self.k)
        self.cos = torch.ones(BUCKET, D // 2, dtype=dtype, device=DEV)
        self.sin = torch.zeros_like(self.cos)
        self.wq = (torch.rand(D, generator=gen) + 0.5).to(dtype).to(DEV)
        self.wk = (torch.rand(D, generator=gen) + 0.5).to(dtype).to(DEV)
        self.q_rot = torch.empty_like(self.q)
        self.out = torch.empty_like(self.q)
        self.graph = None

    def step(self):
        lengths = self.positions + 1
        for layer in range(LAYERS):
            key_pages, value_pages = self.cache.layer(layer)
            if self.mode == "scatter":
                write_kv_cache_batch(key_pages, value_pages, self.tables, self.positions, self.k[layer],
                                     self.v[layer], BLOCK, backend="hip", validate=False)
                query = self.q[layer]
            elif self.mode == "decode_write":
                # Norm/RoPE, KV write and attention in one launch.
                paged_attention_decode_write(self.q[layer], key_pages, value_pages, self.tables, lengths, BLOCK,
                                             self.k[layer], self.v[layer], q_weight=self.wq, k_weight=self.wk,
                                             cos=self.cos, sin=self.sin, q_out=self.q_rot[layer], validate=False,
                                             out=self.out[layer])
                continue
            else:
                query = qk_norm_rope_write_kv(self.q[layer], self.k[layer], self.v[layer], self.wq, self.wk,
                                              self.cos, self.sin, key_pages, value_pages,
                                              block_tables=self.tables, positions=self.positions,
                                              validate=False, out=self.q_rot[layer])
            paged_attention(query, key_pages, value_pages, self.tables, lengths, BLOCK, backend="hip",
                            validate=False, out=self.out[layer])

    def capture(self, warmup=3):
        self.tables.copy_(self.padding_tables)
        self.positions.zero_()
        for _ in range(warmup):
            self.step()
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.step()

    def stage(self, positions, tables, gen):
        """Copy a new batch into the captured buffers (padding rows reset)."""
        active = len(positions)
        host_pos = torch.zeros(BUCKET, dtype=torch.int64)
        host_pos[:active] = torch.tensor(positions)
        host_tables = self.padding_tables.clone()
        host_tables[:active] = tables
        self.positions.copy_(host_pos)
        self.tables.copy_(host_tables)
        self.q.copy_(torch.randn(self.q.shape, generator=gen).to(self.dtype))
        self.k.copy_(torch.randn(self.k.shape, generator=gen).to(self.dtype))
        self.v.copy_(torch.randn(self.v.shape, generator=gen).to(self.dtype))
        angles = torch.randn(BUCKET, D // 2, generator=gen) * 3
        self.cos.copy_(angles.cos().to(self.dtype))
        self.sin.copy_(angles.sin().to(self.dtype))
        return host_pos, host_tables


def new_batch(bucket, active, gen):
    """Active rows: private live pages, a random decode position, -1 past it."""
    order = torch.randperm(bucket.live_pages, generator=gen)
    positions, tables = [], torch.full((active, bucket.width), -1, dtype=torch.int64)
    for r in range(active):
        pos = int(torch.randint(0, bucket.width * BLOCK, (1,), generator=gen))
        used = pos // BLOCK + 1 + int(torch.randint(0, 2, (1,), generator=gen))
        used = min(used, bucket.width)
        tables[r, :used] = order[r * bucket.width:r * bucket.width + used]
        positions.append(pos)
    return positions, tables


def expected_after(bucket, before_k, before_v, host_pos, host_tables):
    """Oracle writes of every layer on CPU copies of the cache before the replay."""
    exp_k, exp_v, rot_q = before_k.clone(), before_v.clone(), []
    for layer in range(LAYERS):
        q, k, v = bucket.q[layer].cpu(), bucket.k[layer].cpu(), bucket.v[layer].cpu()
        if bucket.mode == "scatter":
            paged_oracle.write_kv_cache_batch(exp_k[layer], exp_v[layer], host_tables, host_pos, k, v, BLOCK)
            rot_q.append(q)
        else:
            rot_q.append(paged_oracle.qk_norm_rope_write_kv(
                q, k, v, bucket.wq.cpu(), bucket.wk.cpu(), bucket.cos.cpu(), bucket.sin.cpu(), exp_k[layer],
                exp_v[layer], block_tables=host_tables, positions=host_pos))
    return exp_k, exp_v, rot_q


@pytest.mark.parametrize("mode", ["scatter", "fused", "decode_write"])
@pytest.mark.parametrize("dtype,width", [(torch.bfloat16, 6), (torch.float16, 80)])
def test_decode_bucket_replays_with_new_metadata_and_padding(mode, dtype, width):
    """width 6 (96 tokens): whole-sequence decode; width 80 (1280 tokens, 8
    sequences): split-K with its workspace and merge inside the graph."""
    print(f"graph bucket mode={mode} dtype={dtype} width={width}", flush=True)
    bucket = DecodeBucket(mode, dtype, width, live_pages=BUCKET * width)
    bucket.capture()
    gen = torch.Generator().manual_seed(100 + width)
    for active in (BUCKET, 5, 3):
        positions, tables = new_batch(bucket, active, gen)
        host_pos, host_tables = bucket.stage(positions, tables, gen)
        torch.cuda.synchronize()
        before_k, before_v = bucket.cache.key.cpu(), bucket.cache.value.cpu()
        bucket.graph.replay()
        torch.cuda.synchronize()
        got_k, got_v = bucket.cache.key.cpu(), bucket.cache.value.cpu()
        got_out, got_q = bucket.out.cpu(), bucket.q_rot.cpu()

        exp_k, exp_v, rot_q = expected_after(bucket, before_k, before_v, host_pos, host_tables)
        assert torch.equal(got_v, exp_v)
        slots = host_tables[torch.arange(BUCKET), host_pos // BLOCK] * BLOCK + host_pos % BLOCK
        if mode == "scatter":
            assert torch.equal(got_k, exp_k)
        else:
            untouched = torch.ones(got_k.shape[1] * BLOCK, dtype=torch.bool)
            untouched[slots] = False
            for layer in range(LAYERS):
                rows_got = got_k[layer].view(-1, HKV, D)
                rows_exp = exp_k[layer].view(-1, HKV, D)
                assert torch.equal(rows_got[untouched], rows_exp[untouched])
                normed = paged_oracle.rms_norm(bucket.k[layer].cpu(), bucket.wk.cpu())
                assert_rope_close(rows_got[slots], rows_exp[slots], normed, dtype)
        # Padding rows wrote only row 0 of their reserved pages.
        changed = ~(got_v == before_v).all(-1).all(-1)  # [layer, page, row]
        pad_pages = bucket.padding_pages[active:]
        assert changed[:, pad_pages, 0].all() and not changed[:, pad_pages, 1:].any()
        assert not changed[:, bucket.padding_pages[:active]].any()
        assert int(changed.sum()) == LAYERS * BUCKET

        lengths = host_pos + 1
        group = HQ // HKV
        for layer in range(LAYERS):
            q = rot_q[layer] if mode == "scatter" else got_q[layer]
            if mode != "scatter":
                normed = paged_oracle.rms_norm(bucket.q[layer].cpu(), bucket.wq.cpu())
                assert_rope_close(got_q[layer], rot_q[layer], normed, dtype)
            tensors = dict(zip(paged_oracle.TENSOR_NAMES, (q[:active], got_k[layer], got_v[layer],
                                                            host_tables[:active], lengths[:active])))
            want = paged_oracle.fp32_oracle(tensors, BLOCK)
            err = (got_out[layer, :active].float() - want).abs().max().item()
            assert err <= GATE[dtype], (layer, active, err)
            for r in range(active, BUCKET):  # one-token context -> its value row
                row = got_v[layer, bucket.padding_pages[r], 0].repeat_interleave(group, dim=0)
                assert torch.equal(got_out[layer, r], row)

        # The same step, eagerly, from the same cache state: bit-identical.
        bucket.cache.key.copy_(before_k.to(DEV))
        bucket.cache.value.copy_(before_v.to(DEV))
        bucket.out.zero_()
        bucket.step()
        torch.cuda.synchronize()
        assert torch.equal(bucket.cache.key.cpu(), got_k) and torch.equal(bucket.cache.value.cpu(), got_v)
        assert torch.equal(bucket.out.cpu(), got_out)
        if mode != "scatter":
            assert torch.equal(bucket.q_rot.cpu(), got_q)
