"""MI355X (gfx950) paged-attention path for mini_engine's Qwen3 engine.

A drop-in ``hip`` backend for the reference's paged KV-cache hot path:
KV scatter, GQA decode attention over block tables, ragged chunked paged
prefill and dense suffix prefill, the fused q/k RMSNorm + RoPE + KV write
before them, and the decode-batch output projection and greedy sampling
after them, each a hand-written HIP kernel behind the C ABI of
``libmvme_paged.so`` (declared in ``include/mvme_paged.h``).
"""

from .kernels.paged import paged_attention
from .kernels.data import write_kv_cache, write_kv_cache_batch, write_kv_cache_slots
from .kernels.prefill import paged_prefill_attention, prefill_attention
from .kernels.rope import qk_norm_rope_write_kv
from .kernels.linear import HipLinear, linear_rows
from .sampling import greedy_argmax, sample_next_token

__all__ = ["paged_attention", "write_kv_cache", "write_kv_cache_batch", "write_kv_cache_slots",
           "paged_prefill_attention", "prefill_attention", "qk_norm_rope_write_kv", "HipLinear", "linear_rows",
           "greedy_argmax", "sample_next_token"]
