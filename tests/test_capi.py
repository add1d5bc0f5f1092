"""C-ABI library checks that need no GPU.

The library must load, export every entry point that include/mvme_paged.h
declares, report its ABI version, and reject bad arguments with a status
code and a message *before* launching anything (these calls never reach a
kernel).  The Python layer must fail loudly when the library is missing.
"""

import ctypes
from pathlib import Path
import re

import pytest

from mini_engine_hip import build as hip_build
from mini_engine_hip.kernels import hip_extension as ext

HEADER = Path(__file__).resolve().parents[1] / "include" / "mvme_paged.h"


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mvme_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return ext.load_hip_extension()


def test_library_exports_every_declared_symbol(lib):
    symbols = declared_symbols()
    assert len(symbols) == 18
    raw = ctypes.CDLL(str(hip_build.library_path()))
    for name in symbols:
        assert hasattr(raw, name), name
    assert set(ext.SIGNATURES) == set(symbols)


def test_abi_version(lib):
    assert lib._lib.mvme_abi_version() == ext.ABI_VERSION == 2


def test_workspace_size_is_a_host_function(lib):
    # Headline decode (B=32, ctx 2048, block 256): one work-group per unit, no split.
    assert lib.workspace_size(32, 16, 8, 128, 256, 8, 0) == 0
    # Few units: split-K partials of fp32 (acc[D] + max + sum) per partition.
    size = lib.workspace_size(1, 16, 8, 128, 16, 256, 512)
    assert size == 1 * 16 * 8 * (128 + 2) * 4
    assert lib.workspace_size(1, 16, 8, 100, 16, 256, 0) == 0  # unsupported head dim
    # Shapes the entry point refuses report no workspace instead of an
    # overflowed size: capacity above 1M tokens, batch * heads above 2^31 - 1,
    # and products that would overflow int64.
    assert lib.workspace_size(1, 16, 8, 128, 16, 65537, 0) == 0
    assert lib.workspace_size(1, 16, 8, 128, 1 << 62, 4, 0) == 0
    assert lib.workspace_size(1 << 31, 2, 1, 128, 16, 256, 64) == 0
    assert lib.workspace_size(1 << 40, 1 << 40, 1, 128, 16, 256, 64) == 0
    assert lib.workspace_size(1, 16, 8, 128, 16, 65536, 64) == 16 * 16384 * 130 * 4


def _status(lib, name, *args):
    return getattr(lib._lib, name)(*args)


def test_decode_rejects_bad_arguments_before_launch(lib):
    base = dict(batch=2, q_heads=16, kv_heads=8, head_dim=128, num_blocks=4, block_size=16, table_width=2)

    def call(**kw):
        a = {**base, **kw}
        return _status(lib, "mvme_paged_attention", 1, 1, 1, 1, 1, 1, a["batch"], a["q_heads"], a["kv_heads"],
                       a["head_dim"], a["num_blocks"], a["block_size"], a["table_width"], 0, kw.get("dtype", 0),
                       None, 0, None)

    assert call(dtype=7) == ext.EINVAL and "FP16/BF16" in lib.last_error()
    assert call(head_dim=100) == ext.EINVAL and "head_dim" in lib.last_error()
    assert call(q_heads=12, kv_heads=8) == ext.EINVAL and "GQA" in lib.last_error()
    assert call(table_width=70000, block_size=16) == ext.EINVAL and "1M" in lib.last_error()
    assert call(batch=0) == ext.EINVAL and "empty" in lib.last_error()
    # Split-K shape without workspace.
    status = _status(lib, "mvme_paged_attention", 1, 1, 1, 1, 1, 1, 1, 16, 8, 128, 64, 16, 256, 512, 0, None, 0,
                     None)
    assert status == ext.EWORKSPACE and "workspace" in lib.last_error()
    assert _status(lib, "mvme_paged_attention", None, 1, 1, 1, 1, 1, 2, 16, 8, 128, 4, 16, 2, 0, 0, None, 0,
                   None) == ext.EINVAL


def test_noalloc_decode_rejects_before_touching_the_device(lib):
    """The allocation-free decode entry checks shapes and its fixed 8 MiB
    scratch limit before any HIP call (this container has no GPU)."""
    def call(batch, width, partition, **kw):
        return _status(lib, "mvme_paged_attention_noalloc", kw.get("out", 1), 1, 1, 1, 1, 1, batch, 16, 8, 128,
                       4096, 256, width, partition, kw.get("dtype", 0), None)

    assert lib.workspace_size(64, 16, 8, 128, 256, 64, 64) > 8 << 20
    assert call(64, 64, 64) == ext.EWORKSPACE
    assert "8388608" in lib.last_error() and "no-alloc" in lib.last_error()
    assert call(2, 16, 0, dtype=7) == ext.EINVAL and "FP16/BF16" in lib.last_error()
    assert call(2, 16, 0, out=None) == ext.EINVAL and "null pointer" in lib.last_error()


def test_decode_write_rejects_before_touching_the_device(lib):
    """The fused KV-write decode entry checks shapes, pointers, head_dim,
    norm inputs, strides and alignment before any HIP call."""
    def call(head_dim=128, q_weight=None, k_weight=None, cos=None, sin=None, eps=1e-6, k_stride=None,
             q_stride=None, ptr=256, new_k=256, query=None, q_out=None, parts=0, width=2):
        k_stride = 8 * head_dim if k_stride is None else k_stride
        q_stride = 16 * head_dim if q_stride is None else q_stride
        query = ptr if query is None else query
        return _status(lib, "mvme_paged_attention_decode_write", ptr, query, ptr, ptr, ptr, ptr, 2, 16, 8,
                       head_dim, 4, 16, width, parts, 0, new_k, ptr, k_stride, 8 * head_dim, q_weight, k_weight, cos, sin,
                       eps, q_stride, q_out, None, 0, None)

    assert call(head_dim=80) == ext.EINVAL and "16,32,64,128,256" in lib.last_error()
    assert call(new_k=None) == ext.EINVAL and "null pointer" in lib.last_error()
    assert call(q_weight=256) == ext.EINVAL and "q_weight, k_weight, cos and sin" in lib.last_error()
    assert call(q_weight=256, k_weight=256, cos=256, sin=256, eps=0.0) == ext.EINVAL
    assert "eps" in lib.last_error()
    assert call(k_stride=100) == ext.EINVAL and "stride" in lib.last_error()
    assert call(q_weight=256, k_weight=256, cos=256, sin=256, q_stride=1000) == ext.EINVAL
    assert "stride" in lib.last_error()
    assert call(ptr=258) == ext.EINVAL and "16-byte aligned" in lib.last_error()
    assert call(k_stride=8 * 128 + 4) == ext.EINVAL and "16-byte aligned" in lib.last_error()
    # q_out must not overlap the raw query rows (2 tokens, 3072 elements apart,
    # 2048 elements each): every work-group reads them while one writes q_out.
    rope = dict(q_weight=256, k_weight=256, cos=256, sin=256, q_stride=3072, query=1 << 20)
    for q_out in ((1 << 20), (1 << 20) + (3072 + 2048) * 2 - 16, (1 << 20) - 2 * 2 * 2048 + 16):
        assert call(**rope, q_out=q_out) == ext.EINVAL and "overlap" in lib.last_error()
    # Adjacent ranges are disjoint: the call passes the overlap check and
    # stops at the next one, the missing workspace of a split plan.
    for q_out in ((1 << 20) + (3072 + 2048) * 2, (1 << 20) - 2 * 2 * 2048):
        assert call(**rope, q_out=q_out, parts=16, width=8) == ext.EWORKSPACE


def test_scatter_and_prefill_reject_bad_arguments(lib):
    assert _status(lib, "mvme_write_kv_cache_slots", 1, 1, 0, 16, 8, 128, 1, 1, 1, 4, 1024, 1024, 0, None) == ext.EINVAL
    assert _status(lib, "mvme_write_kv_cache_slots", 1, 1, 4, 16, 8, 128, 1, 1, 1, 4, 100, 1024, 0, None) == ext.EINVAL
    assert "stride" in lib.last_error()
    assert _status(lib, "mvme_write_kv_cache", 1, 1, 4, 16, 8, 128, 1, 2, 30, 1, 1, 5, 1, None) == ext.EINVAL
    assert "exceeds" in lib.last_error()
    assert _status(lib, "mvme_paged_prefill_attention", 1, 1, 1, 1, 1, 1, 1, 1, 1, 4, 16, 8, 2048, 4, 16, 1, 0, 0,
                   None, 0, None) == ext.EINVAL
    assert "1024" in lib.last_error()
    # Few query blocks + long table: key-chunk split needs a workspace.
    need = lib.prefill_workspace_size(8, 1024, 16, 8, 128, 256, 16, 0, ext.FP16)
    assert need == 1024 * 16 * 8 * (128 + 2) * 4 + 1024 * 4
    # bf16 inputs keep bf16 partials: 2 bytes per partial element.
    assert lib.prefill_workspace_size(8, 1024, 16, 8, 128, 256, 16, 0, ext.BF16) == \
        1024 * 16 * 8 * (128 * 2 + 2 * 4) + 1024 * 4
    # head_dim 256: partial rows 256 wide; narrower heads pad to 128.
    assert lib.prefill_workspace_size(8, 1024, 16, 8, 256, 256, 16, 0, ext.BF16) == \
        1024 * 16 * 8 * (256 * 2 + 2 * 4) + 1024 * 4
    assert lib.prefill_workspace_size(8, 1024, 16, 8, 64, 256, 16, 0, ext.BF16) == \
        1024 * 16 * 8 * (128 * 2 + 2 * 4) + 1024 * 4
    assert lib.prefill_workspace_size(8, 1024, 16, 8, 192, 256, 16, 0, ext.BF16) == \
        1024 * 16 * 8 * (256 * 2 + 2 * 4) + 1024 * 4
    assert lib.prefill_workspace_size(8, 1024, 16, 8, 264, 256, 16, 0, ext.BF16) == 0  # scalar kernel, no split
    assert lib.prefill_workspace_size(8, 1024, 16, 8, 128, 256, 16, 0, 9) == 0  # no such type
    assert lib.prefill_workspace_size(8, 1 << 40, 1 << 30, 8, 128, 256, 16, 0, ext.BF16) == 0  # refused shape
    assert _status(lib, "mvme_paged_prefill_attention", 1, 1, 1, 1, 1, 1, 1, 1, 8, 1024, 16, 8, 128, 200, 256, 16,
                   0, 0, None, 0, None) == ext.EWORKSPACE
    # Many query blocks: no split, no workspace.
    assert lib.prefill_workspace_size(8, 1 << 16, 16, 8, 128, 256, 16, 0, ext.BF16) == 0
    # Empty inputs are legal no-ops.
    assert _status(lib, "mvme_write_kv_cache_slots", 1, 1, 4, 16, 8, 128, None, None, None, 0, 1024, 1024, 1,
                   None) == ext.OK
    assert _status(lib, "mvme_paged_prefill_attention", None, None, None, None, None, None, None, None, 0, 0, 16, 8,
                   128, 4, 16, 0, 0, 1, None, 0, None) == ext.OK


def test_dense_prefill_plan_and_rejections(lib):
    """mvme_prefill_attention (dense suffix prefill): its workspace plan and
    argument checks, all before any launch (the pointers are never read)."""
    bf16 = ext.BF16
    # One 4096-token square prompt, Hq16/Hkv8/D128: 32 query blocks per kv
    # head do not fill the CUs, so keys split into chunks of 512 (8 chunks).
    rows = 4096 * 16
    assert lib.dense_prefill_workspace_size(1, 4096, 16, 8, 128, 0, bf16) == \
        8 * rows * 128 * 2 + 8 * rows * 2 * 4 + 4096 * 4
    assert lib.dense_prefill_workspace_size(8, 4096, 16, 8, 128, 0, bf16) == 0  # enough blocks: no split
    assert lib.dense_prefill_workspace_size(1, 4096, 16, 8, 20, 0, bf16) == 0  # generic kernel
    assert lib.dense_prefill_workspace_size(1, 4096, 12, 8, 128, 0, bf16) == 0  # GQA mismatch
    assert lib.dense_prefill_workspace_size(1, 64, 16, 8, 128, -1, bf16) == 0
    assert lib.dense_prefill_workspace_size(1, 64, 16, 8, 128, 1 << 20, bf16) == 0  # context over 2^20
    assert lib.dense_prefill_workspace_size(1, 64, 16, 8, 128, 0, 9) == 0

    def call(batch=1, q_heads=16, kv_heads=8, tokens=64, kv_tokens=64, head_dim=128, start=0, ptr=256, out=256,
             q_strides=None, kv_strides=None, out_strides=None, dtype=bf16, workspace=None, workspace_bytes=0):
        q_strides = q_strides or (q_heads * tokens * head_dim, tokens * head_dim, head_dim)
        kv_strides = kv_strides or (kv_heads * kv_tokens * head_dim, kv_tokens * head_dim, head_dim)
        out_strides = out_strides or (q_heads * tokens * head_dim, tokens * head_dim, head_dim)
        return _status(lib, "mvme_prefill_attention", out, ptr, ptr, ptr, batch, q_heads, kv_heads, tokens, kv_tokens,
                       head_dim, start, *q_strides, *kv_strides, *out_strides, dtype, workspace, workspace_bytes,
                       None)

    assert call(dtype=7) == ext.EINVAL and "FP16/BF16" in lib.last_error()
    assert call(q_heads=12) == ext.EINVAL and "GQA" in lib.last_error()
    assert call(head_dim=1032) == ext.EINVAL and "1024" in lib.last_error()
    assert call(start=1) == ext.EINVAL and "query range exceeds KV sequence" in lib.last_error()
    assert call(tokens=0) == ext.EINVAL and "query range" in lib.last_error()
    assert call(ptr=None) == ext.EINVAL and "null pointer" in lib.last_error()
    assert call(ptr=258) == ext.EINVAL and "16-byte aligned" in lib.last_error()
    assert call(q_strides=(16 * 64 * 128, 64 * 128, 132)) == ext.EINVAL and "multiples of 8" in lib.last_error()
    assert call(q_strides=(0, -8, 128)) == ext.EINVAL and "strides out of range" in lib.last_error()
    assert call(kv_strides=(1 << 50, 64 * 128, 128), batch=4096) == ext.EINVAL and "out of range" in lib.last_error()
    # Output rows must be distinct: an expanded head dim, heads 64 elements
    # apart (inside a 128-element row), tokens overlapping the heads.
    for strides in ((16 * 64 * 128, 0, 128), (16 * 64 * 128, 64, 64 * 64), (16 * 64 * 128, 128, 8 * 128)):
        assert call(out_strides=strides) == ext.EINVAL and "overlap" in lib.last_error()
    # A split plan without (or with too small) a workspace.
    assert call(tokens=4096, kv_tokens=4096) == ext.EWORKSPACE and "workspace" in lib.last_error()
    assert call(tokens=4096, kv_tokens=4096, workspace=256, workspace_bytes=1024) == ext.EWORKSPACE


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """No silent fallback: without a buildable library every call raises."""
    ext.load_hip_extension.cache_clear()
    monkeypatch.setattr(hip_build, "library_path", lambda: tmp_path / "libmissing.so")

    def refuse(**_):
        raise RuntimeError("hipcc not found: the HIP library cannot be built")

    monkeypatch.setattr(hip_build, "build_library", refuse)
    try:
        with pytest.raises(RuntimeError, match="cannot be built"):
            ext.load_hip_extension()
    finally:
        ext.load_hip_extension.cache_clear()


def test_stale_library_is_refused(tmp_path):
    """A library whose recorded source digest differs from the sources beside it
    (or that has none) is refused before it is loaded."""
    current = hip_build.source_digest()
    digest = tmp_path / "SOURCE_DIGEST"
    with pytest.raises(RuntimeError, match="no build digest"):
        ext.check_build_digest(digest, current)
    digest.write_text("0" * 64 + "\n")
    with pytest.raises(RuntimeError, match="stale HIP library"):
        ext.check_build_digest(digest, current)
    digest.write_text(current + "\n")
    ext.check_build_digest(digest, current)
    # The in-tree build carries the digest of the current sources.
    assert hip_build.digest_path().read_text().strip() == current


def test_loader_checks_the_digest(monkeypatch, tmp_path):
    ext.load_hip_extension.cache_clear()
    planted = tmp_path / "SOURCE_DIGEST"
    planted.write_text("f" * 64)
    monkeypatch.setattr(hip_build, "digest_path", lambda: planted)
    try:
        with pytest.raises(RuntimeError, match="stale HIP library"):
            ext.load_hip_extension()
    finally:
        ext.load_hip_extension.cache_clear()


def test_argmax_workspace_plan(lib):
    # Enough slices per row to cover the CUs twice (>= 2048 elements each), a single slice otherwise.
    assert lib.argmax_workspace_size(32, 151936) == 32 * 16 * 8
    assert lib.argmax_workspace_size(1, 151936) == 75 * 8
    assert lib.argmax_workspace_size(600, 151936) == 0
    assert lib.argmax_workspace_size(5, 1) == 0
    assert lib.argmax_workspace_size(0, 10) == 0
    status = lib._lib.mvme_greedy_argmax(None, None, 32, 151936, 151936, 1, None, 0, None)
    assert status == ext.EINVAL
    status = lib._lib.mvme_greedy_argmax(1, 1, 32, 151936, 151936, 1, None, 0, None)
    assert status == ext.EWORKSPACE and "workspace" in lib.last_error()
    assert lib._lib.mvme_greedy_argmax(1, 1, 2, 10, 9, 1, None, 0, None) == ext.EINVAL
    assert lib._lib.mvme_greedy_argmax(1, 1, 2, 10, 10, 7, None, 0, None) == ext.EINVAL


def test_prefill_workspace_bytes_helper(lib):
    """The Python sizing helper a layer loop uses for its one shared buffer is
    the library's plan: the 8 x 128 bf16 batch (capacity 4096 keys, 512-key
    chunks, 8 chunk planes of 1024 tokens x 16 heads x (256 + 8) bytes, plus
    one int per token); fp16 keeps fp32 partials."""
    import torch

    from mini_engine_hip.kernels.prefill import paged_prefill_workspace_bytes

    bf16 = paged_prefill_workspace_bytes(8, 1024, 16, 8, 128, 256, 16, torch.bfloat16)
    assert bf16 == lib.prefill_workspace_size(8, 1024, 16, 8, 128, 256, 16, 0, ext.dtype_code(torch.bfloat16))
    assert 8 * 1024 * 16 * (256 + 8) + 4096 <= bf16 < 8 * 1024 * 16 * (256 + 8) + 4096 + 64
    fp16 = paged_prefill_workspace_bytes(8, 1024, 16, 8, 128, 256, 16, torch.float16)
    assert 8 * 1024 * 16 * (512 + 8) + 4096 <= fp16 < 8 * 1024 * 16 * (512 + 8) + 4096 + 64
