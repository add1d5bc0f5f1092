"""ctypes binding of oracle/paged_ref.c -- TEST INFRASTRUCTURE ONLY.

Takes and returns torch CPU tensors; computes in float64.
"""

from __future__ import annotations

import ctypes
import functools
from pathlib import Path
import subprocess

import torch

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "build" / "liboracle_paged.so"

_p = ctypes.c_void_p
_i = ctypes.c_int64


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


@functools.lru_cache(maxsize=1)
def _lib():
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.oracle_f16_to_f32.restype = ctypes.c_float
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_bf16_to_f32.restype = ctypes.c_float
    lib.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_convert.argtypes = [_p, _p, _i, ctypes.c_int]
    lib.oracle_paged_decode.argtypes = [_p, _p, _p, _p, _p, _p] + [_i] * 7 + [_p]
    lib.oracle_paged_prefill.argtypes = [_p] * 8 + [_i] * 7 + [_p]
    lib.oracle_scatter_slots.argtypes = [_p] * 5 + [_i] * 3
    lib.oracle_prefill_slots.argtypes = [_p] * 4 + [_i] * 3
    return lib


def _addr(t: torch.Tensor) -> int:
    assert t.device.type == "cpu" and t.is_contiguous()
    return t.data_ptr()


def to_float32(t: torch.Tensor) -> torch.Tensor:
    """Bit-level fp16/bf16 -> fp32 conversion done by the C routines."""
    if t.dtype == torch.float32:
        return t.contiguous()
    src = t.contiguous().view(torch.int16)
    out = torch.empty(t.shape, dtype=torch.float32)
    _lib().oracle_convert(_addr(src), _addr(out), t.numel(), int(t.dtype == torch.bfloat16))
    return out


def scalar_f16(bits: int) -> float:
    return _lib().oracle_f16_to_f32(bits)


def scalar_bf16(bits: int) -> float:
    return _lib().oracle_bf16_to_f32(bits)


def paged_decode(query, key_cache, value_cache, block_tables, context_lens, block_size):
    q, kc, vc = (to_float32(t.cpu()) for t in (query, key_cache, value_cache))
    tables = block_tables.cpu().to(torch.int64).contiguous()
    lens = context_lens.cpu().to(torch.int64).contiguous()
    b, hq, d = q.shape
    nb, _, hkv, _ = kc.shape
    out = torch.zeros((b, hq, d), dtype=torch.float64)
    scratch = torch.empty(max(1, tables.shape[1] * block_size), dtype=torch.float64)
    _lib().oracle_paged_decode(_addr(out), _addr(q), _addr(kc), _addr(vc), _addr(tables), _addr(lens),
                               b, hq, hkv, d, nb, block_size, tables.shape[1], _addr(scratch))
    return out


def paged_prefill(q, key_cache, value_cache, cu_seqlens_q, query_starts, block_tables, context_lens,
                  block_size):
    qf, kc, vc = (to_float32(t.cpu()) for t in (q, key_cache, value_cache))
    meta = [t.cpu().to(torch.int64).contiguous() for t in (cu_seqlens_q, query_starts, block_tables,
                                                           context_lens)]
    cu, starts, tables, lens = meta
    t, hq, d = qf.shape
    nb, _, hkv, _ = kc.shape
    out = torch.zeros((t, hq, d), dtype=torch.float64)
    scratch = torch.empty(max(1, tables.shape[1] * block_size), dtype=torch.float64)
    _lib().oracle_paged_prefill(_addr(out), _addr(qf), _addr(kc), _addr(vc), _addr(cu), _addr(starts),
                                _addr(tables), _addr(lens), starts.numel(), hq, hkv, d, nb, block_size,
                                tables.shape[1], _addr(scratch))
    return out


def scatter_slots(key_cache, value_cache, slot_mapping, key, value):
    """Returns scattered copies of the caches (inputs untouched)."""
    kc = key_cache.cpu().contiguous().clone().view(torch.int16)
    vc = value_cache.cpu().contiguous().clone().view(torch.int16)
    k = key.cpu().contiguous().view(torch.int16)
    v = value.cpu().contiguous().view(torch.int16)
    slots = slot_mapping.cpu().to(torch.int64).contiguous()
    row = key_cache.shape[2] * key_cache.shape[3]
    cap = key_cache.shape[0] * key_cache.shape[1]
    _lib().oracle_scatter_slots(_addr(kc), _addr(vc), _addr(slots), _addr(k), _addr(v), slots.numel(), cap,
                                row)
    return kc.view(key_cache.dtype), vc.view(value_cache.dtype)


def prefill_slots(cu_seqlens_q, query_starts, block_tables, block_size):
    cu, starts, tables = (t.cpu().to(torch.int64).contiguous() for t in (cu_seqlens_q, query_starts,
                                                                        block_tables))
    out = torch.empty(int(cu[-1]), dtype=torch.int64)
    _lib().oracle_prefill_slots(_addr(out), _addr(cu), _addr(starts), _addr(tables), starts.numel(),
                                tables.shape[1], block_size)
    return out
