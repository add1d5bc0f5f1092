"""Greedy sampling, ``backend="hip"`` (mini_engine/sampling.py:4-17).

``sample_next_token`` keeps the reference's signature; the hip backend
serves temperature 0 (greedy) through ``mvme_greedy_argmax`` and raises the
reference's errors otherwise (ValueError for the Python-side contract,
RuntimeError for the native checks of bindings.cpp:186-193).
"""

from __future__ import annotations

import torch

from .kernels import hip_extension as ext

_DTYPES = {torch.float16: ext.FP16, torch.bfloat16: ext.BF16, torch.float32: ext.FP32}


def greedy_argmax(logits, *, out=None, workspace=None):
    """Row-wise argmax of ``logits [batch, vocab]`` with torch.argmax's tie and NaN rules.

    ``workspace``: optional device buffer of at least
    ``mvme_greedy_argmax_workspace_size(batch, vocab)`` bytes (allocated per
    call when omitted).
    """
    if not logits.is_cuda or not logits.is_contiguous():
        raise RuntimeError("greedy logits must be contiguous CUDA tensors")
    if logits.ndim != 2:
        raise RuntimeError("greedy logits must be [batch, nonempty vocab]")
    if logits.shape[1] == 0:
        raise RuntimeError("greedy logits must be [batch, nonempty vocab]")
    if logits.dtype not in _DTYPES:
        raise RuntimeError("greedy supports FP32/FP16/BF16")
    if logits.shape[0] > 65535 or logits.shape[1] > 2147483647:
        raise RuntimeError("greedy logits shape too large")
    if out is None:
        out = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
    elif out.shape != (logits.shape[0],) or out.dtype != torch.int64 or not out.is_contiguous() \
            or out.device != logits.device:
        raise ValueError("out must be a contiguous int64 tensor [batch]")
    if logits.shape[0] == 0:
        return out
    lib = ext.load_hip_extension()
    need = lib.argmax_workspace_size(logits.shape[0], logits.shape[1])
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=logits.device)
    elif need and (workspace.device != logits.device or workspace.numel() * workspace.element_size() < need):
        raise ValueError("greedy argmax workspace too small")
    with torch.cuda.device(logits.device):
        lib.call("mvme_greedy_argmax", out.data_ptr(), logits.data_ptr(), logits.shape[0], logits.shape[1],
                 logits.shape[1], _DTYPES[logits.dtype], workspace.data_ptr() if need else None, need,
                 ext.current_stream(logits.device))
    return out


def sample_next_token(logits, temperature=0.0, top_k=0, top_p=1.0, *, backend="hip"):
    """Greedy next tokens ``[batch]`` (temperature 0 only on the hip backend)."""
    if logits.ndim != 2:
        raise ValueError("logits must have shape [batch, vocab]")
    if backend != "hip":
        raise ValueError("sampling backend must be hip")
    if temperature != 0:
        raise ValueError("HIP sampling currently supports greedy temperature=0 only")
    return greedy_argmax(logits)
