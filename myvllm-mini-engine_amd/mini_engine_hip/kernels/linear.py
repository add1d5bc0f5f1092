"""Linear layer, ``backend="hip"`` (mini_engine/kernels/linear.py:14-30).

``HipLinear`` keeps ``CudaLinear``'s interface and errors: an ``nn.Linear``
with the ``[out_features, in_features]`` weight, whose forward flattens the
input to rows.  Up to 64 rows (a decode batch) go through
``mvme_linear_rows``, which reads the weight once at HBM rate; larger
inputs (prefill) are plain GEMMs and take the library matmul, as the
reference's CudaLinear does for every size.
"""

from __future__ import annotations

import torch
from torch import nn

from . import hip_extension as ext

MAX_ROWS = 64


def linear_rows(x, weight, bias=None, *, out=None):
    """out[m] = x[m] @ weight.T (+ bias) for a 2-D ``x`` of at most 64 rows."""
    if not x.is_cuda or not weight.is_cuda:
        raise ValueError("HipLinear requires CUDA input and weights")
    if x.ndim != 2 or weight.ndim != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("input feature dimension does not match Linear")
    if x.dtype not in (torch.float16, torch.bfloat16) or weight.dtype != x.dtype:
        raise ValueError("HIP linear rows supports matching FP16/BF16 input and weights")
    if x.shape[0] > MAX_ROWS:
        raise ValueError("HIP linear rows supports at most 64 rows")
    if x.stride(1) != 1 or not weight.is_contiguous():
        raise ValueError("HIP linear rows needs row-major input and a contiguous weight")
    if bias is not None and (bias.shape != (weight.shape[0],) or bias.dtype != x.dtype or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous [out_features] tensor of the input dtype")
    if weight.device != x.device or (bias is not None and bias.device != x.device):
        raise ValueError("input, weight and bias must share a device")
    rows, out_features = x.shape[0], weight.shape[0]
    if out is None:
        out = torch.empty(rows, out_features, dtype=x.dtype, device=x.device)
    elif (out.shape != (rows, out_features) or out.dtype != x.dtype or not out.is_contiguous()
          or out.device != x.device):
        raise ValueError("out must be a contiguous [rows, out_features] tensor of the input dtype and device")
    lib = ext.load_hip_extension()
    with torch.cuda.device(x.device):
        lib.call("mvme_linear_rows", out.data_ptr(), x.data_ptr(), weight.data_ptr(),
                 bias.data_ptr() if bias is not None else None, rows, x.shape[1], out_features, x.stride(0),
                 ext.dtype_code(x.dtype), ext.current_stream(x.device))
    return out


def _rows_supported(flat, weight):
    return (flat.shape[0] <= MAX_ROWS and flat.dtype in (torch.float16, torch.bfloat16)
            and weight.dtype == flat.dtype and flat.shape[1] % 32 == 0 and weight.shape[0] % 16 == 0
            and flat.stride(1) == 1 and flat.stride(0) % 8 == 0 and weight.is_contiguous()
            and flat.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0)


class HipLinear(nn.Linear):
    """Inference Linear with the HIP decode-batch kernel (CudaLinear's interface)."""

    backend = "hip"

    def forward(self, x):
        if not x.is_cuda or not self.weight.is_cuda:
            raise ValueError("HipLinear requires CUDA input and weights")
        original_shape = x.shape
        if x.shape[-1] != self.in_features:
            raise ValueError("input feature dimension does not match Linear")
        flat = x.reshape(-1, self.in_features)
        if _rows_supported(flat, self.weight):
            output = linear_rows(flat, self.weight, self.bias)
        else:
            output = torch.mm(flat, self.weight.t())
            if self.bias is not None:
                output = output + self.bias
        return output.reshape(*original_shape[:-1], self.out_features)
