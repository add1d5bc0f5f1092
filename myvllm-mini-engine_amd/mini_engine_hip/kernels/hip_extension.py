"""ctypes binding of libmvme_paged.so (the C ABI declared in include/mvme_paged.h).

Plays the role of the reference's ``load_cuda_extension``
(mini_engine/kernels/cuda_extension.py:14-66): one cached handle per
process.  There is no fallback: a missing or unloadable library raises.
"""

from __future__ import annotations

import ctypes
import functools

import torch

from .. import build as _build

FP16, BF16, FP32 = 0, 1, 2
OK, EINVAL, ELAUNCH, EWORKSPACE = 0, 1, 2, 3
ABI_VERSION = 2

_i64, _vp, _int, _size = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/mvme_paged.h.
SIGNATURES = {
    "mvme_abi_version": (_int, []),
    "mvme_last_error": (ctypes.c_char_p, []),
    "mvme_write_kv_cache_slots": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64,
                                         _i64, _i64, _int, _vp]),
    "mvme_write_kv_cache_batch": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp,
                                         _i64, _int, _vp]),
    "mvme_write_kv_cache": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                                   _int, _vp]),
    "mvme_gather_kv_cache": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _int,
                                    _vp]),
    "mvme_paged_attention_workspace_size": (_size, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "mvme_paged_attention": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                    _i64, _i64, _int, _vp, _size, _vp]),
    "mvme_paged_attention_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                            _i64, _i64, _i64, _int, _vp]),
    "mvme_paged_attention_decode_write": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                                 _i64, _i64, _i64, _int, _vp, _vp, _i64, _i64, _vp, _vp, _vp,
                                                 _vp, ctypes.c_float, _i64, _vp, _vp, _size, _vp]),
    "mvme_paged_prefill_workspace_size": (_size, [_i64] * 8 + [_int]),
    "mvme_paged_prefill_attention": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                            _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp, _size, _vp]),
    "mvme_prefill_attention_workspace_size": (_size, [_i64] * 6 + [_int]),
    "mvme_prefill_attention": (_int, [_vp, _vp, _vp, _vp] + [_i64] * 16 + [_int, _vp, _size, _vp]),
    "mvme_qk_norm_rope_write_kv": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp,
                                          _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64,
                                          ctypes.c_float, _int, _vp]),
    "mvme_greedy_argmax_workspace_size": (_size, [_i64, _i64]),
    "mvme_greedy_argmax": (_int, [_vp, _vp, _i64, _i64, _i64, _int, _vp, _size, _vp]),
    "mvme_linear_rows": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp]),
}


class HipLibrary:
    """Typed handle on the shared object; every call checks its status."""

    def __init__(self, lib: ctypes.CDLL, path):
        self._lib = lib
        self.path = path
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.mvme_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libmvme_paged ABI version {version}, expected {ABI_VERSION}")

    def last_error(self) -> str:
        message = self._lib.mvme_last_error()
        return message.decode() if message else ""

    def call(self, name: str, *args):
        status = getattr(self._lib, name)(*args)
        if status != OK:
            raise RuntimeError(f"{name}: {self.last_error()} (status {status})")

    def workspace_size(self, *args) -> int:
        return int(self._lib.mvme_paged_attention_workspace_size(*args))

    def prefill_workspace_size(self, *args) -> int:
        return int(self._lib.mvme_paged_prefill_workspace_size(*args))

    def dense_prefill_workspace_size(self, *args) -> int:
        return int(self._lib.mvme_prefill_attention_workspace_size(*args))

    def argmax_workspace_size(self, *args) -> int:
        return int(self._lib.mvme_greedy_argmax_workspace_size(*args))


def check_build_digest(digest_file, expected: str) -> None:
    """Refuse a library built from other sources than the ones beside it.

    ``build_library`` writes the sha256 of the HIP sources and headers next to
    the library; a missing or different digest means the library is stale.
    """
    try:
        recorded = digest_file.read_text().strip()
    except OSError as error:
        raise RuntimeError(f"no build digest at {digest_file}: rebuild the HIP library "
                           f"(python -m mini_engine_hip.build)") from error
    if recorded != expected:
        raise RuntimeError(f"stale HIP library: the sources changed since it was built "
                           f"(digest {recorded[:12]} != {expected[:12]}); rebuild with "
                           f"python -m mini_engine_hip.build")


@functools.lru_cache(maxsize=1)
def load_hip_extension() -> HipLibrary:
    """Load the prebuilt library; build it first only if no build exists.

    An existing library must carry the digest of the current sources.
    """
    path = _build.library_path()
    if not path.exists():
        _build.build_library()
    check_build_digest(_build.digest_path(), _build.source_digest())
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as error:
        raise RuntimeError(f"cannot load the HIP paged-attention library {path}: {error}") from error
    return HipLibrary(lib, path)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return FP16
    if dtype == torch.bfloat16:
        return BF16
    raise ValueError("HIP kernels support FP16/BF16")


def current_stream(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(tensor: torch.Tensor) -> int:
    return tensor.data_ptr()
