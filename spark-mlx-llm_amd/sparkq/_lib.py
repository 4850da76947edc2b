"""ctypes binding of libsparkq.so (include/sparkq.h).

The library is loaded from this package directory. A missing or unloadable
library raises ImportError-style RuntimeError at first use: there is no
fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

__all__ = [
    "F32", "F16", "BF16", "KV_S8_F16SCALE", "KV_AFFINE_U8",
    "lib", "library_path", "dtype_code", "call", "stream_handle", "workspace",
    "SparkqError",
]

F32, F16, BF16 = 0, 1, 2
KV_S8_F16SCALE, KV_AFFINE_U8, KV_AFFINE_U4, KV_AFFINE_U2 = 0, 1, 2, 3
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_DEVICE, ERR_WORKSPACE = 0, -1, -2, -3, -4

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_LOCK = threading.Lock()

P, I64, I, F, SZ = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float,
                    ctypes.c_size_t)

# name -> (restype, argtypes); mirrors include/sparkq.h
SIGNATURES = {
    "sparkq_last_error": (ctypes.c_char_p, []),
    "sparkq_abi_version": (I, []),
    "sparkq_is_available": (I, []),
    "sparkq_w4a16_workspace_bytes": (SZ, [I64, I64, I64, I]),
    "sparkq_w4a16_linear": (I, [P, P, P, P, P, I64, I64, I64, I, I, I, I, P, SZ, P]),
    "sparkq_w4a16_prepared_bytes": (SZ, [I64, I64, I]),
    "sparkq_w4a16_prepare": (I, [P, P, P, SZ, I64, I64, I, I, P]),
    "sparkq_w4a16_linear_prepared": (I, [P, P, P, P, P, P, I64, I64, I64, I, I, I, I, P, SZ,
                                         P]),
    "sparkq_w4a16_dequantize": (I, [P, P, P, P, I64, I64, I, I, P]),
    "sparkq_w4_quantize": (I, [P, P, P, P, I64, I64, I, I, P]),
    "sparkq_a8_quantize_per_token": (I, [P, P, P, I64, I64, I, P]),
    "sparkq_int8_matmul_workspace_bytes": (SZ, [I64, I64, I64]),
    "sparkq_int8_matmul_i32": (I, [P, P, P, I64, I64, I64, P, SZ, P]),
    "sparkq_w8a8_workspace_bytes": (SZ, [I64, I64, I64]),
    "sparkq_w8a8_linear": (I, [P, P, P, P, I, P, I64, I64, I64, I, I, P, SZ, P]),
    "sparkq_w8a16_linear": (I, [P, P, P, P, I64, I64, I64, I, I, P]),
    "sparkq_w8_affine_linear": (I, [P, P, P, P, P, I64, I64, I64, I, I, I, I, P]),
    "sparkq_int8kv_sdpa_workspace_bytes": (SZ, [I64, I64, I64, I64]),
    "sparkq_int8kv_sdpa_decode": (I, [P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64,
                                      I, I, I, I, F, P, P, SZ, P]),
    "sparkq_int8kv_sdpa_decode_noalloc": (I, [P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64,
                                              I, I, I, I, F, P, P]),
    "sparkq_kv_quantize_s8": (I, [P, P, P, I64, I64, I, P]),
    "sparkq_kv_append": (I, [P, P, P, P, I64, I64, I64, I64, I64, I, I, I, P, P]),
    "sparkq_int8kv_sdpa_prefill": (I, [P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I, I,
                                       I, F, P, P]),
    "sparkq_int8kv_sdpa_prefill_affine": (I, [P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64,
                                              I64, I, I, I, I, F, P, P, SZ, P]),
    "sparkq_int8kv_sdpa_prefill_affine_workspace_bytes": (SZ, [I64, I64, I64, I64, I64, I64, I]),
    "sparkq_ffn_workspace_bytes": (SZ, [I64, I64, I64, I]),
    "sparkq_ffn": (I, [P, P, P, F, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I, I, P, SZ, P]),
    "sparkq_qkv_rope_workspace_bytes": (SZ, [I64, I, I, I, I]),
    "sparkq_qkv_rope": (I, [P, P, P, P, P, P, P, I64, I, I, I, I, I, I, F, I64, I, I, I, P, SZ,
                            P]),
    "sparkq_rope": (I, [P, P, I64, I64, I64, I, I, F, F, I64, I, P]),
    "sparkq_rms_norm": (I, [P, P, P, F, P, P, I64, I64, I, P]),
    "sparkq_attention_gate": (I, [P, P, P, P, P, I64, I64, I64, I64, I64, I, P]),
    "sparkq_quantized_sdpa_workspace_bytes": (SZ, [I64, I64, I64, I64, I64, I64]),
    "sparkq_quantized_sdpa": (I, [P, P, P, P, P, P, P, P, I, I, P, P, I64, I64, I64, I64, I64,
                                  I64, I64, I, I, I, I, F, P, P, SZ, P]),
}


class SparkqError(RuntimeError):
    """A HIP runtime failure reported by libsparkq."""


def library_path() -> str:
    return os.path.join(_HERE, "libsparkq.so")


def lib():
    global _LIB
    if _LIB is None:
        with _LOCK:
            if _LIB is None:
                path = library_path()
                if not os.path.exists(path):
                    raise RuntimeError(
                        f"libsparkq.so is not built ({path}); run "
                        "python spark-mlx-llm_amd/build.py")
                handle = ctypes.CDLL(path)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _LIB = handle
    return _LIB


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[dtype]
    except KeyError:
        raise ValueError(f"unsupported floating dtype {dtype}") from None


def stream_handle(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def call(name: str, *args, device: Optional[torch.device] = None) -> None:
    """Call an entry point and map its status to the reference's exception types
    (validation -> ValueError, runtime -> SparkqError). With `device` (the
    tensors' GPU) the call runs with that device current: the library
    launches on the current device."""
    if device is not None and device.type == "cuda" and device.index is not None \
            and device.index != torch.cuda.current_device():
        with torch.cuda.device(device):
            rc = getattr(lib(), name)(*args)
    else:
        rc = getattr(lib(), name)(*args)
    if rc == OK:
        return
    msg = (lib().sparkq_last_error() or b"").decode(errors="replace")
    if rc in (ERR_INVALID, ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise SparkqError(f"{name}: {msg}")


_WS: dict = {}


def workspace_buffer(device: torch.device, nbytes: int, kind: str) -> torch.Tensor:
    """The uint8 buffer behind workspace() (at least nbytes)."""
    workspace(device, nbytes, kind)
    return _WS[(device.index, torch.cuda.current_stream(device).cuda_stream, kind)]


def workspace(device: torch.device, nbytes: int, kind: str):
    """Scratch buffer per (device, stream, entry-point kind). Reuse is safe
    because every user enqueues on that same stream. Buffers start zeroed:
    split-K entry points keep tile counters at the front of their workspace,
    which must be zero before the first call (every call leaves them zero)."""
    if nbytes <= 0:
        return None, 0
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream, kind)
    buf = _WS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WS[key] = buf
    return ctypes.c_void_p(buf.data_ptr()), buf.numel()
