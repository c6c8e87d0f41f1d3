"""ctypes binding of librocm_qlora_amd.so (the C ABI in include/rocm_qlora_amd.h).

The reference loads its HIP library the same way -- ctypes.CDLL plus argtypes
(hip_kernels/build_utils.py:232-262) -- but compiles it at first use; this
library is built ahead of time (rocm-qlora_amd/build.py) and only loaded here.
There is no fallback: if the library is missing, every GPU operation raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "librocm_qlora_amd.so")

# dtype codes (include/rocm_qlora_amd.h)
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
C2_FP8_E4M3FNUZ, C2_INT8 = 0, 1
WEIGHT_NF4, WEIGHT_INT8 = 0, 1
MERGE_SUM_THEN_ROUND, MERGE_ROUND_THEN_SUM = 0, 1

_P, _I64, _I32, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

# name -> argtypes (all return int status unless listed in _RESTYPE)
SIGNATURES = {
    "rq_status_string": [_I32],
    "rq_version": [],
    "rq_build_arch": [],
    "rq_nf4_quantize": [_P, _I32, _I64, _I64, _P, _P, _P],
    "rq_nf4_dequantize": [_P, _P, _I32, _I64, _I64, _P, _I32, _I64, _P],
    "rq_dq_quantize": [_P, _I32, _I64, _I64, _I32, _P, _P, _P],
    "rq_dq_dequantize": [_P, _P, _I32, _P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P],
    "rq_int8_quantize": [_P, _I32, _I64, _I64, _I64, _P, _P, _P],
    "rq_int8_dequantize": [_P, _P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P],
    "rq_nf4_linear_workspace_size": [_I32, _I64, _I64, _I64, _I64, _P],
    "rq_nf4_linear": [_P, _I32, _I64, _I64, _I64,            # x, dtype, M, K, ldx
                      _P, _I64, _I64, _P, _I32,              # packed, N, block, absmax, dtype
                      _P, _I32, _I64,                        # c2, c2 format, block2
                      _P, _I32,                              # bias, dtype
                      _P, _I64, _P, _P, _I64, _I32, _I64, _F32,  # lora x, ld, A, B, ldB, dtype, rank, scaling
                      _P, _I64, _P, _I64, _P],               # y, ldy, workspace, bytes, stream
    "rq_nf4_linear_noalloc": [_P, _I32, _I64, _I64, _I64,    # x, dtype, M, K, ldx
                              _P, _I64, _I64, _P, _I32,      # packed, N, block, absmax, dtype
                              _P, _I32, _I64,                # c2, c2 format, block2
                              _P, _I32,                      # bias, dtype
                              _P, _I64, _P, _P, _I64, _I32, _I64, _F32,  # lora x, ld, A, B, ldB, dtype, rank, scaling
                              _P, _I64, _P],                 # y, ldy, stream
    "rq_set_gemv_wait_us": [ctypes.c_uint32],
    "rq_gemm_tile_config": [_P],
    "rq_stream_capture_id": [_P, _P],
    "rq_nf4_linear_dx_workspace_size": [_I32, _I64, _I64, _I64, _I64, _P],
    "rq_nf4_linear_dx": [_P, _I32, _I64, _I64, _I64,         # dy, dtype, M, N, lddy
                         _P, _I64, _I64, _P, _I32,           # packed, K, block, absmax, dtype
                         _P, _I32, _I64,                     # c2, c2 format, block2
                         _P, _P, _I64, _I32, _I64, _F32,     # A, B, ldB, dtype, rank, scaling
                         _P, _I64, _F32,                     # dropout mask, ld, mask scale
                         _P, _I64, _P, _I64, _P],            # dx, lddx, workspace, bytes, stream
    "rq_int8_linear": [_P, _I32, _I64, _I64, _I64,           # x, dtype, M, K, ldx
                       _P, _I64, _I64, _P, _I32,             # q, N, block, scales, dtype
                       _P, _I32, _P, _I64, _P],              # bias, dtype, y, ldy, stream
    "rq_int8_linear_dx": [_P, _I32, _I64, _I64, _I64,        # dy, dtype, M, N, lddy
                          _P, _I64, _I64, _P, _I32,          # q, K, block, scales, dtype
                          _P, _I64, _P],                     # dx, lddx, stream
    "rq_merge_lora": [_P, _I32, _I64, _I64, _I64,           # w, format, N, K, block
                      _P, _I32, _P, _I32, _I64,             # scales, dtype, c2, c2 format, block2
                      _P, _P, _I64, _I32, _I64, _F32,       # A, B, ldB, dtype, rank, scaling
                      _I32, _P, _I32, _I64, _P],            # mode, out, dtype, ld, stream
    "rq_fp8_quantize_workspace_size": [_P],
    "rq_fp8_quantize": [_P, _I32, _I64, _I64, _I64, _P, _P, _P, _I64, _P],
    "rq_fp8_fnuz_to_e4m3fn": [_P, _I64, _P, _P],
    "rq_fp8_linear_workspace_size": [_I64, _I64, _P],
    "rq_fp8_linear": [_P, _I32, _I64, _I64, _I64,            # x, dtype, M, K, ldx
                      _P, _I64, _P, _P, _I32,                # codes, N, w scale, bias, dtype
                      _P, _I64, _P, _I64, _P],               # y, ldy, workspace, bytes, stream
    "rq_int8_quantize_rows": [_P, _I32, _I64, _I64, _I64, _P, _P, _P],
    "rq_adamw_step": [_P, _I64, _P, _I64, _I64, _I64, _P, _P, _P],  # table, n, dev table, bytes,
                                                                  # chunks [b, e), m, v, stream
    "rq_int8_linear_w8a8_workspace_size": [_I64, _I64, _P],
    "rq_int8_linear_w8a8": [_P, _I32, _I64, _I64, _I64,      # x, dtype, M, K, ldx
                            _P, _I64, _P, _I32, _P, _I32,    # w, N, w scales, dtype, bias, dtype
                            _P, _I64, _P, _I64, _P],         # y, ldy, workspace, bytes, stream
}
_RESTYPE = {"rq_status_string": ctypes.c_char_p, "rq_build_arch": ctypes.c_char_p,
            "rq_set_gemv_wait_us": ctypes.c_uint32}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


class NativeLibraryError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the prebuilt library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryError(
                    f"{LIB_PATH} is missing: build it with `python rocm-qlora_amd/build.py` "
                    "(rocm_qlora_amd has no non-HIP execution path)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPE.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def available() -> bool:
    try:
        load()
        return True
    except (NativeLibraryError, OSError):
        return False


def status_string(status: int) -> str:
    return load().rq_status_string(status).decode()


def call(name: str, *args) -> None:
    """Call an rq_* entry point and raise RuntimeError on a non-zero status."""
    status = getattr(load(), name)(*args)
    if status != 0:
        raise RuntimeError(f"{name} failed: {status_string(status)} (status {status})")


def set_gemv_wait_us(us: int) -> int:
    """Test hook: microseconds the decode GEMV waits for its in-launch LoRA
    down-projection before a workgroup computes it itself (0 forces that).
    Returns the previous value."""
    return int(load().rq_set_gemv_wait_us(us))


def capture_id(device: torch.device) -> int:
    """Identifier of the graph capture active on the current stream (0: none)."""
    return stream_capture_id(stream_handle(device))


def stream_capture_id(handle: int) -> int:
    """Identifier of the graph capture active on a raw HIP stream (0: none)."""
    cid = ctypes.c_uint64(0)
    call("rq_stream_capture_id", handle, ctypes.byref(cid))
    return int(cid.value)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return DTYPE_F32
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float16:
        return DTYPE_F16
    raise TypeError(f"unsupported dtype {dt}: expected float32, bfloat16 or float16")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: Optional[torch.Tensor]) -> torch.device:
    """All tensors must live on one GPU; returns that device."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"rocm_qlora_amd kernels run on the GPU; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no tensor given")
    return dev
