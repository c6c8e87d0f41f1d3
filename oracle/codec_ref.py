"""ORACLE -- test infrastructure only.  ctypes access to oracle/codec_ref.c
(the bit-level C restatement); built by `make -C oracle`."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libcodec_ref.so")
DT = {"f32": 0, "bf16": 1, "f16": 2}

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.ref_nf4_argmin.argtypes = [ctypes.c_float]
        L.ref_nf4_argmin.restype = I32
        L.ref_fnuz_from_f32.argtypes = [ctypes.c_float]
        L.ref_fnuz_from_f32.restype = ctypes.c_uint8
        L.ref_fnuz_to_f32.argtypes = [ctypes.c_uint8]
        L.ref_fnuz_to_f32.restype = ctypes.c_float
        L.ref_round_bf16.argtypes = [ctypes.c_float]
        L.ref_round_bf16.restype = ctypes.c_float
        L.ref_nf4_table.argtypes = [P]
        L.ref_nf4_quantize.argtypes = [P, I32, I64, I64, P, P]
        L.ref_nf4_dequantize.argtypes = [P, P, I32, I64, I64, P, I32, I64]
        L.ref_dq_quantize.argtypes = [P, I32, I64, I64, I32, P, P]
        L.ref_dq_dequantize.argtypes = [P, P, I32, P, I32, I64, I64, I64, P, I32, I64]
        L.ref_int8_quantize.argtypes = [P, I32, I64, I64, I64, P, P]
        L.ref_fnuz_encode.argtypes = [P, I64, P]
        L.ref_round_array.argtypes = [P, I64, I32, P]
        L.ref_nf4_exhaustive.argtypes = [P, P, I32, I32, P]
        L.ref_nf4_exhaustive.restype = I64
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _raw(t):
    """torch CPU tensor -> (numpy view of its storage bytes as the right width, dtype code)."""
    import torch
    if t.dtype == torch.float32:
        return t.contiguous().numpy(), DT["f32"]
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16), DT["bf16"]
    if t.dtype == torch.float16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16), DT["f16"]
    raise TypeError(t.dtype)


def _empty_like_dt(n, code):
    return np.empty(n, dtype=np.float32 if code == 0 else np.uint16)


def to_torch(a: np.ndarray, code: int):
    import torch
    if code == 0:
        return torch.from_numpy(a.astype(np.float32))
    t = torch.from_numpy(a.view(np.int16).copy())
    return t.view(torch.bfloat16 if code == 1 else torch.float16)


def nf4_table() -> np.ndarray:
    out = np.empty(16, dtype=np.float32)
    lib().ref_nf4_table(_p(out))
    return out


def nf4_quantize(t, block_size=64):
    src, code = _raw(t.flatten())
    n = src.size
    nb = -(-n // block_size)
    packed = np.empty(nb * block_size // 2, dtype=np.uint8)
    absmax = _empty_like_dt(nb, code)
    lib().ref_nf4_quantize(_p(src), code, n, block_size, _p(packed), _p(absmax))
    return packed, to_torch(absmax, code)


def nf4_dequantize(packed: np.ndarray, absmax, block_size, out_dtype="f32", n_out=None):
    s, scode = _raw(absmax.flatten())
    n_out = 2 * packed.size if n_out is None else n_out
    ocode = DT[out_dtype]
    out = _empty_like_dt(n_out, ocode)
    lib().ref_nf4_dequantize(_p(np.ascontiguousarray(packed)), _p(s), scode, packed.size, block_size,
                             _p(out), ocode, n_out)
    return to_torch(out, ocode)


def dq_quantize(c1, block2=256, int8=False):
    src, code = _raw(c1.flatten())
    n = src.size
    nb = -(-n // block2)
    c2 = np.empty(nb * block2, dtype=np.uint8)
    c2s = _empty_like_dt(nb, code)
    lib().ref_dq_quantize(_p(src), code, n, block2, int(int8), _p(c2), _p(c2s))
    return c2, to_torch(c2s, code)


def dq_dequantize(packed, c2, c2s, block1, block2, int8=False, out_dtype="f32", n_out=None):
    s, scode = _raw(c2s.flatten())
    n_out = 2 * packed.size if n_out is None else n_out
    ocode = DT[out_dtype]
    out = _empty_like_dt(n_out, ocode)
    lib().ref_dq_dequantize(_p(np.ascontiguousarray(packed)), _p(np.ascontiguousarray(c2)), int(int8),
                            _p(s), scode, packed.size, block1, block2, _p(out), ocode, n_out)
    return to_torch(out, ocode)


def int8_quantize(t, rows, cols, block_size):
    src, code = _raw(t.flatten())
    if block_size > 0:
        nseg = -(-rows * cols // block_size)
        q = np.empty(nseg * block_size, dtype=np.int8)
    else:
        nseg = rows
        q = np.empty(rows * cols, dtype=np.int8)
    s = _empty_like_dt(nseg, code)
    lib().ref_int8_quantize(_p(src), code, rows, cols, block_size, _p(q), _p(s))
    return q, to_torch(s, code)


def fnuz_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.uint8)
    lib().ref_fnuz_encode(_p(x), x.size, _p(out))
    return out


def round_array(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().ref_round_array(_p(x), x.size, DT[dtype], _p(out))
    return out


def nf4_exhaustive(cell_thr: np.ndarray, cell_base: np.ndarray, part: int, nparts: int):
    first = np.zeros(1, dtype=np.uint32)
    bad = lib().ref_nf4_exhaustive(_p(np.ascontiguousarray(cell_thr, dtype=np.uint32)),
                                   _p(np.ascontiguousarray(cell_base, dtype=np.uint8)),
                                   part, nparts, _p(first))
    return int(bad), int(first[0])
