"""NF4 and INT8 blockwise codecs, run as HIP kernels on gfx950.

Same names, arguments, return values, dtypes and flat layouts as the
reference's quantization/quant_ops.py, so QuantLinear buffers and state_dicts
interchange bit-for-bit.  The arithmetic lives in csrc/codec.hip.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from rocm_qlora import _native as nat
from rocm_qlora._device import on, to_gpu

# NF4 code book (quant_ops.py:10-15).  A format constant, so identical values.
NF4_VALUES = [
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
]


def _squeeze_scales(s: torch.Tensor) -> torch.Tensor:
    # the reference returns `scales.squeeze()` of a [nb, 1] tensor
    return s.view(-1, 1).squeeze()


def _check_block(block_size: int) -> None:
    if block_size < 2 or block_size % 2:
        raise ValueError(f"block_size must be even and >= 2, got {block_size}")


def quantize_int8(tensor: torch.Tensor, block_size: int = 64, per_channel: bool = False
                  ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Blockwise (flat, zero-padded) or per-row absmax INT8 -- quant_ops.py:17-53.

    scale = clamp(absmax / 127, 1e-12) in the input dtype; q = round(w / scale).
    Returns (int8 flat [numel_padded] or [rows, cols], scales squeezed)."""
    nat.dtype_code(tensor.dtype)
    src, home = to_gpu(tensor)
    with on(src.device):
        if per_channel:
            if src.dim() != 2:
                raise ValueError("per_channel quantization expects a 2-D [out, in] weight")
            w = src.contiguous()
            rows, cols = w.shape
            q = torch.empty((rows, cols), dtype=torch.int8, device=w.device)
            s = torch.empty((rows,), dtype=w.dtype, device=w.device)
            nat.call("rq_int8_quantize", w.data_ptr(), nat.dtype_code(w.dtype), rows, cols, 0,
                     q.data_ptr(), s.data_ptr(), nat.stream_handle(w.device))
        else:
            if block_size < 1:
                raise ValueError("block_size must be >= 1")
            w = src.contiguous().view(-1)
            numel = w.numel()
            nb = -(-numel // block_size)
            q = torch.empty((nb * block_size,), dtype=torch.int8, device=w.device)
            s = torch.empty((nb,), dtype=w.dtype, device=w.device)
            if numel:
                nat.call("rq_int8_quantize", w.data_ptr(), nat.dtype_code(w.dtype), 1, numel,
                         block_size, q.data_ptr(), s.data_ptr(), nat.stream_handle(w.device))
    return q.to(home), _squeeze_scales(s).to(home)


def dequantize_int8(int8_tensor: torch.Tensor, scales: torch.Tensor, block_size: int = 64
                    ) -> torch.Tensor:
    """fp32 reconstruction -- quant_ops.py:55-78 (per-row when the tensor is 2-D
    and has one scale per row, else blockwise over the flat tensor)."""
    q, home = to_gpu(int8_tensor)
    s = scales.to(q.device)
    with on(q.device):
        per_channel = q.dim() == 2 and s.numel() == q.size(0)
        qf = q.contiguous()
        sf = s.contiguous().view(-1)
        out = torch.empty(qf.shape if q.dim() == 2 else (qf.numel(),), dtype=torch.float32,
                          device=q.device)
        if per_channel:
            rows, cols = qf.shape
            bs = 0
        else:
            rows, cols, bs = 1, qf.numel(), block_size
            if bs < 1 or qf.numel() % bs or sf.numel() * bs < qf.numel():
                raise RuntimeError(
                    f"shape mismatch: {qf.numel()} int8 values, {sf.numel()} scales, block {bs}")
        if out.numel():
            nat.call("rq_int8_dequantize", qf.data_ptr(), sf.data_ptr(), nat.dtype_code(sf.dtype),
                     rows, cols, bs, out.data_ptr(), nat.DTYPE_F32, out.numel(),
                     nat.stream_handle(q.device))
        if not per_channel and q.dim() != 2:
            out = out.view(-1)
    return out.to(home)


def quantize_int4(tensor: torch.Tensor, block_size: int = 64) -> Tuple[torch.Tensor, torch.Tensor]:
    """NF4 blockwise quantization -- quant_ops.py:80-126.

    Returns (packed uint8 [numel_padded / 2], absmax squeezed, in the input
    dtype).  Byte j holds element 2j in its low nibble and 2j+1 in its high
    nibble."""
    _check_block(block_size)
    nat.dtype_code(tensor.dtype)
    src, home = to_gpu(tensor)
    with on(src.device):
        w = src.contiguous().view(-1)
        numel = w.numel()
        nb = -(-numel // block_size)
        packed = torch.empty((nb * block_size // 2,), dtype=torch.uint8, device=w.device)
        absmax = torch.empty((nb,), dtype=w.dtype, device=w.device)
        if numel:
            nat.call("rq_nf4_quantize", w.data_ptr(), nat.dtype_code(w.dtype), numel, block_size,
                     packed.data_ptr(), absmax.data_ptr(), nat.stream_handle(w.device))
    return packed.to(home), _squeeze_scales(absmax).to(home)


def nf4_dequantize_to(packed: torch.Tensor, scales: torch.Tensor, block_size: int,
                      out_dtype: torch.dtype = torch.float32, n_out: Optional[int] = None
                      ) -> torch.Tensor:
    """GPU-only: the first n_out dequantized weights, rounded to out_dtype
    (dequantize_int4 followed by the caller's `[:n].to(dtype)`)."""
    dev = nat.require_gpu(packed, scales)
    with on(dev):
        p = packed.contiguous().view(-1)
        s = scales.contiguous().view(-1)
        total = 2 * p.numel()
        n = total if n_out is None else int(n_out)
        if total % block_size or s.numel() * block_size < total:
            raise RuntimeError(f"shape mismatch: {p.numel()} packed bytes, {s.numel()} scales, "
                               f"block {block_size}")
        out = torch.empty((n,), dtype=out_dtype, device=dev)
        if n:
            nat.call("rq_nf4_dequantize", p.data_ptr(), s.data_ptr(), nat.dtype_code(s.dtype),
                     p.numel(), block_size, out.data_ptr(), nat.dtype_code(out_dtype), n,
                     nat.stream_handle(dev))
    return out


def dequantize_int4(packed: torch.Tensor, scales: torch.Tensor, block_size: int = 64) -> torch.Tensor:
    """NF4 reconstruction, fp32 flat [2 * numel_packed] -- quant_ops.py:128-150."""
    p, home = to_gpu(packed)
    return nf4_dequantize_to(p, scales.to(p.device), block_size).to(home)
