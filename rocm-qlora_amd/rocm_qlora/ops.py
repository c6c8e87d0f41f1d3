"""Functional entry points of the MI355X quantized-linear path.

Each function validates and lays out torch tensors, then calls one C-ABI
entry point of librocm_qlora_amd.so on the current HIP stream.  There is no
CPU or library fallback for any activation dtype or shape: a tensor off the
GPU, or a missing library, raises.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from rocm_qlora import _native as nat
from rocm_qlora._device import on

# activation rows up to which the NF4 linear runs as a weight-streaming GEMV
# (kGemvMaxM in csrc/rq_linear.h); above it, the MFMA GEMM
GEMV_MAX_M = 16
# largest N * (row stride of LoRA B) the decode GEMV addresses (2^29 elements)
GEMV_MAX_B_ELEMS = 1 << 29


def _rows(t: torch.Tensor, K: int) -> Tuple[torch.Tensor, int]:
    """[..., K] -> 2-D [rows, K] view with unit inner stride, and its row stride."""
    t2 = t.reshape(-1, K)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < K):
        t2 = t2.contiguous()
    return t2, (t2.stride(0) if t2.shape[0] > 1 else K)


# rq_nf4_linear's workspace.  Its first RQ_LINEAR_SYNC_BYTES
# (include/rocm_qlora_amd.h) are a synchronization area that must be zero
# before the buffer's first call and that every call leaves ready for the
# next one once its kernels are done, so one buffer, zeroed once on the
# stream that uses it, serves every call ordered on that stream.  Calls that may run at the same time need buffers of their
# own, hence the keys:
#   * eager calls: one buffer per (device, stream), zeroed by a fill kernel
#     on that stream when it is created; it grows by reallocation (a dropped
#     buffer returns to torch's caching allocator, which hands it out again
#     only in stream order);
#   * graph capture: one buffer per (device, capture, stream) -- the branches
#     of a capture that forks side streams each get their own.  It is taken
#     from a pool of pre-zeroed buffers (_CAPTURE_POOL_ENTRIES of
#     _CAPTURE_POOL_BYTES per device, zeroed at the device's first eager
#     call; and every eager call that finds no free entry as large as its own
#     workspace adds one, zeroed, with one stream synchronization, up to
#     _CAPTURE_POOL_LIMIT bytes per device), so the graph needs no fill node:
#     it holds zeros before the first replay and every replay leaves it ready
#     for the next.  Captures are normally preceded by an eager warm-up call
#     of the same work, which leaves an entry of the size the capture needs.
#     Such a buffer is held for the life of the process (the graph may replay
#     it at any time).  A capture on a device without the pool, or finding
#     no free entry large enough, allocates one from the graph's private
#     memory pool (so it lives exactly as long as the graph), zeroed by a
#     fill kernel recorded in the graph, which every replay runs before the
#     captured calls.
LINEAR_SYNC_BYTES = 131328
_LINEAR_WS: dict = {}
_CAPTURE_WS: dict = {}
_WS_MIN_BYTES = 1 << 20
_CAPTURE_POOL_ENTRIES = 32
# 2 MiB holds the decode GEMV's largest workspace (M = 16 with its K-split
# partials) for the common layer shapes, so that a capture's calls share one
# pre-zeroed buffer rather than recording a fill kernel at each larger need
_CAPTURE_POOL_BYTES = 2 << 20
_CAPTURE_POOL_LIMIT = 1 << 30  # pre-zeroed capture buffers per device, at most (bytes)
_CAPTURE_POOL: dict = {}       # device index -> pre-zeroed buffers not yet handed out
_CAPTURE_POOL_BASE: dict = {}  # device index -> the allocations they are views of (kept for good)
_CAPTURE_POOL_TOTAL: dict = {}  # device index -> bytes of those allocations


def _ensure_capture_pool(dev, idx: int, need: int) -> None:
    """The device's pool exists and holds a free entry of at least `need`
    bytes (while the pool stays within _CAPTURE_POOL_LIMIT)."""
    if idx not in _CAPTURE_POOL_BASE:
        base = torch.zeros(_CAPTURE_POOL_ENTRIES * _CAPTURE_POOL_BYTES, dtype=torch.uint8, device=dev)
        torch.cuda.current_stream(dev).synchronize()  # zero before any later capture, on any stream, replays it
        _CAPTURE_POOL_BASE[idx] = [base]
        _CAPTURE_POOL_TOTAL[idx] = base.numel()
        _CAPTURE_POOL[idx] = [base[i * _CAPTURE_POOL_BYTES:(i + 1) * _CAPTURE_POOL_BYTES]
                              for i in range(_CAPTURE_POOL_ENTRIES)]
    pool = _CAPTURE_POOL[idx]
    if any(e.numel() >= need for e in pool):
        return
    size = -(-max(need, _CAPTURE_POOL_BYTES) // _CAPTURE_POOL_BYTES) * _CAPTURE_POOL_BYTES
    if _CAPTURE_POOL_TOTAL[idx] + size > _CAPTURE_POOL_LIMIT:
        return
    buf = torch.zeros(size, dtype=torch.uint8, device=dev)
    torch.cuda.current_stream(dev).synchronize()
    _CAPTURE_POOL_BASE[idx].append(buf)
    _CAPTURE_POOL_TOTAL[idx] += size
    pool.append(buf)


def _zeroed_area(nbytes: int, dev, min_bytes: int = _WS_MIN_BYTES) -> torch.Tensor:
    ws = torch.empty(max(nbytes, min_bytes), dtype=torch.uint8, device=dev)
    ws[:LINEAR_SYNC_BYTES].zero_()
    return ws


def _workspace(x_dtype: torch.dtype, M: int, K: int, N: int, rank: int, dev) -> Optional[torch.Tensor]:
    import ctypes
    nbytes = ctypes.c_int64(0)
    nat.call("rq_nf4_linear_workspace_size", nat.dtype_code(x_dtype), M, K, N, rank, ctypes.byref(nbytes))
    need = nbytes.value
    if need == 0:
        return None
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(dev).cuda_stream
    if torch.cuda.is_current_stream_capturing():
        cid = nat.capture_id(dev)
        # the buffers of captures that have ended belong to their graphs'
        # pools and are dropped here; a capture still running (on another
        # stream or thread) keeps its buffer, since its pool could otherwise
        # hand the memory to a later allocation of the same capture
        for k in [k for k in _CAPTURE_WS if k[0] == idx and k[1] != cid]:
            if nat.stream_capture_id(k[2]) != k[1]:
                del _CAPTURE_WS[k]
        key = (idx, cid, stream)
        ws = _CAPTURE_WS.get(key)
        if ws is None or ws.numel() < need:
            # a larger buffer replaces a smaller one for the calls captured
            # from here on; calls captured before keep theirs
            pool = _CAPTURE_POOL.get(idx) or []
            fits = [i for i, e in enumerate(pool) if e.numel() >= need]
            if fits:
                ws = pool.pop(min(fits, key=lambda i: pool[i].numel()))
            else:
                ws = _zeroed_area(need, dev, min_bytes=LINEAR_SYNC_BYTES)
            _CAPTURE_WS[key] = ws
        return ws
    _ensure_capture_pool(dev, idx, need)
    key = (idx, stream)
    ws = _LINEAR_WS.get(key)
    if ws is None or ws.numel() < need:
        ws = _zeroed_area(max(need, 2 * ws.numel() if ws is not None else 0), dev)
        _LINEAR_WS[key] = ws
    return ws


def nf4_linear(x: torch.Tensor, weight_quant: torch.Tensor, weight_scales: Optional[torch.Tensor],
               out_features: int, block_size: int = 64, bias: Optional[torch.Tensor] = None, *,
               c2: Optional[torch.Tensor] = None, c2_scales: Optional[torch.Tensor] = None,
               blocksize_2: int = 256, use_fp8_c2: bool = True,
               lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
               scaling: float = 0.0, lora_x: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x . dequant(W)^T + bias (+ LoRA) for an NF4 weight stored flat
    (quant_linear.py:182-197 and lora_layer.py:60-70 in one kernel launch
    sequence).  x: [..., K] bf16/fp16 (bf16/fp16 MFMA kernels) or fp32 (the
    fp32-MFMA kernel, everything in fp32 as the reference computes it) on the
    GPU; output has x's dtype.  Any K and block size: shapes the specialized
    kernels do not take (K % 64 != 0, other block sizes, fp32 with rank > 64)
    run on the library's generic kernels with the same roundings."""
    K = x.shape[-1]
    N = int(out_features)
    xcode = nat.dtype_code(x.dtype)
    dq = c2 is not None
    scales = c2_scales if dq else weight_scales
    dev = nat.require_gpu(x, weight_quant, scales, bias, lora_a, lora_b, c2)
    packed = weight_quant.reshape(-1)
    if packed.dtype != torch.uint8:
        raise TypeError(f"NF4 weight_quant must be uint8, got {packed.dtype}")
    if packed.numel() * 2 < N * K:
        raise RuntimeError(f"weight_quant holds {packed.numel() * 2} codes, need {N}x{K}")
    packed = packed.contiguous()
    scales = scales.reshape(-1).contiguous()
    if block_size < 1:
        raise RuntimeError(f"block_size must be positive, got {block_size}")
    n_blocks = -(-N * K // block_size)
    if dq:
        if c2.numel() < n_blocks or scales.numel() * blocksize_2 < n_blocks:
            raise RuntimeError("c2 / c2_scales too short for the weight")
    elif scales.numel() < n_blocks:
        raise RuntimeError(f"weight_scales holds {scales.numel()} values, need {n_blocks}")
    lead = x.shape[:-1]
    with on(dev):
        x2, ldx = _rows(x, K)
        M = x2.shape[0]
        if (M > GEMV_MAX_M or x.dtype == torch.float32) and K % 64 == 0:  # 16-byte activation loads
            x2, ldx = _aligned_rows(x2, K)
        y = torch.empty((M, N), dtype=x.dtype, device=dev)
        if M == 0:
            return y.reshape(*lead, N)
        rank = 0
        la = lb = xl = None
        ldxl = ldb = 0
        lcode = 0
        if lora_a is not None and lora_b is not None and lora_a.shape[0] > 0:
            rank = lora_a.shape[0]
            if lora_a.shape[1] != K or lora_b.shape != (N, rank):
                raise RuntimeError(f"LoRA shapes {tuple(lora_a.shape)} / {tuple(lora_b.shape)} do not fit "
                                   f"{N}x{K}")
            if lora_a.dtype not in (torch.float32, x.dtype):
                lora_a = lora_a.float()
            if lora_b.dtype != lora_a.dtype:
                lora_b = lora_b.to(lora_a.dtype)
            la = lora_a.contiguous()
            # B rows may be strided (a column slice of a wider parameter);
            # the decode GEMV addresses B with 32-bit offsets, so a stride
            # that would overflow them is packed first
            lb, ldb = _rows(lora_b, rank)
            if M <= GEMV_MAX_M and N * ldb > GEMV_MAX_B_ELEMS:
                lb, ldb = lb.contiguous(), rank
            lcode = nat.dtype_code(la.dtype)
            if lora_x is not None:
                # the GEMM's and the fp32 path's LoRA operand kernels load 16
                # bytes at a time
                wide = (M > GEMV_MAX_M or x.dtype == torch.float32) and K % 64 == 0
                xl, ldxl = (_aligned_rows if wide else _rows)(lora_x.to(x.dtype), K)
        b = bias.contiguous() if bias is not None else None
        ws = _workspace(x.dtype, M, K, N, rank, dev)
        codes = c2.reshape(-1).view(torch.uint8).contiguous() if dq else None
        nat.call("rq_nf4_linear",
                 x2.data_ptr(), xcode, M, K, ldx,
                 packed.data_ptr(), N, block_size, scales.data_ptr(), nat.dtype_code(scales.dtype),
                 nat.ptr(codes), nat.C2_FP8_E4M3FNUZ if use_fp8_c2 else nat.C2_INT8, blocksize_2,
                 nat.ptr(b), nat.dtype_code(b.dtype) if b is not None else 0,
                 nat.ptr(xl), ldxl, nat.ptr(la), nat.ptr(lb), ldb, lcode, rank, float(scaling),
                 y.data_ptr(), N, nat.ptr(ws), ws.numel() if ws is not None else 0,
                 nat.stream_handle(dev))
    return y.reshape(*lead, N)


def nf4_linear_dx(dy: torch.Tensor, weight_quant: torch.Tensor, weight_scales: Optional[torch.Tensor],
                  in_features: int, block_size: int = 64, *,
                  c2: Optional[torch.Tensor] = None, c2_scales: Optional[torch.Tensor] = None,
                  blocksize_2: int = 256, use_fp8_c2: bool = True,
                  lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
                  scaling: float = 0.0, lora_mask: Optional[torch.Tensor] = None,
                  mask_scale: float = 1.0) -> torch.Tensor:
    """dX = dY . dequant(W) (+ the LoRA term ((dY * s) . B) . A) for an NF4
    weight stored flat (dequant_matmul.py:338-351, lora_layer.py:67
    differentiated).  With lora_mask (the dropout mask of the adapter's input,
    [..., K] bool), the LoRA term goes through dropout's backward: times
    mask * mask_scale.  dy: [..., N] fp32/bf16/fp16 on the GPU; output
    [..., K] in dy's dtype.  Shapes outside the MFMA dX kernel's (N or K not
    multiples of 64, other block sizes, fp32 dy) run on the generic kernels."""
    N = dy.shape[-1]
    K = int(in_features)
    dq = c2 is not None
    scales = c2_scales if dq else weight_scales
    dev = nat.require_gpu(dy, weight_quant, scales, lora_a, lora_b, c2)
    packed = weight_quant.reshape(-1)
    if packed.dtype != torch.uint8:
        raise TypeError(f"NF4 weight_quant must be uint8, got {packed.dtype}")
    if packed.numel() * 2 < N * K:
        raise RuntimeError(f"weight_quant holds {packed.numel() * 2} codes, need {N}x{K}")
    packed = packed.contiguous()
    scales = scales.reshape(-1).contiguous()
    lead = dy.shape[:-1]
    with on(dev):
        # the dX kernel loads dY rows 16 bytes at a time
        dy2, lddy = _aligned_rows(dy, N) if N % 64 == 0 else _rows(dy, N)
        M = dy2.shape[0]
        dx = torch.empty((M, K), dtype=dy.dtype, device=dev)
        if M == 0:
            return dx.reshape(*lead, K)
        rank = 0
        la = lb = None
        ldb = 0
        lcode = 0
        if lora_a is not None and lora_b is not None and lora_a.shape[0] > 0:
            rank = lora_a.shape[0]
            if lora_a.shape[1] != K or lora_b.shape != (N, rank):
                raise RuntimeError(f"LoRA shapes {tuple(lora_a.shape)} / {tuple(lora_b.shape)} do not fit "
                                   f"{N}x{K}")
            if lora_a.dtype not in (torch.float32, dy.dtype):
                lora_a = lora_a.float()
            if lora_b.dtype != lora_a.dtype:
                lora_b = lora_b.to(lora_a.dtype)
            la = lora_a.contiguous()
            # B rows may be strided (a column slice of a wider parameter)
            lb, ldb = _rows(lora_b, rank)
            lcode = nat.dtype_code(la.dtype)
        mk, ldm = None, 0
        if rank > 0 and lora_mask is not None:
            mk, ldm = _rows(lora_mask.reshape(-1, K).view(torch.uint8), K)
            if mk.shape[0] != M:
                raise RuntimeError(f"lora_mask has {mk.shape[0]} rows, dY {M}")
        import ctypes
        nbytes = ctypes.c_int64(0)
        nat.call("rq_nf4_linear_dx_workspace_size", nat.dtype_code(dy.dtype), M, N, K, rank, ctypes.byref(nbytes))
        ws = torch.empty(nbytes.value, dtype=torch.uint8, device=dev) if nbytes.value else None
        codes = c2.reshape(-1).view(torch.uint8).contiguous() if dq else None
        nat.call("rq_nf4_linear_dx",
                 dy2.data_ptr(), nat.dtype_code(dy.dtype), M, N, lddy,
                 packed.data_ptr(), K, block_size, scales.data_ptr(), nat.dtype_code(scales.dtype),
                 nat.ptr(codes), nat.C2_FP8_E4M3FNUZ if use_fp8_c2 else nat.C2_INT8, blocksize_2,
                 nat.ptr(la), nat.ptr(lb), ldb, lcode, rank, float(scaling),
                 nat.ptr(mk), ldm, float(mask_scale),
                 dx.data_ptr(), K, nat.ptr(ws), ws.numel() if ws is not None else 0,
                 nat.stream_handle(dev))
    return dx.reshape(*lead, K)


def _aligned_rows(t: torch.Tensor, K: int) -> Tuple[torch.Tensor, int]:
    """2-D [rows, K] view with a 16-byte aligned base and a row stride that
    keeps every row 16-byte aligned (the MFMA kernels load 16 bytes at a time)."""
    t2, ld = _rows(t, K)
    if t2.data_ptr() % 16 or (ld * t2.element_size()) % 16:
        t2 = t2.contiguous().clone()
        ld = K
    return t2, ld


def int8_linear(x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor, out_features: int,
                block_size: int = 0, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x . (q * scale)^T + bias for int8 weights (quant_ops.py:55-78 then
    quant_linear.py:193-197).  q: [N, K] (or flat N*K) int8; block_size 0 ->
    one scale per output row ([N] scales, the row-absmax recipe), otherwise
    blockwise over the flat weight (QuantLinear bits=8 uses 64).
    x: [..., K] fp32/bf16/fp16 on the GPU; output has x's dtype.  Shapes and
    dtypes the int8 GEMV / MFMA GEMM do not take run on the generic kernels."""
    K = x.shape[-1]
    N = int(out_features)
    dev = nat.require_gpu(x, q, scales, bias)
    if q.dtype != torch.int8:
        raise TypeError(f"int8 weights expected, got {q.dtype}")
    qf = q.reshape(-1).contiguous()
    if qf.numel() < N * K:
        raise RuntimeError(f"q holds {qf.numel()} values, need {N}x{K}")
    sc = scales.reshape(-1).contiguous()
    need = N if block_size == 0 else -(-N * K // block_size)
    if sc.numel() < need:
        raise RuntimeError(f"scales hold {sc.numel()} values, need {need}")
    lead = x.shape[:-1]
    with on(dev):
        x2, ldx = _aligned_rows(x, K) if K % 64 == 0 and x.dtype != torch.float32 else _rows(x, K)
        M = x2.shape[0]
        y = torch.empty((M, N), dtype=x.dtype, device=dev)
        if M == 0:
            return y.reshape(*lead, N)
        b = bias.contiguous() if bias is not None else None
        nat.call("rq_int8_linear", x2.data_ptr(), nat.dtype_code(x.dtype), M, K, ldx,
                 qf.data_ptr(), N, block_size, sc.data_ptr(), nat.dtype_code(sc.dtype),
                 nat.ptr(b), nat.dtype_code(b.dtype) if b is not None else 0,
                 y.data_ptr(), N, nat.stream_handle(dev))
    return y.reshape(*lead, N)


def int8_linear_dx(dy: torch.Tensor, q: torch.Tensor, scales: torch.Tensor, in_features: int,
                   block_size: int = 0) -> torch.Tensor:
    """dX = dY . (q * scale) for int8 weights (the backward of
    dequant_matmul.py:308-324: the dequantized weight rounded to dY's dtype,
    then the product), decoded inside the multiply.  q: [N, K] (or flat)
    int8, scales as for int8_linear; dy: [..., N] fp32/bf16/fp16 on the GPU;
    output [..., K] in dy's dtype."""
    N = dy.shape[-1]
    K = int(in_features)
    dev = nat.require_gpu(dy, q, scales)
    if q.dtype != torch.int8:
        raise TypeError(f"int8 weights expected, got {q.dtype}")
    qf = q.reshape(-1).contiguous()
    if qf.numel() < N * K:
        raise RuntimeError(f"q holds {qf.numel()} values, need {N}x{K}")
    sc = scales.reshape(-1).contiguous()
    need = N if block_size == 0 else -(-N * K // block_size)
    if sc.numel() < need:
        raise RuntimeError(f"scales hold {sc.numel()} values, need {need}")
    lead = dy.shape[:-1]
    with on(dev):
        dy2, lddy = _rows(dy, N)
        M = dy2.shape[0]
        dx = torch.empty((M, K), dtype=dy.dtype, device=dev)
        if M == 0:
            return dx.reshape(*lead, K)
        nat.call("rq_int8_linear_dx", dy2.data_ptr(), nat.dtype_code(dy.dtype), M, N, lddy,
                 qf.data_ptr(), K, block_size, sc.data_ptr(), nat.dtype_code(sc.dtype),
                 dx.data_ptr(), K, nat.stream_handle(dev))
    return dx.reshape(*lead, K)


def fp8_quantize(t: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor e4m3fnuz quantization of fp8_linear.py:33-42 on the GPU:
    returns (codes as torch.float8_e4m3fnuz [rows, cols], fp32 0-dim scale),
    scale = fp32(double(max|t|) / 240), codes = fnuz(RND(t / scale))."""
    dev = nat.require_gpu(t)
    t2 = t.reshape(-1, t.shape[-1]) if t.dim() != 2 else t
    rows, cols = t2.shape
    with on(dev):
        src, ld = _rows(t2, cols)
        codes = torch.empty((rows, cols), dtype=torch.uint8, device=dev)
        scale = torch.empty((), dtype=torch.float32, device=dev)
        import ctypes
        nb = ctypes.c_int64(0)
        nat.call("rq_fp8_quantize_workspace_size", ctypes.byref(nb))
        ws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
        nat.call("rq_fp8_quantize", src.data_ptr(), nat.dtype_code(t.dtype), rows, cols, ld,
                 codes.data_ptr(), scale.data_ptr(), ws.data_ptr(), ws.numel(), nat.stream_handle(dev))
    return codes.view(torch.float8_e4m3fnuz), scale


def fp8_to_e4m3fn(codes: torch.Tensor) -> torch.Tensor:
    """e4m3fnuz codes (fp8_quantize's) -> e4m3fn codes of the same values,
    the format gfx950's fp8 matrix cores read: exact except the 8 odd-mantissa
    magnitudes below 2^-6, which round to the nearest even e4m3fn code (as
    torch's .to(torch.float8_e4m3fn) does); NaN stays NaN."""
    dev = nat.require_gpu(codes)
    src = codes.view(torch.uint8).contiguous()
    with on(dev):
        out = torch.empty(src.shape, dtype=torch.uint8, device=dev)
        nat.call("rq_fp8_fnuz_to_e4m3fn", src.data_ptr(), src.numel(), out.data_ptr(), nat.stream_handle(dev))
    return out.view(torch.float8_e4m3fn)


def fp8_linear(x: torch.Tensor, w_codes: torch.Tensor, w_scale: torch.Tensor,
               bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """_FP8LinearFunc.forward (fp8_linear.py:27-60) for a weight quantized by
    fp8_quantize: x is quantized per tensor, the fp8 products are summed by
    the fp8 matrix cores in fp32, scaled by x_scale * w_scale, rounded to x's
    dtype, and the bias is added.  w_codes: torch.float8_e4m3fn (fp8_to_e4m3fn
    of the quantized weight, used as is) or torch.float8_e4m3fnuz / uint8
    (re-encoded on every call).  x: [..., K] fp32/bf16/fp16 on the GPU (fp32
    x, K % 64 != 0 or unaligned rows: the generic kernels, which decode the
    codes and sum the fp32 products as fp8_linear.py:44-52 does)."""
    K = x.shape[-1]
    dev = nat.require_gpu(x, w_codes, w_scale, bias)
    if w_codes.dtype != torch.float8_e4m3fn:
        if w_codes.dtype not in (torch.float8_e4m3fnuz, torch.uint8):
            raise TypeError(f"fp8 weight codes expected, got {w_codes.dtype}")
        w_codes = fp8_to_e4m3fn(w_codes)
    wc = w_codes.reshape(-1, K).view(torch.uint8).contiguous()
    N = wc.shape[0]
    ws_scale = w_scale.reshape(()).to(torch.float32).contiguous()
    lead = x.shape[:-1]
    with on(dev):
        x2, ldx = _aligned_rows(x, K) if K % 64 == 0 and x.dtype != torch.float32 else _rows(x, K)
        M = x2.shape[0]
        y = torch.empty((M, N), dtype=x.dtype, device=dev)
        if M == 0:
            return y.reshape(*lead, N)
        import ctypes
        nb = ctypes.c_int64(0)
        nat.call("rq_fp8_linear_workspace_size", M, K, ctypes.byref(nb))
        ws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
        b = bias.to(x.dtype).contiguous() if bias is not None else None
        nat.call("rq_fp8_linear", x2.data_ptr(), nat.dtype_code(x.dtype), M, K, ldx,
                 wc.data_ptr(), N, ws_scale.data_ptr(), nat.ptr(b),
                 nat.dtype_code(b.dtype) if b is not None else 0,
                 y.data_ptr(), N, ws.data_ptr(), ws.numel(), nat.stream_handle(dev))
    return y.reshape(*lead, N)


def int8_quantize_rows(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row int8 quantization of 16-bit activations on the GPU: the
    per-row recipe of quantize_int8 (quant_ops.py:29-35) in fp32.  Returns
    (codes int8 [rows, K], scales fp32 [rows]) with scales[m] =
    max(max|x[m]| / 127, 1e-12) and codes = RNE(x / scales[m])."""
    K = x.shape[-1]
    dev = nat.require_gpu(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"bf16/fp16 activations expected, got {x.dtype}")
    with on(dev):
        x2, ldx = _aligned_rows(x, K)
        M = x2.shape[0]
        codes = torch.empty((M, K), dtype=torch.int8, device=dev)
        scales = torch.empty((M,), dtype=torch.float32, device=dev)
        if M:
            nat.call("rq_int8_quantize_rows", x2.data_ptr(), nat.dtype_code(x.dtype), M, K, ldx,
                     codes.data_ptr(), scales.data_ptr(), nat.stream_handle(dev))
    return codes, scales


def int8_linear_w8a8(x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor,
                     bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """W8A8 INT8 mode: x quantized per row to int8 (int8_quantize_rows), the
    int8 products summed exactly in int32 by the int8 matrix cores, then
    y = RND(RND(float(acc) * x_scale[m] * w_scale[n]) + RND(bias)).
    q: [N, K] int8 with one scale per row (quantize_int8(w,
    per_channel=True)); x: [..., K] bf16/fp16 on the GPU, K % 64 == 0.
    Not the reference's INT8 linear (int8_linear: 16-bit activations times
    dequantized weights): a separate, faster mode with activation rounding."""
    K = x.shape[-1]
    dev = nat.require_gpu(x, q, scales, bias)
    if q.dtype != torch.int8:
        raise TypeError(f"int8 weights expected, got {q.dtype}")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"bf16/fp16 activations expected, got {x.dtype}")
    wq = q.reshape(-1, K).contiguous()
    N = wq.shape[0]
    sc = scales.reshape(-1).contiguous()
    if sc.numel() != N:
        raise RuntimeError(f"W8A8 needs one weight scale per row: {sc.numel()} scales for {N} rows")
    lead = x.shape[:-1]
    with on(dev):
        x2, ldx = _aligned_rows(x, K)
        M = x2.shape[0]
        y = torch.empty((M, N), dtype=x.dtype, device=dev)
        if M == 0:
            return y.reshape(*lead, N)
        import ctypes
        nb = ctypes.c_int64(0)
        nat.call("rq_int8_linear_w8a8_workspace_size", M, K, ctypes.byref(nb))
        ws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
        b = bias.to(x.dtype).contiguous() if bias is not None else None
        nat.call("rq_int8_linear_w8a8", x2.data_ptr(), nat.dtype_code(x.dtype), M, K, ldx,
                 wq.data_ptr(), N, sc.data_ptr(), nat.dtype_code(sc.dtype), nat.ptr(b),
                 nat.dtype_code(b.dtype) if b is not None else 0,
                 y.data_ptr(), N, ws.data_ptr(), ws.numel(), nat.stream_handle(dev))
    return y.reshape(*lead, N)


MERGE_MODES = {"sum_then_round": nat.MERGE_SUM_THEN_ROUND, "round_then_sum": nat.MERGE_ROUND_THEN_SUM}


def merge_lora(weight_quant: torch.Tensor, weight_scales: torch.Tensor, out_features: int, in_features: int,
               block_size: int = 64, lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
               scaling: float = 0.0, *, bits: int = 4, c2: Optional[torch.Tensor] = None,
               use_fp8_c2: bool = True, blocksize_2: int = 256, mode: str = "sum_then_round",
               out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """[out, in] 16-bit weight of dequant(W) + (B @ A) * scaling, straight
    from the quantized buffers in one kernel.  mode "sum_then_round":
    RND(W + d) as LoRALinear.merge_lora rounds it (lora_layer.py:84-103);
    "round_then_sum": RND(RND(W) + RND(d)) as the export path does
    (export/gguf_export.py:53-77).  bits 4: NF4 codes with per-block absmax,
    or c2 codes with weight_scales = c2_scales under double quantization;
    bits 8: int8 codes, block_size 0 meaning one scale per row."""
    N, K = int(out_features), int(in_features)
    dev = nat.require_gpu(weight_quant, weight_scales, lora_a, lora_b, c2)
    if mode not in MERGE_MODES:
        raise ValueError(f"mode must be one of {sorted(MERGE_MODES)}, got {mode!r}")
    if out_dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"out_dtype must be float16 or bfloat16, got {out_dtype}")
    w = weight_quant.reshape(-1).contiguous()
    if bits == 4:
        fmt = nat.WEIGHT_NF4
        if w.dtype != torch.uint8 or w.numel() * 2 < N * K:
            raise RuntimeError(f"NF4 weight_quant must hold {N}x{K} codes as uint8")
    elif bits == 8:
        fmt = nat.WEIGHT_INT8
        if w.dtype != torch.int8 or w.numel() < N * K:
            raise RuntimeError(f"INT8 weight_quant must hold {N}x{K} int8 values")
    else:
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    sc = weight_scales.reshape(-1).contiguous()
    rank = 0
    la = lb = None
    ldb = lcode = 0
    if lora_a is not None and lora_b is not None and lora_a.shape[0] > 0:
        rank = lora_a.shape[0]
        if lora_a.shape[1] != K or lora_b.shape != (N, rank):
            raise RuntimeError(f"LoRA shapes {tuple(lora_a.shape)} / {tuple(lora_b.shape)} do not fit {N}x{K}")
        if lora_b.dtype != lora_a.dtype:
            lora_b = lora_b.to(lora_a.dtype)
        la = lora_a.detach().contiguous()
        lb, ldb = _rows(lora_b.detach(), rank)
        lcode = nat.dtype_code(la.dtype)
    codes = c2.reshape(-1).view(torch.uint8).contiguous() if c2 is not None else None
    with on(dev):
        out = torch.empty((N, K), dtype=out_dtype, device=dev)
        nat.call("rq_merge_lora", w.data_ptr(), fmt, N, K, block_size, sc.data_ptr(), nat.dtype_code(sc.dtype),
                 nat.ptr(codes), nat.C2_FP8_E4M3FNUZ if use_fp8_c2 else nat.C2_INT8, blocksize_2,
                 nat.ptr(la), nat.ptr(lb), ldb, lcode, rank, float(scaling), MERGE_MODES[mode],
                 out.data_ptr(), nat.dtype_code(out_dtype), K, nat.stream_handle(dev))
    return out
