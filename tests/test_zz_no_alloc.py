"""rq_nf4_linear_noalloc (the allocation-free variant of rq_nf4_linear, its
workspace a static device array) called through the C ABI: bit-identical to
rq_nf4_linear with an allocated workspace on two calls in a row, the second
with a smaller input, then on the other paths that use the workspace (the
MFMA GEMM with LoRA and K splits, fp32 activations); a call that would need
more than the array is rejected before anything runs."""
import math

import pytest
import torch

from rocm_qlora import _native as nat
from rocm_qlora import ops
from rocm_qlora.quantization import quantize_int4

pytestmark = pytest.mark.gpu

SCRATCH_LIMIT = 8  # RQ_ERR_SCRATCH_LIMIT


def _layer(N, K, rank, seed, dev):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    a = torch.empty(rank, K)
    torch.nn.init.kaiming_uniform_(a, a=math.sqrt(5), generator=g)
    b = torch.randn(N, rank, generator=g) * 0.01
    bias = torch.randn(N, generator=g) * 0.1
    packed, absmax = quantize_int4(w.to(dev), 64)
    return packed, absmax, a.to(dev), b.to(dev), bias.to(dev)


def _noalloc(x, packed, absmax, N, a, b, scaling, bias=None):
    M, K = x.shape
    y = torch.empty(M, N, dtype=x.dtype, device=x.device)
    st = nat.load().rq_nf4_linear_noalloc(
        x.data_ptr(), nat.dtype_code(x.dtype), M, K, K,
        packed.data_ptr(), N, 64, absmax.data_ptr(), nat.dtype_code(absmax.dtype),
        None, 0, 256,
        nat.ptr(bias), nat.dtype_code(bias.dtype) if bias is not None else 0,
        None, 0, a.data_ptr(), b.data_ptr(), b.shape[1], nat.dtype_code(a.dtype), a.shape[0], float(scaling),
        y.data_ptr(), N, nat.stream_handle(x.device))
    return st, y


@pytest.mark.parametrize("cases", [[(2, 4096, 4096, 16), (1, 1024, 512, 16)]])
def test_noalloc_matches_workspace_entry_two_calls(dev, cases):
    """Two calls in a row (the second smaller): decode GEMV with the LoRA
    down-projection inside the launch, which uses the array's
    synchronization area."""
    for i, (M, K, N, rank) in enumerate(cases):
        print(f"noalloc call {i}: M={M} K={K} N={N} rank={rank}", flush=True)
        packed, absmax, a, b, bias = _layer(N, K, rank, seed=10 + i, dev=dev)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16).to(dev)
        st, y = _noalloc(x, packed, absmax, N, a, b, 2.0, bias)
        assert st == 0, nat.status_string(st)
        want = ops.nf4_linear(x, packed, absmax, N, 64, bias, lora_a=a, lora_b=b, scaling=2.0)
        torch.cuda.synchronize(dev)
        assert torch.equal(y, want), f"call {i} differs from rq_nf4_linear"


def test_noalloc_gemm_and_fp32_paths(dev):
    """The MFMA GEMM (LoRA operand, K splits on the k/v shape) and the fp32
    path, each twice in a row."""
    for M, K, N, dt in [(300, 4096, 1024, torch.bfloat16), (300, 4096, 1024, torch.bfloat16),
                        (16, 1024, 512, torch.float32), (3, 1024, 512, torch.float32)]:
        print(f"noalloc M={M} K={K} N={N} {dt}", flush=True)
        packed, absmax, a, b, _ = _layer(N, K, 16, seed=M + N, dev=dev)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(dt).to(dev)
        st, y = _noalloc(x, packed, absmax, N, a, b, 0.5)
        assert st == 0, nat.status_string(st)
        want = ops.nf4_linear(x, packed, absmax, N, 64, lora_a=a, lora_b=b, scaling=0.5)
        torch.cuda.synchronize(dev)
        assert torch.equal(y, want)


def test_noalloc_rejects_oversized_call(dev):
    """A GEMM whose workspace exceeds the array even without K splits (its
    16-bit LoRA operand alone, M x rank x 2 bytes, is 32 MiB here) returns
    RQ_ERR_SCRATCH_LIMIT before launching anything (the output keeps its
    sentinel)."""
    M, K, N, rank = 65536, 4096, 1024, 256
    assert M * rank * 2 >= 32 << 20
    packed, absmax, a, b, _ = _layer(N, K, rank, seed=3, dev=dev)
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)  # 512 MiB
    y = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=dev)
    st = nat.load().rq_nf4_linear_noalloc(
        x.data_ptr(), nat.DTYPE_BF16, M, K, K, packed.data_ptr(), N, 64, absmax.data_ptr(),
        nat.dtype_code(absmax.dtype), None, 0, 256, None, 0, None, 0, a.data_ptr(), b.data_ptr(), rank,
        nat.DTYPE_F32, rank, 1.0, y.data_ptr(), N, nat.stream_handle(dev))
    torch.cuda.synchronize(dev)
    assert st == SCRATCH_LIMIT
    assert bool((y == 7.0).all())
