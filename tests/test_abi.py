"""The C-ABI library loads, exports every symbol include/rocm_qlora_amd.h
declares, and validates arguments before touching the GPU.  CPU only: every
call here returns before any HIP call."""
import ctypes
import re
from pathlib import Path

import pytest

from rocm_qlora import _native as nat

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "rocm_qlora_amd.h"


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b((?:rq|launch)_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = nat.load()
    syms = declared_symbols()
    assert len(syms) >= 8
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_python_signatures_cover_header():
    assert set(declared_symbols()) <= set(nat.SIGNATURES)


def test_linear_sync_area_size_matches_header():
    from rocm_qlora import ops
    m = re.search(r"#define RQ_LINEAR_SYNC_BYTES (\d+)", HEADER.read_text())
    assert m and int(m.group(1)) == ops.LINEAR_SYNC_BYTES


def test_linear_workspace_holds_sync_area():
    """A GEMV with LoRA needs at least the synchronization area; a GEMM that
    needs workspace gets it after the area."""
    from rocm_qlora import ops
    nb = ctypes.c_int64(0)
    nat.call("rq_nf4_linear_workspace_size", nat.DTYPE_BF16, 1, 4096, 4096, 16, ctypes.byref(nb))
    assert nb.value >= ops.LINEAR_SYNC_BYTES
    nat.call("rq_nf4_linear_workspace_size", nat.DTYPE_BF16, 1, 4096, 4096, 0, ctypes.byref(nb))
    assert nb.value == 0
    nat.call("rq_nf4_linear_workspace_size", nat.DTYPE_BF16, 2048, 4096, 4096, 64, ctypes.byref(nb))
    assert nb.value > ops.LINEAR_SYNC_BYTES


def test_status_strings_and_version():
    assert nat.status_string(0) == "ok"
    assert "dtype" in nat.status_string(2)
    assert nat.load().rq_version() >= 100
    assert nat.load().rq_build_arch() == b"gfx950"


def _raw(name):
    return getattr(nat.load(), name)


def test_argument_validation_without_gpu():
    nf4q = _raw("rq_nf4_quantize")
    assert nf4q(None, 7, 64, 64, None, None, None) == 2            # bad dtype
    assert nf4q(None, 0, 64, 3, None, None, None) == 3             # odd block
    assert nf4q(None, 0, 0, 64, None, None, None) == 0             # empty is a no-op
    assert nf4q(None, 0, 64, 64, None, None, None) == 1            # null pointers
    deq = _raw("rq_nf4_dequantize")
    assert deq(None, None, 0, 32, 64, None, 0, 65, None) == 3      # n_out > 2 * n_packed
    assert deq(None, None, 0, 30, 64, None, 0, 60, None) == 3      # ragged block
    assert deq(None, None, 0, 32, 64, None, 0, 64, None) == 1
    dq = _raw("rq_dq_quantize")
    assert dq(None, 0, 10, 256, 9, None, None, None) == 2          # bad c2 format
    i8 = _raw("rq_int8_quantize")
    assert i8(None, 0, -1, 4, 0, None, None, None) == 3


def test_cpu_tensor_without_gpu_raises():
    import torch
    from rocm_qlora.quantization import quantize_int4
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(RuntimeError, match="GPU"):
        quantize_int4(torch.randn(128))
