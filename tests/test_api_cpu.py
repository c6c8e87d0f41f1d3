"""Host-side checks of the Python API mirror (names, buffers, flags, model
surgery, error behaviour) that need no GPU.  Model surgery is exercised with
QuantLinear.from_linear patched to the oracle's quantizer, so the module-tree
logic of quantize_model is tested here; the real quantizer and every forward
pass are covered by the GPU tests."""
import math

import pytest
import torch
import torch.nn as nn

import rocm_qlora
from oracle import qlora_ref as R
from rocm_qlora import QuantLinear, LoRALinear, quantize_model, enable_all_kernels


def test_public_names_of_the_reference_api():
    # rocm_qlora/__init__.py, quantization/__init__.py:5-23, kernels/__init__.py:5-23,
    # hip_kernels/__init__.py:22-36, fp8/__init__.py of the reference
    import rocm_qlora.quantization as q
    import rocm_qlora.kernels as k
    import rocm_qlora.hip_kernels as h
    import rocm_qlora.fp8 as f
    import rocm_qlora.lora as lo
    import rocm_qlora.model as mo
    for mod, names in [
        (q, ["quantize_int4", "dequantize_int4", "quantize_int8", "dequantize_int8", "NF4_VALUES",
             "QuantLinear", "DoubleQuantState", "double_quantize", "double_dequantize",
             "patch_quant_linear_for_double_quant", "estimate_double_quant_savings"]),
        (k, ["fused_dequant_nf4_matmul", "fused_dequant_int8_matmul", "dequantize_nf4_triton",
             "get_kernel_config", "get_device_info", "is_triton_available"]),
        (h, ["is_hip_kernel_available", "enable_hip_kernels", "hip_dequant_int4_matmul",
             "hip_dequant_int8_matmul", "benchmark_hip_vs_triton"]),
        (f, ["detect_fp8_support", "FP8Config", "get_fp8_dtype", "get_fp8_recipe", "FP8LinearWrapper",
             "wrap_model_for_fp8", "enable_fp8_autocast"]),
        (lo, ["LoRALinear"]),
        (mo, ["quantize_model"]),
        (rocm_qlora, ["QuantLinear", "LoRALinear", "quantize_model", "enable_all_kernels",
                      "fused_dequant_nf4_matmul", "fused_dequant_int8_matmul", "get_device_info",
                      "is_triton_available", "is_hip_kernel_available", "enable_hip_kernels",
                      "hip_dequant_int4_matmul", "hip_dequant_int8_matmul", "benchmark_hip_vs_triton",
                      "find_hipcc", "is_hipcc_available", "compile_hip_kernel", "get_or_compile_int4_kernel"]),
    ]:
        for n in names:
            assert hasattr(mod, n), f"{mod.__name__} lacks {n}"
    from rocm_qlora.model.quantize_model import enable_all_kernels as e2  # noqa: F401
    from rocm_qlora.kernels.kernel_config import TritonKernelConfig  # noqa: F401
    from rocm_qlora.hip_kernels import int4_matmul, build_utils  # noqa: F401


@pytest.mark.parametrize("bits,qdtype", [(8, torch.int8), (4, torch.uint8)])
def test_quant_linear_buffers(bits, qdtype):
    """quant_linear.py:38-53: buffers, dtypes, flags, no parameters."""
    ql = QuantLinear(64, 128, bits=bits)
    sd = ql.state_dict()
    assert {"weight_quant", "weight_scales", "weight_zeros", "bias"} <= set(sd)
    assert ql.weight_quant.dtype == qdtype
    assert ql.merged_fp16_weight is None and ql.merged_mode is False
    assert ql.use_triton_kernel is False and ql.use_double_quant is False
    assert list(ql.parameters()) == []
    assert not hasattr(ql, "weight")
    assert ql.original_shape == (128, 64)
    assert QuantLinear(64, 128, bias=False).bias is None
    assert repr(ql) == f"QuantLinear(in=64, out=128, bits={bits}, block_size=64)"


def test_enable_kernel_returns_bool():
    layer = QuantLinear(64, 64)
    res = layer.enable_kernel()
    assert isinstance(res, bool)
    if res:
        assert layer.use_triton_kernel is True and layer.use_hip_kernel is True


def test_from_linear_rejects_bad_bits():
    with pytest.raises(ValueError, match="Unsupported bit depth"):
        QuantLinear.from_linear(nn.Linear(64, 64), bits=3)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the behaviour without a GPU")
def test_forward_without_gpu_raises():
    """No CPU execution path: a quantized forward on the CPU raises."""
    ql = QuantLinear(64, 128, bits=4)
    packed, absmax = R.quantize_int4(torch.randn(128, 64) * 0.02, 64)
    ql.weight_quant, ql.weight_scales = packed, absmax
    with pytest.raises(RuntimeError, match="GPU"):
        ql(torch.randn(2, 64))
    with pytest.raises(RuntimeError, match="GPU"):
        rocm_qlora.fused_dequant_nf4_matmul(torch.randn(2, 64), packed, absmax)


def test_merged_mode_forward_is_plain_linear():
    """quant_linear.py:126-130: merged fp16 weight -> F.linear, no dequantization."""
    ql = QuantLinear(64, 32, bits=4)
    w16 = (torch.randn(32, 64) * 0.1).to(torch.float16)
    ql.merged_fp16_weight = w16
    ql.merged_mode = True
    ql.bias.normal_()
    x = torch.randn(3, 64)
    assert torch.equal(ql(x), torch.nn.functional.linear(x, w16.float(), ql.bias))


def test_lora_init_and_trainables():
    """lora_layer.py:22-49: A Kaiming-uniform(a=sqrt 5) drawn from the CPU
    generator exactly as nn.init does, B zeros, s = alpha / r, base frozen."""
    ql = QuantLinear(64, 128)
    torch.manual_seed(5)
    lora = LoRALinear(ql, r=8, lora_alpha=32)
    torch.manual_seed(5)
    a = torch.empty(8, 64)
    nn.init.kaiming_uniform_(a, a=math.sqrt(5))
    assert torch.equal(lora.lora_A.data, a)
    assert float(lora.lora_A.detach().abs().max()) <= 1 / math.sqrt(64)
    assert torch.count_nonzero(lora.lora_B) == 0
    assert lora.scaling == 4.0
    names = [n for n, p in lora.named_parameters() if p.requires_grad]
    assert names == ["lora_A", "lora_B"]
    assert lora.get_trainable_params() == 64 * 8 + 128 * 8
    assert isinstance(lora.lora_dropout, nn.Identity)
    assert isinstance(LoRALinear(ql, lora_dropout=0.1).lora_dropout, nn.Dropout)
    assert "scaling=4.0000" in repr(lora)


def test_unmerge_without_merge_raises():
    lora = LoRALinear(QuantLinear(64, 64), r=4)
    with pytest.raises(RuntimeError, match="not merged"):
        lora.unmerge_lora()


class _FakeAttention(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(128, 128)
        self.k_proj = nn.Linear(128, 128)
        self.v_proj = nn.Linear(128, 128)
        self.o_proj = nn.Linear(128, 128)
        self.ff = nn.Linear(128, 512)


class _FakeTransformer(nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([_FakeAttention() for _ in range(4)])
        self.tiny_proj = nn.Linear(32, 32)


@pytest.fixture
def oracle_quantizer(monkeypatch):
    """QuantLinear.from_linear with the oracle's quantizer (CPU), so the
    surgery logic runs without a GPU."""
    def from_linear(cls, linear, bits=8, block_size=64):
        inst = cls(linear.in_features, linear.out_features, bits=bits, bias=linear.bias is not None,
                   block_size=block_size)
        flat = linear.weight.data.flatten()
        q, s = (R.quantize_int8(flat, block_size) if bits == 8 else R.quantize_int4(flat, block_size))
        inst.weight_quant, inst.weight_scales = q, s
        if linear.bias is not None:
            inst.bias = linear.bias.data.clone()
        del linear.weight
        return inst
    monkeypatch.setattr(QuantLinear, "from_linear", classmethod(from_linear))


def test_quantize_model_targets_and_counts(oracle_quantizer, capsys):
    """quantize_model.py:36-123 behaviour: suffix match on target_modules,
    small layers skipped, everything else frozen, only adapters trainable."""
    model = _FakeTransformer()
    quantize_model(model, bits=8, lora_r=8, target_modules=["q_proj", "v_proj", "tiny_proj"])
    for layer in model.layers:
        assert isinstance(layer.q_proj, LoRALinear) and isinstance(layer.v_proj, LoRALinear)
        assert isinstance(layer.k_proj, nn.Linear) and isinstance(layer.ff, nn.Linear)
        assert layer.q_proj.lora_dropout.p == 0.05
    assert isinstance(model.tiny_proj, nn.Linear)  # 32 < 64: skipped
    trainable = sum(p.numel() for p in model.parameters() if p.requires_grad)
    assert trainable == 8 * (8 * 128 + 128 * 8)
    assert not any(p.requires_grad for n, p in model.named_parameters() if "lora_" not in n)
    assert "Model Quantization Summary" in capsys.readouterr().out


def test_quantize_model_invalid_bits():
    with pytest.raises(ValueError, match="Only 4 and 8 bits are supported"):
        quantize_model(_FakeTransformer(), bits=3)


def test_enable_all_kernels_counts_each_layer_once(oracle_quantizer):
    model = _FakeTransformer()
    quantize_model(model, bits=4, target_modules=["q_proj"])
    n = enable_all_kernels(model)
    from rocm_qlora import _native
    assert n == (4 if _native.available() else 0)


def test_kernel_config_and_device_info(monkeypatch):
    from rocm_qlora.kernels import get_kernel_config, get_device_info, is_triton_available
    from rocm_qlora.kernels import kernel_config as kc
    assert isinstance(get_kernel_config(), kc.TritonKernelConfig)
    info = get_device_info()
    assert {"arch", "compute_units", "vram_gb", "wavefront_size", "triton_available"} <= set(info)
    assert is_triton_available() is False

    class _Props:
        name = "AMD Instinct MI355X"
        gcnArchName = "gfx950:sramecc+:xnack-"
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda i=0: _Props())
    assert kc.detect_gpu_arch() == "cdna4"
    cfg = get_kernel_config()
    assert (cfg.BLOCK_M, cfg.BLOCK_N, cfg.BLOCK_K, cfg.wavefront_size) == (256, 128, 64, 64)


def test_cdna4_config_matches_library():
    """get_kernel_config's gfx950 entry describes the GEMM the library runs
    (rq_gemm_tile_config: tile rows, columns, k step, waves, LDS stages)."""
    import ctypes
    from rocm_qlora import _native as nat
    from rocm_qlora.kernels import kernel_config as kc
    out = (ctypes.c_int32 * 5)()
    nat.call("rq_gemm_tile_config", out)
    c = kc.CDNA4_CONFIG
    assert list(out) == [c.BLOCK_M, c.BLOCK_N, c.BLOCK_K, c.num_warps, c.num_stages]


def test_build_utils_and_enable_hip_kernels_without_gpu():
    from rocm_qlora.hip_kernels.build_utils import find_hipcc, is_hipcc_available, compile_hip_kernel
    from rocm_qlora.hip_kernels import enable_hip_kernels, is_hip_kernel_available
    assert find_hipcc() is None or isinstance(find_hipcc(), str)
    assert isinstance(is_hipcc_available(), bool)
    assert compile_hip_kernel("/nonexistent/x.hip", "/tmp/rq_nonexistent.so") is False
    model = nn.Sequential(QuantLinear(32, 64, bits=4), nn.ReLU(), QuantLinear(64, 32, bits=8))
    n = enable_hip_kernels(model)
    assert n == (2 if is_hip_kernel_available() else 0)
    assert all(isinstance(m.use_hip_kernel, bool) for m in model if isinstance(m, QuantLinear))


def test_fp8_config_names():
    from rocm_qlora.fp8 import get_fp8_dtype, FP8Config, detect_fp8_support, get_fp8_recipe
    assert get_fp8_dtype("e4m3") == torch.float8_e4m3fnuz
    assert get_fp8_dtype("e5m2") == torch.float8_e5m2fnuz
    with pytest.raises(ValueError):
        get_fp8_dtype("e3m4")
    cfg = FP8Config()
    assert cfg.enabled and cfg.forward_dtype == "e4m3" and cfg.amax_history_len == 16
    info = detect_fp8_support()
    assert {"fp8_supported", "rocm_version", "arch", "fp8_dtypes_available",
            "transformer_engine_available", "reason"} <= set(info)
    assert get_fp8_recipe(cfg) is None  # no TransformerEngine in this image


def test_estimate_double_quant_savings_closed_form():
    """Bits saved per parameter with 64 / 256 blocks: 32/64 - (8/64 + 32/16384)
    = 0.373046875 (tests/v4/test_double_quant.py:75-81 of the reference)."""
    from rocm_qlora.quantization import estimate_double_quant_savings
    r = estimate_double_quant_savings(torch.empty(4096 * 4096))
    assert abs(r["bits_saved_per_param"] - 0.373046875) < 1e-9


def test_custom_operators_registered_with_fake_shapes():
    """The HIP entry points are torch.library custom operators whose fake
    implementations give the output shapes and dtypes (what torch.compile
    traces with)."""
    import rocm_qlora  # noqa: F401  (registers the operators)
    from torch._subclasses.fake_tensor import FakeTensorMode
    for name in ("nf4_linear", "nf4_linear_dx", "int8_linear", "fp8_quantize", "fp8_linear"):
        assert hasattr(torch.ops.rocm_qlora, name)
    with FakeTensorMode():
        x = torch.empty(3, 5, 256, dtype=torch.bfloat16)
        p = torch.empty(64 * 128, dtype=torch.uint8)
        s = torch.empty(256)
        y = torch.ops.rocm_qlora.nf4_linear(x, p, s, 64, 64, None, None, None, 256, True, None, None, 0.0, None)
        assert y.shape == (3, 5, 64) and y.dtype == torch.bfloat16
        d = torch.ops.rocm_qlora.nf4_linear_dx(y, p, s, 256, 64, None, None, 256, True, None, None, 0.0, None, 1.0)
        assert d.shape == (3, 5, 256) and d.dtype == torch.bfloat16
        q = torch.empty(64, 256, dtype=torch.int8)
        y8 = torch.ops.rocm_qlora.int8_linear(x, q, torch.empty(64), 64, 0, None)
        assert y8.shape == (3, 5, 64)
        c, sc = torch.ops.rocm_qlora.fp8_quantize(x)
        assert c.shape == (15, 256) and c.dtype == torch.float8_e4m3fnuz and sc.shape == () and sc.dtype == torch.float32
        yf = torch.ops.rocm_qlora.fp8_linear(x, torch.empty(64, 256, dtype=torch.float8_e4m3fn), sc, None)
        assert yf.shape == (3, 5, 64) and yf.dtype == torch.bfloat16
