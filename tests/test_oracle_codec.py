"""Pins the oracle (oracle/qlora_ref.py, torch restatement) against the
independent bit-level C restatement (oracle/codec_ref.c), known answers and
closed forms, and pins the HIP kernels' NF4 decision tables exhaustively.
CPU only."""
import math
import re
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import codec_ref as C
from oracle import qlora_ref as R

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "rocm-qlora_amd" / "csrc"


def _header_u32(name, text):
    body = re.search(name + r"\[\d+\] = \{([^}]*)\}", text, re.S).group(1)
    return [int(x, 16) for x in re.findall(r"0x([0-9A-Fa-f]{8})u", body)]


def test_nf4_table_bits_agree_three_ways():
    """torch's fp32 table == C cast of the decimal literals == the kernels' bits."""
    torch_bits = torch.tensor(R.NF4_VALUES, dtype=torch.float32).view(torch.int32).numpy().view(np.uint32)
    c_bits = C.nf4_table().view(np.uint32)
    kern = np.array(_header_u32("kNF4Bits", (CSRC / "rq_common.h").read_text()), dtype=np.uint32)
    assert np.array_equal(torch_bits, c_bits)
    assert np.array_equal(torch_bits, kern)
    assert list(np.diff(torch_bits.view(np.float32)) > 0) == [True] * 15  # sorted, as the tables assume


def test_nf4_decision_tables_exhaustive():
    """The kernels' cell table + one compare equals brute-force argmin for every
    fp32 in [-1, 1] (2.13e9 values)."""
    text = (CSRC / "nf4_tables.h").read_text()
    thr = np.array(_header_u32("kNF4CellThr", text), dtype=np.uint32)
    base = np.array([int(x) for x in re.search(r"kNF4CellBase\[64\] = \{([^}]*)\}", text).group(1).split(",")],
                    dtype=np.uint8)
    assert thr.size == 64 and base.size == 64
    parts = 64
    with ThreadPoolExecutor(8) as ex:
        res = list(ex.map(lambda p: C.nf4_exhaustive(thr, base, p, parts), range(parts)))
    bad = sum(b for b, _ in res)
    first = next((f for b, f in res if b), None)
    assert bad == 0, f"{bad} mismatches, first at 0x{first:08x}"


def test_brute_force_argmin_matches_torch_argmin():
    """The C brute-force rule is torch.argmin's rule (first minimum, NaN -> 0)."""
    g = torch.Generator().manual_seed(1)
    n = torch.cat([torch.rand(20000, generator=g) * 2 - 1,
                   torch.tensor(R.NF4_VALUES), torch.tensor([0.0, -0.0, float("nan")]),
                   # exact midpoints of adjacent levels (ties)
                   (torch.tensor(R.NF4_VALUES[:-1]) + torch.tensor(R.NF4_VALUES[1:])) / 2])
    table = torch.tensor(R.NF4_VALUES, dtype=torch.float32)
    t_idx = torch.argmin(torch.abs(n.unsqueeze(-1) - table), dim=-1)
    c_idx = torch.tensor([C.lib().ref_nf4_argmin(float(v)) for v in n])
    assert torch.equal(t_idx, c_idx)


def _weights(shape, dtype, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(shape, generator=g) * 0.02
    if outliers:
        flat = w.view(-1)
        k = max(1, flat.numel() // 1000)
        pos = torch.randperm(flat.numel(), generator=g)[:k]
        sign = torch.randint(0, 2, (k,), generator=g).float() * 2 - 1
        flat[pos] = 0.16 * sign
    return w.to(dtype)


def _edge_weights(dtype, block):
    """zero blocks, constant blocks, exact code points, a NaN block, tiny values."""
    rows = []
    rows.append(torch.zeros(block))
    rows.append(torch.full((block,), 0.37))
    rows.append(torch.full((block,), -0.37))
    s = 0.05
    rows.append(torch.tensor([R.NF4_VALUES[i % 16] * s for i in range(block)]))
    nan_row = torch.randn(block) * 0.02
    nan_row[3] = float("nan")
    rows.append(nan_row)
    rows.append(torch.randn(block) * 1e-30)
    inf_row = torch.randn(block)
    inf_row[5] = float("inf")
    rows.append(inf_row)
    return torch.cat(rows).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block", [32, 64, 128])
def test_quantize_int4_oracle_vs_c(dtype, block):
    for w in (_weights((37, 300), dtype, 3), _edge_weights(dtype, block)):
        p_t, s_t = R.quantize_int4(w, block)
        p_c, s_c = C.nf4_quantize(w, block)
        assert np.array_equal(p_t.numpy(), p_c)
        same = (s_t.view(torch.int16 if dtype != torch.float32 else torch.int32) ==
                s_c.view(torch.int16 if dtype != torch.float32 else torch.int32))
        assert bool((same | (torch.isnan(s_t) & torch.isnan(s_c))).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dequantize_int4_oracle_vs_c(dtype):
    w = _weights((64, 256), dtype, 5)
    packed, s = R.quantize_int4(w, 64)
    ref = R.dequantize_int4(packed, s, 64)
    for od, code in ((torch.float32, "f32"), (torch.bfloat16, "bf16"), (torch.float16, "f16")):
        c = C.nf4_dequantize(packed.numpy(), s, 64, code)
        assert torch.equal(ref.to(od).float(), c.float())


def test_known_answer_blocks():
    # all-zero block: every code 7 (0x77 bytes), absmax clamped to fp32(1e-12)
    p, s = R.quantize_int4(torch.zeros(64), 64)
    assert p.tolist() == [0x77] * 32 and s.item() == np.float32(1e-12)
    # a block equal to s * T[j] re-quantizes to codes j (identity on codes)
    s0 = 0.0123
    codes = torch.arange(64) % 16
    w = torch.tensor(R.NF4_VALUES)[codes] * s0
    p, _ = R.quantize_int4(w, 64)
    assert torch.equal(p, (codes[0::2] | (codes[1::2] << 4)).to(torch.uint8))
    # constant blocks: +c -> 15, -c -> 0
    assert R.quantize_int4(torch.full((64,), 3.0), 64)[0].tolist() == [0xFF] * 32
    assert R.quantize_int4(torch.full((64,), -3.0), 64)[0].tolist() == [0x00] * 32
    # nibble order: element 2j low, 2j+1 high
    w = torch.zeros(64)
    w[0], w[1] = -1.0, 1.0
    assert R.quantize_int4(w, 64)[0][0].item() == 0xF0
    # padding: 37x73 pads to a multiple of 64
    p, s = R.quantize_int4(torch.randn(37 * 73), 64)
    assert p.numel() == math.ceil(37 * 73 / 64) * 32 and s.numel() == math.ceil(37 * 73 / 64)


def test_nf4_roundtrip_error_bounds():
    """quant_ops invariants: |dequant - w| <= s * (max level gap) / 2, and the
    reference's own roundtrip bound (tests/test_quant_ops.py:47-63)."""
    torch.manual_seed(42)
    w = torch.randn(4096)
    p, s = R.quantize_int4(w, 64)
    d = R.dequantize_int4(p, s, 64)
    gap = max(b - a for a, b in zip(R.NF4_VALUES, R.NF4_VALUES[1:]))
    err = (d - w).abs().view(-1, 64)
    assert bool((err <= s.view(-1, 1) * gap / 2 * (1 + 1e-6)).all())
    assert (d - w).abs().max() < 0.15 * w.abs().max()


def test_fnuz_cast_vs_c_all_bf16_and_dense_fp32():
    """torch's fp32 -> float8_e4m3fnuz cast equals the C nearest-code search on
    every bf16 value and on a dense fp32 sweep of [0, 1] plus each code midpoint."""
    all_bf16 = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    sweep = torch.from_numpy(np.arange(0, 0x3F800001, 97, dtype=np.uint32).view(np.float32))
    vals = torch.tensor([C.lib().ref_fnuz_to_f32(c) for c in range(256) if c != 0x80])
    v_sorted = torch.sort(vals.unique()).values
    mids = ((v_sorted[:-1].double() + v_sorted[1:].double()) / 2).float()
    over = torch.tensor([239.9, 240.0, 247.9, 248.0, 250.0, 255.9, 256.0, 1e6, -248.0])
    for x in (all_bf16, sweep, mids, -mids, over):
        x = x[~torch.isnan(x)]
        t_codes = x.to(torch.float8_e4m3fnuz).view(torch.uint8).numpy()
        c_codes = C.fnuz_encode(x.numpy())
        assert np.array_equal(t_codes, c_codes)


def test_bf16_rounding_vs_c():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(200000, generator=g) * torch.exp(torch.randn(200000, generator=g) * 8)
    # include exact ties
    ties = torch.from_numpy((np.arange(1, 5000, dtype=np.uint32) << 15 | 0x3F800000).view(np.float32))
    x = torch.cat([x, ties, -ties])
    assert np.array_equal(x.to(torch.bfloat16).float().numpy(), C.round_array(x.numpy(), "bf16"))
    x16 = x[x.abs() < 60000]
    assert np.array_equal(x16.to(torch.float16).float().numpy(), C.round_array(x16.numpy(), "f16"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("use_fp8", [True, False])
def test_double_quant_oracle_vs_c(dtype, use_fp8):
    w = _weights((96, 512), dtype, 11)
    packed, c2, c2s, _ = R.double_quantize(w, 64, 256, use_fp8=use_fp8)
    _, c1 = R.quantize_int4(w, 64)
    c2_c, c2s_c = C.dq_quantize(c1, 256, int8=not use_fp8)
    assert np.array_equal(c2.view(torch.uint8).numpy() if use_fp8 else c2.view(torch.uint8).numpy(), c2_c)
    assert torch.equal(c2s.float(), c2s_c.float())
    ref = R.double_dequantize(packed, c2, c2s, w.shape, 64, 256, use_fp8)
    got = C.dq_dequantize(packed.numpy(), c2_c, c2s_c, 64, 256, int8=not use_fp8, n_out=w.numel())
    assert torch.equal(ref.reshape(-1), got)


def test_double_quant_known_answers():
    # the c1 that attains each 256-block max encodes to fnuz 0x40 (= 1.0)
    w = _weights((64, 1024), torch.float32, 2)
    _, c2, c2s, _ = R.double_quantize(w, 64, 256)
    codes = c2.view(torch.uint8).view(-1, 256)
    _, c1 = R.quantize_int4(w, 64)
    amax_pos = c1.view(-1, 256).abs().argmax(dim=1)
    assert bool((codes[torch.arange(codes.shape[0]), amax_pos] == 0x40).all())
    # bits saved closed form 0.5 - (8/64 + 32/(64*256)) = 0.37305 (tests/v4/test_double_quant.py:75-81)
    from rocm_qlora.quantization.double_quant import estimate_double_quant_savings
    est = estimate_double_quant_savings(torch.empty(4096, 4096))
    assert abs(est["bits_saved_per_param"] - (0.5 - (8 / 64 + 32 / (64 * 256)))) < 1e-9


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_int8_oracle_vs_c(dtype):
    w = _weights((48, 200), dtype, 13)
    q_t, s_t = R.quantize_int8(w.flatten(), 64)
    q_c, s_c = C.int8_quantize(w, 1, w.numel(), 64)
    assert np.array_equal(q_t.numpy(), q_c) and torch.equal(s_t.float(), s_c.float())
    q_t, s_t = R.quantize_int8(w, per_channel=True)
    q_c, s_c = C.int8_quantize(w, 48, 200, 0)
    assert np.array_equal(q_t.numpy().reshape(-1), q_c) and torch.equal(s_t.float(), s_c.float())
    # fp32: +-127 at each row's absmax element.  bf16: the scale is rounded to
    # bf16 (relative error <= 2^-9), so absmax / scale lies in 127 * (1 +- 2^-9)
    # and the bf16 quotient rounds to 126.5..127.5 -> 126 or 127 (never 128).
    row_max = q_t.abs().max(dim=1).values
    if dtype == torch.float32:
        assert bool((row_max == 127).all())
    else:
        assert bool(((row_max == 127) | (row_max == 126)).all())


def test_int8_roundtrip_bound():
    """tests/test_quant_ops.py:13-29 -- error < 1% of max with an outlier."""
    torch.manual_seed(42)
    t = torch.randn(1024) * 2.0
    t[0] = 100.0
    q, s = R.quantize_int8(t, 64)
    d = R.dequantize_int8(q, s, 64)
    assert (t - d[:1024]).abs().max() < 0.01 * t.abs().max()


def test_fp8_recipe_known_answers():
    """The absmax element of each tensor encodes to fnuz 0x7F (= 240)."""
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(64, 128, generator=g) * 0.02).to(torch.bfloat16)
    codes, scale = R.fp8_quantize_tensor(w)
    flat = codes.view(torch.uint8).view(-1)
    i = w.float().abs().view(-1).argmax()
    assert flat[i].item() in (0x7F, 0xFF)
    assert scale.dtype == torch.float32
    assert scale.item() == np.float32(w.float().abs().max().item() / 240.0)
