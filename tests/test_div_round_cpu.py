"""The quantizers' shortcut for RND16(x / s) (div_round in csrc/rq_common.h),
checked by brute force on the CPU.

The kernels compute a 16-bit tensor's `x / s` (quant_ops.py:38 `reshaped /
scales`, double_quant.py's `c1 / c2_scale`, fp8_linear.py:37's `x / scale`)
as RND16(RN32(x * RN32(1 / s))) and divide exactly only where the bits of
that product below 16-bit precision lie within 4 of the rounding midpoint,
where it is not finite, or (fp16) where it is below fp16's normal range.
Here every finite bf16 / fp16 value x is tried against about two thousand
scales s (random over many binades, powers of two, all-ones mantissas, the
clamp floor, subnormals, the extremes), with numpy's IEEE float32 operations:
on every element the shortcut keeps, its result must equal the exactly
rounded quotient's, bit for bit.
"""
import numpy as np
import pytest

MID = {"bf16": (0xFFFF, 0x8000), "f16": (0x1FFF, 0x1000)}


def _all_finite(dt):
    bits = np.arange(1 << 16, dtype=np.uint32)
    if dt == "bf16":
        v = (bits << 16).view(np.float32)
    else:
        v = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    return v[np.isfinite(v)]


def _round16(v, dt):
    """RNE of float32 values to the 16-bit dtype, as float32 bit patterns."""
    if dt == "f16":
        with np.errstate(over="ignore"):
            return v.astype(np.float16).astype(np.float32).view(np.uint32)
    b = v.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    r = r.astype(np.uint32)
    nan = np.isnan(v)
    r[nan] = 0x7FC00000
    return r


def _scales(rng):
    s = [np.float32(2.0) ** e for e in range(-40, 20)]
    s += [np.float32((2.0 - 2.0 ** -23) * 2.0 ** e) for e in range(-30, 10)]
    s += [np.float32(1e-12), np.float32(2.0 ** -126), np.float32(2.0 ** -140), np.float32(1.5 * 2.0 ** -149),
          np.float32(3.4e38), np.float32(1.0 / 240.0), np.float32(0.02), np.float32(127.0)]
    mant = rng.uniform(1.0, 2.0, size=1900)
    expo = rng.integers(-30, 12, size=1900)
    s += list((mant * 2.0 ** expo).astype(np.float32))
    return np.array(s, dtype=np.float32)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_div_round_matches_exact_rounded_quotient(dt):
    rng = np.random.default_rng(7)
    x = _all_finite(dt)
    low, mid = MID[dt]
    kept = 0
    with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
        for s in _scales(rng):
            rs = np.float32(1.0) / s
            r = x * rs
            b = r.view(np.uint32)
            exact = (((b & low) - np.uint32(mid - 4)) <= 8) | ((b & 0x7F800000) == 0x7F800000)
            if dt == "f16":
                exact |= (b & 0x7FFFFFFF) < 0x38800000
            q = x / s
            keep = ~exact
            got, want = _round16(r[keep], dt), _round16(q[keep], dt)
            bad = np.nonzero(got != want)[0]
            assert bad.size == 0, (dt, float(s), float(x[keep][bad[0]]))
            kept += int(keep.sum())
    # the shortcut is the common case (fp16: quotients below its normal range,
    # frequent with the large scales here, divide exactly)
    assert kept > 0.9 * len(x) * len(_scales(np.random.default_rng(7)))


def test_div_round_fallback_detects_a_planted_midpoint_case():
    """A quotient whose fast product sits next to a bf16 midpoint is one the
    shortcut hands to the exact division (the planted mistake: a window of 0
    would keep it and round it the wrong way)."""
    rng = np.random.default_rng(3)
    x = _all_finite("bf16")
    low, mid = MID["bf16"]
    found = False
    with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
        for s in _scales(rng)[:400]:
            rs = np.float32(1.0) / s
            r = x * rs
            q = x / s
            fin = np.isfinite(r) & np.isfinite(q)
            diff = _round16(r[fin], "bf16") != _round16(q[fin], "bf16")
            if diff.any():
                b = r[fin][diff].view(np.uint32)
                assert np.all(((b & low) - np.uint32(mid - 4)) <= 8)
                found = True
    assert found, "no scale produced a midpoint case; the window would be untested"
