"""The device quantizer's rounding identity, checked on the CPU.

Every Q8_0 quantizer on the GPU (activation quantize, RMSNorm prologue, GeGLU
epilogue, int8 vector codec) rounds v = x * id with

    q = clamp(cvt_i32(RN(v + copysign(0.49999997, v))), -128, 127)

where cvt_i32 is v_cvt_i32_f32 (truncate toward zero, saturate, NaN -> 0).
BlockQ8_0::from_float (glypr k_quants, via candle) and the int8 codec
(glypr-core/src/util.rs) use Rust's `f32::round(v) as i8`: half away from zero,
saturating, NaN -> 0.  This test holds the two equal on ties, their float
neighbours, specials and a random sample of all bit patterns; with
GLYPR_EXHAUSTIVE=1 it covers all 2^32 patterns (a few minutes).
"""
import os

import numpy as np

HALF_PRED = np.float32(0.49999997)


def ref_round_i8(v):
    """Rust `f32::round(v) as i8`: half away from zero, saturating, NaN -> 0."""
    with np.errstate(invalid="ignore"):
        a = np.abs(v.astype(np.float64))
        r = np.floor(a + 0.5) * np.sign(v)        # exact in f64 for f32 inputs
        r = np.where(np.isnan(v), 0.0, np.clip(r, -128.0, 127.0))
    return r.astype(np.int64)


def device_round_i8(v):
    """RN(v + copysign(pred(0.5), v)) in f32, then v_cvt_i32_f32, then clamp."""
    with np.errstate(invalid="ignore", over="ignore"):
        s = (v + np.copysign(HALF_PRED, v)).astype(np.float32)
        t = np.trunc(s.astype(np.float64))
        t = np.where(np.isnan(s), 0.0, np.clip(t, -2.0 ** 31, 2.0 ** 31 - 1))
    return np.clip(t, -128, 127).astype(np.int64)


def check(v):
    v = np.ascontiguousarray(v, dtype=np.float32)
    a, b = ref_round_i8(v), device_round_i8(v)
    bad = np.flatnonzero(a != b)
    assert bad.size == 0, (f"{bad.size} mismatches, first v={v[bad[0]]!r} "
                           f"ref {a[bad[0]]} device {b[bad[0]]}")


def test_ties_neighbours_and_specials():
    k = np.arange(-300, 301, dtype=np.float32)
    ties = np.concatenate([k + np.float32(0.5), k])
    near = np.concatenate([np.nextafter(ties, np.float32(np.inf)),
                           np.nextafter(ties, np.float32(-np.inf))])
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 1e-45, -1e-45,
                         HALF_PRED, -HALF_PRED, 2.0 ** 23 + 1, -(2.0 ** 23) - 1, 2.0 ** 24,
                         3.0e38, -3.0e38, 127.49999, 127.5, -128.49998, -128.5],
                        dtype=np.float32)
    check(np.concatenate([ties, near, specials]))


def test_random_bit_patterns():
    rng = np.random.default_rng(3)
    check(rng.integers(0, 2 ** 32, size=4_000_000, dtype=np.uint64)
          .astype(np.uint32).view(np.float32))


def test_every_bit_pattern_when_asked():
    if os.environ.get("GLYPR_EXHAUSTIVE") != "1":
        return
    step = 1 << 26
    for start in range(0, 1 << 32, step):
        check(np.arange(start, start + step, dtype=np.uint64).astype(np.uint32)
              .view(np.float32))
