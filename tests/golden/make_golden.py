"""Generate tests/golden/q8_0_kat.json: known-answer vectors for the Q8_0 path.

glypr has no golden vectors at the Q8_0-op level (its only Q8_0 unit test
compares two runtime implementations, metal_kernels/mod.rs:1924-1979, and its
end-to-end goldens need the real EmbeddingGemma weights).  These vectors are
fixed by mathematics alone - exact integer/power-of-two arithmetic and the
special cases of the GGML Q8_0 definition (BlockQ8_0::from_float / to_float /
vec_dot, geglu_scalar_f32's clamps, pool_and_normalize's closed form) - and
are computed here with Python integers and fractions, never with the oracle
or the GPU code they check.

    python tests/golden/make_golden.py      # rewrites q8_0_kat.json
"""
from __future__ import annotations

import json
import math
import os
import struct
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "q8_0_kat.json")


def f32_bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def exact_f32(fr: Fraction) -> int:
    """Bits of an f32 that must equal `fr` exactly (asserted)."""
    v = float(fr)
    b = f32_bits(v)
    assert Fraction(struct.unpack("<f", struct.pack("<I", b))[0]) == fr, fr
    return b


def f16_value(bits: int) -> Fraction:
    s = -1 if bits & 0x8000 else 1
    e = (bits >> 10) & 0x1F
    m = bits & 0x3FF
    assert e != 0x1F
    if e == 0:
        return s * Fraction(m, 1 << 24)
    return s * Fraction(1024 + m, 1024) * Fraction(2) ** (e - 15)


def round_half_away(fr: Fraction) -> int:
    """Rust f32::round on an exactly representable value."""
    a = abs(fr)
    r = int(a) + (1 if a - int(a) >= Fraction(1, 2) else 0)
    return r if fr >= 0 else -r


def exact_product_bits(a: float, b: float) -> int:
    """IEEE product of two values whose exact product fits an f32 (signed zeros
    follow the IEEE sign rule; the magnitude is checked with fractions)."""
    p = a * b
    assert Fraction(p) == Fraction(a) * Fraction(b)
    return exact_f32(Fraction(p)) if p != 0 else f32_bits(p)


def dequant_cases():
    """BlockQ8_0::to_float: y = (f32)q * f32(d) is exact in f32."""
    q = [-128, -127, -64, -1, 0, 1, 2, 3, 63, 64, 100, 126, 127] * 3
    q = q[:32]
    cases = []
    for dbits in [0x3C00, 0x3800, 0xC000, 0x0001, 0x0400, 0x7BFF, 0x0000, 0x8000, 0x3555,
                  0x2E66]:
        d = math.copysign(float(f16_value(dbits)), -1.0 if dbits & 0x8000 else 1.0)
        cases.append({"d_bits": dbits, "qs": q,
                      "y_bits": [exact_product_bits(float(v), d) for v in q]})
    return cases


def quantize_cases():
    """BlockQ8_0::from_float on inputs whose answer is fixed exactly.

    Each case: 32 f32 inputs (bits), expected f16 d bits and int8 qs."""
    cases = []

    def add(name, xs, dbits, qs):
        assert len(xs) == 32 and len(qs) == 32
        cases.append({"name": name, "x_bits": [f32_bits(v) for v in xs], "d_bits": dbits,
                      "qs": qs})

    # all zero: d = 0, id = 0, q = 0
    add("zeros", [0.0] * 32, 0x0000, [0] * 32)
    # amax = 127 -> d = 1 exactly, id = 1: q = round half away from zero (numpy's
    # round-half-even would give 2 for 2.5 and -2 for -2.5).
    xs = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5, 3.5, -3.5, 0.49999997,
          -0.49999997, 4.5, 5.5, -5.5] + [float(i) for i in range(-8, 8)]
    add("half_away_from_zero", xs, 0x3C00, [round_half_away(Fraction(v)) for v in xs])
    # lossless: x = k * 2^e with max |k| = 127 -> d = 2^e exact in f16, q = k.
    for e in (-3, 0, 5, -20):
        ks = [((i * 37) % 255) - 127 for i in range(32)]
        ks[7] = -127
        xs = [float(Fraction(k) * Fraction(2) ** e) for k in ks]
        dbits = {-3: 0x3000, 0: 0x3C00, 5: 0x5000, -20: 0x0010}[e]  # 2^-20 is f16 subnormal
        assert f16_value(dbits) == Fraction(2) ** e
        add(f"lossless_e{e}", xs, dbits, ks)
    # amax at a negative position
    xs = [float(v) for v in range(-127, -95)]
    add("negative_amax", xs, 0x3C00, list(range(-127, -95)))
    # f16 overflow of d: amax = 127 * 65536 -> d = 65536 -> f16 inf; id = 2^-16 exact.
    xs = [127.0 * 65536.0] + [float(v) * 65536.0 for v in range(-15, 16)]
    add("d_overflows_f16", xs, 0x7C00, [127] + list(range(-15, 16)))
    # NaN is ignored by the amax (f32::max) and converts to q = 0 (`NaN as i8`).
    xs = [float("nan"), 127.0] + [float(v) for v in range(30)]
    add("nan_ignored", xs, 0x3C00, [0, 127] + list(range(30)))
    return cases


def vec_dot_cases():
    """Lossless operands (power-of-two scales): the dot is an exact integer sum."""
    cases = []
    for nb, ew, ex in [(1, 0, 0), (4, -7, -3), (24, -8, -6), (36, -10, 2)]:
        k = nb * 32
        wq = [((i * 53 + 11) % 255) - 127 for i in range(k)]
        xq = [((i * 29 + 5) % 255) - 127 for i in range(k)]
        total = sum(a * b for a, b in zip(wq, xq)) * Fraction(2) ** (ew + ex)
        dw = {0: 0x3C00, -7: 0x2000, -8: 0x1C00, -10: 0x1400}[ew]
        dx = {0: 0x3C00, -3: 0x3000, -6: 0x2400, 2: 0x4400}[ex]
        assert f16_value(dw) == Fraction(2) ** ew and f16_value(dx) == Fraction(2) ** ex
        # every per-block partial sum and the running f32 sum stay exact integers
        # times 2^(ew+ex) below 2^24, so f32 arithmetic in any order is exact.
        cases.append({"k": k, "w_d_bits": dw, "x_d_bits": dx, "wq": wq, "xq": xq,
                      "y_bits": exact_f32(total)})
    return cases


def geglu_cases():
    """geglu_scalar_f32's exact points: g <= -10 -> 0; g >= 10 -> g*u; g = 0 -> 0*u."""
    pts = []
    for g, u in [(-10.0, 3.0), (-1e6, -2.0), (-10.5, 0.25), (10.0, 3.0), (12.5, -0.5),
                 (1e3, 0.125), (0.0, 2.0), (0.0, -2.0)]:
        if g <= -10:
            y = 0.0
        elif g >= 10:
            y = float(Fraction(g) * Fraction(u))
        else:  # g == 0: act = (0.5*0)*(1+tanh(0)) = +0, times u keeps u's sign
            y = math.copysign(0.0, u)
        pts.append({"g_bits": f32_bits(g), "u_bits": f32_bits(u), "y_bits": f32_bits(y)})
    return pts


def rmsnorm_cases():
    """Constant row c = +-2^k with eps = 0: sum of squares d*c^2 is exact, inv = 1/|c|
    exactly, so y = sign(c) * w bit-exactly (any reduction order)."""
    cases = []
    for d, c in [(768, 0.25), (768, -8.0), (256, 2.0), (32, -0.5)]:
        w = [float(Fraction(1) + Fraction((i * 7) % 64 - 32, 64)) for i in range(d)]
        y = [math.copysign(1.0, c) * v for v in w]
        cases.append({"d": d, "c_bits": f32_bits(c), "w_bits": [f32_bits(v) for v in w],
                      "y_bits": [f32_bits(v) for v in y]})
    return cases


def pool_cases():
    """All tokens equal to v = 2^k * (3, 4, 0, ...): mean = v exactly (t a power of two),
    L2 -> (3/5, 4/5, 0, ...) correctly rounded; MRL to 1 dim -> (1)."""
    d, t = 64, 512
    v = [0.0] * d
    v[0], v[1] = 3.0 * 0.125, 4.0 * 0.125
    return [{"t": t, "d": d, "v_bits": [f32_bits(x) for x in v],
             "l2_bits": [f32_bits(0.6), f32_bits(0.8)] + [0] * (d - 2),
             "mrl1_bits": [f32_bits(1.0)]}]


def main():
    data = {
        "description": "Known-answer vectors for the Q8_0 path, fixed by exact arithmetic "
                       "(see make_golden.py).",
        "dequant": dequant_cases(),
        "quantize": quantize_cases(),
        "vec_dot": vec_dot_cases(),
        "geglu": geglu_cases(),
        "rmsnorm": rmsnorm_cases(),
        "pool": pool_cases(),
    }
    with open(OUT, "w") as f:
        json.dump(data, f, separators=(",", ":"))
        f.write("\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
