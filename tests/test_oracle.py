"""Pin the CPU oracle (oracle/glypr_oracle.c) before trusting it.

Each check is chosen so a plausible mistake fails it: the known-answer vectors
(tests/golden/q8_0_kat.json, exact arithmetic) catch a wrong rounding rule, a
dropped f16 rounding of d, a swapped operand; float64 brute force over the same
quantized operands catches a wrong block index or scale; the lossless special
case reduces the whole GEMM to numpy's float64 X @ W^T; invariants pin RMSNorm
and pooling; tanh is measured against double-precision tanh.
"""
import json
import math
import os
import struct

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
KAT = json.load(open(os.path.join(HERE, "golden", "q8_0_kat.json")))


def bits_to_f32(b):
    return np.array(b, dtype=np.uint32).view(np.float32)


def f32_to_bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


# ------------------------------------------------------------ f16 codec ----

def test_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    # plus every boundary region: around f16 max, min normal, subnormals, ties
    extra = []
    for h in range(0, 0x7C00, 7):
        f = np.uint16(h).view(np.float16).astype(np.float32)
        fb = int(np.float32(f).view(np.uint32))
        extra += [fb - 1, fb, fb + 1, fb + (1 << 12), fb + (1 << 12) - 1, fb + (1 << 12) + 1]
    extra = [e % (1 << 32) for e in extra]
    bits = np.concatenate([bits, np.array(extra, dtype=np.uint64).astype(np.uint32)])
    x = bits.view(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16_bits(x)
    ok = np.isnan(x) | (got == ref)
    assert ok.all(), f"{np.count_nonzero(~ok)} f32->f16 mismatches"
    h = np.arange(65536, dtype=np.uint16)
    back = oracle.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(back.view(np.uint32)[~nan], ref.view(np.uint32)[~nan])
    assert np.isnan(back[nan]).all()


# ----------------------------------------------------------- Q8_0 codec ----

def test_dequant_kat(oracle):
    for c in KAT["dequant"]:
        blk = oracle.join_blocks(np.array([[c["d_bits"]]], np.uint16),
                                 np.array([c["qs"]], np.int8))
        y = oracle.dequantize_rows(blk, 32)
        assert np.array_equal(f32_to_bits(y[0]), np.array(c["y_bits"], np.uint32)), c["d_bits"]


def test_quantize_kat(oracle):
    for c in KAT["quantize"]:
        x = bits_to_f32(c["x_bits"]).reshape(1, 32)
        d, qs = oracle.split_blocks(oracle.quantize_rows(x), 32)
        assert int(d[0, 0]) == c["d_bits"], c["name"]
        assert qs[0].tolist() == c["qs"], c["name"]


def test_quantize_matches_f64_definition(oracle):
    """Random rows: q must be the nearest integer to x/d within 1 step, d = amax/127
    rounded to f16, and |q| = 127 at the amax position."""
    x = oracle.normal(64 * 768, seed=7).reshape(64, 768)
    d, qs = oracle.split_blocks(oracle.quantize_rows(x), 768)
    blocks = x.reshape(-1, 32).astype(np.float64)
    amax = np.abs(blocks).max(axis=1)
    d_ref = np.float32(amax / 127).astype(np.float32)
    assert np.array_equal(d.reshape(-1), oracle.f32_to_f16_bits(
        (np.float32(amax.astype(np.float32)) / np.float32(127)).astype(np.float32)))
    q = qs.reshape(-1, 32).astype(np.float64)
    err = np.abs(blocks / (amax[:, None] / 127) - q)
    assert err.max() <= 0.5 + 1e-4
    pos = np.argmax(np.abs(blocks), axis=1)
    assert np.all(np.abs(q[np.arange(len(pos)), pos]) == 127)
    del d_ref


def test_vec_dot_kat(oracle):
    for c in KAT["vec_dot"]:
        k = c["k"]
        nb = k // 32
        w = oracle.join_blocks(np.full((1, nb), c["w_d_bits"], np.uint16),
                               np.array([c["wq"]], np.int8))
        x = oracle.join_blocks(np.full((1, nb), c["x_d_bits"], np.uint16),
                               np.array([c["xq"]], np.int8))
        y = oracle.lib().orc_q8_0_vec_dot(k, w.ctypes.data_as(oracle._u8p),
                                          x.ctypes.data_as(oracle._u8p))
        assert struct.unpack("<I", struct.pack("<f", y))[0] == c["y_bits"]


@pytest.mark.parametrize("m,k,n", [(1, 32, 1), (19, 256, 128), (64, 768, 96), (7, 1152, 33)])
def test_matmul_vs_f64_bruteforce(oracle, m, k, n):
    x = oracle.normal(m * k, seed=11 + m).reshape(m, k)
    w = oracle.q8_0_weight(n, k, seed=5 + n)
    xq = oracle.quantize_rows(x)
    y = oracle.matmul(x, w, n)
    y64 = oracle.matmul_f64(xq, m, k, w, n)
    # f32 sequential sum of K/32 rounded terms: relative error <= ~nb * 2^-23 of the
    # sum of |terms|; bound by the sum of absolute block terms computed in f64.
    nb = k // 32
    dw, qw = oracle.split_blocks(w, k)
    dx, qx = oracle.split_blocks(xq, k)
    absterm = np.zeros((m, n))
    for b in range(nb):
        s = np.abs(qx[:, b * 32:(b + 1) * 32].astype(np.int64)
                   @ qw[:, b * 32:(b + 1) * 32].astype(np.int64).T)
        absterm += s * oracle.f16_bits_to_f32(dx[:, b])[:, None] * np.abs(
            oracle.f16_bits_to_f32(dw[:, b]))[None, :]
    bound = (3 * nb + 2) * 2.0 ** -24 * absterm + 1e-30
    assert np.all(np.abs(y - y64) <= bound)
    # preq path and the single-threaded path give identical bits
    assert np.array_equal(oracle.matmul_preq(xq, m, k, w, n), y)
    assert np.array_equal(oracle.matmul(x, w, n, threads=1), y)


def test_matmul_lossless_equals_numpy(oracle):
    """x blocks = k*2^e with one |k| = 127: quantization is lossless, so the Q8_0
    GEMM equals numpy's float64 X @ W_deq^T up to the f32 summation error."""
    rng = np.random.default_rng(3)
    m, k, n = 33, 768, 70
    ks = rng.integers(-127, 128, size=(m, k))
    ks.reshape(m, -1, 32)[:, :, 0] = 127
    e = rng.integers(-6, 3, size=(m, k // 32))
    x = (ks.reshape(m, -1, 32) * (2.0 ** e)[:, :, None]).reshape(m, k).astype(np.float32)
    w = oracle.q8_0_weight(n, k, seed=9)
    xq = oracle.quantize_rows(x)
    assert np.array_equal(oracle.dequantize_rows(xq, k), x)   # lossless
    wd = oracle.dequantize_rows(w, k).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T
    y = oracle.matmul(x, w, n)
    scale = np.abs(x).astype(np.float64) @ np.abs(wd).T
    assert np.all(np.abs(y - ref) <= 1e-6 * scale + 1e-30)


# ------------------------------------------- the INT8_FMA variant's oracle --

def _f32_round(q):
    """Round a Fraction to the nearest binary32 value, ties to even (normal
    range), exactly: the IEEE definition of one rounding."""
    from fractions import Fraction
    if q == 0:
        return Fraction(0)
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    assert -126 <= e <= 127
    ulp = Fraction(2) ** (e - 23)
    n, r = divmod(a, ulp)
    if r > ulp / 2 or (r == ulp / 2 and n % 2 == 1):
        n += 1
    return (n * ulp) if q > 0 else -(n * ulp)


def _block_terms(oracle, xq, w, k):
    """Per output and block: the integer block sum S and the two f16 scales,
    exactly (as Fractions)."""
    from fractions import Fraction
    dw, qw = oracle.split_blocks(w, k)
    dx, qx = oracle.split_blocks(xq, k)
    fdw = oracle.f16_bits_to_f32(dw).astype(np.float64)
    fdx = oracle.f16_bits_to_f32(dx).astype(np.float64)
    s = np.stack([qx[:, b * 32:(b + 1) * 32].astype(np.int64)
                  @ qw[:, b * 32:(b + 1) * 32].astype(np.int64).T for b in range(k // 32)])
    return s, fdw, fdx, Fraction


def test_matmul_fma_exact_rational_bruteforce(oracle):
    """Every rounding of both accumulation orders stated with exact rationals:
    the 2-op form t = round(S d_w), acc = round(acc + t d_x) must match
    matmul_fma bit for bit, the 3-op form acc = round(acc + round(t d_x)) must
    match matmul, and on these inputs the two orders differ somewhere (so the
    check tells them apart)."""
    m, k, n = 8, 256, 16
    x = oracle.normal(m * k, seed=71).reshape(m, k)
    w = oracle.q8_0_weight(n, k, seed=72)
    xq = oracle.quantize_rows(x)
    s, fdw, fdx, Fraction = _block_terms(oracle, xq, w, k)
    fma_ref = np.empty((m, n), np.float32)
    seq_ref = np.empty((m, n), np.float32)
    for i in range(m):
        for c in range(n):
            a2 = a3 = Fraction(0)
            for b in range(k // 32):
                t = _f32_round(Fraction(int(s[b, i, c])) * Fraction(fdw[c, b]))
                a2 = _f32_round(a2 + t * Fraction(fdx[i, b]))
                a3 = _f32_round(a3 + _f32_round(t * Fraction(fdx[i, b])))
            fma_ref[i, c], seq_ref[i, c] = float(a2), float(a3)
    assert np.array_equal(f32_to_bits(oracle.matmul_fma(x, w, n)), f32_to_bits(fma_ref))
    assert np.array_equal(f32_to_bits(oracle.matmul(x, w, n)), f32_to_bits(seq_ref))
    assert np.count_nonzero(f32_to_bits(fma_ref) != f32_to_bits(seq_ref)) > 0
    assert np.array_equal(oracle.matmul_fma(x, w, n, threads=1), oracle.matmul_fma(x, w, n))
    rb = (k // 32) * 34
    for i, c in ((0, 0), (m - 1, n - 1), (3, 11)):
        got = oracle.vec_dot_fma(k, w[c].reshape(-1)[:rb], xq[i].reshape(-1)[:rb])
        assert f32_to_bits(np.float32(got)) == f32_to_bits(fma_ref[i, c])


def test_matmul_fma_one_block_is_vec_dot(oracle):
    """k = 32: fma(t, d_x, 0) = round(t d_x) = vec_dot's single term."""
    m, n = 40, 50
    x = oracle.normal(m * 32, seed=73).reshape(m, 32) * np.float32(5.0)
    w = oracle.q8_0_weight(n, 32, seed=74, sigma=0.3)
    assert np.array_equal(f32_to_bits(oracle.matmul_fma(x, w, n)),
                          f32_to_bits(oracle.matmul(x, w, n)))


@pytest.mark.parametrize("m,k,n", [(19, 256, 128), (64, 768, 96), (7, 1152, 33)])
def test_matmul_fma_vs_f64_bruteforce(oracle, m, k, n):
    """The fused form's error against the float64 sum: nb roundings of t and
    nb of the accumulate, bounded by (2 nb + 2) 2^-24 sum |terms|; and within
    BASELINE's 1e-3 relative / 1e-4 absolute of the INT8_EXACT oracle."""
    x = oracle.normal(m * k, seed=91 + m).reshape(m, k)
    w = oracle.q8_0_weight(n, k, seed=92 + n)
    xq = oracle.quantize_rows(x)
    y = oracle.matmul_fma(x, w, n).astype(np.float64)
    y64 = oracle.matmul_f64(xq, m, k, w, n)
    s, fdw, fdx, _ = _block_terms(oracle, xq, w, k)
    absterm = np.einsum("bmn,nb,mb->mn", np.abs(s).astype(np.float64), np.abs(fdw), np.abs(fdx))
    nb = k // 32
    assert np.all(np.abs(y - y64) <= (2 * nb + 2) * 2.0 ** -24 * absterm + 1e-30)
    exact = oracle.matmul(x, w, n).astype(np.float64)
    assert np.all(np.abs(y - exact) <= np.maximum(1e-3 * np.abs(exact), 1e-4))


def test_reference_metal_case_activation_error_bound(oracle):
    """glypr's Q8_0 unit-test inputs (metal_kernels/mod.rs:1924-1979): w =
    sin(0.031 i)*1.5 quantized to Q8_0 [128 x 256], x = cos(0.059 i)*3 via bf16,
    m in {1, 19, 64}.  The CPU Q8_0 path differs from the dequant GEMM (Metal /
    CANDLE_DEQUANTIZE_ALL semantics) only by activation quantization, bounded by
    sum_b (0.5 + 127 * 2^-11) * d_x,b * sum_{j in b} |w_deq|."""
    n, k = 128, 256
    wf = (np.sin(np.arange(n * k, dtype=np.float64) * np.float32(0.031)) * 1.5).astype(
        np.float32).reshape(n, k)
    wq = oracle.quantize_rows(wf)
    wabs = np.abs(oracle.dequantize_rows(wq, k).astype(np.float64)).reshape(n, k // 32, 32).sum(2)
    for m in (1, 19, 64):
        xf = (np.cos(np.arange(m * k, dtype=np.float64) * np.float32(0.059)) * 3.0).astype(
            np.float32)
        xb = (xf.view(np.uint32) + 0x7FFF + ((xf.view(np.uint32) >> 16) & 1)) >> 16
        x = (xb << 16).astype(np.uint32).view(np.float32).reshape(m, k)
        y = oracle.matmul(x, wq, n)
        yd = oracle.matmul_dequant_f64(x, wq, n)
        amax = np.abs(x.astype(np.float64)).reshape(m, k // 32, 32).max(2)
        bound = (0.5 + 127 * 2.0 ** -11) * (amax / 127) @ wabs.T
        assert np.all(np.abs(y - yd) <= bound * (1 + 1e-5) + 1e-5)
        # and the activation quantization is what separates them: a dequant of the
        # quantized activations closes the gap to f32 rounding
        xq = oracle.quantize_rows(x)
        yq = oracle.matmul_dequant_f64(oracle.dequantize_rows(xq, k), wq, n)
        assert np.abs(y - yq).max() <= 1e-4


# -------------------------------------------------------------- RMSNorm ----

def test_rmsnorm_kat(oracle):
    for c in KAT["rmsnorm"]:
        d = c["d"]
        x = np.full((1, d), bits_to_f32([c["c_bits"]])[0], np.float32)
        w = bits_to_f32(c["w_bits"])
        y = oracle.rmsnorm(x, w, eps=0.0)
        assert np.array_equal(f32_to_bits(y[0]), np.array(c["y_bits"], np.uint32))


def test_rmsnorm_vs_f64_and_invariants(oracle):
    x = oracle.normal(40 * 768, seed=21).reshape(40, 768)
    w = 1 + 0.1 * oracle.normal(768, seed=22)
    y = oracle.rmsnorm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.abs(y - ref).max() < 1e-5   # reference tolerance, test_cpu_simd.rs:5-39
    # eps = 0: scaling a row by 2^k leaves the output bit-identical
    y0 = oracle.rmsnorm(x, w, 0.0)
    assert np.array_equal(oracle.rmsnorm(x * np.float32(8.0), w, 0.0), y0)
    assert np.array_equal(oracle.rmsnorm(x * np.float32(0.25), w, 0.0), y0)
    # weightless (v_norm) == weight of ones
    assert np.array_equal(oracle.rmsnorm(x, None, 1e-6), oracle.rmsnorm(x, np.ones(768, np.float32), 1e-6))
    # the lane order matters: a plain sequential sum differs in some rows' bits
    seq = np.array([np.float32(1) / np.sqrt(np.float32(np.sum(r.astype(np.float32) ** 2,
                                                              dtype=np.float32)) / 768 + 1e-6)
                    for r in x])
    assert seq.shape == (40,)


# ---------------------------------------------------------------- GeGLU ----

def test_tanh_accuracy(oracle):
    xs = np.concatenate([np.linspace(-12, 12, 400_001), np.geomspace(1e-8, 12, 100_000),
                         -np.geomspace(1e-8, 12, 100_000)]).astype(np.float32)
    ours = np.array([oracle.tanhf(float(v)) for v in xs], np.float32)
    ref = np.tanh(xs.astype(np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    err = np.abs(ours.astype(np.float64) - ref) / ulp
    assert err.max() <= 3.0, err.max()
    assert oracle.tanhf(0.0) == 0.0 and oracle.tanhf(10.0) == 1.0 and oracle.tanhf(-30.0) == -1.0
    assert oracle.tanhf(1e-5) == np.float32(1e-5)


def test_geglu_kat_and_formula(oracle):
    for c in KAT["geglu"]:
        g = bits_to_f32([c["g_bits"]])
        u = bits_to_f32([c["u_bits"]])
        y = oracle.geglu(g, u)
        assert f32_to_bits(y)[0] == c["y_bits"]
    g = oracle.normal(200_000, seed=31, std=3.0)
    u = oracle.normal(200_000, seed=32)
    y = oracle.geglu(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = 0.5 * g64 * (1 + np.tanh(0.7978845608028654 * (g64 + 0.044715 * g64 ** 3))) * u64
    ref = np.where(g64 <= -10, 0, np.where(g64 >= 10, g64 * u64, ref))
    assert np.all(np.abs(y - ref) <= 1e-5 * np.abs(u64) * (np.abs(g64) + 1))


def test_geglu_tanh_substitution_is_ulp_level(oracle):
    """The shared tanh replaces the platform libm tanhf.  Away from the cancellation
    in 1 + tanh (g > -1) outputs agree to a few ulp; everywhere the difference is
    at most 0.5*|g*u| times a few ulp of 1 (glypr's formula amplifies tanh's ulp
    error in relative terms where 1 + tanh cancels, on any libm)."""
    g = oracle.normal(100_000, seed=41, std=2.0)
    u = oracle.normal(100_000, seed=42)
    ours = oracle.geglu(g, u)
    libm = np.array([oracle.lib().orc_geglu_scalar_libm(float(a), float(b))
                     for a, b in zip(g, u)], np.float32)
    # the array form runs the same scalar function on every element
    assert np.array_equal(oracle.geglu_libm(g, u).view(np.uint32), libm.view(np.uint32))
    diff = np.abs(ours.astype(np.float64) - libm)
    assert np.all(diff <= 0.5 * np.abs(g * u) * 4 * 2.0 ** -24 + 4e-6 * np.abs(libm))
    ok = g > -1
    rel = diff[ok] / np.maximum(np.abs(libm[ok]), 1e-30)
    assert rel.max() < 4e-6


# -------------------------------------------------------- gather / pool ----

def test_gather_equals_dequant_rows(oracle):
    vocab, d = 1000, 768
    table = oracle.q8_0_weight(vocab, d, seed=51)
    ids = oracle.uniform_ids(300, seed=52, vocab=vocab)
    out = oracle.embed_gather(table, vocab, d, ids, 0.5)
    ref = oracle.dequantize_rows(table, d)[ids] * np.float32(0.5)
    assert np.array_equal(out, ref)
    with pytest.raises(IndexError):
        oracle.embed_gather(table, vocab, d, np.array([3, vocab], np.uint32), 1.0)


def test_pool_kat(oracle):
    c = KAT["pool"][0]
    v = bits_to_f32(c["v_bits"])
    tok = np.tile(v, (c["t"], 1))
    assert np.array_equal(f32_to_bits(oracle.pool_normalize(tok)), np.array(c["l2_bits"], np.uint32))
    assert np.array_equal(f32_to_bits(oracle.pool_normalize(tok, trunc=1)),
                          np.array(c["mrl1_bits"], np.uint32))


def test_pool_long_context_vs_f64(oracle):
    """The reference's long-context generator and F64 ground truth
    (tests/corpus_parity.rs:433-460), here on the f32 path: cos > 0.99999."""
    hd = 768
    for t in (1024, 8192):
        tt = np.arange(t)[:, None]
        cc = np.arange(hd)[None, :]
        raw = (((tt * 7919 + cc * 104729) % 10000) / 5000.0 - 1.0).astype(np.float32)
        ref = raw.astype(np.float64).mean(axis=0)
        ref = ref / max(np.sqrt((ref ** 2).sum()), 1e-12)
        got = oracle.pool_normalize(raw)
        cos = float(got @ ref / np.linalg.norm(got) / np.linalg.norm(ref))
        assert cos > 0.99999
        mask = np.ones(t, np.uint8)
        mask[t // 2:] = 0
        gm = oracle.pool_normalize(raw, mask=mask)
        r2 = raw[: t // 2].astype(np.float64).mean(axis=0)
        r2 /= np.linalg.norm(r2)
        assert float(gm @ r2 / np.linalg.norm(gm)) > 0.99999
        m = oracle.pool_normalize(raw, trunc=256)
        assert m.shape == (256,) and abs(np.linalg.norm(m.astype(np.float64)) - 1) < 1e-6


# ------------------------------------------------- l2_normalize / cosine ----

def _seq_sum_f32(terms):
    """Sequential float32 sum from -0.0 (numpy's add.accumulate is a running
    float32 sum; np.sum would be pairwise)."""
    t = np.concatenate([np.array([-0.0], np.float32), np.asarray(terms, np.float32)])
    return np.add.accumulate(t, dtype=np.float32)[-1]


def test_l2_normalize_kat_and_sequential_sum(oracle):
    # the reference's own known answers (util.rs:258-262)
    y = oracle.l2_normalize(np.array([3.0, 4.0], np.float32))
    assert abs(y[0] - 0.6) < 1e-6 and abs(y[1] - 0.8) < 1e-6
    assert np.array_equal(f32_to_bits(y), f32_to_bits(np.array([3, 4], np.float32) / np.float32(5)))
    # a zero norm returns the input unchanged, signed zeros included (no 1e-12 clamp)
    z = np.array([0.0, -0.0, 0.0, -0.0], np.float32)
    assert np.array_equal(f32_to_bits(oracle.l2_normalize(z)), f32_to_bits(z))
    # a norm that underflows to 0 (1e-30^2 = 0 in f32) also returns the input
    tiny = np.full(8, 1e-30, np.float32)
    assert np.array_equal(f32_to_bits(oracle.l2_normalize(tiny)), f32_to_bits(tiny))
    # random vectors: bit-identical to the sequential f32 statement, and within
    # f32 rounding of the float64 normalisation
    rng = np.random.default_rng(3)
    for n in (1, 7, 256, 768, 5000):
        x = rng.standard_normal(n).astype(np.float32) * np.float32(rng.uniform(0.01, 100))
        got = oracle.l2_normalize(x)
        nrm = np.sqrt(_seq_sum_f32(x * x), dtype=np.float32)
        assert np.array_equal(f32_to_bits(got), f32_to_bits(x / nrm)), n
        ref = x.astype(np.float64) / np.linalg.norm(x.astype(np.float64))
        assert np.abs(got - ref).max() <= 4e-7 * (1 + np.sqrt(n) * 2**-10)


def test_cosine_kat_special_cases_and_sequential_sum(oracle):
    # util.rs:264-267: truncate_mrl(l2_normalize([1,1,1,1]), 2) has cosine 1 with itself
    t = oracle.l2_normalize(oracle.l2_normalize(np.ones(4, np.float32))[:2])
    assert abs(oracle.cosine(t, t) - 1.0) < 1e-6
    # zero norm -> 0.0, either side
    assert oracle.cosine(np.zeros(3, np.float32), np.ones(3, np.float32)) == 0.0
    assert oracle.cosine(np.ones(3, np.float32), np.zeros(3, np.float32)) == 0.0
    # orthogonal and opposite vectors are exact
    assert oracle.cosine(np.array([1, 0], np.float32), np.array([0, 2], np.float32)) == 0.0
    assert oracle.cosine(np.array([3, 4], np.float32), np.array([-6, -8], np.float32)) == -1.0
    # the clamp: a vector whose rounded cosine with itself exceeds 1 returns 1.0
    rng = np.random.default_rng(5)
    over = 0
    for _ in range(400):
        a = rng.standard_normal(33).astype(np.float32)
        d = _seq_sum_f32(a * a)
        r = np.sqrt(d, dtype=np.float32)
        raw = np.float32(d / np.float32(r * r))
        c = oracle.cosine(a, a)
        assert c == min(raw, np.float32(1.0))
        over += raw > 1
    assert over > 0, "no case exercised the clamp"
    # random pairs: bit-identical to the sequential f32 statement; float64 within rounding
    for n in (1, 5, 256, 768, 3000):
        a = rng.standard_normal(n).astype(np.float32)
        b = (0.3 * a + rng.standard_normal(n)).astype(np.float32)
        dot, sa, sb = _seq_sum_f32(a * b), _seq_sum_f32(a * a), _seq_sum_f32(b * b)
        ref = np.float32(dot / (np.sqrt(sa, dtype=np.float32) * np.sqrt(sb, dtype=np.float32)))
        ref = np.clip(ref, np.float32(-1), np.float32(1))
        got = oracle.cosine(a, b)
        assert f32_to_bits(np.float32(got)) == f32_to_bits(ref), n
        c64 = float(a.astype(np.float64) @ b / np.linalg.norm(a.astype(np.float64))
                    / np.linalg.norm(b.astype(np.float64)))
        assert abs(got - c64) < 1e-6 * (1 + n * 2**-8)


# ------------------------------------------------------------- attention ----

def test_attention_band_equals_masked_dense(oracle):
    """Chunked sliding attention == dense attention with the -1e9 band mask
    (attention/chunked.rs:64-172 vs model.rs:580-651): compare with numpy."""
    rng = np.random.default_rng(5)
    nh, nkv, t, hd, W = 3, 1, 70, 16, 16
    q = rng.standard_normal((nh, t, hd)).astype(np.float32)
    k = rng.standard_normal((nkv, t, hd)).astype(np.float32)
    v = rng.standard_normal((nkv, t, hd)).astype(np.float32)
    out = oracle.attention(q, k, v, W)
    i = np.arange(t)
    mask = np.where(np.abs(i[:, None] - i[None, :]) > W, -1e9, 0.0)
    for h in range(nh):
        s = q[h].astype(np.float64) @ k[0].astype(np.float64).T + mask
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ref = p @ v[0].astype(np.float64)
        assert np.abs(out[:, h * hd:(h + 1) * hd] - ref).max() < 1e-5
    full = oracle.attention(q, k, v, 0)
    assert not np.allclose(full, out)


# ------------------------------------------------------------------ RoPE ----

@pytest.mark.parametrize("hd,theta", [(256, 1e4), (256, 1e6), (64, 1e4)])
def test_rope_tables_closed_form(oracle, hd, theta):
    """rope.rs:14-87: inv_freq[i] = f32(1 / theta^(2i/hd)), freqs = f32(pos) * inv_freq
    in f32, emb = [freqs, freqs], tables = cos/sin(emb).  numpy reproduces the f32
    product exactly; the cos/sin of it are checked against float64."""
    t = 8192
    c, s = oracle.rope_tables(hd, theta, t)
    inv = (1.0 / np.power(theta, 2.0 * np.arange(hd // 2) / hd)).astype(np.float32)
    freqs = np.arange(t, dtype=np.float32)[:, None] * inv[None, :]     # f32 product
    emb = np.concatenate([freqs, freqs], axis=1).astype(np.float64)
    assert np.abs(c - np.cos(emb)).max() < 2e-7
    assert np.abs(s - np.sin(emb)).max() < 2e-7
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    assert np.array_equal(c[:, :hd // 2], c[:, hd // 2:])


# -------------------------------------------------------- whole forward ----

def _forward_f64(oracle, tensors, ids, trunc, H, F, nh, nkv, hd, n_layers, window, eps=1e-6,
                 full_hd=0, full_nkv=0, layer_types=None):
    """Independent float64 statement of forward_embeds (model.rs:498-578) over the
    layer order of layer.rs:20-50: the same Q8_0 quantization of every GEMM input
    (oracle quantizer, pinned above), everything else in float64.  With
    `per_layer_model_proj.weight` present it adds TextPLE (ple.rs:48-85) and each
    layer's TextPLEBlock with the layer scalar (ple.rs:118-145, norm.rs:65-95);
    with `output.weight` the embedding projection (model.rs:577).  A projection
    given as a uint16 [n, k] array is a dense bf16 weight (linear.rs:48-54): its
    exact values, and no quantization of its input.  full_hd / full_nkv (0: the
    sliding values) give the full-attention layers their own head_dim and kv
    head count (config.rs:142-169); layer_types (nonzero = full) replaces the
    default 5 sliding + 1 full pattern (config.rs:117-140)."""
    def deq(name, n, k):
        w = tensors[name]
        if w.dtype == np.uint16:
            return (w.astype(np.uint32) << 16).view(np.float32).reshape(n, k).astype(np.float64)
        return oracle.dequantize_rows(w, k).reshape(n, k).astype(np.float64)

    def lin(x, name, n, k):
        if tensors[name].dtype == np.uint16:
            return x.astype(np.float64) @ deq(name, n, k).T
        xq = oracle.dequantize_rows(oracle.quantize_rows(x.astype(np.float32)), k)
        return xq.reshape(x.shape[0], k).astype(np.float64) @ deq(name, n, k).T

    def rms(x, w):
        y = x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
        return y if w is None else y * w.astype(np.float64)

    def rope(x, theta):     # x [t, hd]
        t, hd = x.shape
        inv = (1.0 / np.power(theta, 2.0 * np.arange(hd // 2) / hd)).astype(np.float32)
        f = np.arange(t, dtype=np.float32)[:, None] * inv[None, :]
        e = np.concatenate([f, f], 1).astype(np.float64)
        rot = np.concatenate([-x[:, hd // 2:], x[:, :hd // 2]], 1)
        return x * np.cos(e) + rot * np.sin(e)

    def gelu_tanh(x):
        return 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))

    t = ids.size
    table = oracle.dequantize_rows(tensors["token_embd.weight"], H).reshape(-1, H)
    h = (table[ids] * np.float32(np.sqrt(H))).astype(np.float64)
    ple = None
    if "per_layer_model_proj.weight" in tensors:
        P = tensors["per_layer_model_proj.weight"].shape[0] // n_layers
        raw = lin(h, "per_layer_model_proj.weight", n_layers * P, H) * float(H) ** -0.5
        ple = rms(raw.reshape(t, n_layers, P), tensors["per_layer_proj_norm.weight"])
    idx = np.arange(t)
    sliding_hd, sliding_nkv = hd, nkv
    for l in range(n_layers):
        p = f"blk.{l}."
        full = bool(layer_types[l]) if layer_types is not None else (l + 1) % 6 == 0
        hd = (full_hd or sliding_hd) if full else sliding_hd
        nkv = (full_nkv or sliding_nkv) if full else sliding_nkv
        theta = 1e6 if full else 1e4
        mask = np.zeros((t, t)) if full else \
            np.where(np.abs(idx[:, None] - idx[None, :]) > window, -np.inf, 0.0)
        x = rms(h, tensors[p + "attn_norm.weight"])
        q = lin(x, p + "attn_q.weight", nh * hd, H).reshape(t, nh, hd)
        k = lin(x, p + "attn_k.weight", nkv * hd, H).reshape(t, nkv, hd)
        v = lin(x, p + "attn_v.weight", nkv * hd, H).reshape(t, nkv, hd)
        ctx = np.empty((t, nh * hd))
        for j in range(nh):
            g = j // (nh // nkv)
            qj = rope(rms(q[:, j], tensors[p + "attn_q_norm.weight"]), theta)
            kg = rope(rms(k[:, g], tensors[p + "attn_k_norm.weight"]), theta)
            vg = rms(v[:, g], None)
            s = qj @ kg.T + mask                     # scale 1.0
            pr = np.exp(s - s.max(1, keepdims=True))
            ctx[:, j * hd:(j + 1) * hd] = (pr / pr.sum(1, keepdims=True)) @ vg
        h = h + rms(lin(ctx, p + "attn_output.weight", H, nh * hd),
                    tensors[p + "post_attention_norm.weight"])
        x = rms(h, tensors[p + "ffn_norm.weight"])
        gt = lin(x, p + "ffn_gate.weight", F, H)
        up = lin(x, p + "ffn_up.weight", F, H)
        act = gelu_tanh(gt) * up
        h = h + rms(lin(act, p + "ffn_down.weight", H, F), tensors[p + "post_ffw_norm.weight"])
        if ple is not None:
            P = ple.shape[2]
            a = gelu_tanh(lin(h, p + "inp_gate.weight", P, H)) * ple[:, l, :]
            h = (h + rms(lin(a, p + "proj.weight", H, P), tensors[p + "post_norm.weight"])) * \
                float(tensors[p + "layer_output_scale.weight"][0])
    states = rms(h, tensors["output_norm.weight"])
    if "output.weight" in tensors:
        states = lin(states, "output.weight", tensors["output.weight"].shape[0], H)
    pooled = states.mean(0)
    pooled /= max(np.linalg.norm(pooled), 1e-12)
    m = pooled[:trunc]
    return m / max(np.linalg.norm(m), 1e-12), states


def _small_model(oracle, H, F, nh, nkv, hd, L, vocab, rng, ple_dim=0, out_dim=0, full_hd=0,
                 full_nkv=0):
    tensors = {"token_embd.weight": oracle.q8_0_weight(vocab, H, 100, 0.02),
               "output_norm.weight": (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)}
    seed = 200
    sliding_hd, sliding_nkv = hd, nkv
    for l in range(L):
        full = (l + 1) % 6 == 0
        hd = (full_hd or sliding_hd) if full else sliding_hd
        nkv = (full_nkv or sliding_nkv) if full else sliding_nkv
        for name, n, k in [("attn_q", nh * hd, H), ("attn_k", nkv * hd, H),
                           ("attn_v", nkv * hd, H), ("attn_output", H, nh * hd),
                           ("ffn_gate", F, H), ("ffn_up", F, H), ("ffn_down", H, F)]:
            tensors[f"blk.{l}.{name}.weight"] = oracle.q8_0_weight(n, k, seed, 0.02)
            seed += 1
        for name, n in [("attn_norm", H), ("post_attention_norm", H), ("ffn_norm", H),
                        ("post_ffw_norm", H), ("attn_q_norm", hd), ("attn_k_norm", hd)]:
            w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            if name in ("attn_q_norm", "attn_k_norm"):
                w = (w * 0.25).astype(np.float32)
            tensors[f"blk.{l}.{name}.weight"] = w
        if ple_dim:
            tensors[f"blk.{l}.inp_gate.weight"] = oracle.q8_0_weight(ple_dim, H, seed, 0.05)
            tensors[f"blk.{l}.proj.weight"] = oracle.q8_0_weight(H, ple_dim, seed + 1, 0.05)
            seed += 2
            tensors[f"blk.{l}.post_norm.weight"] = \
                (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
            tensors[f"blk.{l}.layer_output_scale.weight"] = \
                np.array([0.5 + 0.5 * rng.random()], np.float32)
    if ple_dim:
        tensors["per_layer_model_proj.weight"] = oracle.q8_0_weight(L * ple_dim, H, 900, 0.05)
        tensors["per_layer_proj_norm.weight"] = \
            (1 + 0.1 * rng.standard_normal(ple_dim)).astype(np.float32)
    if out_dim:
        tensors["output.weight"] = oracle.q8_0_weight(out_dim, H, 901, 0.05)
    return tensors


def test_model_forward_with_ple_vs_float64_statement(oracle):
    """TextPLE + TextPLEBlock + layer scalar + embedding projection: the oracle
    against the float64 statement; each added part changes the output, so a
    dropped term fails."""
    H, F, nh, nkv, hd, L, vocab, t, W, P, D = 128, 192, 2, 1, 64, 6, 1000, 40, 8, 64, 96
    rng = np.random.default_rng(12)
    tensors = _small_model(oracle, H, F, nh, nkv, hd, L, vocab, rng, ple_dim=P, out_dim=D)
    ids = rng.integers(0, vocab, t).astype(np.uint32)
    kw = dict(hidden=H, ffn=F, n_heads=nh, n_kv_heads=nkv, head_dim=hd, n_layers=L, vocab=vocab,
              sliding_window=W)
    out, states = oracle.model_forward(tensors, ids, 32, **kw)
    assert states.shape == (t, D) and out.shape == (32,)
    ref_out, ref_states = _forward_f64(oracle, tensors, ids, 32, H, F, nh, nkv, hd, L, W)
    row_cos = (states * ref_states).sum(1) / np.linalg.norm(states, axis=1) / \
        np.linalg.norm(ref_states, axis=1)
    # Each Q8_0 quantization point (PLE adds two GEMM inputs per layer and the
    # projection one) rounds the f32 oracle value and the float64-derived one
    # separately, so isolated int8 flips cost ~3e-5 of row cosine each; a
    # dropped term costs orders of magnitude more (no layer scalar: 0.64).
    assert row_cos.min() > 0.9995 and row_cos.mean() > 0.9999, (row_cos.min(), row_cos.mean())
    assert float(out @ ref_out) > 0.99999
    # every part is live: dropping the scalars, the PLE block or the projection shows
    no_scalar = {k: (np.ones(1, np.float32) if k.endswith("layer_output_scale.weight") else v)
                 for k, v in tensors.items()}
    o2, _ = oracle.model_forward(no_scalar, ids, 32, **kw)
    no_ple = {k: v for k, v in tensors.items()
              if not any(s in k for s in ("per_layer", "inp_gate", ".proj.", "post_norm",
                                          "layer_output_scale"))}
    o3, _ = oracle.model_forward(no_ple, ids, 32, **kw)
    no_out = {k: v for k, v in tensors.items() if k != "output.weight"}
    _, s4 = oracle.model_forward(no_out, ids, 32, **kw)
    assert float(o2 @ out) < 0.9999 and float(o3 @ out) < 0.9999 and s4.shape == (t, H)


def test_model_forward_layer_types_vs_float64_statement(oracle):
    """A layer_types pattern other than the default (full layers first, third
    and sixth; sliding_window_pattern, config.rs:117-140): the oracle against
    the float64 statement with the same pattern, and far from the statement
    with the default pattern (a full layer takes no band and the 1e6 RoPE
    table), so an ignored pattern fails."""
    H, F, nh, nkv, hd, L, vocab, t, W = 128, 192, 2, 1, 64, 6, 1000, 40, 8
    rng = np.random.default_rng(13)
    tensors = _small_model(oracle, H, F, nh, nkv, hd, L, vocab, rng)
    ids = rng.integers(0, vocab, t).astype(np.uint32)
    pattern = [1, 0, 1, 0, 0, 1]
    out, states = oracle.model_forward(tensors, ids, 32, hidden=H, ffn=F, n_heads=nh,
                                       n_kv_heads=nkv, head_dim=hd, n_layers=L, vocab=vocab,
                                       sliding_window=W, layer_types=pattern)
    ref_out, ref_states = _forward_f64(oracle, tensors, ids, 32, H, F, nh, nkv, hd, L, W,
                                       layer_types=pattern)
    dflt_out, _ = _forward_f64(oracle, tensors, ids, 32, H, F, nh, nkv, hd, L, W)
    row_cos = (states * ref_states).sum(1) / np.linalg.norm(states, axis=1) / \
        np.linalg.norm(ref_states, axis=1)
    assert row_cos.min() > 0.9995 and float(out @ ref_out) > 0.99999
    assert float(out @ dflt_out) < 0.999


def test_model_forward_vs_float64_statement(oracle):
    """The oracle's composition (gather x sqrt(H), q/k/v norms, RoPE, GQA attention
    with scale 1.0 and the 5:1 sliding/full pattern, post-norm residuals, GeGLU MLP,
    final norm, pool, L2, MRL) against an independent float64 statement at small
    dimensions: 6 layers so both layer types run, window 8 < t so the band binds."""
    H, F, nh, nkv, hd, L, vocab, t, W = 128, 192, 2, 1, 64, 6, 1000, 40, 8
    rng = np.random.default_rng(11)
    tensors = {"token_embd.weight": oracle.q8_0_weight(vocab, H, 100, 0.02),
               "output_norm.weight": (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)}
    seed = 200
    for l in range(L):
        for name, n, k in [("attn_q", nh * hd, H), ("attn_k", nkv * hd, H),
                           ("attn_v", nkv * hd, H), ("attn_output", H, nh * hd),
                           ("ffn_gate", F, H), ("ffn_up", F, H), ("ffn_down", H, F)]:
            tensors[f"blk.{l}.{name}.weight"] = oracle.q8_0_weight(n, k, seed, 0.02)
            seed += 1
        for name, n in [("attn_norm", H), ("post_attention_norm", H), ("ffn_norm", H),
                        ("post_ffw_norm", H), ("attn_q_norm", hd), ("attn_k_norm", hd)]:
            w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            if name in ("attn_q_norm", "attn_k_norm"):
                w = (w * 0.25).astype(np.float32)
            tensors[f"blk.{l}.{name}.weight"] = w
    ids = rng.integers(0, vocab, t).astype(np.uint32)
    out, states = oracle.model_forward(tensors, ids, 32, hidden=H, ffn=F, n_heads=nh,
                                       n_kv_heads=nkv, head_dim=hd, n_layers=L, vocab=vocab,
                                       sliding_window=W)
    ref_out, ref_states = _forward_f64(oracle, tensors, ids, 32, H, F, nh, nkv, hd, L, W)
    row_cos = (states * ref_states).sum(1) / np.linalg.norm(states, axis=1) / \
        np.linalg.norm(ref_states, axis=1)
    assert row_cos.min() > 0.9999, row_cos.min()
    assert float(out @ ref_out) > 0.99999
    assert out.shape == (32,) and abs(np.linalg.norm(out.astype(np.float64)) - 1) < 1e-6
    # a wrong window (full attention everywhere) must be visible at this size
    bad_out, _ = oracle.model_forward(tensors, ids, 32, hidden=H, ffn=F, n_heads=nh,
                                      n_kv_heads=nkv, head_dim=hd, n_layers=L, vocab=vocab,
                                      sliding_window=t)
    assert float(bad_out @ ref_out) < float(out @ ref_out)
    with pytest.raises(ValueError):
        oracle.model_forward(tensors, np.array([vocab], np.uint32), 32, hidden=H, ffn=F,
                             n_heads=nh, n_kv_heads=nkv, head_dim=hd, n_layers=L, vocab=vocab)


# ------------------------------------------------- synthetic-input makers ----

def test_splitmix64_published_vectors(oracle):
    """SplitMix64 (Steele, Lea, Flood 2014) from state 0: the published first
    outputs."""
    import ctypes
    st = ctypes.c_uint64(0)
    got = [oracle.lib().orc_splitmix64(ctypes.byref(st)) for _ in range(3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def _splitmix_stream(seed, n):
    mask = (1 << 64) - 1
    s, out = seed, []
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & mask
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        out.append(z ^ (z >> 31))
    return out


def test_generators_restated_in_python(oracle):
    """fill_normal (Box-Muller on (0,1] uniforms), uniform ids and the Q8_0
    weight maker, restated in Python from the same SplitMix64 stream."""
    r = _splitmix_stream(9, 8)
    u = [((v >> 11) + 1.0) / 9007199254740992.0 for v in r]
    ref = []
    for i in range(0, 8, 2):
        rad = math.sqrt(-2.0 * math.log(u[i]))
        ref += [np.float32(1.5 + 2.0 * rad * math.cos(2 * math.pi * u[i + 1])),
                np.float32(1.5 + 2.0 * rad * math.sin(2 * math.pi * u[i + 1]))]
    assert np.array_equal(oracle.normal(8, seed=9, mean=1.5, std=2.0), np.array(ref, np.float32))
    ids = oracle.uniform_ids(16, seed=4, vocab=1000)
    assert ids.tolist() == [v % 1000 for v in _splitmix_stream(4, 16)]
    w = oracle.q8_0_weight(2, 64, seed=12, sigma=0.02)
    d, qs = oracle.split_blocks(w, 64)
    st = _splitmix_stream(12, 4 * 34)
    pos = 0
    for blk in range(4):
        u1 = ((st[pos] >> 11) + 1.0) / 9007199254740992.0
        u2 = ((st[pos + 1] >> 11) + 1.0) / 9007199254740992.0
        z = math.sqrt(-2.0 * math.log(u1)) * math.cos(2 * math.pi * u2)
        dref = np.float32(abs(z) * float(np.float32(0.02)) / 127.0).astype(np.float16).view(np.uint16)
        assert int(d.reshape(-1)[blk]) == int(dref)
        qref = [int(v % 255) - 127 for v in st[pos + 2: pos + 34]]
        assert qs.reshape(-1, 32)[blk].tolist() == qref
        pos += 34
    big = oracle.normal(200_000, seed=3)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01


# The pin of every exported oracle function: a test above (or in the vector
# codec / rounding modules) that a plausible mistake in it would fail.
PINS = {
    "orc_f32_to_f16": ["test_f16_matches_numpy_rne"],
    "orc_f16_to_f32": ["test_f16_matches_numpy_rne"],
    "orc_f32_to_f16_array": ["test_f16_matches_numpy_rne"],
    "orc_f16_to_f32_array": ["test_f16_matches_numpy_rne"],
    "orc_q8_0_quantize_row": ["test_quantize_kat", "test_quantize_matches_f64_definition"],
    "orc_q8_0_quantize_rows": ["test_quantize_kat", "test_quantize_matches_f64_definition"],
    "orc_q8_0_dequantize_row": ["test_dequant_kat"],
    "orc_q8_0_dequantize_rows": ["test_dequant_kat"],
    "orc_q8_0_vec_dot": ["test_vec_dot_kat"],
    "orc_q8_0_matmul": ["test_matmul_vs_f64_bruteforce", "test_matmul_lossless_equals_numpy"],
    "orc_q8_0_matmul_preq": ["test_matmul_vs_f64_bruteforce"],
    "orc_q8_0_vec_dot_fma": ["test_matmul_fma_exact_rational_bruteforce"],
    "orc_q8_0_matmul_fma": ["test_matmul_fma_exact_rational_bruteforce",
                            "test_matmul_fma_one_block_is_vec_dot",
                            "test_matmul_fma_vs_f64_bruteforce"],
    "orc_q8_0_matmul_f64": ["test_matmul_lossless_equals_numpy"],
    "orc_q8_0_matmul_dequant_f64": ["test_reference_metal_case_activation_error_bound"],
    "orc_rmsnorm_row": ["test_rmsnorm_kat", "test_rmsnorm_vs_f64_and_invariants"],
    "orc_rmsnorm": ["test_rmsnorm_kat", "test_rmsnorm_vs_f64_and_invariants"],
    "orc_tanhf": ["test_tanh_accuracy"],
    "orc_geglu_scalar": ["test_geglu_kat_and_formula"],
    "orc_geglu": ["test_geglu_kat_and_formula"],
    "orc_geglu_scalar_libm": ["test_geglu_tanh_substitution_is_ulp_level"],
    "orc_geglu_libm": ["test_geglu_tanh_substitution_is_ulp_level"],
    "orc_embed_gather": ["test_gather_equals_dequant_rows"],
    "orc_pool_normalize": ["test_pool_kat", "test_pool_long_context_vs_f64"],
    "orc_l2_normalize": ["test_l2_normalize_kat_and_sequential_sum"],
    "orc_cosine": ["test_cosine_kat_special_cases_and_sequential_sum"],
    "orc_quantize_binary": ["test_reference_known_answers", "test_quantize_binary_matches_packbits"],
    "orc_hamming": ["test_reference_known_answers", "test_hamming_matches_unpackbits_and_invariants"],
    "orc_binary_cosine": ["test_reference_known_answers", "test_binary_cosine_against_float64"],
    "orc_quantize_int8": ["test_reference_known_answers",
                          "test_quantize_int8_round_half_away_and_saturation"],
    "orc_int8_dot": ["test_reference_known_answers",
                     "test_int8_dot_and_cosine_against_int64_and_float64"],
    "orc_int8_cosine": ["test_reference_known_answers",
                        "test_int8_dot_and_cosine_against_int64_and_float64"],
    "orc_splitmix64": ["test_splitmix64_published_vectors"],
    "orc_fill_normal": ["test_generators_restated_in_python"],
    "orc_fill_uniform_ids": ["test_generators_restated_in_python"],
    "orc_make_q8_0_weight": ["test_generators_restated_in_python"],
    "orc_layer_is_full": ["test_model_forward_vs_float64_statement"],
    "orc_rope_tables": ["test_rope_tables_closed_form"],
    "orc_attention": ["test_attention_band_equals_masked_dense"],
    "orc_encoder_layer": ["test_model_forward_vs_float64_statement",
                          "test_model_forward_per_layer_geometry_vs_float64_statement"],
    "orc_model_forward": ["test_model_forward_vs_float64_statement",
                          "test_model_forward_with_ple_vs_float64_statement"],
}


def test_every_oracle_export_is_pinned():
    import re
    hdr = open(os.path.join(os.path.dirname(HERE), "oracle", "glypr_oracle.h")).read()
    exports = set(re.findall(r"\b(orc_[a-z0-9_]+)\s*\(", hdr))
    missing = sorted(exports - set(PINS))
    assert not missing, f"oracle functions with no pin: {missing}"
    stale = sorted(set(PINS) - exports)
    assert not stale, f"pins name functions the header no longer exports: {stale}"
    names = set()
    for mod in ("test_oracle.py", "test_vec_codecs.py", "test_round.py"):
        names |= set(re.findall(r"^def (test_[a-z0-9_]+)", open(os.path.join(HERE, mod)).read(),
                                re.M))
    for fn, tests in PINS.items():
        for t in tests:
            assert t in names, f"{fn}: pin {t} does not exist"


def test_model_forward_per_layer_geometry_vs_float64_statement(oracle):
    """The released EmbeddingGemma-2 layout in miniature: sliding layers with 2
    kv heads of head_dim 32, the full layer (5) with 1 kv head of head_dim 64
    and its own RoPE table (config.rs:142-169, model.rs:278-287): the oracle
    against the float64 statement.  Using the sliding geometry for the full
    layer is a shape error, and a uniform-geometry model embeds differently."""
    H, F, nh, nkv, hd, fhd, fnkv, L, vocab, t, W = 128, 192, 4, 2, 32, 64, 1, 6, 1000, 40, 8
    rng = np.random.default_rng(21)
    tensors = _small_model(oracle, H, F, nh, nkv, hd, L, vocab, rng, full_hd=fhd, full_nkv=fnkv)
    assert tensors["blk.5.attn_q.weight"].shape[0] == nh * fhd
    assert tensors["blk.5.attn_k.weight"].shape[0] == fnkv * fhd
    ids = rng.integers(0, vocab, t).astype(np.uint32)
    kw = dict(hidden=H, ffn=F, n_heads=nh, n_kv_heads=nkv, head_dim=hd, n_layers=L, vocab=vocab,
              sliding_window=W, full_head_dim=fhd, full_n_kv_heads=fnkv)
    out, states = oracle.model_forward(tensors, ids, 32, **kw)
    ref_out, ref_states = _forward_f64(oracle, tensors, ids, 32, H, F, nh, nkv, hd, L, W,
                                       full_hd=fhd, full_nkv=fnkv)
    row_cos = (states * ref_states).sum(1) / np.linalg.norm(states, axis=1) / \
        np.linalg.norm(ref_states, axis=1)
    assert row_cos.min() > 0.9995 and row_cos.mean() > 0.9999, (row_cos.min(), row_cos.mean())
    assert float(out @ ref_out) > 0.99999
    # the full layer's geometry matters: the same tensors with the full layer's
    # q/k/v/o cut to the sliding geometry give another embedding
    cut = dict(tensors)
    cut["blk.5.attn_q.weight"] = tensors["blk.5.attn_q.weight"].reshape(nh, fhd, -1)[:, :hd] \
        .reshape(nh * hd, -1).copy()
    cut["blk.5.attn_k.weight"] = np.concatenate([tensors["blk.5.attn_k.weight"][:hd]] * nkv)
    cut["blk.5.attn_v.weight"] = np.concatenate([tensors["blk.5.attn_v.weight"][:hd]] * nkv)
    o = tensors["blk.5.attn_output.weight"]
    nbk = o.shape[1] // 34
    cut["blk.5.attn_output.weight"] = o.reshape(H, nh, fhd // 32, 34)[:, :, :hd // 32] \
        .reshape(H, -1).copy()
    cut["blk.5.attn_q_norm.weight"] = tensors["blk.5.attn_q_norm.weight"][:hd].copy()
    cut["blk.5.attn_k_norm.weight"] = tensors["blk.5.attn_k_norm.weight"][:hd].copy()
    del nbk
    uni = dict(kw, full_head_dim=0, full_n_kv_heads=0)
    o2, _ = oracle.model_forward(cut, ids, 32, **uni)
    assert float(o2 @ out) < 0.9999
