"""GPU parity of the INT8_FMA variant (GLYPR_Q8_INT8_FMA) through the C ABI.

INT8_FMA has INT8_EXACT's operands and integer block sums and adds each
block's term as acc = fma(round(S * d_w), d_x, acc).  Bars:
  - bit-exact against the oracle's restatement of that order
    (oracle.matmul_fma, pinned in tests/test_oracle.py by exact-rational
    brute force), on every GEMM route (fused prologue, small-M ring, large-M
    128 x 128, register-staged) and through the GeGLU epilogue;
  - matmul: BASELINE's tolerance, 1e-3 relative with a 1e-4 absolute floor,
    against the INT8_EXACT oracle and against the float64 brute force, and
    the float64 error bound of the fused order, (2 nb + 2) 2^-24 sum |terms|;
  - MLP: BASELINE's tolerance against the INT8_EXACT chain plus the effect of
    the bytes of Q8_0(h) that an ulp of gate / up moved (mlp_vs_exact_chain).
"""
import sys

import numpy as np
import pytest
import torch

from glypr_amd import ops
from glypr_amd.ops import INT8_EXACT, INT8_FMA, Q8Weight

pytestmark = pytest.mark.gpu

C3_M, C3_H, C3_F = 16384, 768, 1152


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bits_equal(got, ref, what):
    g, r = bits(got), bits(ref)
    bad = np.count_nonzero(g != r)
    assert bad == 0, f"{what}: {bad} of {g.size} values differ; max |d| = " \
                     f"{np.abs(got.astype(np.float64) - ref).max()}"


def within_baseline(got, ref, what):
    """BASELINE: max relative error 1e-3 with an absolute floor of 1e-4."""
    ref = np.asarray(ref, np.float64)
    err = np.abs(got.astype(np.float64) - ref)
    lim = np.maximum(1e-3 * np.abs(ref), 1e-4)
    assert np.all(err <= lim), f"{what}: max |d| = {err.max()}, worst d/lim = {(err / lim).max()}"


def fma_bound_vs_f64(oracle, got, x, wb, n):
    """|y - y64| <= (2 nb + 2) 2^-24 sum_b |S_b d_w d_x| over the same
    quantized operands (nb roundings of t, nb of the accumulate)."""
    m, k = x.shape
    xq = oracle.quantize_rows(x)
    y64 = oracle.matmul_f64(xq, m, k, wb, n)
    dw, qw = oracle.split_blocks(wb, k)
    dx, qx = oracle.split_blocks(xq, k)
    fdw = np.abs(oracle.f16_bits_to_f32(dw).astype(np.float64))
    fdx = np.abs(oracle.f16_bits_to_f32(dx).astype(np.float64))
    absterm = np.zeros((m, n))
    for b in range(k // 32):
        s = np.abs(qx[:, b * 32:(b + 1) * 32].astype(np.int64)
                   @ qw[:, b * 32:(b + 1) * 32].astype(np.int64).T)
        absterm += s * fdx[:, b][:, None] * fdw[:, b][None, :]
    nb = k // 32
    assert np.all(np.abs(got.astype(np.float64) - y64)
                  <= (2 * nb + 2) * 2.0 ** -24 * absterm + 1e-30)
    within_baseline(got, y64, "vs float64")


# (m, k, n) per route: fused quantize prologue (m <= 1024, k <= 1152), the
# small-M ring (m <= 2048; k up to 2048), the large-M 128 x 128 kernel and the
# register-staged kernel (k not a multiple of 128; 64- and 128-wide tiles)
ROUTES = [(1, 768, 1152), (33, 256, 70), (512, 768, 1152), (1500, 768, 1152),
          (64, 2048, 768), (3000, 1152, 129), (2177, 256, 300), (2049, 96, 200),
          (4096, 96, 2304)]


@pytest.mark.parametrize("m,k,n", ROUTES)
def test_matmul_int8_fma(ctx, oracle, m, k, n):
    say(f"matmul INT8_FMA m={m} k={k} n={n}")
    x = oracle.normal(m * k, seed=900 + m).reshape(m, k)
    wb = oracle.q8_0_weight(n, k, seed=910 + n)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    y = host(ops.q8_0_matmul(ctx, w, dev(x), INT8_FMA))
    assert_bits_equal(y, oracle.matmul_fma(x, wb, n), f"INT8_FMA {m}x{k}x{n}")
    within_baseline(y, oracle.matmul(x, wb, n), "vs the INT8_EXACT oracle")
    rows = np.arange(m) if m <= 512 else np.random.default_rng(m).choice(m, 256, False)
    fma_bound_vs_f64(oracle, y[rows], x[rows], wb, n)


def test_matmul_int8_fma_is_not_exact(ctx, oracle):
    """The variant runs its own epilogue: at C2's shape some outputs differ in
    their last bits from INT8_EXACT's (the single rounding of the fused form),
    and the same call repeated gives the same bits."""
    m, k, n = 512, 768, 1152
    x = oracle.normal(m * k, seed=931).reshape(m, k)
    wb = oracle.q8_0_weight(n, k, seed=932)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    xd = dev(x)
    ye = host(ops.q8_0_matmul(ctx, w, xd, INT8_EXACT))
    yf = host(ops.q8_0_matmul(ctx, w, xd, INT8_FMA))
    yf2 = host(ops.q8_0_matmul(ctx, w, xd, INT8_FMA))
    assert np.array_equal(bits(yf), bits(yf2))
    differ = np.count_nonzero(bits(ye) != bits(yf))
    say(f"  outputs whose bits differ from INT8_EXACT: {differ} of {ye.size}")
    assert differ > 0


@pytest.mark.parametrize("m", [1, 200, 512])
def test_rmsnorm_matmul_int8_fma(ctx, oracle, m):
    """RMSNorm prologue (fused for m <= 256) under the fused epilogue."""
    k, n = 768, 1152
    say(f"rmsnorm_q8_0_matmul INT8_FMA m={m}")
    x = oracle.normal(m * k, seed=940 + m).reshape(m, k)
    nw = 1 + 0.1 * oracle.normal(k, seed=941)
    wb = oracle.q8_0_weight(n, k, seed=942)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    y = host(ops.rmsnorm_q8_0_matmul(ctx, w, dev(x), dev(nw), 1e-6, INT8_FMA))
    xn = oracle.rmsnorm(x, nw, 1e-6)
    assert_bits_equal(y, oracle.matmul_fma(xn, wb, n), "rmsnorm INT8_FMA")
    within_baseline(y, oracle.matmul(xn, wb, n), "vs the INT8_EXACT oracle")


def test_noalloc_matmul_int8_fma(ctx, oracle):
    """The no-allocation entry point takes the variant too, with the same bits."""
    k, n = 768, 1152
    wb = oracle.q8_0_weight(n, k, seed=951)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    for m in (2500, 700):
        say(f"q8_0_matmul_noalloc INT8_FMA m={m}")
        x = dev(oracle.normal(m * k, seed=950 + m).reshape(m, k))
        a = host(ops.q8_0_matmul(ctx, w, x, INT8_FMA))
        b = host(ops.q8_0_matmul_noalloc(ctx, w, x, INT8_FMA))
        assert np.array_equal(bits(a), bits(b))


def _mlp_fma_ref(oracle, xn, gb, ub, db, H, F):
    gate, up = oracle.matmul_fma(xn, gb, F), oracle.matmul_fma(xn, ub, F)
    return oracle.matmul_fma(oracle.geglu(gate, up), db, H)


def mlp_vs_exact_chain(oracle, got, xn, gb, ub, db, H, F, what):
    """The MLP under INT8_FMA against the INT8_EXACT oracle chain.  gate / up
    may differ in their last bit, and that can move a value of h across a
    Q8_0 rounding boundary: one byte of Q8_0(h) then differs by one step d_h,
    and y by d_h * |w_down| for that column (a last-bit difference in gate / up
    from any other summation order does the same).  So the bound is BASELINE's
    1e-3 relative / 1e-4 absolute plus
    sum_j |deq Q8_0(h_fma) - deq Q8_0(h_exact)|_j |w_j|; with no flipped byte
    it is BASELINE's tolerance alone."""
    h_f = oracle.geglu(oracle.matmul_fma(xn, gb, F), oracle.matmul_fma(xn, ub, F))
    h_e = oracle.geglu(oracle.matmul(xn, gb, F), oracle.matmul(xn, ub, F))
    ref = oracle.matmul(h_e, db, H).astype(np.float64)
    dq_f = oracle.dequantize_rows(oracle.quantize_rows(h_f), F).astype(np.float64)
    dq_e = oracle.dequantize_rows(oracle.quantize_rows(h_e), F).astype(np.float64)
    flip = np.abs(dq_f - dq_e) @ np.abs(oracle.dequantize_rows(db, F).astype(np.float64)).T
    err = np.abs(got.astype(np.float64) - ref)
    lim = np.maximum(1e-3 * np.abs(ref), 1e-4)
    n_flip = int(np.count_nonzero(dq_f != dq_e))
    over = int(np.count_nonzero(err > lim))
    say(f"  {what}: Q8_0(h) values that differ from the exact chain's: {n_flip} of {dq_f.size}; "
        f"outputs beyond 1e-3/1e-4: {over} of {err.size}, max |d| = {err.max():.3g}")
    assert np.all(err <= lim + flip * (1 + 1e-6)), (err - lim - flip).max()
    if n_flip == 0:
        assert over == 0


@pytest.mark.parametrize("m,H,F", [(1, 768, 1152), (512, 768, 1152), (1500, 256, 96),
                                   (2200, 256, 96), (4096, 768, 1152), (2500, 128, 160)])
def test_mlp_int8_fma(ctx, oracle, m, H, F):
    """gate/up GeGLU epilogue (+ Q8_0 of h) and down, every route, bit-exact
    against the fused-order oracle chain and within BASELINE's tolerance of
    the INT8_EXACT chain."""
    say(f"mlp INT8_FMA m={m} H={H} F={F}")
    x = oracle.normal(m * H, seed=960 + m).reshape(m, H)
    gb, ub = oracle.q8_0_weight(F, H, seed=961), oracle.q8_0_weight(F, H, seed=962)
    db = oracle.q8_0_weight(H, F, seed=963)
    g, u = Q8Weight.from_gguf(ctx, gb, F, H), Q8Weight.from_gguf(ctx, ub, F, H)
    d = Q8Weight.from_gguf(ctx, db, H, F)
    gu, _ = Q8Weight.concat(ctx, [g, u])
    y = host(ops.mlp(ctx, gu, d, dev(x), INT8_FMA))
    rows = np.arange(m) if m <= 512 else np.sort(np.random.default_rng(m).choice(m, 256, False))
    assert_bits_equal(y[rows], _mlp_fma_ref(oracle, x[rows], gb, ub, db, H, F), "mlp INT8_FMA")
    mlp_vs_exact_chain(oracle, y[rows], x[rows], gb, ub, db, H, F, "mlp")


def test_c3_rmsnorm_mlp_int8_fma(ctx, oracle):
    """C3's RMSNorm -> gate/up GeGLU -> down at M = 16384 under INT8_FMA: two
    runs bit-identical, 128 sampled rows bit-exact against the fused-order
    chain and within BASELINE's tolerance of the INT8_EXACT chain."""
    say(f"C3 INT8_FMA rmsnorm_mlp m={C3_M}")
    x = oracle.normal(C3_M * C3_H, seed=971).reshape(C3_M, C3_H)
    nw = 1 + 0.1 * oracle.normal(C3_H, seed=972)
    gb, ub = oracle.q8_0_weight(C3_F, C3_H, seed=973), oracle.q8_0_weight(C3_F, C3_H, seed=974)
    db = oracle.q8_0_weight(C3_H, C3_F, seed=975)
    g, u = Q8Weight.from_gguf(ctx, gb, C3_F, C3_H), Q8Weight.from_gguf(ctx, ub, C3_F, C3_H)
    d = Q8Weight.from_gguf(ctx, db, C3_H, C3_F)
    gu, _ = Q8Weight.concat(ctx, [g, u])
    xd, nwd = dev(x), dev(nw)
    y1 = host(ops.rmsnorm_mlp(ctx, gu, d, xd, nwd, 1e-6, INT8_FMA))
    y2 = host(ops.rmsnorm_mlp(ctx, gu, d, xd, nwd, 1e-6, INT8_FMA))
    assert np.array_equal(bits(y1), bits(y2))
    rows = np.sort(np.random.default_rng(976).choice(C3_M, 128, replace=False))
    rows[:2] = [0, C3_M - 1]
    xn = oracle.rmsnorm(x[rows], nw, 1e-6)
    assert_bits_equal(y1[rows], _mlp_fma_ref(oracle, xn, gb, ub, db, C3_H, C3_F), "C3 mlp rows")
    mlp_vs_exact_chain(oracle, y1[rows], xn, gb, ub, db, C3_H, C3_F, "C3 mlp")
