"""GPU parity of the Q8_0 hot path (through the C ABI) against the CPU oracle.

Bar: bit-exact for dequantization, activation quantization, RMSNorm, GeGLU,
gather, pooling and the INT8_EXACT GEMM (+ its fused prologue/epilogues);
BASELINE's tolerance (max relative error 1e-3, absolute floor 1e-4) is also
asserted against the float64 brute force.  The BF16_DEQUANT variant is held to
a bf16 bound against the float64 dequant oracle.
"""
import json
import os
import sys

import numpy as np
import pytest
import torch

from glypr_amd import _lib
from glypr_amd import ops
from glypr_amd.ops import BF16_DEQUANT, INT8_EXACT, Q8Weight

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
KAT = json.load(open(os.path.join(HERE, "golden", "q8_0_kat.json")))


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


def baseline_tolerance(got, ref64):
    """BASELINE: max relative error 1e-3 with an absolute floor of 1e-4."""
    err = np.abs(got.astype(np.float64) - ref64)
    assert np.all(err <= np.maximum(1e-3 * np.abs(ref64), 1e-4)), err.max()


# ------------------------------------------------------------------ codec --

def test_dequant_kat_and_random(ctx, oracle):
    say("dequant: KAT blocks + random [300 x 768]")
    for c in KAT["dequant"]:
        blk = oracle.join_blocks(np.array([[c["d_bits"]]], np.uint16), np.array([c["qs"]], np.int8))
        w = Q8Weight.from_gguf(ctx, blk, 1, 32)
        y = host(ops.dequantize(ctx, w))
        assert np.array_equal(bits(y[0]), np.array(c["y_bits"], np.uint32)), c["d_bits"]
    wb = oracle.q8_0_weight(300, 768, seed=3)
    w = Q8Weight.from_gguf(ctx, wb, 300, 768)
    assert w.shape() == (300, 768)
    assert_bits_equal(host(ops.dequantize(ctx, w)), oracle.dequantize_rows(wb, 768), "dequant")


def test_quantize_kat_and_random(ctx, oracle):
    say("quantize: KAT blocks + N(0,1) [517 x 1152]")
    for c in KAT["quantize"]:
        x = np.array(c["x_bits"], np.uint32).view(np.float32).reshape(1, 32)
        d, qs = oracle.split_blocks(host(ops.quantize(ctx, dev(x))), 32)
        assert int(d[0, 0]) == c["d_bits"], c["name"]
        assert qs[0].tolist() == c["qs"], c["name"]
    x = oracle.normal(517 * 1152, seed=8).reshape(517, 1152) * np.float32(3.7)
    x[5, 100:140] = 0.0
    x[9, 0] = 1e30
    got = host(ops.quantize(ctx, dev(x)))
    assert np.array_equal(got, oracle.quantize_rows(x))


# ----------------------------------------------------------------- GEMMs ---

SHAPES = [(1, 32, 1), (19, 256, 128), (33, 96, 70), (64, 768, 1280), (100, 1152, 768),
          (512, 768, 1152), (300, 768, 256), (7, 128, 33)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_int8_bit_exact(ctx, oracle, m, k, n):
    say(f"matmul INT8_EXACT m={m} k={k} n={n}")
    x = oracle.normal(m * k, seed=100 + m).reshape(m, k)
    wb = oracle.q8_0_weight(n, k, seed=200 + n)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    y = host(ops.q8_0_matmul(ctx, w, dev(x), INT8_EXACT))
    ref = oracle.matmul(x, wb, n)
    assert_bits_equal(y, ref, f"matmul {m}x{k}x{n}")
    baseline_tolerance(y, oracle.matmul_f64(oracle.quantize_rows(x), m, k, wb, n))


def test_matmul_int8_large_tile_path(ctx, oracle):
    m, k, n = 4096, 768, 2304
    say(f"matmul INT8_EXACT large-tile path m={m} k={k} n={n}")
    x = oracle.normal(m * k, seed=7).reshape(m, k)
    wb = oracle.q8_0_weight(n, k, seed=77)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    y = host(ops.q8_0_matmul(ctx, w, dev(x), INT8_EXACT))
    assert_bits_equal(y, oracle.matmul(x, wb, n), "large-tile matmul")


@pytest.mark.parametrize("m,k,n", [(2100, 128, 70), (2177, 256, 300), (3000, 1152, 129),
                                   (2049, 96, 200)])
def test_matmul_int8_large_m_ragged(ctx, oracle, m, k, n):
    """Large-M kernels with partial row/column tiles, one K stage, and K that is not a
    multiple of 128 (the register-staged fallback)."""
    say(f"matmul INT8_EXACT large-M ragged m={m} k={k} n={n}")
    x = oracle.normal(m * k, seed=300 + m).reshape(m, k)
    wb = oracle.q8_0_weight(n, k, seed=400 + n)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    y = host(ops.q8_0_matmul(ctx, w, dev(x), INT8_EXACT))
    assert_bits_equal(y, oracle.matmul(x, wb, n), f"matmul {m}x{k}x{n}")


@pytest.mark.parametrize("m,H,F", [(2200, 256, 96), (2500, 128, 160)])
def test_mlp_large_m_ragged(ctx, oracle, m, H, F):
    """GeGLU epilogue of the large-M kernel when the last tile holds a partial h block
    pair (F not a multiple of 64) and M is not a multiple of 128."""
    say(f"mlp large-M ragged m={m} H={H} F={F}")
    x = oracle.normal(m * H, seed=m + 6).reshape(m, H)
    gb, ub, db = (oracle.q8_0_weight(F, H, seed=21), oracle.q8_0_weight(F, H, seed=22),
                  oracle.q8_0_weight(H, F, seed=23))
    g = Q8Weight.from_gguf(ctx, gb, F, H)
    u = Q8Weight.from_gguf(ctx, ub, F, H)
    d = Q8Weight.from_gguf(ctx, db, H, F)
    gu, views = Q8Weight.concat(ctx, [g, u])
    y = host(ops.mlp(ctx, gu, d, dev(x), INT8_EXACT))
    assert_bits_equal(y, _mlp_ref(oracle, x, gb, ub, db, H, F), "mlp")


def test_matmul_deterministic_and_c3_rows(ctx, oracle):
    """C3 size (M = 16384): two runs are bit-identical (no LDS race) and 64 random
    rows match the oracle bit for bit."""
    m, k, n = 16384, 768, 1152
    say(f"matmul C3 size m={m} k={k} n={n}")
    x = oracle.normal(m * k, seed=31).reshape(m, k)
    wb = oracle.q8_0_weight(n, k, seed=32)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    xd = dev(x)
    y1 = host(ops.q8_0_matmul(ctx, w, xd, INT8_EXACT))
    y2 = host(ops.q8_0_matmul(ctx, w, xd, INT8_EXACT))
    assert np.array_equal(bits(y1), bits(y2))
    rows = np.random.default_rng(0).choice(m, 64, replace=False)
    assert_bits_equal(y1[rows], oracle.matmul(x[rows], wb, n), "C3 rows")


def test_rmsnorm_bit_exact(ctx, oracle):
    # dims 256 NV (every staged chunk used) and between (the chain's zero-padded
    # tail), with one to six read batches of the chain
    for rows, dim, with_w in [(37, 768, True), (512, 768, True), (96, 256, True), (40, 256, False),
                              (5, 1152, True), (33, 512, True), (17, 640, True), (9, 1024, True),
                              (7, 2048, True), (11, 1792, False), (5, 1312, True),
                              (3, 20, True), (6, 21, True), (4, 3000, False)]:
        say(f"rmsnorm rows={rows} dim={dim} weight={with_w}")
        x = oracle.normal(rows * dim, seed=rows + dim).reshape(rows, dim) * np.float32(2.5)
        w = (1 + 0.1 * oracle.normal(dim, seed=9)) if with_w else None
        y = host(ops.rmsnorm(ctx, dev(x), None if w is None else dev(w), 1e-6))
        assert_bits_equal(y, oracle.rmsnorm(x, w, 1e-6), f"rmsnorm {rows}x{dim}")
    # in place (x == y) and the KAT rows
    x = oracle.normal(64 * 768, seed=4).reshape(64, 768)
    xd = dev(x)
    ops.rmsnorm(ctx, xd, None, 1e-6, out=xd)
    assert_bits_equal(host(xd), oracle.rmsnorm(x, None, 1e-6), "rmsnorm in place")
    for c in KAT["rmsnorm"]:
        d = c["d"]
        x = np.full((2, d), np.array([c["c_bits"]], np.uint32).view(np.float32)[0], np.float32)
        w = np.array(c["w_bits"], np.uint32).view(np.float32)
        y = host(ops.rmsnorm(ctx, dev(x), dev(w), 0.0))
        assert np.array_equal(bits(y[1]), np.array(c["y_bits"], np.uint32))


@pytest.mark.parametrize("m", [1, 19, 512, 2048])
def test_rmsnorm_matmul_bit_exact(ctx, oracle, m):
    k, n = 768, 1280
    say(f"rmsnorm_q8_0_matmul m={m}")
    x = oracle.normal(m * k, seed=m).reshape(m, k) * np.float32(4.0)
    nw = 1 + 0.1 * oracle.normal(k, seed=1)
    wb = oracle.q8_0_weight(n, k, seed=2)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    y = host(ops.rmsnorm_q8_0_matmul(ctx, w, dev(x), dev(nw), 1e-6, INT8_EXACT))
    ref = oracle.matmul(oracle.rmsnorm(x, nw, 1e-6), wb, n)
    assert_bits_equal(y, ref, "rmsnorm+matmul")


def _prologue_rows(oracle, m, k, seed):
    """Activations that stress the quantize prologue: random rows plus, where m
    allows, an all-zero row (amax 0: scale 0, inverse 0), a row of huge values,
    a row of denormal-sized values and a row with one outlier per block."""
    x = oracle.normal(m * k, seed=seed).reshape(m, k) * np.float32(3.0)
    if m >= 5:
        x[1] = 0.0
        x[2] *= np.float32(1e5)
        x[3] *= np.float32(1e-38)
        x[4, ::32] = np.float32(-5e4)
    return x


@pytest.mark.parametrize("m,k,n", [(1, 128, 1), (17, 256, 70), (33, 384, 129), (16, 1152, 300),
                                   (200, 640, 128), (256, 768, 1280), (257, 768, 1280),
                                   (600, 512, 200), (1024, 768, 768), (1025, 768, 768),
                                   (2048, 896, 257)])
def test_fused_prologue_matmul_bit_exact(ctx, oracle, m, k, n):
    """Small-M matmuls with the quantize / RMSNorm prologue inside the GEMM
    (quantize up to M = 1024, RMSNorm up to M = 256) and the two-launch route
    just past those bounds: ragged M and N tiles, every K stage count from 1
    to 7, special rows, and RMSNorm with and without a weight."""
    say(f"fused-prologue matmul m={m} k={k} n={n}")
    x = _prologue_rows(oracle, m, k, seed=500 + m)
    wb = oracle.q8_0_weight(n, k, seed=600 + n)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    xd = dev(x)
    y = host(ops.q8_0_matmul(ctx, w, xd, INT8_EXACT))
    assert_bits_equal(y, oracle.matmul(x, wb, n), "quantize prologue")
    nw = 1 + 0.1 * oracle.normal(k, seed=k)
    y = host(ops.rmsnorm_q8_0_matmul(ctx, w, xd, dev(nw), 1e-6, INT8_EXACT))
    assert_bits_equal(y, oracle.matmul(oracle.rmsnorm(x, nw, 1e-6), wb, n), "rmsnorm prologue")
    y = host(ops.rmsnorm_q8_0_matmul(ctx, w, xd, None, 1e-5, INT8_EXACT))
    assert_bits_equal(y, oracle.matmul(oracle.rmsnorm(x, None, 1e-5), wb, n),
                      "rmsnorm prologue, no weight")


@pytest.mark.parametrize("m,H,F", [(1, 128, 32), (19, 256, 96), (64, 1152, 160),
                                   (300, 512, 64), (2048, 768, 1152)])
def test_mlp_ragged_small_m_bit_exact(ctx, oracle, m, H, F):
    """Small-M gate/up GEMM with the GeGLU epilogue: h widths that end inside a
    GeGLU tile, partial M tiles and the special activation rows."""
    say(f"mlp ragged m={m} H={H} F={F}")
    x = _prologue_rows(oracle, m, H, seed=700 + m)
    gb, ub, db = (oracle.q8_0_weight(F, H, seed=21), oracle.q8_0_weight(F, H, seed=22),
                  oracle.q8_0_weight(H, F, seed=23))
    g = Q8Weight.from_gguf(ctx, gb, F, H)
    u = Q8Weight.from_gguf(ctx, ub, F, H)
    d = Q8Weight.from_gguf(ctx, db, H, F)
    gu, _ = Q8Weight.concat(ctx, [g, u])
    xd = dev(x)
    y = host(ops.mlp(ctx, gu, d, xd, INT8_EXACT))
    assert_bits_equal(y, _mlp_ref(oracle, x, gb, ub, db, H, F), "mlp")
    nw = 1 + 0.1 * oracle.normal(H, seed=H + 1)
    y = host(ops.rmsnorm_mlp(ctx, gu, d, xd, dev(nw), 1e-6, INT8_EXACT))
    assert_bits_equal(y, _mlp_ref(oracle, oracle.rmsnorm(x, nw, 1e-6), gb, ub, db, H, F),
                      "rmsnorm+mlp")


def test_rmsnorm_calls_repeat_and_interleave(ctx, oracle):
    """RMSNorm-prologue matmul and MLP calls at H = 768, F = 1152 repeated and
    interleaved on one context (one shared activation workspace), across the
    fused-prologue and two-launch routes: ragged M and N and the special rows
    stay bit-exact on every call."""
    H, F = 768, 1152
    gb, ub, db = (oracle.q8_0_weight(F, H, seed=31), oracle.q8_0_weight(F, H, seed=32),
                  oracle.q8_0_weight(H, F, seed=33))
    g = Q8Weight.from_gguf(ctx, gb, F, H)
    u = Q8Weight.from_gguf(ctx, ub, F, H)
    d = Q8Weight.from_gguf(ctx, db, H, F)
    gu, _ = Q8Weight.concat(ctx, [g, u])
    nw = 1 + 0.1 * oracle.normal(H, seed=34)
    nwd = dev(nw)
    plain = {n: (oracle.q8_0_weight(n, H, seed=40 + n), None) for n in (70, 1280)}
    plain = {n: (wb, Q8Weight.from_gguf(ctx, wb, n, H)) for n, (wb, _) in plain.items()}
    cases = [(3, 70), (512, 1280), (37, 1280), (2047, 70), (512, 1280), (1, 1280), (130, 70)]
    for rep, (m, n) in enumerate(cases):
        say(f"rmsnorm call {rep}: m={m} n={n}")
        x = _prologue_rows(oracle, m, H, seed=900 + rep)
        xd = dev(x)
        xn = oracle.rmsnorm(x, nw, 1e-6)
        wb, w = plain[n]
        y = host(ops.rmsnorm_q8_0_matmul(ctx, w, xd, nwd, 1e-6, INT8_EXACT))
        assert_bits_equal(y, oracle.matmul(xn, wb, n), f"rmsnorm+matmul call {rep}")
        y = host(ops.rmsnorm_mlp(ctx, gu, d, xd, nwd, 1e-6, INT8_EXACT))
        assert_bits_equal(y, _mlp_ref(oracle, xn, gb, ub, db, H, F), f"rmsnorm+mlp call {rep}")


def test_geglu_bit_exact(ctx, oracle):
    say("geglu elementwise [512 x 1152] + KAT points")
    g = oracle.normal(512 * 1152, seed=61, std=3.0)
    u = oracle.normal(512 * 1152, seed=62)
    g[:8] = [-10.0, 10.0, 0.0, -0.0, 9.99, -9.99, 1e-6, -50.0]
    y = host(ops.geglu(ctx, dev(g), dev(u)))
    assert_bits_equal(y, oracle.geglu(g, u), "geglu")
    for c in KAT["geglu"]:
        gg = np.array([c["g_bits"]], np.uint32).view(np.float32)
        uu = np.array([c["u_bits"]], np.uint32).view(np.float32)
        assert bits(host(ops.geglu(ctx, dev(gg), dev(uu))))[0] == c["y_bits"]


def _mlp_ref(oracle, x, gb, ub, db, H, F):
    gate = oracle.matmul(x, gb, F)
    up = oracle.matmul(x, ub, F)
    return oracle.matmul(oracle.geglu(gate, up), db, H)


@pytest.mark.parametrize("m", [1, 33, 512, 4096])
def test_mlp_bit_exact(ctx, oracle, m):
    H, F = 768, 1152
    say(f"mlp (gate/up GeGLU epilogue + down) m={m}")
    x = oracle.normal(m * H, seed=m + 5).reshape(m, H)
    gb, ub, db = (oracle.q8_0_weight(F, H, seed=11), oracle.q8_0_weight(F, H, seed=12),
                  oracle.q8_0_weight(H, F, seed=13))
    g = Q8Weight.from_gguf(ctx, gb, F, H)
    u = Q8Weight.from_gguf(ctx, ub, F, H)
    d = Q8Weight.from_gguf(ctx, db, H, F)
    gu, views = Q8Weight.concat(ctx, [g, u])
    y = host(ops.mlp(ctx, gu, d, dev(x), INT8_EXACT))
    assert_bits_equal(y, _mlp_ref(oracle, x, gb, ub, db, H, F), "mlp")
    nw = 1 + 0.1 * oracle.normal(H, seed=14)
    y2 = host(ops.rmsnorm_mlp(ctx, gu, d, dev(x), dev(nw), 1e-6, INT8_EXACT))
    assert_bits_equal(y2, _mlp_ref(oracle, oracle.rmsnorm(x, nw, 1e-6), gb, ub, db, H, F),
                      "rmsnorm+mlp")


def test_concat_views_share_the_fused_buffer(ctx, oracle):
    m, H = 77, 768
    say("try_concat q/k/v: fused output == separate outputs; views == parts")
    x = oracle.normal(m * H, seed=90).reshape(m, H)
    parts = [oracle.q8_0_weight(n, H, seed=91 + i) for i, n in enumerate((768, 256, 256))]
    ws = [Q8Weight.from_gguf(ctx, p, p.shape[0], H) for p in parts]
    fused, views = Q8Weight.concat(ctx, ws)
    assert fused.shape() == (1280, H) and [v.shape() for v in views] == [(768, H), (256, H),
                                                                          (256, H)]
    xd = dev(x)
    yf = host(ops.q8_0_matmul(ctx, fused, xd))
    off = 0
    for p, v in zip(parts, views):
        n = p.shape[0]
        yv = host(ops.q8_0_matmul(ctx, v, xd))
        ref = oracle.matmul(x, p, n)
        assert_bits_equal(yv, ref, "view")
        assert_bits_equal(yf[:, off:off + n], ref, "fused slice")
        off += n
    sub = views[0].view(100, 50)
    assert_bits_equal(host(ops.dequantize(ctx, sub)),
                      oracle.dequantize_rows(parts[0][100:150], H), "narrow view")
    # parts can be released; views keep the fused buffer alive
    for wv in ws:
        wv.close()
    fused.close()
    assert_bits_equal(host(ops.q8_0_matmul(ctx, views[2], xd)), oracle.matmul(x, parts[2], 256),
                      "view after fused handle released")


@pytest.mark.parametrize("n_ids", [1, 512, 768, 769, 3000])
def test_gather_bit_exact_and_range(ctx, oracle, n_ids):
    """Up to 768 ids ride in the kernel arguments, more are uploaded first:
    both routes against the oracle, bit for bit."""
    vocab, d = 50_000, 768
    say(f"embed gather vocab={vocab} d={d} ids={n_ids}")
    tb = oracle.q8_0_weight(vocab, d, seed=71)
    table = Q8Weight.from_gguf(ctx, tb, vocab, d)
    ids = oracle.uniform_ids(n_ids, seed=72, vocab=vocab)
    ids[:4] = [0, vocab - 1, 7, 7][:n_ids]
    scale = float(np.float32(np.sqrt(768.0)))
    y = host(ops.embed_gather(ctx, table, ids, scale))
    assert_bits_equal(y, oracle.embed_gather(tb, vocab, d, ids, scale), "gather")
    with pytest.raises(_lib.GlyprError) as e:
        ops.embed_gather(ctx, table, np.array([1, vocab], np.uint32), 1.0)
    assert e.value.code == _lib.GLYPR_ERR_RANGE


def test_pool_vs_f64_and_oracle(ctx, oracle):
    """pool_and_normalize: the GPU sums tokens in 64-token chunks (fixed order), so
    it is held to the float64 mean (|err| <= 1e-6 of the largest component) and
    to the sequential-sum oracle at cosine > 1 - 1e-10, not bit-exactness."""
    for t, d, trunc, masked in [(512, 768, 256, False), (512, 768, 0, False), (19, 768, 128, True),
                                (8192, 768, 256, False), (1000, 768, 0, True)]:
        say(f"pool_normalize t={t} d={d} trunc={trunc} masked={masked}")
        tok = oracle.normal(t * d, seed=t + trunc).reshape(t, d) + np.float32(0.05)
        mask = None
        if masked:
            mask = (np.arange(t) % 3 != 1).astype(np.uint8)
        y = host(ops.pool_normalize(ctx, dev(tok), mask, trunc))
        sel = tok.astype(np.float64) if mask is None else tok[mask.astype(bool)].astype(np.float64)
        ref = sel.mean(0)
        ref = ref / np.linalg.norm(ref)
        if 0 < trunc < d:
            ref = ref[:trunc] / np.linalg.norm(ref[:trunc])
        assert np.abs(y - ref).max() <= 1e-6 * np.abs(ref).max()
        orc = oracle.pool_normalize(tok, mask, trunc)
        cos = float(y.astype(np.float64) @ orc / np.linalg.norm(y) / np.linalg.norm(orc))
        assert cos > 1 - 1e-10
    c = KAT["pool"][0]
    v = np.array(c["v_bits"], np.uint32).view(np.float32)
    tok = np.tile(v, (c["t"], 1))
    assert np.array_equal(bits(host(ops.pool_normalize(ctx, dev(tok)))),
                          np.array(c["l2_bits"], np.uint32))


# ------------------------------------------------------------ bf16 variant -

@pytest.mark.parametrize("m,k,n", [(19, 256, 128), (512, 768, 1152), (4096, 768, 1152),
                                   (300, 1152, 768), (2049, 64, 300), (3000, 1152, 70),
                                   (4100, 768, 1280), (2500, 96, 257)])
def test_matmul_bf16_dequant_within_bf16_bound(ctx, oracle, m, k, n):
    """BF16_DEQUANT vs the float64 dequant oracle: both operands rounded to bf16
    (relative error <= 2^-8 each), f32 accumulation:
    |y - y64| <= 2^-7 * (|x| @ |w_deq|^T) + f32 accumulation slack."""
    say(f"matmul BF16_DEQUANT m={m} k={k} n={n}")
    x = oracle.normal(m * k, seed=300 + m).reshape(m, k)
    wb = oracle.q8_0_weight(n, k, seed=301)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    y = host(ops.q8_0_matmul(ctx, w, dev(x), BF16_DEQUANT))
    y64 = oracle.matmul_dequant_f64(x, wb, n)
    wd = np.abs(oracle.dequantize_rows(wb, k).astype(np.float64))
    bound = 2.0 ** -7 * (np.abs(x).astype(np.float64) @ wd.T) * (1 + 1e-3) + 1e-6
    assert np.all(np.abs(y - y64) <= bound)
    cos = (y * y64).sum(1) / np.linalg.norm(y, axis=1) / np.linalg.norm(y64, axis=1)
    assert cos.min() > 0.9999
    # A5': the same output against glypr's CPU Q8_0 path (INT8_EXACT oracle,
    # activations quantized per 32-block).  The gap is the oracle's own
    # activation-quantization error, ~0.5 % relative per element, so the
    # per-row cosine sits near 1 - (0.005)^2 / 2.
    rows = np.arange(m) if m <= 512 else np.random.default_rng(m).choice(m, 256, replace=False)
    y8 = oracle.matmul(x[rows], wb, n).astype(np.float64)
    c8 = (y[rows] * y8).sum(1) / np.linalg.norm(y[rows], axis=1) / np.linalg.norm(y8, axis=1)
    say(f"  cosine to the INT8_EXACT oracle: min {c8.min():.7f} mean {c8.mean():.7f}")
    assert c8.min() > 0.999


@pytest.mark.parametrize("m,k,n", [(1, 64, 1), (100, 768, 1152), (600, 1152, 257),
                                   (4100, 768, 1280), (8192, 768, 768), (4095, 768, 1024)])
def test_dense_bf16_weight_matmul_within_bound(ctx, oracle, m, k, n):
    """LinearOp::forward over a dense bf16 weight: x rounded to bf16 (relative
    error <= 2^-9), exact bf16 weights, f32 accumulation:
    |y - y64| <= 2^-8 * (|x| @ |w|^T) + 1e-6 against float64 x @ w^T."""
    say(f"dense bf16 matmul m={m} k={k} n={n}")
    x = oracle.normal(m * k, seed=900 + m).reshape(m, k)
    wf = 0.02 * oracle.normal(n * k, seed=901 + n).reshape(n, k)
    bits = ops.f32_to_bf16_bits(wf)
    w64 = (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    w = ops.BF16Weight.from_bf16(ctx, bits)
    y = host(ops.bf16_matmul(ctx, w, dev(x)))
    y64 = x.astype(np.float64) @ w64.T
    bound = 2.0 ** -8 * (np.abs(x).astype(np.float64) @ np.abs(w64).T) + 1e-6
    assert np.all(np.abs(y - y64) <= bound)
    w.close()


def test_dense_bf16_weight_shape_errors(ctx, oracle):
    bits = ops.f32_to_bf16_bits(np.ones((4, 96), np.float32))
    with pytest.raises(_lib.GlyprError) as e:
        ops.BF16Weight.from_bf16(ctx, bits)
    assert e.value.code == _lib.GLYPR_ERR_UNSUPPORTED


@pytest.mark.parametrize("m,H,F", [(512, 768, 1152), (2200, 256, 96), (3000, 768, 1152)])
def test_mlp_bf16_dequant(ctx, oracle, m, H, F):
    """BF16_DEQUANT gate/up + GeGLU + down vs the float64 dequant oracle; the
    large-M shapes run the 128 x 256 tile kernel (partial h tiles for F = 96)."""
    say(f"mlp BF16_DEQUANT m={m} H={H} F={F}")
    x = oracle.normal(m * H, seed=400).reshape(m, H)
    gb, ub, db = (oracle.q8_0_weight(F, H, seed=41), oracle.q8_0_weight(F, H, seed=42),
                  oracle.q8_0_weight(H, F, seed=43))
    g, u, d = (Q8Weight.from_gguf(ctx, gb, F, H), Q8Weight.from_gguf(ctx, ub, F, H),
               Q8Weight.from_gguf(ctx, db, H, F))
    gu, _ = Q8Weight.concat(ctx, [g, u])
    y = host(ops.mlp(ctx, gu, d, dev(x), BF16_DEQUANT))
    gate = oracle.matmul_dequant_f64(x, gb, F).astype(np.float32)
    up = oracle.matmul_dequant_f64(x, ub, F).astype(np.float32)
    ref = oracle.matmul_dequant_f64(oracle.geglu(gate, up), db, H)
    cos = (y * ref).sum(1) / np.linalg.norm(y, axis=1) / np.linalg.norm(ref, axis=1)
    assert cos.min() > 0.999, cos.min()


def test_zero_rows_and_shape_errors(ctx, oracle):
    say("m = 0 no-op and shape errors")
    wb = oracle.q8_0_weight(64, 64, seed=1)
    w = Q8Weight.from_gguf(ctx, wb, 64, 64)
    x = torch.zeros((0, 64), dtype=torch.float32, device="cuda")
    assert ops.q8_0_matmul(ctx, w, x).shape == (0, 64)
    other = Q8Weight.from_gguf(ctx, oracle.q8_0_weight(8, 96, seed=2), 8, 96)
    with pytest.raises(_lib.GlyprError) as e:
        Q8Weight.concat(ctx, [w, other])
    assert e.value.code == _lib.GLYPR_ERR_SHAPE
    with pytest.raises(_lib.GlyprError) as e:
        ops.mlp(ctx, w, other, torch.zeros((4, 64), device="cuda"))
    assert e.value.code == _lib.GLYPR_ERR_SHAPE


# ------------------------------------------------------ C3 (M = 16384) ------

C3_M, C3_H, C3_F = 16384, 768, 1152


def _c3_weights(ctx, oracle):
    qb = oracle.q8_0_weight(1280, C3_H, seed=501)        # q | k | v of one layer
    gb, ub = oracle.q8_0_weight(C3_F, C3_H, seed=502), oracle.q8_0_weight(C3_F, C3_H, seed=503)
    db = oracle.q8_0_weight(C3_H, C3_F, seed=504)
    wq = Q8Weight.from_gguf(ctx, qb, 1280, C3_H)
    g, u = Q8Weight.from_gguf(ctx, gb, C3_F, C3_H), Q8Weight.from_gguf(ctx, ub, C3_F, C3_H)
    d = Q8Weight.from_gguf(ctx, db, C3_H, C3_F)
    gu, _ = Q8Weight.concat(ctx, [g, u])
    return (qb, gb, ub, db), (wq, gu, d)


def test_c3_int8_rmsnorm_geglu_mlp(ctx, oracle):
    """C3's RMSNorm -> gate/up GeGLU -> down at M = 16384 (the large-M GeGLU
    epilogue kernel): two runs bit-identical, 64 sampled rows bit-exact."""
    say(f"C3 INT8_EXACT rmsnorm_mlp m={C3_M}")
    x = oracle.normal(C3_M * C3_H, seed=505).reshape(C3_M, C3_H)
    nw = 1 + 0.1 * oracle.normal(C3_H, seed=506)
    (qb, gb, ub, db), (wq, gu, d) = _c3_weights(ctx, oracle)
    xd, nwd = dev(x), dev(nw)
    y1 = host(ops.rmsnorm_mlp(ctx, gu, d, xd, nwd, 1e-6, INT8_EXACT))
    y2 = host(ops.rmsnorm_mlp(ctx, gu, d, xd, nwd, 1e-6, INT8_EXACT))
    assert np.array_equal(bits(y1), bits(y2))
    rows = np.random.default_rng(5).choice(C3_M, 64, replace=False)
    rows[:2] = [0, C3_M - 1]
    xn = oracle.rmsnorm(x[rows], nw, 1e-6)
    assert_bits_equal(y1[rows], _mlp_ref(oracle, xn, gb, ub, db, C3_H, C3_F), "C3 mlp rows")


def test_c3_bf16_dequant_qkv_and_mlp(ctx, oracle):
    """C3's BF16_DEQUANT launches at M = 16384 (RMSNorm -> bf16 prologue, the
    128 x 256 large-M kernels, the bf16 GeGLU epilogue): sampled rows against
    the float64 dequant oracle within the bf16 bound, and the per-row cosine to
    glypr's CPU Q8_0 path (INT8_EXACT oracle) reported (A5')."""
    say(f"C3 BF16_DEQUANT qkv + mlp m={C3_M}")
    x = oracle.normal(C3_M * C3_H, seed=507).reshape(C3_M, C3_H)
    nw = 1 + 0.1 * oracle.normal(C3_H, seed=508)
    (qb, gb, ub, db), (wq, gu, d) = _c3_weights(ctx, oracle)
    xd, nwd = dev(x), dev(nw)
    y = host(ops.rmsnorm_q8_0_matmul(ctx, wq, xd, nwd, 1e-6, BF16_DEQUANT))
    z = host(ops.rmsnorm_mlp(ctx, gu, d, xd, nwd, 1e-6, BF16_DEQUANT))
    again = host(ops.rmsnorm_q8_0_matmul(ctx, wq, xd, nwd, 1e-6, BF16_DEQUANT))
    assert np.array_equal(bits(y), bits(again))
    rows = np.random.default_rng(6).choice(C3_M, 96, replace=False)
    rows[:2] = [0, C3_M - 1]
    xn = oracle.rmsnorm(x[rows], nw, 1e-6)
    y64 = oracle.matmul_dequant_f64(xn, qb, 1280)
    wd = np.abs(oracle.dequantize_rows(qb, C3_H).astype(np.float64))
    bound = 2.0 ** -7 * (np.abs(xn).astype(np.float64) @ wd.T) * (1 + 1e-3) + 1e-6
    assert np.all(np.abs(y[rows] - y64) <= bound)
    y8 = oracle.matmul(xn, qb, 1280).astype(np.float64)
    c8 = (y[rows] * y8).sum(1) / np.linalg.norm(y[rows], axis=1) / np.linalg.norm(y8, axis=1)
    say(f"  qkv cosine to the INT8_EXACT oracle: min {c8.min():.7f} mean {c8.mean():.7f}")
    assert c8.min() > 0.999
    gate = oracle.matmul_dequant_f64(xn, gb, C3_F).astype(np.float32)
    up = oracle.matmul_dequant_f64(xn, ub, C3_F).astype(np.float32)
    ref = oracle.matmul_dequant_f64(oracle.geglu(gate, up), db, C3_H)
    cz = (z[rows] * ref).sum(1) / np.linalg.norm(z[rows], axis=1) / np.linalg.norm(ref, axis=1)
    assert cz.min() > 0.999, cz.min()
    z8 = _mlp_ref(oracle, xn, gb, ub, db, C3_H, C3_F).astype(np.float64)
    c8 = (z[rows] * z8).sum(1) / np.linalg.norm(z[rows], axis=1) / np.linalg.norm(z8, axis=1)
    say(f"  mlp cosine to the INT8_EXACT oracle: min {c8.min():.7f} mean {c8.mean():.7f}")
    assert c8.min() > 0.998


# ------------------------------------- against glypr's platform-tanh numerics --
# glypr's CPU GeGLU calls the platform tanhf (cpu_simd/geglu.rs:6-18).  This
# library and its oracle share their own tanh instead, a few ulp from glibc's
# (test_geglu_tanh_substitution_is_ulp_level).  Where such an ulp moves an h
# value across a rounding boundary of its Q8_0 block, one int8 of the down
# projection's input changes by 1: these tests hold the GPU path to an oracle
# built on glibc's tanhf (geglu_libm), at BASELINE's tolerance, and report how
# many bytes of Q8_0(h) the substitution changed.

def _mlp_ref_libm(oracle, xn, gb, ub, db, H, F):
    gate, up = oracle.matmul(xn, gb, F), oracle.matmul(xn, ub, F)
    h_ours, h_libm = oracle.geglu(gate, up), oracle.geglu_libm(gate, up)
    flips = int(np.count_nonzero(oracle.quantize_rows(h_ours) != oracle.quantize_rows(h_libm)))
    return oracle.matmul(h_libm, db, H), flips


@pytest.mark.parametrize("m", [512, C3_M])
def test_mlp_vs_platform_tanh(ctx, oracle, m):
    """The INT8_EXACT RMSNorm -> gate/up GeGLU -> down MLP at C2's M = 512 (every
    row) and C3's M = 16384 (256 sampled rows) against the glibc-tanhf oracle."""
    H, F = 768, 1152
    say(f"INT8_EXACT rmsnorm_mlp m={m} vs the platform-tanh oracle")
    x = oracle.normal(m * H, seed=611).reshape(m, H)
    nw = 1 + 0.1 * oracle.normal(H, seed=612)
    gb, ub, db = (oracle.q8_0_weight(F, H, seed=613), oracle.q8_0_weight(F, H, seed=614),
                  oracle.q8_0_weight(H, F, seed=615))
    g, u = Q8Weight.from_gguf(ctx, gb, F, H), Q8Weight.from_gguf(ctx, ub, F, H)
    d = Q8Weight.from_gguf(ctx, db, H, F)
    gu, _ = Q8Weight.concat(ctx, [g, u])
    y = host(ops.rmsnorm_mlp(ctx, gu, d, dev(x), dev(nw), 1e-6, INT8_EXACT))
    rows = np.arange(m) if m <= 512 else np.sort(np.random.default_rng(7).choice(m, 256, False))
    ref, flips = _mlp_ref_libm(oracle, oracle.rmsnorm(x[rows], nw, 1e-6), gb, ub, db, H, F)
    err = np.abs(y[rows].astype(np.float64) - ref)
    rel = err / np.maximum(np.abs(ref), 1e-4)
    say(f"  bytes of Q8_0(h) changed by the tanh substitution: {flips} of {len(rows) * F}; "
        f"max |d| {err.max():.3g}, max relative (1e-4 floor) {rel.max():.3g}")
    baseline_tolerance(y[rows], ref.astype(np.float64))


def test_c2_layer_vs_platform_tanh(ctx, oracle):
    """C2, one layer's seven projections at T = 512 (RMSNorm -> q|k|v, o,
    RMSNorm -> gate/up GeGLU -> down), against the glibc-tanhf oracle: the
    projections without a GeGLU stay bit-exact, the MLP meets BASELINE's
    tolerance."""
    m, H, F = 512, 768, 1152
    say("C2 layer projections vs the platform-tanh oracle")
    x = oracle.normal(m * H, seed=621).reshape(m, H)
    ctxv = oracle.normal(m * H, seed=622).reshape(m, H)
    n1, n2 = 1 + 0.1 * oracle.normal(H, seed=623), 1 + 0.1 * oracle.normal(H, seed=624)
    qkvb = oracle.q8_0_weight(1280, H, seed=625)
    ob = oracle.q8_0_weight(H, H, seed=626)
    gb, ub, db = (oracle.q8_0_weight(F, H, seed=627), oracle.q8_0_weight(F, H, seed=628),
                  oracle.q8_0_weight(H, F, seed=629))
    wqkv, wo = Q8Weight.from_gguf(ctx, qkvb, 1280, H), Q8Weight.from_gguf(ctx, ob, H, H)
    g, u = Q8Weight.from_gguf(ctx, gb, F, H), Q8Weight.from_gguf(ctx, ub, F, H)
    d = Q8Weight.from_gguf(ctx, db, H, F)
    gu, _ = Q8Weight.concat(ctx, [g, u])
    qkv = host(ops.rmsnorm_q8_0_matmul(ctx, wqkv, dev(x), dev(n1), 1e-6, INT8_EXACT))
    o = host(ops.q8_0_matmul(ctx, wo, dev(ctxv), INT8_EXACT))
    y = host(ops.rmsnorm_mlp(ctx, gu, d, dev(x), dev(n2), 1e-6, INT8_EXACT))
    assert_bits_equal(qkv, oracle.matmul(oracle.rmsnorm(x, n1, 1e-6), qkvb, 1280), "qkv")
    assert_bits_equal(o, oracle.matmul(ctxv, ob, H), "o")
    ref, flips = _mlp_ref_libm(oracle, oracle.rmsnorm(x, n2, 1e-6), gb, ub, db, H, F)
    say(f"  bytes of Q8_0(h) changed by the tanh substitution: {flips} of {m * F}")
    baseline_tolerance(y, ref.astype(np.float64))
