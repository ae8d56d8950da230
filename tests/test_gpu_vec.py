"""GPU parity of the output-vector codecs (glypr-core util.rs:52-197) through
the C ABI against the CPU oracle.

Bar: bit-exact everywhere.  The encodings and the hamming / int8 dot sums are
integers; int8_cosine uses only IEEE-rounded f32 ops (i32 -> f32, sqrt, *, /);
binary_cosine reads a table the host fills with the same libm cosf the oracle
calls.  Shapes cover the word counts with a register-resident kernel (1, 2, 4,
8, 12, 16) and the generic one (5, 40), int8 dims on the 8-byte fast path and
the byte path, and row counts that leave partial tiles.
"""
import sys

import numpy as np
import pytest
import torch

from glypr_amd import ops

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_quantize_binary_and_int8(ctx, oracle):
    rng = np.random.default_rng(11)
    for n, dim in [(1, 64), (3, 768), (37, 256), (5, 320)]:
        say(f"quantize_binary n={n} dim={dim}")
        x = rng.standard_normal((n, dim)).astype(np.float32)
        x[0, :6] = [0.0, -0.0, np.nan, np.inf, -np.inf, 1e-45]
        got = host(ops.quantize_binary(ctx, dev(x))).view(np.uint64)
        assert np.array_equal(got, oracle.quantize_binary(x))
    # more 256-element chunks than one pass of the capped grid (16384 blocks x
    # 4 waves x 4 chunks = 262144): the grid-stride loop runs a second round
    n = 262144 + 300
    say(f"quantize_binary n={n} dim=256 (grid-stride)")
    x = rng.standard_normal((n, 256)).astype(np.float32)
    got = host(ops.quantize_binary(ctx, dev(x))).view(np.uint64)
    assert np.array_equal(got, oracle.quantize_binary(x))
    with pytest.raises(Exception):
        ops.quantize_binary(ctx, dev(np.ones((1, 65), np.float32)))
    for count in (5, 1001, 768 * 33):
        say(f"quantize_int8 count={count}")
        x = rng.uniform(-1.3, 1.3, count).astype(np.float32)
        x[:5] = [np.nan, np.inf, -np.inf, 0.5, -5.0]
        got = host(ops.quantize_int8(ctx, dev(x)))
        assert np.array_equal(got, oracle.quantize_int8(x))
    got = host(ops.quantize_int8(ctx, dev(np.array([1.0, -1.0, 0.0, 0.5], np.float32))))
    assert got.tolist() == [127, -127, 0, 64]            # tests/quantization.rs:28-30


@pytest.mark.parametrize("words", [1, 2, 4, 5, 8, 12, 16, 40])
def test_hamming_and_binary_cosine(ctx, oracle, words):
    say(f"hamming / binary_cosine words={words}")
    rng = np.random.default_rng(100 + words)
    na, nb = 5, 300
    a = rng.integers(0, 2**64, size=(na, words), dtype=np.uint64)
    b = rng.integers(0, 2**64, size=(nb, words), dtype=np.uint64)
    b[0] = a[0]
    b[1] = ~a[0]
    da, db = dev(a.view(np.int64)), dev(b.view(np.int64))
    h = host(ops.hamming(ctx, da, db)).view(np.uint32)
    assert np.array_equal(h, oracle.hamming(a, b))
    assert h[0, 0] == 0 and h[0, 1] == 64 * words
    c = host(ops.binary_cosine(ctx, da, db))
    assert np.array_equal(c.view(np.uint32), oracle.binary_cosine(a, b).view(np.uint32))


def test_binary_cosine_every_distance(ctx, oracle):
    """Every h in [0, dim] for the MRL dims: the table equals the oracle's cosf."""
    for words in (1, 2, 4, 8, 12):
        dim = 64 * words
        say(f"binary_cosine exhaustive dim={dim}")
        a = np.zeros((1, words), np.uint64)
        b = np.zeros((dim + 1, words), np.uint64)
        for h in range(dim + 1):           # first h bits set
            for w in range(words):
                nbit = min(max(h - 64 * w, 0), 64)
                b[h, w] = np.uint64((1 << nbit) - 1) if nbit < 64 else np.uint64(2**64 - 1)
        c = host(ops.binary_cosine(ctx, dev(a.view(np.int64)), dev(b.view(np.int64))))
        assert np.array_equal(c.view(np.uint32), oracle.binary_cosine(a, b).view(np.uint32))


@pytest.mark.parametrize("na,nb,dim", [(1, 1, 4), (3, 70, 768), (64, 129, 256),
                                       (70, 33, 100), (17, 500, 1024), (2, 40, 7)])
def test_int8_dot_and_cosine(ctx, oracle, na, nb, dim):
    say(f"int8_dot / int8_cosine na={na} nb={nb} dim={dim}")
    rng = np.random.default_rng(na * 1000 + dim)
    a = rng.integers(-127, 128, size=(na, dim), dtype=np.int8)
    b = rng.integers(-127, 128, size=(nb, dim), dtype=np.int8)
    b[0] = 0                                   # zero norm -> cosine 0
    if na > 1:
        a[1] = -127                            # largest |sums|
        b[-1] = 127
    d = host(ops.int8_dot(ctx, dev(a), dev(b)))
    assert np.array_equal(d, oracle.int8_dot(a, b))
    c = host(ops.int8_cosine(ctx, dev(a), dev(b)))
    assert np.array_equal(c.view(np.uint32), oracle.int8_cosine(a, b).view(np.uint32))


def test_end_to_end_encode_and_search(ctx, oracle):
    """Embeddings -> int8 / binary codes -> all-pairs similarity, on the GPU,
    equal to the reference functions applied row by row."""
    rng = np.random.default_rng(12)
    emb = rng.standard_normal((200, 256)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    e = dev(emb)
    q8 = ops.quantize_int8(ctx, e)
    qb = ops.quantize_binary(ctx, e)
    ci = host(ops.int8_cosine(ctx, q8[:8].contiguous(), q8))
    cb = host(ops.binary_cosine(ctx, qb[:8].contiguous(), qb))
    ref_q8 = oracle.quantize_int8(emb)
    ref_qb = oracle.quantize_binary(emb)
    assert np.array_equal(ci.view(np.uint32),
                          oracle.int8_cosine(ref_q8[:8], ref_q8).view(np.uint32))
    assert np.array_equal(cb.view(np.uint32),
                          oracle.binary_cosine(ref_qb[:8], ref_qb).view(np.uint32))
    # each query's best match is itself
    assert np.array_equal(np.argmax(ci, axis=1), np.arange(8))
