"""Oracle pinning for the output-vector codecs (glypr-core util.rs:52-197).

Known answers are the reference's own (tests/quantization.rs:10-31,
util.rs:273-306); everything else is checked against an independent statement:
numpy's packbits / unpackbits for the bit codecs, int64 matmul for the int8
dot, float64 for the cosines, and the f32 round-half-away formula written with
floor for quantize_int8."""
import numpy as np
import pytest

from oracle import pyoracle as o


def test_reference_known_answers():
    # tests/quantization.rs:12-25, util.rs:273-290
    for dim in (63, 65):
        with pytest.raises(ValueError):
            o.quantize_binary(np.ones(dim, np.float32))
    assert o.quantize_binary(np.full(128, 0.1, np.float32)).shape == (1, 2)
    ones = o.quantize_binary(np.ones(64, np.float32))
    neg = o.quantize_binary(-np.ones(64, np.float32))
    assert ones.shape == (1, 1) and int(ones[0, 0]) == 2**64 - 1
    assert int(neg[0, 0]) == 0
    assert o.hamming(ones, neg)[0, 0] == 64
    assert o.hamming(ones, ones)[0, 0] == 0
    assert abs(o.binary_cosine(ones, neg)[0, 0] - (-1.0)) < 1e-6
    assert abs(o.binary_cosine(ones, ones)[0, 0] - 1.0) < 1e-6
    # tests/quantization.rs:28-31, util.rs:293-306
    q = o.quantize_int8(np.array([1.0, -1.0, 0.0, 0.5], np.float32))
    assert q.tolist() == [127, -127, 0, 64]
    qb = o.quantize_int8(np.array([1.0, 1.0, 0.0, 0.5], np.float32))
    assert o.int8_dot(q, qb)[0, 0] == 64 * 64
    assert abs(o.int8_cosine(q, q)[0, 0] - 1.0) < 1e-5


def _packbits_u64(x):
    """Independent statement: bit i of word i/64 = x[i] > 0 via numpy packbits."""
    bits = np.packbits(np.asarray(x) > 0, axis=-1, bitorder="little")
    return np.ascontiguousarray(bits).view("<u8")


def test_quantize_binary_matches_packbits():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 768)).astype(np.float32)
    x[0, :10] = [0.0, -0.0, np.nan, -np.nan, np.inf, -np.inf, 1e-45, -1e-45, 1e-38, -1e-38]
    assert np.array_equal(o.quantize_binary(x), _packbits_u64(x))


def test_hamming_matches_unpackbits_and_invariants():
    rng = np.random.default_rng(6)
    a = rng.integers(0, 2**64, size=(5, 12), dtype=np.uint64)
    b = rng.integers(0, 2**64, size=(9, 12), dtype=np.uint64)
    h = o.hamming(a, b)
    ref = np.unpackbits((a[:, None, :] ^ b[None, :, :]).view(np.uint8), axis=-1).sum(-1)
    assert np.array_equal(h, ref.astype(np.uint32))
    assert np.array_equal(o.hamming(b, a), h.T)                       # symmetry
    assert np.array_equal(np.diag(o.hamming(a, ~a)), np.full(5, 768))  # complement
    # triangle inequality
    hab, hbc, hac = o.hamming(a[:1], b[:1])[0, 0], o.hamming(b[:1], b[1:2])[0, 0], \
        o.hamming(a[:1], b[1:2])[0, 0]
    assert hac <= hab + hbc


def test_binary_cosine_against_float64():
    rng = np.random.default_rng(7)
    for words in (1, 2, 4, 12):
        a = rng.integers(0, 2**64, size=(4, words), dtype=np.uint64)
        b = rng.integers(0, 2**64, size=(6, words), dtype=np.uint64)
        c = o.binary_cosine(a, b)
        h = o.hamming(a, b).astype(np.float64)
        ref = np.cos(np.pi * h / (64 * words))
        assert np.max(np.abs(c.astype(np.float64) - ref)) < 2e-7
    assert o.binary_cosine(np.zeros((1, 0), np.uint64), np.zeros((1, 0), np.uint64))[0, 0] == 1.0


def test_quantize_int8_round_half_away_and_saturation():
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.uniform(-1.2, 1.2, 5000).astype(np.float32),
                        # odd k / 254: x * 127 falls on or next to the k / 2 ties
                        (np.arange(-253, 254, 2, dtype=np.float32) / np.float32(254.0)),
                        np.array([2.0, -5.0, np.inf, -np.inf, np.nan, 0.0, -0.0],
                                 np.float32)])
    v = x * np.float32(127.0)                        # f32 product, as the reference
    with np.errstate(invalid="ignore"):
        ref = np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))
        ref = np.clip(ref, -127, 127)
    ref = np.where(np.isnan(ref), 0, ref).astype(np.int8)
    assert np.array_equal(o.quantize_int8(x), ref)
    assert o.quantize_int8(np.array([-5.0], np.float32))[0] == -127   # not -128


def test_int8_dot_and_cosine_against_int64_and_float64():
    rng = np.random.default_rng(9)
    a = rng.integers(-127, 128, size=(4, 100), dtype=np.int8)
    b = rng.integers(-127, 128, size=(7, 100), dtype=np.int8)
    b[0] = 0
    dot = o.int8_dot(a, b)
    ref = a.astype(np.int64) @ b.astype(np.int64).T
    assert np.array_equal(dot, ref.astype(np.int32))
    c = o.int8_cosine(a, b)
    na = (a.astype(np.int64) ** 2).sum(1)
    nb = (b.astype(np.int64) ** 2).sum(1)
    with np.errstate(invalid="ignore", divide="ignore"):
        ref_c = ref / np.sqrt(np.outer(na, nb).astype(np.float64))
    ref_c = np.where(np.outer(na, nb) == 0, 0.0, np.clip(ref_c, -1, 1))
    assert np.all(c[:, 0] == 0.0)                     # zero vector -> 0
    assert np.max(np.abs(c - ref_c)) < 3e-7
    assert np.all(np.abs(np.diag(o.int8_cosine(a, a)) - 1.0) < 1e-6)
