"""ctypes + numpy binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker.  The product package
(glypr_amd) never imports this module.

The oracle restates glypr's CPU Q8_0 path (candle k_quants Q8_0 + glypr's
cpu_simd ops); see glypr_oracle.h for the per-function reference citations.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
QK8_0 = 32
BLOCK_BYTES = 34

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", HERE, "liboracle.so"], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB_PATH


class ModelConfig(ctypes.Structure):
    _fields_ = [("hidden", _i64), ("ffn", _i64), ("n_heads", _i64), ("n_kv_heads", _i64),
                ("head_dim", _i64), ("n_layers", _i64), ("vocab", _i64),
                ("sliding_window", _i64), ("eps", ctypes.c_float),
                ("rope_theta_sliding", ctypes.c_double), ("rope_theta_full", ctypes.c_double),
                ("ple_dim", _i64), ("out_dim", _i64), ("full_head_dim", _i64),
                ("full_n_kv_heads", _i64), ("layer_types", ctypes.c_void_p)]


class LayerWeights(ctypes.Structure):
    _fields_ = [(n, _u8p) for n in ("q", "k", "v", "o", "gate", "up", "down")] + \
               [(n, _f32p) for n in ("input_norm", "post_attn_norm", "pre_ffn_norm",
                                     "post_ffn_norm", "q_norm", "k_norm")] + \
               [("ple_gate", _u8p), ("ple_proj", _u8p), ("ple_post_norm", _f32p),
                ("layer_scalar", _f32p)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16_array": (None, [_f32p, _u16p, _i64]),
            "orc_f16_to_f32_array": (None, [_u16p, _f32p, _i64]),
            "orc_q8_0_quantize_rows": (None, [_f32p, _i64, _i64, _u8p]),
            "orc_q8_0_dequantize_rows": (None, [_u8p, _i64, _i64, _f32p]),
            "orc_q8_0_vec_dot": (ctypes.c_float, [_i64, _u8p, _u8p]),
            "orc_q8_0_matmul": (None, [_f32p, _i64, _i64, _u8p, _i64, _f32p, ctypes.c_int]),
            "orc_q8_0_matmul_preq": (None, [_u8p, _i64, _i64, _u8p, _i64, _f32p, ctypes.c_int]),
            "orc_q8_0_vec_dot_fma": (ctypes.c_float, [_i64, _u8p, _u8p]),
            "orc_q8_0_matmul_fma": (None, [_f32p, _i64, _i64, _u8p, _i64, _f32p, ctypes.c_int]),
            "orc_q8_0_matmul_f64": (None, [_u8p, _i64, _i64, _u8p, _i64, _f64p]),
            "orc_q8_0_matmul_dequant_f64": (None, [_f32p, _i64, _i64, _u8p, _i64, _f64p,
                                                   ctypes.c_int]),
            "orc_rmsnorm": (None, [_f32p, _f32p, ctypes.c_float, _f32p, _i64, _i64,
                                   ctypes.c_int]),
            "orc_tanhf": (ctypes.c_float, [ctypes.c_float]),
            "orc_geglu_scalar": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "orc_geglu_scalar_libm": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "orc_geglu_libm": (None, [_f32p, _f32p, _f32p, _i64, ctypes.c_int]),
            "orc_geglu": (None, [_f32p, _f32p, _f32p, _i64, ctypes.c_int]),
            "orc_embed_gather": (ctypes.c_int, [_u8p, _i64, _i64, _u32p, _i64, ctypes.c_float,
                                                _f32p]),
            "orc_pool_normalize": (None, [_f32p, _u8p, _i64, _i64, _i64, _f32p]),
            "orc_l2_normalize": (None, [_f32p, _i64, _f32p]),
            "orc_cosine": (ctypes.c_float, [_f32p, _f32p, _i64]),
            "orc_quantize_binary": (ctypes.c_int, [_f32p, _i64, _u64p]),
            "orc_hamming": (ctypes.c_uint32, [_u64p, _u64p, _i64]),
            "orc_binary_cosine": (ctypes.c_float, [_u64p, _u64p, _i64]),
            "orc_quantize_int8": (None, [_f32p, _i64, _i8p]),
            "orc_int8_dot": (ctypes.c_int32, [_i8p, _i8p, _i64]),
            "orc_int8_cosine": (ctypes.c_float, [_i8p, _i8p, _i64]),
            "orc_splitmix64": (ctypes.c_uint64, [ctypes.POINTER(ctypes.c_uint64)]),
            "orc_fill_normal": (None, [_f32p, _i64, ctypes.c_uint64, ctypes.c_float,
                                       ctypes.c_float]),
            "orc_fill_uniform_ids": (None, [_u32p, _i64, ctypes.c_uint64, ctypes.c_uint32]),
            "orc_make_q8_0_weight": (None, [_u8p, _i64, _i64, ctypes.c_uint64, ctypes.c_float]),
            "orc_layer_is_full": (ctypes.c_int, [_i64]),
            "orc_rope_tables": (None, [_i64, ctypes.c_double, _i64, _f32p, _f32p]),
            "orc_attention": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _f32p,
                                     ctypes.c_int]),
            "orc_encoder_layer": (None, [ctypes.POINTER(ModelConfig),
                                         ctypes.POINTER(LayerWeights), _i64, _f32p, _f32p, _i64,
                                         ctypes.c_int]),
            "orc_model_forward": (ctypes.c_int, [ctypes.POINTER(ModelConfig),
                                                 _u8p, ctypes.POINTER(LayerWeights), _f32p,
                                                 _u8p, _f32p, _u8p, _u32p,
                                                 _i64, _i64, _f32p, _f32p, ctypes.c_int]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: Optional[np.ndarray], ptype):
    if a is None:
        return ctypes.cast(None, ptype)
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ptype)


# ---------------------------------------------------------------- codec ----

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


def quantize_rows(x: np.ndarray) -> np.ndarray:
    """f32 [m,k] -> GGUF Q8_0 blocks uint8 [m, k/32*34]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    out = np.empty((m, k // QK8_0 * BLOCK_BYTES), np.uint8)
    lib().orc_q8_0_quantize_rows(_p(x, _f32p), m, k, _p(out, _u8p))
    return out


def dequantize_rows(blocks: np.ndarray, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows = blocks.size // (k // QK8_0 * BLOCK_BYTES)
    out = np.empty((rows, k), np.float32)
    lib().orc_q8_0_dequantize_rows(_p(blocks, _u8p), rows, k, _p(out, _f32p))
    return out


def split_blocks(blocks: np.ndarray, k: int):
    """GGUF Q8_0 bytes [rows, k/32*34] -> (d f16 bits uint16 [rows, nb], qs int8 [rows, k])."""
    nb = k // QK8_0
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, nb, BLOCK_BYTES)
    d = b[:, :, :2].copy().view(np.uint16).reshape(-1, nb)
    qs = b[:, :, 2:].copy().view(np.int8).reshape(-1, k)
    return d, qs


def join_blocks(d_bits: np.ndarray, qs: np.ndarray) -> np.ndarray:
    rows, k = qs.shape
    nb = k // QK8_0
    out = np.empty((rows, nb, BLOCK_BYTES), np.uint8)
    out[:, :, :2] = np.ascontiguousarray(d_bits, dtype=np.uint16).reshape(rows, nb, 1).view(
        np.uint8)
    out[:, :, 2:] = np.ascontiguousarray(qs, dtype=np.int8).reshape(rows, nb, QK8_0).view(np.uint8)
    return out.reshape(rows, nb * BLOCK_BYTES)


# ---------------------------------------------------------------- GEMM -----

def matmul(x: np.ndarray, w_blocks: np.ndarray, n: int, threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    y = np.empty((m, n), np.float32)
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    lib().orc_q8_0_matmul(_p(x, _f32p), m, k, _p(w, _u8p), n, _p(y, _f32p), threads)
    return y


def matmul_fma(x: np.ndarray, w_blocks: np.ndarray, n: int, threads: int = 0) -> np.ndarray:
    """The INT8_FMA variant: matmul's operands, each block's term added with
    one fused multiply-add (orc_q8_0_vec_dot_fma)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    y = np.empty((m, n), np.float32)
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    lib().orc_q8_0_matmul_fma(_p(x, _f32p), m, k, _p(w, _u8p), n, _p(y, _f32p), threads)
    return y


def vec_dot_fma(k: int, w_blocks: np.ndarray, x_blocks: np.ndarray) -> float:
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    xb = np.ascontiguousarray(x_blocks, dtype=np.uint8)
    return float(lib().orc_q8_0_vec_dot_fma(k, _p(w, _u8p), _p(xb, _u8p)))


def matmul_preq(xq: np.ndarray, m: int, k: int, w_blocks: np.ndarray, n: int,
                threads: int = 0) -> np.ndarray:
    y = np.empty((m, n), np.float32)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    lib().orc_q8_0_matmul_preq(_p(xq, _u8p), m, k, _p(w, _u8p), n, _p(y, _f32p), threads)
    return y


def matmul_f64(xq: np.ndarray, m: int, k: int, w_blocks: np.ndarray, n: int) -> np.ndarray:
    y = np.empty((m, n), np.float64)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    lib().orc_q8_0_matmul_f64(_p(xq, _u8p), m, k, _p(w, _u8p), n, _p(y, _f64p))
    return y


def matmul_dequant_f64(x: np.ndarray, w_blocks: np.ndarray, n: int, threads: int = 0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    y = np.empty((m, n), np.float64)
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    lib().orc_q8_0_matmul_dequant_f64(_p(x, _f32p), m, k, _p(w, _u8p), n, _p(y, _f64p), threads)
    return y


# ------------------------------------------------------------- elementwise --

def rmsnorm(x: np.ndarray, weight: Optional[np.ndarray], eps: float = 1e-6,
            threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    rows = x.size // d
    y = np.empty_like(x)
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.float32)
    lib().orc_rmsnorm(_p(x, _f32p), _p(w, _f32p), ctypes.c_float(eps), _p(y, _f32p), rows, d,
                      threads)
    return y


def tanhf(x: float) -> float:
    return lib().orc_tanhf(ctypes.c_float(x))


def geglu(gate: np.ndarray, up: np.ndarray, threads: int = 0) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    assert g.shape == u.shape
    out = np.empty_like(g)
    lib().orc_geglu(_p(g, _f32p), _p(u, _f32p), _p(out, _f32p), g.size, threads)
    return out


def geglu_libm(gate: np.ndarray, up: np.ndarray, threads: int = 0) -> np.ndarray:
    """geglu with the platform tanhf (glypr's own CPU numerics on glibc)."""
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    assert g.shape == u.shape
    out = np.empty_like(g)
    lib().orc_geglu_libm(_p(g, _f32p), _p(u, _f32p), _p(out, _f32p), g.size, threads)
    return out


def embed_gather(table_blocks: np.ndarray, vocab: int, d: int, ids: np.ndarray,
                 scale: float) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.empty((ids.size, d), np.float32)
    t = np.ascontiguousarray(table_blocks, dtype=np.uint8)
    rc = lib().orc_embed_gather(_p(t, _u8p), vocab, d, _p(ids, _u32p), ids.size,
                                ctypes.c_float(scale), _p(out, _f32p))
    if rc != 0:
        raise IndexError("token id out of range")
    return out


def pool_normalize(tokens: np.ndarray, mask: Optional[np.ndarray] = None,
                   trunc: int = 0) -> np.ndarray:
    tok = np.ascontiguousarray(tokens, dtype=np.float32)
    t, d = tok.shape
    td = trunc if 0 < trunc < d else d
    out = np.empty(td, np.float32)
    mk = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    lib().orc_pool_normalize(_p(tok, _f32p), _p(mk, _u8p), t, d, trunc, _p(out, _f32p))
    return out


def l2_normalize(x: np.ndarray) -> np.ndarray:
    """util.rs:22-29 (orc_l2_normalize)."""
    v = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty_like(v)
    lib().orc_l2_normalize(_p(v, _f32p), v.size, _p(out, _f32p))
    return out


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    """util.rs:32-41 (orc_cosine), as an f32."""
    va = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    vb = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
    assert va.size == vb.size
    return np.float32(lib().orc_cosine(_p(va, _f32p), _p(vb, _f32p), va.size))


# --------------------------------------------------------- vector codecs ----
# glypr-core util.rs:52-197; the C restatement holds the citations.

def quantize_binary(x: np.ndarray) -> np.ndarray:
    """f32 [n, dim] -> u64 [n, dim/64]; ValueError when dim % 64 != 0."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    n, dim = x.shape
    out = np.zeros((n, max(dim // 64, 0)), np.uint64)
    for r in range(n):
        row = np.ascontiguousarray(x[r])
        dst = out[r] if dim >= 64 else np.zeros(1, np.uint64)
        if lib().orc_quantize_binary(_p(row, _f32p), dim, _p(dst, _u64p)) != 0:
            raise ValueError(f"binary quantization requires a multiple of 64, got {dim}")
    return out


def hamming(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """All pairs: u64 [na, w], [nb, w] -> u32 [na, nb]."""
    a = np.ascontiguousarray(np.atleast_2d(a), dtype=np.uint64)
    b = np.ascontiguousarray(np.atleast_2d(b), dtype=np.uint64)
    out = np.empty((a.shape[0], b.shape[0]), np.uint32)
    for i in range(a.shape[0]):
        for j in range(b.shape[0]):
            out[i, j] = lib().orc_hamming(_p(a[i], _u64p), _p(b[j], _u64p), a.shape[1])
    return out


def binary_cosine(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(np.atleast_2d(a), dtype=np.uint64)
    b = np.ascontiguousarray(np.atleast_2d(b), dtype=np.uint64)
    out = np.empty((a.shape[0], b.shape[0]), np.float32)
    for i in range(a.shape[0]):
        for j in range(b.shape[0]):
            out[i, j] = lib().orc_binary_cosine(_p(a[i], _u64p), _p(b[j], _u64p), a.shape[1])
    return out


def quantize_int8(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.int8)
    lib().orc_quantize_int8(_p(x, _f32p), x.size, _p(out, _i8p))
    return out


def int8_dot(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """All pairs: i8 [na, d], [nb, d] -> i32 [na, nb]."""
    a = np.ascontiguousarray(np.atleast_2d(a), dtype=np.int8)
    b = np.ascontiguousarray(np.atleast_2d(b), dtype=np.int8)
    out = np.empty((a.shape[0], b.shape[0]), np.int32)
    for i in range(a.shape[0]):
        for j in range(b.shape[0]):
            out[i, j] = lib().orc_int8_dot(_p(a[i], _i8p), _p(b[j], _i8p), a.shape[1])
    return out


def int8_cosine(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(np.atleast_2d(a), dtype=np.int8)
    b = np.ascontiguousarray(np.atleast_2d(b), dtype=np.int8)
    out = np.empty((a.shape[0], b.shape[0]), np.float32)
    for i in range(a.shape[0]):
        for j in range(b.shape[0]):
            out[i, j] = lib().orc_int8_cosine(_p(a[i], _i8p), _p(b[j], _i8p), a.shape[1])
    return out


# ------------------------------------------------------------ synthetic ----

def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(_p(out, _f32p), n, seed, ctypes.c_float(mean), ctypes.c_float(std))
    return out


def uniform_ids(n: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().orc_fill_uniform_ids(_p(out, _u32p), n, seed, vocab)
    return out


def q8_0_weight(n: int, k: int, seed: int, sigma: float = 0.02) -> np.ndarray:
    """GGUF Q8_0 bytes [n, k/32*34] with BASELINE's synthetic distribution."""
    out = np.empty((n, k // QK8_0 * BLOCK_BYTES), np.uint8)
    lib().orc_make_q8_0_weight(_p(out, _u8p), n, k, seed, ctypes.c_float(sigma))
    return out


def rope_tables(head_dim: int, theta: float, t: int):
    c = np.empty((t, head_dim), np.float32)
    s = np.empty((t, head_dim), np.float32)
    lib().orc_rope_tables(head_dim, theta, t, _p(c, _f32p), _p(s, _f32p))
    return c, s


def attention(q, k, v, window: int, threads: int = 0):
    """q [nh,t,hd], k/v [nkv,t,hd] -> ctx [t, nh*hd]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    nh, t, hd = q.shape
    nkv = k.shape[0]
    out = np.empty((t, nh * hd), np.float32)
    lib().orc_attention(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), nh, nkv, t, hd, window,
                        _p(out, _f32p), threads)
    return out


def model_forward(tensors: dict, ids: np.ndarray, trunc: int, *, hidden: int, ffn: int,
                  n_heads: int, n_kv_heads: int, head_dim: int, n_layers: int, vocab: int,
                  sliding_window: int = 512, eps: float = 1e-6, theta_sliding: float = 1e4,
                  theta_full: float = 1e6, full_head_dim: int = 0, full_n_kv_heads: int = 0,
                  threads: int = 0, layer_types=None):
    """orc_model_forward over GGUF-named tensors {name: array} (Q8_0 tensors as
    block bytes, norms as f32).  The PLE block runs when
    `per_layer_model_proj.weight` is present (ple_dim = its rows / n_layers),
    the embedding projection when `output.weight` is.  layer_types (n_layers
    values, nonzero = full attention) replaces the default 5 sliding + 1 full
    pattern.  Returns (pooled [trunc or out dim], unpooled token embeddings
    [t, out dim])."""
    ple_dim = 0
    if "per_layer_model_proj.weight" in tensors:
        ple_dim = tensors["per_layer_model_proj.weight"].shape[0] // n_layers
    out_dim = tensors["output.weight"].shape[0] if "output.weight" in tensors else 0
    cfg = ModelConfig(hidden=hidden, ffn=ffn, n_heads=n_heads, n_kv_heads=n_kv_heads,
                      head_dim=head_dim, n_layers=n_layers, vocab=vocab,
                      sliding_window=sliding_window, eps=eps, rope_theta_sliding=theta_sliding,
                      rope_theta_full=theta_full, ple_dim=ple_dim, out_dim=out_dim,
                      full_head_dim=full_head_dim, full_n_kv_heads=full_n_kv_heads)
    keep = []
    if layer_types is not None:
        lt = np.ascontiguousarray(np.asarray(layer_types) != 0, dtype=np.uint8)
        assert lt.size == n_layers
        keep.append(lt)
        cfg.layer_types = lt.ctypes.data

    def arr(name, dt, ptype):
        if name not in tensors:
            return ctypes.cast(None, ptype)
        a = np.ascontiguousarray(tensors[name], dtype=dt)
        keep.append(a)
        return _p(a, ptype)

    layers = (LayerWeights * n_layers)()
    for i in range(n_layers):
        p = f"blk.{i}."
        layers[i] = LayerWeights(
            *[arr(p + n + ".weight", np.uint8, _u8p) for n in
              ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")],
            *[arr(p + n + ".weight", np.float32, _f32p) for n in
              ("attn_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm", "attn_q_norm",
               "attn_k_norm")],
            arr(p + "inp_gate.weight", np.uint8, _u8p), arr(p + "proj.weight", np.uint8, _u8p),
            arr(p + "post_norm.weight", np.float32, _f32p),
            arr(p + "layer_output_scale.weight", np.float32, _f32p))
    ids = np.ascontiguousarray(ids, np.uint32)
    t = ids.size
    d = out_dim or hidden
    out = np.empty(trunc if 0 < trunc < d else d, np.float32)
    states = np.empty((t, d), np.float32)
    rc = lib().orc_model_forward(ctypes.byref(cfg), arr("token_embd.weight", np.uint8, _u8p),
                                 layers, arr("output_norm.weight", np.float32, _f32p),
                                 arr("per_layer_model_proj.weight", np.uint8, _u8p),
                                 arr("per_layer_proj_norm.weight", np.float32, _f32p),
                                 arr("output.weight", np.uint8, _u8p),
                                 _p(ids, _u32p), t, trunc, _p(out, _f32p), _p(states, _f32p),
                                 threads)
    if rc != 0:
        raise ValueError("orc_model_forward: token id out of range")
    return out, states
