"""Torch-tensor helpers over the C ABI (tests, bench, smoke).

PyTorch only provides device memory and the current HIP stream here; every
computation is a libglypr_hip.so kernel.  Tensors must be contiguous and live
on the context's device.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np
import torch

from ._lib import (BF16_DEQUANT, GLYPR_ERR_UNSUPPORTED, INT8_EXACT, INT8_FMA, GlyprError, check,
                   lib)

__all__ = ["Context", "Q8Weight", "BF16Weight", "INT8_EXACT", "BF16_DEQUANT", "INT8_FMA",
           "q8_0_matmul", "bf16_matmul", "f32_to_bf16_bits",
           "rmsnorm_q8_0_matmul", "rmsnorm", "geglu", "mlp", "rmsnorm_mlp", "dequantize",
           "quantize", "embed_gather", "pool_normalize"]


def _ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


class Context:
    """glypr_hip_ctx for one device."""

    def __init__(self, device: int = 0):
        self.device = device
        h = ctypes.c_void_p()
        check(lib().glypr_hip_ctx_create(device, ctypes.byref(h)))
        self.handle = h

    @property
    def stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    def sync(self):
        check(lib().glypr_hip_sync(self.handle, self.stream))

    def reserve(self, rows: int):
        """glypr_hip_ctx_reserve: size the workspace for `rows` activation rows."""
        check(lib().glypr_hip_ctx_reserve(self.handle, rows))

    def close(self):
        if self.handle:
            lib().glypr_hip_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check_tensor(self, t: torch.Tensor, name: str, dtype=torch.float32):
        if t.device.type != "cuda" or t.device.index != self.device:
            raise ValueError(f"{name} must be on cuda:{self.device}")
        if t.dtype != dtype:
            raise ValueError(f"{name} must be {dtype}")


class Q8Weight:
    """Opaque Q8_0 weight handle (LinearOp::from_gguf_tensor / try_concat)."""

    def __init__(self, handle, n: int, k: int):
        self.handle = handle
        self.n = n
        self.k = k

    @classmethod
    def from_gguf(cls, ctx: Context, blocks: np.ndarray, n: int, k: int) -> "Q8Weight":
        b = np.ascontiguousarray(blocks, dtype=np.uint8)
        if b.size != n * (k // 32) * 34:
            raise ValueError("blocks size does not match (n, k)")
        h = ctypes.c_void_p()
        check(lib().glypr_hip_q8_0_weight_create(ctx.handle, b.ctypes.data_as(ctypes.c_void_p),
                                                 n, k, ctypes.byref(h)))
        return cls(h, n, k)

    @classmethod
    def concat(cls, ctx: Context, parts: Sequence["Q8Weight"]):
        arr = (ctypes.c_void_p * len(parts))(*[p.handle for p in parts])
        views = (ctypes.c_void_p * len(parts))()
        f = ctypes.c_void_p()
        check(lib().glypr_hip_q8_0_weight_concat(ctx.handle, arr, len(parts), ctypes.byref(f),
                                                 views))
        fused = cls(f, sum(p.n for p in parts), parts[0].k)
        vs = [cls(ctypes.c_void_p(views[i]), parts[i].n, parts[i].k) for i in range(len(parts))]
        return fused, vs

    def view(self, row0: int, rows: int) -> "Q8Weight":
        h = ctypes.c_void_p()
        check(lib().glypr_hip_q8_0_weight_view(self.handle, row0, rows, ctypes.byref(h)))
        return Q8Weight(h, rows, self.k)

    def shape(self):
        n = ctypes.c_int64()
        k = ctypes.c_int64()
        check(lib().glypr_hip_q8_0_weight_shape(self.handle, ctypes.byref(n), ctypes.byref(k)))
        return n.value, k.value

    def close(self):
        if self.handle:
            lib().glypr_hip_q8_0_weight_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BF16Weight:
    """Opaque dense bf16 weight handle (LinearOp over an F16/BF16 tensor)."""

    def __init__(self, handle, n: int, k: int):
        self.handle = handle
        self.n = n
        self.k = k

    @classmethod
    def from_bf16(cls, ctx: Context, rows: np.ndarray) -> "BF16Weight":
        """rows: uint16 [n, k] holding bf16 bit patterns."""
        b = np.ascontiguousarray(rows, dtype=np.uint16)
        if b.ndim != 2:
            raise ValueError("rows must be [n, k]")
        h = ctypes.c_void_p()
        check(lib().glypr_hip_bf16_weight_create(ctx.handle, b.ctypes.data_as(ctypes.c_void_p),
                                                 b.shape[0], b.shape[1], ctypes.byref(h)))
        return cls(h, b.shape[0], b.shape[1])

    def close(self):
        if self.handle:
            lib().glypr_hip_bf16_weight_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 (nearest even) and return the uint16 bit patterns."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_matmul(ctx: Context, w: BF16Weight, x: torch.Tensor,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ctx._check_tensor(x, "x")
    m = x.numel() // w.k
    y = _out(x, (*x.shape[:-1], w.n), out)
    check(lib().glypr_hip_bf16_matmul(ctx.handle, w.handle, _ptr(x), _ptr(y), m, ctx.stream))
    return y


def _out(x: torch.Tensor, shape, out: Optional[torch.Tensor]):
    if out is None:
        return torch.empty(shape, dtype=torch.float32, device=x.device)
    return out


def q8_0_matmul(ctx: Context, w: Q8Weight, x: torch.Tensor, variant: int = INT8_EXACT,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ctx._check_tensor(x, "x")
    m = x.numel() // w.k
    y = _out(x, (*x.shape[:-1], w.n), out)
    check(lib().glypr_hip_q8_0_matmul(ctx.handle, w.handle, _ptr(x), _ptr(y), m, variant,
                                      ctx.stream))
    return y


def q8_0_matmul_noalloc(ctx: Context, w: Q8Weight, x: torch.Tensor, variant: int = INT8_EXACT,
                        out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """glypr_hip_q8_0_matmul_noalloc: the same GEMM with its activation operand
    in the library's fixed per-device scratch array (no device allocation)."""
    ctx._check_tensor(x, "x")
    m = x.numel() // w.k
    y = _out(x, (*x.shape[:-1], w.n), out)
    check(lib().glypr_hip_q8_0_matmul_noalloc(ctx.handle, w.handle, _ptr(x), _ptr(y), m, variant,
                                              ctx.stream))
    return y


def rmsnorm_q8_0_matmul(ctx: Context, w: Q8Weight, x: torch.Tensor,
                        norm_weight: Optional[torch.Tensor], eps: float = 1e-6,
                        variant: int = INT8_EXACT,
                        out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ctx._check_tensor(x, "x")
    m = x.numel() // w.k
    y = _out(x, (*x.shape[:-1], w.n), out)
    check(lib().glypr_hip_rmsnorm_q8_0_matmul(ctx.handle, w.handle, _ptr(x), _ptr(norm_weight),
                                              eps, _ptr(y), m, variant, ctx.stream))
    return y


def rmsnorm(ctx: Context, x: torch.Tensor, weight: Optional[torch.Tensor], eps: float = 1e-6,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ctx._check_tensor(x, "x")
    d = x.shape[-1]
    y = _out(x, x.shape, out)
    check(lib().glypr_hip_rmsnorm(ctx.handle, _ptr(x), _ptr(weight), eps, _ptr(y),
                                  x.numel() // d, d, ctx.stream))
    return y


def geglu(ctx: Context, gate: torch.Tensor, up: torch.Tensor,
          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ctx._check_tensor(gate, "gate")
    ctx._check_tensor(up, "up")
    if gate.shape != up.shape:
        raise ValueError("gate/up shape mismatch")
    y = _out(gate, gate.shape, out)
    check(lib().glypr_hip_geglu(ctx.handle, _ptr(gate), _ptr(up), _ptr(y), gate.numel(),
                                ctx.stream))
    return y


def mlp(ctx: Context, gate_up: Q8Weight, down: Q8Weight, x: torch.Tensor,
        variant: int = INT8_EXACT, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ctx._check_tensor(x, "x")
    m = x.numel() // gate_up.k
    y = _out(x, (*x.shape[:-1], down.n), out)
    check(lib().glypr_hip_mlp(ctx.handle, gate_up.handle, down.handle, _ptr(x), _ptr(y), m,
                              variant, ctx.stream))
    return y


def rmsnorm_mlp(ctx: Context, gate_up: Q8Weight, down: Q8Weight, x: torch.Tensor,
                norm_weight: Optional[torch.Tensor], eps: float = 1e-6,
                variant: int = INT8_EXACT, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ctx._check_tensor(x, "x")
    m = x.numel() // gate_up.k
    y = _out(x, (*x.shape[:-1], down.n), out)
    check(lib().glypr_hip_rmsnorm_mlp(ctx.handle, gate_up.handle, down.handle, _ptr(x),
                                      _ptr(norm_weight), eps, _ptr(y), m, variant, ctx.stream))
    return y


def dequantize(ctx: Context, w: Q8Weight) -> torch.Tensor:
    y = torch.empty((w.n, w.k), dtype=torch.float32, device=f"cuda:{ctx.device}")
    check(lib().glypr_hip_q8_0_dequantize(ctx.handle, w.handle, _ptr(y), ctx.stream))
    return y


def quantize(ctx: Context, x: torch.Tensor) -> torch.Tensor:
    ctx._check_tensor(x, "x")
    k = x.shape[-1]
    m = x.numel() // k
    out = torch.empty((m, k // 32 * 34), dtype=torch.uint8, device=x.device)
    check(lib().glypr_hip_q8_0_quantize(ctx.handle, _ptr(x), m, k, _ptr(out), ctx.stream))
    return out


def embed_gather(ctx: Context, table: Q8Weight, ids, scale: float,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    if out is None:
        out = torch.empty((ids.size, table.k), dtype=torch.float32, device=f"cuda:{ctx.device}")
    check(lib().glypr_hip_q8_0_embed_gather(ctx.handle, table.handle,
                                            ids.ctypes.data_as(ctypes.c_void_p), ids.size,
                                            scale, _ptr(out), ctx.stream))
    return out


def pool_normalize(ctx: Context, tokens: torch.Tensor, mask=None, trunc: int = 0,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ctx._check_tensor(tokens, "tokens")
    t, d = tokens.shape
    td = trunc if 0 < trunc < d else d
    if out is None:
        out = torch.empty(td, dtype=torch.float32, device=tokens.device)
    mk = None
    if mask is not None:
        mk = np.ascontiguousarray(mask, dtype=np.uint8)
    check(lib().glypr_hip_pool_normalize(
        ctx.handle, _ptr(tokens),
        None if mk is None else mk.ctypes.data_as(ctypes.c_void_p), t, d, trunc, _ptr(out),
        ctx.stream))
    return out


# ---- output-vector codecs (glypr-core util.rs:52-197) ----------------------
# Binary codes are u64 words carried in int64 tensors (same bits); hamming
# distances come back as int32 (they never exceed 2^31).

def quantize_binary(ctx: Context, x: torch.Tensor, out: Optional[torch.Tensor] = None
                    ) -> torch.Tensor:
    """quantize_binary (util.rs:52-71) per row: f32 [n, dim] -> words [n, dim/64]."""
    ctx._check_tensor(x, "x")
    n, dim = x.shape
    if out is None:
        out = torch.empty((n, dim // 64), dtype=torch.int64, device=x.device)
    check(lib().glypr_hip_quantize_binary(ctx.handle, _ptr(x), n, dim, _ptr(out), ctx.stream))
    return out


def quantize_int8(ctx: Context, x: torch.Tensor, out: Optional[torch.Tensor] = None
                  ) -> torch.Tensor:
    """quantize_int8 (util.rs:128-133), elementwise."""
    ctx._check_tensor(x, "x")
    if out is None:
        out = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    check(lib().glypr_hip_quantize_int8(ctx.handle, _ptr(x), x.numel(), _ptr(out), ctx.stream))
    return out


def _pairs(ctx: Context, a: torch.Tensor, b: torch.Tensor, dtype, name: str):
    ctx._check_tensor(a, "a", dtype)
    ctx._check_tensor(b, "b", dtype)
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[1]:
        raise ValueError(f"{name}: a [na, d] and b [nb, d] must share d")
    return a.shape[0], b.shape[0], a.shape[1]


def hamming(ctx: Context, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """hamming_distance (util.rs:75-109) for all pairs -> int32 [na, nb]."""
    na, nb, w = _pairs(ctx, a, b, torch.int64, "hamming")
    out = torch.empty((na, nb), dtype=torch.int32, device=a.device)
    check(lib().glypr_hip_hamming(ctx.handle, _ptr(a), na, _ptr(b), nb, w, _ptr(out),
                                  ctx.stream))
    return out


def binary_cosine(ctx: Context, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """binary_cosine_similarity (util.rs:112-119) for all pairs -> f32 [na, nb]."""
    na, nb, w = _pairs(ctx, a, b, torch.int64, "binary_cosine")
    out = torch.empty((na, nb), dtype=torch.float32, device=a.device)
    check(lib().glypr_hip_binary_cosine(ctx.handle, _ptr(a), na, _ptr(b), nb, w, _ptr(out),
                                        ctx.stream))
    return out


def int8_dot(ctx: Context, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """int8_dot_product (util.rs:137-176) for all pairs -> int32 [na, nb]."""
    na, nb, d = _pairs(ctx, a, b, torch.int8, "int8_dot")
    out = torch.empty((na, nb), dtype=torch.int32, device=a.device)
    check(lib().glypr_hip_int8_dot(ctx.handle, _ptr(a), na, _ptr(b), nb, d, _ptr(out),
                                   ctx.stream))
    return out


def int8_cosine(ctx: Context, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """int8_cosine_similarity (util.rs:181-197) for all pairs -> f32 [na, nb]."""
    na, nb, d = _pairs(ctx, a, b, torch.int8, "int8_cosine")
    out = torch.empty((na, nb), dtype=torch.float32, device=a.device)
    check(lib().glypr_hip_int8_cosine(ctx.handle, _ptr(a), na, _ptr(b), nb, d, _ptr(out),
                                      ctx.stream))
    return out


def attention(ctx: Context, qkv: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor,
              eps: float, cos_t: torch.Tensor, sin_t: torch.Tensor, n_heads: int, n_kv_heads: int,
              head_dim: int = 256, window: int = 0,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """SelfAttention core: per-head norms, RoPE, GQA attention -> ctx [t, n_heads*head_dim]."""
    ctx._check_tensor(qkv, "qkv")
    t = qkv.shape[0]
    y = _out(qkv, (t, n_heads * head_dim), out)
    check(lib().glypr_hip_attention(ctx.handle, _ptr(qkv), _ptr(q_norm), _ptr(k_norm), eps,
                                    _ptr(cos_t), _ptr(sin_t), t, n_heads, n_kv_heads, head_dim,
                                    window, _ptr(y), ctx.stream))
    return y


class ModelConfig(ctypes.Structure):
    """glypr_model_config (include/glypr_hip.h)."""
    _fields_ = [("hidden", ctypes.c_int64), ("ffn", ctypes.c_int64), ("n_heads", ctypes.c_int64),
                ("n_kv_heads", ctypes.c_int64), ("head_dim", ctypes.c_int64),
                ("n_layers", ctypes.c_int64), ("vocab", ctypes.c_int64),
                ("sliding_window", ctypes.c_int64), ("eps", ctypes.c_float),
                ("rope_theta_sliding", ctypes.c_double), ("rope_theta_full", ctypes.c_double),
                ("ple_dim", ctypes.c_int64), ("out_dim", ctypes.c_int64),
                ("full_head_dim", ctypes.c_int64), ("full_n_kv_heads", ctypes.c_int64),
                ("max_seq_len", ctypes.c_int64), ("max_batch_tokens", ctypes.c_int64),
                ("layer_types", ctypes.c_void_p)]


class Gguf:
    """A memory-mapped, parsed GGUF v2/v3 file (glypr_gguf_*); host only."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib().glypr_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self.handle = h

    def version(self):
        v, a = ctypes.c_uint32(), ctypes.c_uint32()
        check(lib().glypr_gguf_version(self.handle, ctypes.byref(v), ctypes.byref(a)))
        return v.value, a.value

    def tensors(self):
        """[{name, type, dims (ne order), nbytes, data (address or None)}]"""
        n = ctypes.c_int64()
        check(lib().glypr_gguf_tensor_count(self.handle, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            name, typ, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
            ne = (ctypes.c_int64 * 4)()
            data, nb = ctypes.c_void_p(), ctypes.c_int64()
            check(lib().glypr_gguf_tensor_info(self.handle, i, ctypes.byref(name),
                                               ctypes.byref(typ), ctypes.byref(nd), ne,
                                               ctypes.byref(data), ctypes.byref(nb)))
            out.append({"name": name.value.decode(), "type": typ.value,
                        "dims": tuple(ne[:nd.value]), "nbytes": nb.value, "data": data.value})
        return out

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A copy of the tensor's bytes as stored in the file."""
        idx = ctypes.c_int64()
        check(lib().glypr_gguf_find_tensor(self.handle, name.encode(), ctypes.byref(idx)))
        t = self.tensors()[idx.value]
        if t["data"] is None:
            raise GlyprError(GLYPR_ERR_UNSUPPORTED, f"tensor {name!r} has an unsized ggml type")
        return np.ctypeslib.as_array((ctypes.c_uint8 * t["nbytes"]).from_address(t["data"])).copy()

    def u64(self, key: str) -> int:
        v = ctypes.c_uint64()
        check(lib().glypr_gguf_get_u64(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def f64(self, key: str) -> float:
        v = ctypes.c_double()
        check(lib().glypr_gguf_get_f64(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def str(self, key: str) -> str:
        v = ctypes.c_char_p()
        check(lib().glypr_gguf_get_str(self.handle, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    def array_u64(self, key: str):
        et, n = ctypes.c_int(), ctypes.c_int64()
        check(lib().glypr_gguf_get_array(self.handle, key.encode(), ctypes.byref(et),
                                         ctypes.byref(n)))
        out = []
        for i in range(n.value):
            v = ctypes.c_uint64()
            check(lib().glypr_gguf_get_array_u64(self.handle, key.encode(), i, ctypes.byref(v)))
            out.append(v.value)
        return out

    def close(self):
        if self.handle:
            lib().glypr_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """The text backbone (glypr_hip_model_*): tensors by their GGUF names."""

    @classmethod
    def from_gguf(cls, ctx: Context, path: str) -> "Model":
        """glypr_hip_model_load_gguf: config and tensors from a GGUF file."""
        with Gguf(path) as g:
            hidden = g.u64("gemma-embedding2.embedding_length")
            dims = {t["name"]: t["dims"] for t in g.tensors()}
        m = cls.__new__(cls)
        m.ctx = ctx
        out = dims.get("output.weight")
        m.cfg = {"hidden": hidden, "out_dim": out[1] if out else 0}
        h = ctypes.c_void_p()
        m.handle = None
        check(lib().glypr_hip_model_load_gguf(ctx.handle, os.fsencode(path), ctypes.byref(h)))
        m.handle = h
        return m

    def __init__(self, ctx: Context, layer_types=None, **cfg):
        """layer_types: n_layers values, nonzero = a full-attention layer
        (sliding_window_pattern, config.rs:117-140); None = the default
        5 sliding + 1 full pattern."""
        defaults = dict(hidden=768, ffn=1152, n_heads=3, n_kv_heads=1, head_dim=256, n_layers=24,
                        vocab=262144, sliding_window=512, eps=1e-6, rope_theta_sliding=10000.0,
                        rope_theta_full=1e6, ple_dim=0, out_dim=0, full_head_dim=0,
                        full_n_kv_heads=0, max_seq_len=0, max_batch_tokens=0)
        defaults.update(cfg)
        self.cfg = defaults
        self.ctx = ctx
        c = ModelConfig(**defaults)
        if layer_types is not None:
            lt = np.ascontiguousarray(np.asarray(layer_types) != 0, dtype=np.uint8)
            if lt.size != defaults["n_layers"]:
                raise ValueError("layer_types needs one entry per layer")
            c.layer_types = lt.ctypes.data   # read by glypr_hip_model_create only
        h = ctypes.c_void_p()
        check(lib().glypr_hip_model_create(ctx.handle, ctypes.byref(c), ctypes.byref(h)))
        self.handle = h

    def set_tensor(self, name: str, data: np.ndarray, rows: int, cols: int, q8_0: bool):
        """q8_0: data holds GGUF Q8_0 blocks; otherwise f32 values, or, for a
        layer projection given as a uint16 array, dense bf16 bit patterns."""
        a = np.ascontiguousarray(data)
        dtype = 1 if q8_0 else (2 if a.dtype == np.uint16 else 0)
        if dtype == 0:
            a = np.ascontiguousarray(a, dtype=np.float32)
        check(lib().glypr_hip_model_set_tensor(self.handle, name.encode(),
                                               a.ctypes.data_as(ctypes.c_void_p), rows, cols,
                                               dtype))

    def finalize(self):
        check(lib().glypr_hip_model_finalize(self.handle))

    def set_variant(self, variant: int):
        """glypr_hip_model_set_variant: INT8_EXACT (default) or INT8_FMA for
        every Q8_0 projection of the later embed calls."""
        check(lib().glypr_hip_model_set_variant(self.handle, variant))

    def embed(self, ids, trunc: int = 0, hidden: Optional[torch.Tensor] = None,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        H = self.cfg.get("out_dim") or self.cfg["hidden"]   # embedding width
        td = trunc if 0 < trunc < H else H
        if out is None:
            out = torch.empty(td, dtype=torch.float32, device=f"cuda:{self.ctx.device}")
        check(lib().glypr_hip_model_embed(self.handle, ids.ctypes.data_as(ctypes.c_void_p),
                                          ids.size, trunc, _ptr(out), _ptr(hidden),
                                          self.ctx.stream))
        return out

    def embed_batch(self, seqs, trunc: int = 0, out: Optional[torch.Tensor] = None):
        """glypr_hip_model_embed_batch: a list of id arrays -> [n, width]."""
        lens = np.array([len(q) for q in seqs], dtype=np.int64)
        ids = np.ascontiguousarray(np.concatenate([np.asarray(q, np.uint32) for q in seqs]),
                                   dtype=np.uint32)
        H = self.cfg.get("out_dim") or self.cfg["hidden"]
        td = trunc if 0 < trunc < H else H
        if out is None:
            out = torch.empty((len(seqs), td), dtype=torch.float32,
                              device=f"cuda:{self.ctx.device}")
        check(lib().glypr_hip_model_embed_batch(self.handle, ids.ctypes.data_as(ctypes.c_void_p),
                                                lens.ctypes.data_as(ctypes.c_void_p), len(seqs),
                                                trunc, _ptr(out), self.ctx.stream))
        return out

    def close(self):
        if self.handle:
            lib().glypr_hip_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
