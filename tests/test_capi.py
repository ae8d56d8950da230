"""C ABI checks that need no GPU: the library loads, exports every symbol that
include/glypr_hip.h declares, and rejects bad arguments before touching a
device (the reference's bail! paths: linear.rs:46, cpu_simd/rmsnorm.rs:72,
cpu_simd/geglu.rs:35-57, metal_kernels/mod.rs:1294-1300)."""
import ctypes
import os
import re

import pytest

from glypr_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "glypr_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(glypr_(?:hip|gguf)_\w+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name
    assert L.glypr_hip_abi_version() == 8


def _has_gpu():
    try:
        import torch
        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device error path")
def test_ctx_create_without_device_fails_cleanly():
    L = _lib.lib()
    h = ctypes.c_void_p()
    rc = L.glypr_hip_ctx_create(0, ctypes.byref(h))
    assert rc == _lib.GLYPR_ERR_DEVICE
    assert h.value is None
    assert "device" in _lib.last_error()


FAKE = ctypes.c_void_p(0x1000)       # never dereferenced: validation fails first
MISALIGNED = ctypes.c_void_p(0x1004)
NULL = None


def test_weight_create_validation():
    L = _lib.lib()
    out = ctypes.c_void_p()
    blocks = (ctypes.c_uint8 * 34)()
    assert L.glypr_hip_q8_0_weight_create(NULL, blocks, 1, 33, ctypes.byref(out)) == \
        _lib.GLYPR_ERR_SHAPE
    assert "multiple of 32" in _lib.last_error()
    assert L.glypr_hip_q8_0_weight_create(NULL, blocks, 0, 32, ctypes.byref(out)) == \
        _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_q8_0_weight_create(NULL, NULL, 1, 32, ctypes.byref(out)) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_q8_0_weight_create(NULL, blocks, 1, 32, ctypes.byref(out)) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert "ctx" in _lib.last_error()


def test_matmul_validation_order():
    L = _lib.lib()
    assert L.glypr_hip_q8_0_matmul(NULL, NULL, NULL, NULL, -1, 0, NULL) == _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_q8_0_matmul(NULL, NULL, NULL, NULL, 4, 7, NULL) == \
        _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_q8_0_matmul(NULL, NULL, FAKE, FAKE, 4, 0, NULL) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_q8_0_matmul(NULL, FAKE, MISALIGNED, FAKE, 4, 0, NULL) == \
        _lib.GLYPR_ERR_ALIGNMENT
    assert L.glypr_hip_q8_0_matmul(NULL, FAKE, FAKE, FAKE, 4, 0, NULL) == \
        _lib.GLYPR_ERR_INVALID_ARG   # ctx NULL
    assert L.glypr_hip_rmsnorm_q8_0_matmul(NULL, FAKE, FAKE, MISALIGNED, 1e-6, FAKE, 4, 0,
                                           NULL) == _lib.GLYPR_ERR_ALIGNMENT
    assert L.glypr_hip_mlp(NULL, FAKE, FAKE, FAKE, FAKE, 4, 9, NULL) == \
        _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_mlp(NULL, NULL, FAKE, FAKE, FAKE, 4, 0, NULL) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_rmsnorm_mlp(NULL, FAKE, FAKE, MISALIGNED, NULL, 1e-6, FAKE, 4, 1,
                                   NULL) == _lib.GLYPR_ERR_ALIGNMENT
    # the three variants pass the variant check (and fail later, on the NULL
    # weight); the next value does not
    for v in (_lib.INT8_EXACT, _lib.BF16_DEQUANT, _lib.INT8_FMA):
        assert L.glypr_hip_q8_0_matmul(NULL, NULL, FAKE, FAKE, 4, v, NULL) == \
            _lib.GLYPR_ERR_INVALID_ARG
        assert L.glypr_hip_mlp(NULL, NULL, FAKE, FAKE, FAKE, 4, v, NULL) == \
            _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_q8_0_matmul(NULL, NULL, FAKE, FAKE, 4, 3, NULL) == \
        _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_mlp(NULL, FAKE, FAKE, FAKE, FAKE, 4, 3, NULL) == \
        _lib.GLYPR_ERR_UNSUPPORTED


def test_noalloc_matmul_validation():
    """glypr_hip_q8_0_matmul_noalloc validates like glypr_hip_q8_0_matmul (its
    scratch-size check needs the weight handle, so it runs on the GPU)."""
    L = _lib.lib()
    assert L.glypr_hip_q8_0_matmul_noalloc(NULL, NULL, NULL, NULL, -1, 0, NULL) == \
        _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_q8_0_matmul_noalloc(NULL, NULL, NULL, NULL, 4, 7, NULL) == \
        _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_q8_0_matmul_noalloc(NULL, NULL, FAKE, FAKE, 4, 0, NULL) == \
        _lib.GLYPR_ERR_INVALID_ARG


def test_elementwise_validation():
    L = _lib.lib()
    assert L.glypr_hip_rmsnorm(NULL, FAKE, NULL, 1e-6, FAKE, -1, 768, NULL) == \
        _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_rmsnorm(NULL, NULL, NULL, 1e-6, FAKE, 4, 768, NULL) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_geglu(NULL, FAKE, NULL, FAKE, 16, NULL) == _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_q8_0_quantize(NULL, FAKE, 4, 48, FAKE, NULL) == _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_q8_0_quantize(NULL, MISALIGNED, 4, 64, FAKE, NULL) == \
        _lib.GLYPR_ERR_ALIGNMENT
    assert L.glypr_hip_pool_normalize(NULL, FAKE, NULL, 0, 768, 256, FAKE, NULL) == \
        _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_q8_0_embed_gather(NULL, NULL, FAKE, 4, 1.0, FAKE, NULL) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_q8_0_embed_gather(NULL, FAKE, FAKE, -1, 1.0, FAKE, NULL) == \
        _lib.GLYPR_ERR_SHAPE


def test_vector_codec_validation():
    """quantize_binary bails on dims that are not a multiple of 64
    (util.rs:53-59, tests/quantization.rs:12-14); the all-pairs searches reject
    negative sizes, NULL and misaligned buffers, and int8 dims whose i32 sums
    could wrap, all before touching a device."""
    L = _lib.lib()
    for dim in (63, 65):
        assert L.glypr_hip_quantize_binary(NULL, FAKE, 1, dim, FAKE, NULL) == \
            _lib.GLYPR_ERR_SHAPE
        assert "multiple of 64" in _lib.last_error()
    assert L.glypr_hip_quantize_binary(NULL, FAKE, 1, 128, FAKE, NULL) == \
        _lib.GLYPR_ERR_INVALID_ARG   # shape accepted; ctx NULL
    assert L.glypr_hip_quantize_binary(NULL, MISALIGNED, 1, 128, FAKE, NULL) == \
        _lib.GLYPR_ERR_ALIGNMENT
    assert L.glypr_hip_quantize_int8(NULL, FAKE, -1, FAKE, NULL) == _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_quantize_int8(NULL, NULL, 4, FAKE, NULL) == _lib.GLYPR_ERR_INVALID_ARG
    for fn in (L.glypr_hip_hamming, L.glypr_hip_binary_cosine, L.glypr_hip_int8_dot,
               L.glypr_hip_int8_cosine):
        assert fn(NULL, FAKE, -1, FAKE, 1, 4, FAKE, NULL) == _lib.GLYPR_ERR_SHAPE
        assert fn(NULL, FAKE, 1, NULL, 1, 4, FAKE, NULL) == _lib.GLYPR_ERR_INVALID_ARG
        assert fn(NULL, FAKE, 1, FAKE, 1, 4, MISALIGNED, NULL) == _lib.GLYPR_ERR_ALIGNMENT
        assert fn(NULL, FAKE, 1, FAKE, 1, 4, FAKE, NULL) == _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_int8_dot(NULL, FAKE, 1, FAKE, 1, 65537, FAKE, NULL) == \
        _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_int8_cosine(NULL, FAKE, 1, FAKE, 1, 65537, FAKE, NULL) == \
        _lib.GLYPR_ERR_SHAPE


def test_embed_batch_validation():
    L = _lib.lib()
    lens = (ctypes.c_int64 * 2)(3, 4)
    assert L.glypr_hip_model_embed_batch(NULL, FAKE, lens, 2, 256, FAKE, NULL) == \
        _lib.GLYPR_ERR_INVALID_ARG


def test_handle_lifecycle_validation():
    L = _lib.lib()
    assert L.glypr_hip_q8_0_weight_destroy(NULL) == _lib.GLYPR_OK
    assert L.glypr_hip_ctx_destroy(NULL) == _lib.GLYPR_OK
    out = ctypes.c_void_p()
    parts = (ctypes.c_void_p * 1)(FAKE.value)
    assert L.glypr_hip_q8_0_weight_concat(NULL, parts, 1, ctypes.byref(out), NULL) == \
        _lib.GLYPR_ERR_SHAPE   # try_concat needs >= 2 parts (linear.rs:83-85)
    assert L.glypr_hip_q8_0_weight_view(NULL, 0, 1, ctypes.byref(out)) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_q8_0_weight_shape(NULL, NULL, NULL) == _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_sync(NULL, NULL) == _lib.GLYPR_ERR_INVALID_ARG


def test_product_has_no_oracle_dependency():
    """The product library must not link or load the oracle."""
    import subprocess
    out = subprocess.run(["ldd", _lib.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle" not in out
    for root, _, files in os.walk(os.path.join(ROOT, "glypr_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".hpp", ".h")):
                text = open(os.path.join(root, f)).read()
                assert "pyoracle" not in text and "liboracle" not in text, f


def test_reserve_validation():
    L = _lib.lib()
    assert L.glypr_hip_ctx_reserve(NULL, 0) == _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_ctx_reserve(NULL, -5) == _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_ctx_reserve(NULL, 8320) == _lib.GLYPR_ERR_INVALID_ARG   # ctx NULL


def _cfg(**kw):
    from glypr_amd.ops import ModelConfig
    base = dict(hidden=768, ffn=1152, n_heads=3, n_kv_heads=1, head_dim=256, n_layers=24,
                vocab=262144, sliding_window=512, eps=1e-6, rope_theta_sliding=1e4,
                rope_theta_full=1e6, ple_dim=0, out_dim=0, full_head_dim=0, full_n_kv_heads=0,
                max_seq_len=0)
    base.update(kw)
    return ModelConfig(**base)


def test_attention_geometry_validation():
    """Geometries the attention kernels do not run are refused before anything
    is launched or allocated: more than 4 q heads per kv head, or head dims
    other than 256."""
    L = _lib.lib()
    out = ctypes.c_void_p()
    # the BASELINE geometry passes validation (then fails on the NULL ctx)
    assert L.glypr_hip_model_create(NULL, ctypes.byref(_cfg()), ctypes.byref(out)) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_model_create(NULL, ctypes.byref(_cfg(n_heads=5, n_kv_heads=1)),
                                    ctypes.byref(out)) == _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_model_create(NULL, ctypes.byref(_cfg(n_heads=4, full_n_kv_heads=3)),
                                    ctypes.byref(out)) == _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_model_create(NULL, ctypes.byref(_cfg(head_dim=128)),
                                    ctypes.byref(out)) == _lib.GLYPR_ERR_UNSUPPORTED
    # the released geometry: full layers with head_dim 512 and one kv head pass
    real = _cfg(hidden=512, ffn=2048, n_heads=4, n_kv_heads=2, full_head_dim=512,
                full_n_kv_heads=1)
    assert L.glypr_hip_model_create(NULL, ctypes.byref(real), ctypes.byref(out)) == \
        _lib.GLYPR_ERR_INVALID_ARG
    assert L.glypr_hip_model_create(NULL, ctypes.byref(_cfg(full_head_dim=384)),
                                    ctypes.byref(out)) == _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_model_create(NULL, ctypes.byref(_cfg(max_seq_len=-1)),
                                    ctypes.byref(out)) == _lib.GLYPR_ERR_SHAPE
    # row capacities at which the attention kernels' 32-bit per-lane byte
    # offsets (2 head_dim padded_rows) would reach 2^31 are refused: 2^22 rows
    # of head_dim 256, 2^21 of 512 (the released full layers), as batch
    # capacity or as sequence length; a batch capacity one 64-row step below
    # passes validation
    for cap, geometry in (((1 << 22), _cfg()), ((1 << 21), real)):
        for field in ("max_batch_tokens", "max_seq_len"):
            setattr(geometry, field, cap)
            assert L.glypr_hip_model_create(NULL, ctypes.byref(geometry),
                                            ctypes.byref(out)) == _lib.GLYPR_ERR_SHAPE
            assert "2^31" in _lib.last_error()
            setattr(geometry, field, 0)
        geometry.max_batch_tokens = cap - 64
        assert L.glypr_hip_model_create(NULL, ctypes.byref(geometry),
                                        ctypes.byref(out)) == _lib.GLYPR_ERR_INVALID_ARG
        geometry.max_batch_tokens = 0
    # glypr_hip_attention: the same geometry rule, checked before the pointers
    args = lambda nq, nkv, hd: (NULL, FAKE, FAKE, FAKE, 1e-6, FAKE, FAKE, 512, nq, nkv, hd, 0,
                                FAKE, NULL)
    assert L.glypr_hip_attention(*args(5, 1, 256)) == _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_attention(*args(3, 1, 128)) == _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_attention(*args(3, 2, 256)) == _lib.GLYPR_ERR_SHAPE
    assert L.glypr_hip_attention(*args(4, 1, 256)) == _lib.GLYPR_ERR_INVALID_ARG   # ctx NULL
    assert L.glypr_hip_attention(*args(4, 1, 512)) == _lib.GLYPR_ERR_INVALID_ARG
    big = lambda t, hd: (NULL, FAKE, FAKE, FAKE, 1e-6, FAKE, FAKE, t, 3, 1, hd, 0, FAKE, NULL)
    assert L.glypr_hip_attention(*big(1 << 22, 256)) == _lib.GLYPR_ERR_UNSUPPORTED
    assert L.glypr_hip_attention(*big(1 << 21, 512)) == _lib.GLYPR_ERR_UNSUPPORTED


def test_gemm_routing():
    """The INT8_EXACT GEMM routes (k_gemm_i8.hip): the LDS-ring small-M kernel
    and the 128 x 128 large-M kernel address operands with 32-bit offsets, so a
    weight of 2^31 or more bytes (N * K) takes the int64-offset kernel."""
    L = _lib.lib()
    route = L.glypr_internal_gemm_i8_route
    route.restype = ctypes.c_int
    route.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
    SMALL, BIG, REG128, REG64, PRO = 0, 1, 2, 3, 4
    assert route(512, 1280, 768, 0) == SMALL           # C2 qkv
    assert route(512, 2304, 768, 0) == SMALL           # C2 gate|up
    assert route(2048, 768, 1152, 0) == SMALL
    assert route(2049, 768, 1152, 0) == BIG
    assert route(16384, 1280, 768, 0) == BIG           # C3
    big_n = (1 << 31) // 1024                          # N * K = 2^31
    assert route(512, big_n, 1024, 0) == REG128
    assert route(512, big_n - 1, 1024, 0) == SMALL
    assert route(4096, big_n, 1024, 0) == REG128
    assert route(4096, big_n - 1, 1024, 0) == BIG
    assert route(64, 64, 1024, 0) == SMALL
    assert route(4096, 64, 96, 0) in (REG128, REG64)   # K % 128 != 0
    # the released EmbeddingGemma-2 widths: K = 2048 (down, full-layer o) stays small-M
    assert route(512, 512, 2048, 0) == SMALL and route(512, 512, 1536, 0) == SMALL
    assert route(512, 512, 1280, 0) == BIG               # no 40-block small instantiation
    assert route(512, 512, 2048, 1) == -1                 # the fused prologue stops at 1152
    # the fused prologue: quantize up to M = 1024, RMSNorm up to M = 256
    assert route(1024, 768, 768, 1) == PRO and route(1025, 768, 768, 1) == -1
    assert route(256, 1280, 768, 2) == PRO and route(257, 1280, 768, 2) == -1
    assert route(256, big_n, 1024, 2) == -1


# ---- the model-config struct: C header, ctypes mirror and the Rust binding ----

_C_FIELDS = re.compile(r"^\s*(int64_t|float|double|const uint8_t\*)\s+(\w+);", re.M)


def _header_struct_fields():
    text = open(HEADER).read()
    body = text[text.index("typedef struct glypr_model_config {"):]
    body = body[:body.index("} glypr_model_config;")]
    return [(t, n) for t, n in _C_FIELDS.findall(body)]


def test_model_config_layout_probe():
    """sizeof / offsetof of glypr_model_config compiled by the C compiler
    against include/glypr_hip.h equal the ctypes mirror (ops.ModelConfig)."""
    import subprocess
    import tempfile
    from glypr_amd.ops import ModelConfig
    fields = _header_struct_fields()
    assert [n for _, n in fields] == [f[0] for f in ModelConfig._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", '#include "glypr_hip.h"',
           "int main(void) {", 'printf("size %zu\\n", sizeof(glypr_model_config));']
    for _, n in fields:
        src.append(f'printf("{n} %zu %zu\\n", offsetof(glypr_model_config, {n}), '
                   f'sizeof(((glypr_model_config*)0)->{n}));')
    src.append("return 0; }")
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "probe.c")
        open(c, "w").write("\n".join(src))
        exe = os.path.join(d, "probe")
        subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), c,
                        "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    got = dict((l.split()[0], tuple(int(v) for v in l.split()[1:])) for l in out if l)
    assert got["size"] == (ctypes.sizeof(ModelConfig),)
    for name, ctype in ModelConfig._fields_:
        assert got[name] == (getattr(ModelConfig, name).offset, ctypes.sizeof(ctype)), name


def test_integration_rust_struct_matches_header():
    """The Rust #[repr(C)] glypr_model_config in INTEGRATION.md lists the C
    struct's fields in order with matching types, so a Rust caller's struct is
    exactly as large as the one glypr_hip_model_create reads."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    body = text[text.index("pub struct glypr_model_config {"):]
    body = body[len("pub struct glypr_model_config {"):body.index("}")]
    rust = [(n, " ".join(t.split())) for n, t in
            re.findall(r"pub\s+(\w+)\s*:\s*(\*const\s+\w+|\w+)", body)]
    rmap = {"int64_t": "i64", "float": "f32", "double": "f64", "const uint8_t*": "*const u8"}
    assert [(n, t) for n, t in rust] == [(n, rmap[t]) for t, n in _header_struct_fields()]
