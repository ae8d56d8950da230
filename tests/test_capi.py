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
    assert L.glypr_hip_abi_version() == 4


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
