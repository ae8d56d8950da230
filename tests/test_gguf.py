"""GGUF v3 reader (glypr_gguf_*): parsing, metadata and tensor access, and the
error paths of corrupt files.  Host only, so these run without a GPU.  The
files are written by tests/gguf_util.py from the published GGUF layout."""
import struct

import numpy as np
import pytest

from glypr_amd import _lib
from glypr_amd._lib import GlyprError
from glypr_amd.ops import Gguf

import gguf_util as gu


def _sample(tmp_path, alignment=None):
    rng = np.random.default_rng(3)
    q8 = rng.integers(0, 256, size=(5, 2 * 34), dtype=np.uint8)    # 5 rows of 64 Q8_0 values
    f32 = rng.standard_normal(7).astype(np.float32)
    f16 = rng.standard_normal((3, 4)).astype(np.float16)
    meta = [("general.architecture", gu.STR, "gemma-embedding2"),
            ("a.u32", gu.U32, 4000000000), ("a.i32", gu.I32, 17), ("a.neg", gu.I32, -5),
            ("a.u64", gu.U64, 1 << 40), ("a.f32", gu.F32, 1.5), ("a.f64", gu.F64, 1e-6),
            ("a.bool", gu.BOOL, True), ("a.arr", gu.ARR, (gu.U32, [3, 1, 4, 1, 5])),
            ("a.strs", gu.ARR, (gu.STR, ["x", "yz"]))]
    if alignment:
        meta.append(("general.alignment", gu.U32, alignment))
    tensors = [("w.q8", gu.GGML_Q8_0, (64, 5), q8.tobytes()),
               ("n.f32", gu.GGML_F32, (7,), f32.tobytes()),
               ("h.f16", gu.GGML_F16, (4, 3), f16.tobytes())]
    p = tmp_path / "m.gguf"
    raw = gu.write_gguf(p, meta, tensors, alignment=alignment or 32)
    return p, raw, q8, f32, f16


@pytest.mark.parametrize("alignment", [None, 64])
def test_parse_metadata_and_tensors(tmp_path, alignment):
    p, raw, q8, f32, f16 = _sample(tmp_path, alignment)
    with Gguf(str(p)) as g:
        assert g.version() == (3, alignment or 32)
        t = {x["name"]: x for x in g.tensors()}
        assert [x["name"] for x in g.tensors()] == ["w.q8", "n.f32", "h.f16"]
        assert t["w.q8"]["type"] == 8 and t["w.q8"]["dims"] == (64, 5) and t["w.q8"]["nbytes"] == 340
        assert t["n.f32"]["dims"] == (7,) and t["n.f32"]["nbytes"] == 28
        assert t["h.f16"]["type"] == 1 and t["h.f16"]["nbytes"] == 24
        assert np.array_equal(g.tensor_bytes("w.q8"), q8.reshape(-1))
        assert np.array_equal(g.tensor_bytes("n.f32").view(np.float32), f32)
        assert np.array_equal(g.tensor_bytes("h.f16").view(np.float16), f16.reshape(-1))
        assert g.u64("a.u32") == 4000000000 and g.u64("a.i32") == 17 and g.u64("a.u64") == 1 << 40
        assert g.u64("a.bool") == 1
        assert g.f64("a.f32") == 1.5 and g.f64("a.f64") == 1e-6 and g.f64("a.i32") == 17.0
        assert g.str("general.architecture") == "gemma-embedding2"
        assert g.array_u64("a.arr") == [3, 1, 4, 1, 5]
        with pytest.raises(GlyprError) as e:
            g.u64("a.missing")
        assert e.value.code == _lib.GLYPR_ERR_NOT_FOUND
        with pytest.raises(GlyprError) as e:
            g.u64("a.neg")
        assert e.value.code == _lib.GLYPR_ERR_UNSUPPORTED
        with pytest.raises(GlyprError) as e:
            g.str("a.u32")
        assert e.value.code == _lib.GLYPR_ERR_UNSUPPORTED
        with pytest.raises(GlyprError) as e:
            g.tensor_bytes("nope")
        assert e.value.code == _lib.GLYPR_ERR_NOT_FOUND


def test_data_offsets_follow_alignment(tmp_path):
    p, raw, q8, f32, f16 = _sample(tmp_path, 64)
    with Gguf(str(p)) as g:
        base = min(x["data"] for x in g.tensors())
        for x in g.tensors():
            assert (x["data"] - base) % 64 == 0
        # the data section starts at an aligned file offset: the first tensor's bytes
        first = g.tensor_bytes("w.q8").tobytes()
        assert raw.index(first) % 64 == 0


def test_corrupt_files_fail_cleanly(tmp_path):
    p, raw, *_ = _sample(tmp_path)
    cases = {
        "bad magic": b"GGUX" + raw[4:],
        "version 1": raw[:4] + struct.pack("<I", 1) + raw[8:],
        "header only": raw[:24],
        "cut in metadata": raw[:60],
        "cut in tensor table": raw[:raw.index(b"h.f16") + 3],
        "cut in data": raw[:-10],
        "huge tensor count": raw[:8] + struct.pack("<Q", 1 << 40) + raw[16:],
    }
    expect = {"version 1": _lib.GLYPR_ERR_UNSUPPORTED}
    for name, blob in cases.items():
        q = tmp_path / "bad.gguf"
        q.write_bytes(blob)
        with pytest.raises(GlyprError) as e:
            Gguf(str(q))
        assert e.value.code == expect.get(name, _lib.GLYPR_ERR_SHAPE), name
    with pytest.raises(GlyprError) as e:
        Gguf(str(tmp_path / "absent.gguf"))
    assert e.value.code == _lib.GLYPR_ERR_INVALID_ARG


def test_misaligned_tensor_offset_rejected(tmp_path):
    p, raw, *_ = _sample(tmp_path)
    # the second tensor's offset field follows its type: move it off the grid
    i = raw.index(b"n.f32") + len(b"n.f32")
    i += 4 + 8 + 4          # n_dims, ne[0], type
    off = struct.unpack_from("<Q", raw, i)[0]
    bad = raw[:i] + struct.pack("<Q", off + 4) + raw[i + 8:]
    q = tmp_path / "mis.gguf"
    q.write_bytes(bad)
    with pytest.raises(GlyprError) as e:
        Gguf(str(q))
    assert e.value.code == _lib.GLYPR_ERR_SHAPE


def test_model_load_needs_a_context(tmp_path):
    p, *_ = _sample(tmp_path)
    import ctypes
    h = ctypes.c_void_p()
    rc = _lib.lib().glypr_hip_model_load_gguf(None, str(p).encode(), ctypes.byref(h))
    assert rc != _lib.GLYPR_OK and not h.value
