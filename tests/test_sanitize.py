"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

The GGUF parser (gguf.cpp), the model driver (model.cpp) and the C ABI
(capi.hip) are compiled for the host only, with both sanitizers and no error
recovery, and linked with tests/sanitize/driver.cpp.  The driver then parses
valid, truncated and corrupt GGUF files (every prefix of a valid file, flipped
header bytes, overflowing dimensions, oversized arrays and strings) and calls
each entry point with invalid arguments.  Any out-of-bounds access, leak,
overflow or other undefined behaviour fails the test.  No GPU is touched: the
kernel launchers come from the built library and are never reached.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

import gguf_util as gu

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "glypr_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
# host-only objects; each sanitizer flag goes to the host pass
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all"]
HOST_SOURCES = ["capi.hip", "model.cpp", "gguf.cpp"]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    from glypr_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libglypr_hip.so is not built (python -m glypr_amd.build)")
    d = tmp_path_factory.mktemp("san")
    objs = []
    common = ["-x", "hip", "--cuda-host-only", "-std=c++17", "-O1", "-g",
              "-fno-omit-frame-pointer", *SAN, f"-I{ROOT}/include", f"-I{CSRC}"]
    procs = []
    for src in HOST_SOURCES + [os.path.join(HERE, "sanitize", "driver.cpp")]:
        path = src if os.path.isabs(src) else os.path.join(CSRC, src)
        obj = str(d / (os.path.basename(path) + ".o"))
        objs.append(obj)
        procs.append(subprocess.Popen([HIPCC, *common, "-c", path, "-o", obj],
                                      stdout=subprocess.PIPE, stderr=subprocess.STDOUT))
    for p in procs:
        out = p.communicate()[0].decode()
        assert p.returncode == 0, out
    exe = str(d / "driver")
    r = subprocess.run([HIPCC, "--cuda-host-only", *SAN, *objs, f"-L{os.path.dirname(_lib.LIB_PATH)}",
                        "-lglypr_hip", f"-Wl,-rpath,{os.path.dirname(_lib.LIB_PATH)}", "-o", exe],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return exe


def _run(exe, args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe, *args], capture_output=True, text=True, errors="replace", env=env,
                       timeout=300)
    report = r.stdout + r.stderr
    assert "AddressSanitizer" not in report and "runtime error" not in report and \
        "LeakSanitizer" not in report, report[-4000:]
    assert r.returncode == 0, report[-4000:]
    return r.stdout


def _valid(path):
    rng = np.random.default_rng(9)
    q8 = rng.integers(0, 256, size=(5, 2 * 34), dtype=np.uint8)
    meta = [("general.architecture", gu.STR, "gemma-embedding2"), ("a.u32", gu.U32, 7),
            ("a.i32", gu.I32, -3), ("a.f64", gu.F64, 0.5), ("a.bool", gu.BOOL, True),
            ("a.arr", gu.ARR, (gu.U32, [3, 1, 4])), ("a.strs", gu.ARR, (gu.STR, ["x", "yz"])),
            ("gemma-embedding2.attention.head_count_kv", gu.ARR, (gu.I32, [2, 2, -1]))]
    tensors = [("w.q8", gu.GGML_Q8_0, (64, 5), q8.tobytes()),
               ("n.f32", gu.GGML_F32, (7,), rng.standard_normal(7).astype(np.float32).tobytes())]
    return gu.write_gguf(path, meta, tensors)


def test_validation_paths_under_sanitizers(driver):
    out = _run(driver, ["--validate"])
    assert "validation failures 0" in out


def test_gguf_parser_under_sanitizers(driver, tmp_path):
    raw = _valid(tmp_path / "ok.gguf")
    files = [str(tmp_path / "ok.gguf")]
    # every prefix of the valid file
    for n in range(len(raw)):
        p = tmp_path / f"cut{n}.gguf"
        p.write_bytes(raw[:n])
        files.append(str(p))
    # single-byte corruptions over the header, metadata and tensor table
    data_start = raw.index(b"w.q8") + 60
    rng = np.random.default_rng(1)
    for i in range(0, data_start, 3):
        b = bytearray(raw)
        b[i] ^= int(rng.integers(1, 256))
        p = tmp_path / f"flip{i}.gguf"
        p.write_bytes(bytes(b))
        files.append(str(p))
    # an overflowing element count: four dims of 2^39 each
    big = gu.write_gguf(tmp_path / "tmp.gguf", [], [("t", gu.GGML_F32, (1, 1, 1, 1), b"\0" * 4)])
    i = big.index(b"t") + 1 + 4
    dims = struct.pack("<4Q", *([1 << 39] * 4))
    (tmp_path / "ovf.gguf").write_bytes(big[:i] + dims + big[i + 32:])
    files.append(str(tmp_path / "ovf.gguf"))
    # arrays and strings whose counts exceed the file
    hdr = b"GGUF" + struct.pack("<IQQ", 3, 0, 1)
    key = struct.pack("<Q", 5) + b"a.big"
    for body in (struct.pack("<IIQ", 9, 4, 1 << 62),               # u32 array, 2^62 elements
                 struct.pack("<IIQ", 9, 8, 1 << 40) + b"\0" * 64,  # string array
                 struct.pack("<IQ", 8, 1 << 60) + b"xyz",          # string
                 struct.pack("<II", 9, 9) + struct.pack("<Q", 1) + struct.pack("<IQ", 4, 1)):
        p = tmp_path / f"arr{len(files)}.gguf"
        p.write_bytes(hdr + key + body + b"\0" * 32)
        files.append(str(p))
    out = _run(driver, files)
    lines = [l for l in out.splitlines() if l.startswith("open ")]
    assert len(lines) == len(files)
    assert lines[0].endswith("-> 0 "), lines[0]
    assert f"open {tmp_path / 'ovf.gguf'} -> 2" in out       # GLYPR_ERR_SHAPE
    # a prefix that cuts into the last tensor's bytes, or anything before them,
    # is refused; only the trailing alignment padding may be cut
    data_end = len(raw) - 4   # n.f32's 28 bytes end 4 bytes before the 32-byte padding
    for n, l in enumerate(lines[1:len(raw) + 1]):
        assert (" -> 0 " in l) == (n >= data_end), l
