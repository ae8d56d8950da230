"""glypr_hip_q8_0_matmul_noalloc, the matmul for callers that cannot allocate:
through the C ABI, its output equals glypr_hip_q8_0_matmul's bit for bit (both
variants), on two calls in a row with the second input smaller (the shared
per-device scratch keeps the first call's contents), on a second context of the
same device (which shares the array) and with profiling on; sizes beyond the
scratch are refused with GLYPR_ERR_SHAPE before anything runs; a call on a
second stream while the first stream's call is still pending is refused with
GLYPR_ERR_BUSY, and accepted once that call has finished."""
import ctypes

import numpy as np
import pytest
import torch

from glypr_amd import _lib, ops
from glypr_amd.ops import BF16_DEQUANT, INT8_EXACT, Q8Weight

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def bits(t):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("variant", [INT8_EXACT, BF16_DEQUANT])
def test_noalloc_matmul_equals_matmul(variant):
    from oracle import pyoracle as po
    ctx = ops.Context(0)
    n, k = 1280, 768
    wb = po.q8_0_weight(n, k, seed=71)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    # M = 3000 runs the separate quantize (or bf16) launch into the scratch;
    # M = 700 then the prologue-fused GEMM (INT8_EXACT) on a smaller input
    for m in (3000, 700):
        say(f"no-alloc matmul variant={variant} m={m}")
        x = torch.from_numpy(po.normal(m * k, seed=m).reshape(m, k)).cuda()
        ref = ops.q8_0_matmul(ctx, w, x, variant)
        got = ops.q8_0_matmul_noalloc(ctx, w, x, variant)
        assert np.array_equal(bits(got), bits(ref)), f"m={m}"
    # a smaller call after a larger one on the separate-launch route too
    x2 = torch.from_numpy(po.normal(2100 * k, seed=5).reshape(2100, k)).cuda()
    assert np.array_equal(bits(ops.q8_0_matmul_noalloc(ctx, w, x2, variant)),
                          bits(ops.q8_0_matmul(ctx, w, x2, variant)))
    # a second context on the device shares the array; profiling records nothing
    ctx2 = ops.Context(0)
    _lib.check(_lib.lib().glypr_hip_profile_enable(ctx2.handle, 1))
    w2 = Q8Weight.from_gguf(ctx2, wb, n, k)
    got2 = ops.q8_0_matmul_noalloc(ctx2, w2, x2, variant)
    assert np.array_equal(bits(got2), bits(ops.q8_0_matmul(ctx, w, x2, variant)))
    tot = (ctypes.c_double * _lib.KERNEL_COUNT)()
    cnt = (ctypes.c_int64 * _lib.KERNEL_COUNT)()
    _lib.check(_lib.lib().glypr_hip_profile_read(ctx2.handle, tot, cnt))
    assert sum(cnt) == 0
    w2.close()
    ctx2.close()
    w.close()
    ctx.close()


def test_noalloc_matmul_rejects_oversized():
    from oracle import pyoracle as po
    ctx = ops.Context(0)
    k = 2048
    w = Q8Weight.from_gguf(ctx, po.q8_0_weight(64, k, seed=72), 64, k)
    # BF16_DEQUANT needs 2 m k bytes: m = 16384 fits 64 MiB exactly, one more row does not
    m_ok = (64 << 20) // (2 * k)
    x = torch.zeros((m_ok + 1, k), dtype=torch.float32, device="cuda")
    y = torch.empty((m_ok + 1, 64), dtype=torch.float32, device="cuda")
    L = _lib.lib()
    rc = L.glypr_hip_q8_0_matmul_noalloc(ctx.handle, w.handle, ops._ptr(x), ops._ptr(y),
                                         m_ok + 1, BF16_DEQUANT, ctx.stream)
    assert rc == _lib.GLYPR_ERR_SHAPE and "scratch" in _lib.last_error()
    # row counts whose byte count m k would wrap 64 bits are refused the same
    # way (the bound on m comes before the product); x and y are not touched
    for m_huge in (1 << 55, (1 << 63) - 1):
        for variant in (INT8_EXACT, BF16_DEQUANT):
            rc = L.glypr_hip_q8_0_matmul_noalloc(ctx.handle, w.handle, ops._ptr(x), ops._ptr(y),
                                                 ctypes.c_int64(m_huge), variant, ctx.stream)
            assert rc == _lib.GLYPR_ERR_SHAPE and "scratch" in _lib.last_error()
    rc = L.glypr_hip_q8_0_matmul_noalloc(ctx.handle, w.handle, ops._ptr(x), ops._ptr(y), m_ok,
                                         BF16_DEQUANT, ctx.stream)
    assert rc == _lib.GLYPR_OK
    torch.cuda.synchronize()
    w.close()
    ctx.close()


def test_noalloc_matmul_rejects_overlap_on_another_stream():
    """Stream A is held by a bounded spin kernel (torch.cuda._sleep), so the
    no-allocation call queued behind it is pending when stream B calls: B's
    call must fail with GLYPR_ERR_BUSY and launch nothing.  Calls on A itself
    stay accepted (one stream orders them), and after A has finished B's call
    runs and gives the matmul's bits."""
    from oracle import pyoracle as po
    ctx = ops.Context(0)
    n, k, m = 1152, 768, 512
    wb = po.q8_0_weight(n, k, seed=81)
    w = Q8Weight.from_gguf(ctx, wb, n, k)
    x = torch.from_numpy(po.normal(m * k, seed=82).reshape(m, k)).cuda()
    ref = ops.q8_0_matmul(ctx, w, x, INT8_EXACT)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    ya = torch.empty((m, n), dtype=torch.float32, device="cuda")
    yb = torch.full((m, n), -1.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    L = _lib.lib()
    fn = L.glypr_hip_q8_0_matmul_noalloc

    def call(y, stream):
        return fn(ctx.handle, w.handle, ctypes.c_void_p(x.data_ptr()),
                  ctypes.c_void_p(y.data_ptr()), m, INT8_EXACT,
                  ctypes.c_void_p(stream.cuda_stream))

    # the spin kernel counts GPU clock ticks: time a short spin first, so the
    # hold below lasts ~300 ms of wall time whatever the clock runs at
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(sa):
        e0.record()
        torch.cuda._sleep(10_000_000)
        e1.record()
    e1.synchronize()
    ticks_per_ms = 10_000_000 / max(e0.elapsed_time(e1), 1e-3)
    hold = int(min(max(300 * ticks_per_ms, 1e7), 4e9))
    say(f"no-alloc overlap: stream A held by a {hold}-tick spin (~300 ms), then a call on A "
        "and one on B")
    with torch.cuda.stream(sa):
        torch.cuda._sleep(hold)
    assert call(ya, sa) == _lib.GLYPR_OK
    assert call(ya, sa) == _lib.GLYPR_OK    # the same stream: ordered, accepted
    rc = call(yb, sb)
    assert not sa.query(), "stream A finished before B's call: the hold did not cover it"
    assert rc == _lib.GLYPR_ERR_BUSY, (rc, _lib.last_error())
    assert "another stream" in _lib.last_error()
    sa.synchronize()
    sb.synchronize()
    assert np.all(yb.cpu().numpy() == -1.0)  # the refused call launched nothing
    assert call(yb, sb) == _lib.GLYPR_OK     # A has finished: accepted
    assert np.array_equal(bits(ya), bits(ref))
    assert np.array_equal(bits(yb), bits(ref))
    w.close()
    ctx.close()
