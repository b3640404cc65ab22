"""The allocation-free matmul (arfq_matmul_noalloc) against arfq_matmul, through the
C ABI: the same kernels with scratch from the library's fixed per-GPU array, so the
outputs must be bit-identical; two calls in a row, the second on a smaller input (the
array keeps the last call's contents)."""
import sys

import numpy as np
import pytest

import arf_amd
from arf_amd import arfq

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _both(ctx, qtype, n, k, m, seed, x_dtype=np.float32):
    """y from arfq_matmul and from arfq_matmul_noalloc on the same inputs."""
    from arf_amd import QType, synth
    raw = synth.weight(qtype, n, k, seed=seed)
    x = synth.activations(m, k, seed=seed + 1).astype(x_dtype)
    w = ctx.upload(QType[qtype.upper()], raw, n, k)
    xd = ctx.to_device(x)
    y0 = ctx.empty((m, n), np.float32)
    y1 = ctx.empty((m, n), np.float32)
    ctx.matmul(w, xd, m, y0)
    dt = arf_amd.DType.F32 if x_dtype == np.float32 else arf_amd.DType.F16
    st = arf_amd.load_library().arfq_matmul_noalloc(ctx.handle, w.handle, 0, m, xd.ptr, int(dt), y1.ptr)
    assert st == arfq.ARFQ_OK, arf_amd.load_library().arfq_last_error(ctx.handle)
    got, want = y1.numpy(), y0.numpy()
    w.free()
    return got, want


@pytest.mark.parametrize("cases", [
    # C3's Q6_K shape at m = 8 (x preparation + split-K partials in the scratch), then smaller
    [("q6_k", 5120, 17408, 8, np.float32), ("q6_k", 96, 2048, 5, np.float32)],
    # Q4_K prefill tile (x f16 sums + split partials), then a skinny f32 product
    [("q4_k", 512, 2048, 160, np.float16), ("q4_k", 256, 1024, 12, np.float32)],
    # Q8_0 / IQ4_XS skinny, then a decode GEMV (no scratch)
    [("iq4_xs", 1024, 4096, 40, np.float32), ("q4_k", 300, 5120, 1, np.float32)],
])
def test_noalloc_matches_matmul(gpu_ctx, cases):
    for i, (qtype, n, k, m, xdt) in enumerate(cases):
        _say("case: noalloc", i, qtype, n, k, m, np.dtype(xdt).name)
        got, want = _both(gpu_ctx, qtype, n, k, m, seed=1000 + 7 * i + n, x_dtype=xdt)
        assert np.all(np.isfinite(got))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_rejects_products_above_its_scratch(gpu_ctx):
    # C4's prefill (2048 x 5120 f16 x, 17408 rows) needs more than the fixed array
    from arf_amd import QType, synth
    _say("case: noalloc over limit")
    n, k, m = 17408, 5120, 2048
    w = gpu_ctx.upload(QType.Q4_K, synth.weight("q4_k", n, k, seed=5), n, k)
    x = gpu_ctx.empty((m, k), np.float16)
    y = gpu_ctx.empty((m, n), np.float32)
    L = arf_amd.load_library()
    st = L.arfq_matmul_noalloc(gpu_ctx.handle, w.handle, 0, m, x.ptr, int(arf_amd.DType.F16), y.ptr)
    assert st == arfq.ARFQ_E_UNSUPPORTED
    assert b"scratch" in L.arfq_last_error(gpu_ctx.handle)
    w.free()


def test_noalloc_allocates_nothing():
    # a fresh context that has never run arfq_matmul: the allocation-free entry point
    # must leave the context's scratch at 0 bytes and, after the runtime's own one-time
    # set-up in the first call, the device's free memory (hipMemGetInfo) unchanged over
    # further calls -- two products that use scratch (x preparation and split-K
    # partials), the second smaller; the outputs then match arfq_matmul's bit for bit
    from arf_amd import QType, synth
    _say("case: noalloc allocates nothing")
    ctx = arf_amd.Context(0)
    try:
        L = arf_amd.load_library()
        shapes = [("q6_k", 2048, 8192, 8), ("q6_k", 2048, 8192, 8), ("q6_k", 96, 2048, 5)]
        ws, xs, ys = [], [], []
        for i, (qtype, n, k, m) in enumerate(shapes):
            ws.append(ctx.upload(QType[qtype.upper()], synth.weight(qtype, n, k, seed=77 + i), n, k))
            xs.append(ctx.to_device(synth.activations(m, k, seed=78 + i)))
            ys.append(ctx.empty((m, n), np.float32))
        ctx.sync()
        free0 = None
        for i, (qtype, n, k, m) in enumerate(shapes):
            st = L.arfq_matmul_noalloc(ctx.handle, ws[i].handle, 0, m, xs[i].ptr, int(arf_amd.DType.F32),
                                       ys[i].ptr)
            assert st == arfq.ARFQ_OK, L.arfq_last_error(ctx.handle)
            ctx.sync()
            scratch, free, _ = ctx.memory()
            assert scratch == 0
            if i == 0:
                free0 = free
            else:
                assert free == free0, (free0, free)
        got = [y.numpy() for y in ys]
        for i, (qtype, n, k, m) in enumerate(shapes):
            want = ctx.empty((m, n), np.float32)
            ctx.matmul(ws[i], xs[i], m, want)
            assert np.array_equal(got[i].view(np.uint32), want.numpy().view(np.uint32))
        assert ctx.memory()[0] > 0  # arfq_matmul grew the context's scratch
    finally:
        ctx.close()
