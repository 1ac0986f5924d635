"""The allocation-free entry point laya_layernorm_bwd_noalloc against laya_layernorm_bwd, through the C-ABI:
identical bits on two calls in a row (the second smaller, so the shared scratch holds the first call's
partials), no growth of the context's allocations, and a clear error beyond the scratch's limit."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev(ctx, a):
    from laya_amd.device import DeviceArray
    return DeviceArray.from_numpy(ctx, np.ascontiguousarray(a, np.float32))


def _call(fn, ctx, x, w, dy, dx0, rows, n, with_stats, bias):
    """One backward through `fn` on fresh output buffers; returns dx, dγ, dβ on the host."""
    from laya_amd._native import check
    from laya_amd.device import DeviceArray
    rng = np.random.default_rng(rows)
    dx = _dev(ctx, dx0)
    dg = _dev(ctx, rng.standard_normal(n))  # gradients accumulate: start from non-zero values
    db = _dev(ctx, rng.standard_normal(n)) if bias else None
    mean = rstd = None
    if with_stats:
        xs = x.numpy().astype(np.float64)
        mu = xs.mean(axis=1)
        mean = _dev(ctx, mu)
        rstd = _dev(ctx, 1.0 / np.sqrt(((xs - mu[:, None]) ** 2).mean(axis=1) + 1e-5))
    check(fn(ctx.handle, x.ptr, rows, n, w.ptr, ctypes.c_float(1e-5), dy.ptr, dx.ptr, dg.ptr,
             None if db is None else db.ptr, None if mean is None else mean.ptr, None if rstd is None else rstd.ptr))
    out = (dx.numpy(), dg.numpy(), None if db is None else db.numpy())
    for a in (dx, dg, db, mean, rstd):
        if isinstance(a, DeviceArray):
            a.free()
    return out


def test_noalloc_layernorm_backward_matches_the_allocating_entry_point():
    from laya_amd._native import ERR_ARGUMENT, lib
    from laya_amd.device import Context
    print("no-alloc LayerNorm backward: fresh context", flush=True)
    ctx = Context(0)
    try:
        L = lib()
        rng = np.random.default_rng(3)
        # Two calls in a row, the second with fewer rows and a narrower row than the first.
        for rows, n, with_stats, bias in ((13871, 768, True, False), (300, 1024, False, True), (37, 96, True, True)):
            print(f"  rows={rows} n={n} stats={with_stats} bias={bias}", flush=True)
            x = _dev(ctx, rng.standard_normal((rows, n)))
            w = _dev(ctx, 1 + 0.2 * rng.standard_normal(n))
            dy = _dev(ctx, rng.standard_normal((rows, n)))
            dx0 = rng.standard_normal((rows, n)).astype(np.float32)
            held = ctx.memory_in_use()
            got = _call(L.laya_layernorm_bwd_noalloc, ctx, x, w, dy, dx0, rows, n, with_stats, bias)
            ctx.sync()
            # The outputs were allocated and freed by the test; the entry point itself allocated nothing.
            assert ctx.memory_in_use() == held
            want = _call(L.laya_layernorm_bwd, ctx, x, w, dy, dx0, rows, n, with_stats, bias)
            for a, b in zip(got, want):
                if b is not None:
                    np.testing.assert_array_equal(a, b)
            for a in (x, w, dy):
                a.free()
        # Beyond the static scratch (rows wider than 2048): refused before any launch.
        x = _dev(ctx, np.zeros((2, 4096)))
        w = _dev(ctx, np.ones(4096))
        assert L.laya_layernorm_bwd_noalloc(ctx.handle, x.ptr, 2, 4096, w.ptr, ctypes.c_float(1e-5), x.ptr, x.ptr,
                                            w.ptr, None, None, None) == ERR_ARGUMENT
        assert b"2048" in L.laya_last_error()
    finally:
        ctx.close()
