"""Failure paths of the library, each forced from the host: non-finite gradients, the allocation cap,
a missing tensor, bad arguments. Every kernel still runs to completion on ordinary (if NaN) data;
nothing here faults or hangs the device.

The reference does not detect NaN/Inf gradients: Gradients.ClipByGlobalNorm computes a NaN norm, its
`coefficient < 1` test is false, so the gradients stay unscaled and AdamW applies them
(AdamW.cs:103-130, 29-73). The library does the same arithmetic and adds a flag the host can read."""
import ctypes
import json
import os
import shutil

import numpy as np
import pytest

import oracle
from fixtures import TINY, tiny_batch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from laya_amd.device import Context
    print("failure-path tests: creating context on device 0", flush=True)
    c = Context(0)
    yield c
    c.close()


def _dev(ctx, a):
    from laya_amd.device import DeviceArray
    return DeviceArray.from_numpy(ctx, a)


def _adamw(ctx, p, g, m, v, n, lr, step, coef):
    from laya_amd._native import check, lib
    begin, end = (ctypes.c_size_t * 1)(0), (ctypes.c_size_t * 1)(n)
    lrs = (ctypes.c_double * 1)(lr)
    check(lib().laya_adamw(ctx.handle, p.ptr, g.ptr, m.ptr, v.ptr, 1, begin, end, lrs, 0.9, 0.999, 1e-8, 0.01, step,
                           coef.ptr, 0))


def test_status_before_any_norm_is_a_state_error():
    from laya_amd._native import ERR_STATE, lib
    from laya_amd.device import Context
    c = Context(0)
    try:
        assert lib().laya_grad_norm_status(c.handle) == ERR_STATE
    finally:
        c.close()


def test_a_nan_gradient_is_flagged_and_applied_as_the_reference_applies_it(ctx):
    """One NaN gradient element: the norm is NaN, the coefficient stays 1 (no scaling), the status reports
    LAYA_ERR_NOT_FINITE, and AdamW turns exactly that parameter into NaN while every other element takes
    the reference's update bit for bit."""
    from laya_amd._native import ERR_NOT_FINITE, OK, check, lib
    rng = np.random.default_rng(31)
    n = 4096
    p = rng.standard_normal(n).astype(np.float32)
    g = (5 * rng.standard_normal(n)).astype(np.float32)
    g[1234] = np.nan
    pd, gd = _dev(ctx, p), _dev(ctx, g)
    md, vd = _dev(ctx, np.zeros(n, np.float32)), _dev(ctx, np.zeros(n, np.float32))
    norm, coef = _dev(ctx, np.zeros(2, np.float32)), _dev(ctx, np.zeros(1, np.float32))
    check(lib().laya_grad_norm(ctx.handle, gd.ptr, n, 1.0, norm.ptr, coef.ptr))
    assert lib().laya_grad_norm_status(ctx.handle) == ERR_NOT_FINITE
    assert b"not finite" in lib().laya_last_error()
    assert np.isnan(norm.numpy().view(np.float64)[0])
    assert coef.numpy()[0] == 1.0
    # The oracle's clip on the host: NaN norm, gradients untouched.
    gc = g.copy()
    assert np.isnan(oracle.clip([gc], 1.0))
    np.testing.assert_array_equal(gc.view(np.uint32), g.view(np.uint32))
    _adamw(ctx, pd, gd, md, vd, n, 1e-3, 1, coef)
    pr, mr, vr = p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    oracle.adamw_tensor(pr, gc, mr, vr, 1e-3, 1)
    got = pd.numpy()
    assert np.isnan(got[1234]) and np.isnan(pr[1234])
    assert np.isfinite(np.delete(got, 1234)).all()
    np.testing.assert_array_equal(got, pr)  # NaN positions compare equal in assert_array_equal
    np.testing.assert_array_equal(md.numpy(), mr)
    np.testing.assert_array_equal(vd.numpy(), vr)
    # A finite gradient clears the flag.
    gd.upload(np.ones(n, np.float32))
    check(lib().laya_grad_norm(ctx.handle, gd.ptr, n, 1.0, norm.ptr, coef.ptr))
    assert lib().laya_grad_norm_status(ctx.handle) == OK


def test_an_infinite_gradient_is_flagged(ctx):
    from laya_amd._native import ERR_NOT_FINITE, check, lib
    g = np.ones(1000, np.float32)
    g[7] = np.inf
    gd = _dev(ctx, g)
    norm, coef = _dev(ctx, np.zeros(2, np.float32)), _dev(ctx, np.zeros(1, np.float32))
    check(lib().laya_grad_norm(ctx.handle, gd.ptr, g.size, 1.0, norm.ptr, coef.ptr))
    assert lib().laya_grad_norm_status(ctx.handle) == ERR_NOT_FINITE
    assert np.isinf(norm.numpy().view(np.float64)[0])
    # max/(inf + 1e-6) = 0 < 1: the reference scales by 0 here, and so does the coefficient.
    assert coef.numpy()[0] == 0.0


def test_adamw_step_is_bit_identical_to_the_reference_formula(ctx):
    """AdamW.cs:61-68 rounds every float operation on its own; the kernel does too (no multiply-add
    contraction, correctly rounded division and square root), so three steps with no clipping match the
    oracle's restatement (built with contraction off) bit for bit."""
    from laya_amd._native import check, lib
    rng = np.random.default_rng(32)
    n = 50_000
    p = rng.standard_normal(n).astype(np.float32)
    pd = _dev(ctx, p)
    md, vd = _dev(ctx, np.zeros(n, np.float32)), _dev(ctx, np.zeros(n, np.float32))
    norm, coef = _dev(ctx, np.zeros(2, np.float32)), _dev(ctx, np.zeros(1, np.float32))
    pr, mr, vr = p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for step in (1, 2, 3):
        g = (rng.standard_normal(n) * 10.0 ** rng.uniform(-6, 1, n)).astype(np.float32)
        gd = _dev(ctx, g)
        check(lib().laya_grad_norm(ctx.handle, gd.ptr, n, 1e30, norm.ptr, coef.ptr))
        _adamw(ctx, pd, gd, md, vd, n, 3e-4, step, coef)
        oracle.adamw_tensor(pr, g.copy(), mr, vr, 3e-4, step)
    np.testing.assert_array_equal(pd.numpy(), pr)
    np.testing.assert_array_equal(md.numpy(), mr)
    np.testing.assert_array_equal(vd.numpy(), vr)


def test_model_clip_reports_a_nan_gradient(ctx):
    """A NaN logit gradient poisons every gradient below it: the model's clip returns the NaN norm (as
    ClipByGlobalNorm does), check_gradients_finite raises, and the C-ABI clip with a norm output returns
    LAYA_ERR_NOT_FINITE. A finite backward afterwards clears the flag."""
    from laya_amd._native import ERR_NOT_FINITE, LayaNotFiniteError, lib
    from laya_amd.model import TrainableDecisionModel
    m = TrainableDecisionModel.from_directory(TINY, ctx)
    batch, coeff, _ = tiny_batch()
    m.forward(batch)
    bad = coeff.copy()
    bad[0] = np.nan
    m.backward(bad)
    assert np.isnan(m.clip_grad_norm(1.0))
    with pytest.raises(LayaNotFiniteError):
        m.check_gradients_finite()
    v = ctypes.c_double()
    assert lib().laya_model_clip_grad_norm(m.handle, 1.0, ctypes.byref(v)) == ERR_NOT_FINITE
    m.zero_gradients()
    m.forward(batch)
    m.backward(coeff)
    assert np.isfinite(m.clip_grad_norm(1.0))
    m.check_gradients_finite()
    m.close()


def test_the_memory_cap_turns_an_allocation_into_an_out_of_memory_error():
    """laya_ctx_set_memory_cap: an allocation that would exceed the cap fails with LAYA_ERR_MEMORY before
    reaching the device allocator, and a model that does not fit leaves nothing allocated behind."""
    from laya_amd._native import LayaMemoryError
    from laya_amd.config import modernbert_base
    from laya_amd.device import Context, DeviceArray
    from laya_amd.model import TrainableDecisionModel
    c = Context(0)
    try:
        c.set_memory_cap(64 << 20)
        a = DeviceArray(c, (1 << 20,))  # 4 MiB: fits
        with pytest.raises(LayaMemoryError) as e:
            DeviceArray(c, (16 << 20,))  # 64 MiB more: over the cap
        assert "cap" in str(e.value)
        held = c.memory_in_use()
        with pytest.raises(LayaMemoryError):
            TrainableDecisionModel(modernbert_base(), c)  # 656 MB of parameters alone
        assert c.memory_in_use() == held
        a.free()
        c.set_memory_cap(0)
        DeviceArray(c, (16 << 20,)).free()
    finally:
        c.close()


def test_a_checkpoint_missing_a_tensor_is_rejected(ctx, tmp_path):
    """InvalidDataException for a missing tensor (TrainableDecisionModel.cs:184-186): LAYA_ERR_MISSING."""
    from laya_amd._native import LayaMissingError, check, lib
    from laya_amd.model import TrainableDecisionModel
    from laya_amd.safetensors_io import SafetensorsFile, write
    d = tmp_path / "ckpt"
    shutil.copytree(TINY, d)
    st = SafetensorsFile(os.path.join(TINY, "model.safetensors"))
    keep = [n for n in st.names_in_file_order() if n != "head.layers.1.norm2.weight"]
    write(str(d / "model.safetensors"), [(n, st.read_float32(n).shape, st.read_float32(n), "F32") for n in keep])
    with pytest.raises(LayaMissingError) as e:
        TrainableDecisionModel.from_directory(str(d), ctx)
    assert "head.layers.1.norm2.weight" in str(e.value)
    m = TrainableDecisionModel.from_directory(TINY, ctx)
    idx = ctypes.c_int()
    with pytest.raises(LayaMissingError):
        check(lib().laya_model_find_param(m.handle, b"encoder.layers.99.attn.Wqkv.weight", ctypes.byref(idx)))
    m.close()


def test_size_mismatches_are_argument_errors(ctx):
    """ArgumentException for sizes (PackedMatrix.cs:124-126): checked on the host before any launch."""
    from laya_amd._native import ERR_ARGUMENT, lib
    x = _dev(ctx, np.zeros((4, 8), np.float32))
    w = _dev(ctx, np.zeros((3, 8), np.float32))
    y = _dev(ctx, np.zeros((4, 3), np.float32))
    L = lib()
    assert L.laya_linear_fwd(ctx.handle, x.ptr, -1, 8, w.ptr, 3, None, None, y.ptr) == ERR_ARGUMENT
    assert L.laya_linear_fwd(ctx.handle, x.ptr, 4, 8, None, 3, None, None, y.ptr) == ERR_ARGUMENT
    assert L.laya_layernorm_fwd(ctx.handle, x.ptr, 4, 0, w.ptr, None, ctypes.c_float(1e-5), y.ptr, None,
                                None) == ERR_ARGUMENT
    assert L.laya_adamw(ctx.handle, x.ptr, x.ptr, x.ptr, x.ptr, 5, None, None, None, 0.9, 0.999, 1e-8, 0.01, 1, None,
                        0) == ERR_ARGUMENT
