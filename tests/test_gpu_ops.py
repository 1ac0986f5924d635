"""Op-level parity of the HIP kernels against the oracle, through the C-ABI.

Floating-point ops are compared with the fp64 oracle by relative L2 (fp32 bar 1e-4, the targets
here are tighter); integer work (dropout masks, row gathers, scatter order) is compared bit-exactly.
"""
import numpy as np
import pytest

import oracle
from fixtures import rel_l2

pytestmark = pytest.mark.gpu

laya = pytest.importorskip("laya_amd.ops")


@pytest.fixture(scope="module")
def ctx():
    from laya_amd.device import Context
    print("GPU op tests: creating context on device 0", flush=True)
    c = Context(0)
    yield c
    c.close()


def dev(ctx, a):
    from laya_amd.device import DeviceArray
    return DeviceArray.from_numpy(ctx, np.asarray(a))


def param(ctx, name, a, trainable=True):
    return laya.Parameter(ctx, name, np.asarray(a, np.float32), trainable)


@pytest.mark.parametrize("policy", ["fp32", "fp32-split3", "fp32-mfma"])
@pytest.mark.parametrize("rows,inn,out", [(37, 96, 130), (300, 128, 384), (1000, 768, 2304), (5, 768, 1),
                                          (2048, 1152, 768), (333, 100, 260),
                                          # large enough for the balanced static schedule of dX + dW
                                          (8000, 768, 768), (9000, 768, 2304),
                                          # dW tiles outnumber the workers: a worker's dW run would cover a
                                          # whole tile, which the schedule must not take
                                          (4096, 2944, 2944),
                                          # 516 forward tiles: three workgroups per CU with 16-deep K
                                          # stages (the second with a ragged last stage); the backward
                                          # pair on 256 x 256 tiles (ragged columns, ragged last dW unit)
                                          (11000, 768, 768), (11000, 1148, 768),
                                          # the backward pair on 256 x 256 tiles at the model's shapes,
                                          # and with rows of x and dX that are not float4-aligned
                                          (13871, 768, 2304), (13871, 1152, 768), (11000, 1150, 768),
                                          # the forward on 192 x 256 tiles (with the residual, the
                                          # 2304-wide cases above run two and three rounds of them): a
                                          # ragged last row and column tile, and whole tiles with a
                                          # 4-stage K loop
                                          (12345, 768, 700), (13824, 64, 768)])
def test_linear_forward_and_backward(ctx, rows, inn, out, policy):
    """Every fp32 implementation (the default: two-piece fp16 products on 256-wide tiles, exact bf16
    splits elsewhere; exact bf16 splits everywhere; the fp32 matrix cores) at the fp64 oracle's result to
    1e-6, widened as √K for reductions longer than 2048 terms (fp32 rounding of a K-term sum grows as √K)."""
    print(f"linear rows={rows} in={inn} out={out} {policy}", flush=True)
    ctx.set_matmul_precision(policy)
    rng = np.random.default_rng(rows + inn + out)
    x = rng.standard_normal((rows, inn)).astype(np.float32)
    W = (0.05 * rng.standard_normal((out, inn))).astype(np.float32)
    b = rng.standard_normal(out).astype(np.float32)
    res = rng.standard_normal((rows, out)).astype(np.float32)
    dy = rng.standard_normal((rows, out)).astype(np.float32)
    w, bias = param(ctx, "w", W), param(ctx, "b", b)
    dx_, y_ = dev(ctx, np.zeros((rows, inn), np.float32)), dev(ctx, np.zeros((rows, out), np.float32))
    xd, rd, dyd = dev(ctx, x), dev(ctx, res), dev(ctx, dy)
    laya.linear(w, bias, xd, rows, y_, residual=rd)
    y_ref = oracle.linear(x, W, b, double=True) + res
    assert rel_l2(y_ref, y_.numpy()) < 1e-6
    # Accumulation: two backward calls add twice into dW/db; dx is overwritten.
    laya.linear_backward(w, bias, xd, dyd, rows, dx_)
    laya.linear_backward(w, bias, xd, dyd, rows, dx_)
    dW = np.zeros((out, inn)); db = np.zeros(out)
    dx_ref = oracle.linear_backward(x, dy, W, True, dW, db, double=True)
    tol = 1e-6 * max(1.0, (max(rows, out) / 2048) ** 0.5)
    assert rel_l2(dx_ref, dx_.numpy()) < tol
    assert rel_l2(2 * dW, w.gradient.numpy()) < tol
    assert rel_l2(2 * db, bias.gradient.numpy()) < tol
    ctx.set_matmul_precision("fp32")


@pytest.mark.parametrize("rows,inn,out,with_bias", [(6000, 768, 2304, True), (6000, 1152, 2100, False),
                                                    (13871, 768, 2304, True)])
def test_linear_forward_on_wide_tiles(ctx, rows, inn, out, with_bias):
    """Grids whose rounds are shorter on 256 × 256 tiles (no residual): ragged rows and columns, with
    and without bias, at the fp64 oracle's result to 1e-6."""
    print(f"linear (wide tiles) rows={rows} in={inn} out={out} bias={with_bias}", flush=True)
    rng = np.random.default_rng(rows + inn + out)
    x = rng.standard_normal((rows, inn)).astype(np.float32)
    W = (0.05 * rng.standard_normal((out, inn))).astype(np.float32)
    b = rng.standard_normal(out).astype(np.float32) if with_bias else None
    w = param(ctx, "w", W)
    bias = param(ctx, "b", b) if with_bias else None
    y_ = dev(ctx, np.zeros((rows, out), np.float32))
    laya.linear(w, bias, dev(ctx, x), rows, y_)
    y_ref = oracle.linear(x, W, b if with_bias else np.zeros(out, np.float32), double=True)
    assert rel_l2(y_ref, y_.numpy()) < 1e-6


def test_wide_tile_products_are_bitwise_deterministic(ctx):
    """The 256 x 256 forward tiles and the wide backward pair (whose dW tiles several workers share, summed
    by the fixup in worker order) give the same bits on every call."""
    rows, inn, out = 13871, 768, 2304
    print(f"wide tiles twice: rows={rows} in={inn} out={out}", flush=True)
    rng = np.random.default_rng(5)
    x = dev(ctx, rng.standard_normal((rows, inn)).astype(np.float32))
    dy = dev(ctx, rng.standard_normal((rows, out)).astype(np.float32))
    W = (0.05 * rng.standard_normal((out, inn))).astype(np.float32)
    results = []
    for _ in range(2):
        w = param(ctx, "w", W)
        y = dev(ctx, np.zeros((rows, out), np.float32))
        dx = dev(ctx, np.zeros((rows, inn), np.float32))
        laya.linear(w, None, x, rows, y)
        laya.linear_backward(w, None, x, dy, rows, dx)
        results.append((y.numpy(), dx.numpy(), w.gradient.numpy()))
    for a, b in zip(*results):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("sx,sw,sdy", [(1e-20, 1.0, 1.0), (1e20, 1e-3, 1.0), (1.0, 1e15, 1e-25),
                                        (1e-30, 1e-7, 1e30), (0.0, 1.0, 1.0)])
def test_two_piece_products_across_magnitudes(ctx, sx, sw, sdy):
    """The two-piece fp16 products scale each operand by a power of two taken from its largest magnitude,
    so operands far from 1 (and all-zero ones) keep fp32 accuracy: forward, dX and dW on the 256-wide
    kernels (13871 x 768 -> 2304 and 768 wide) at the fp64 oracle's result to 1e-6, with rows whose
    magnitudes spread over six decades; row by row, every y and dX row within 2e-5 of its own exact value
    (rows far below the operand's largest lose relative precision: the model's backward switches to
    three-piece splits before its rows can span more than 2^14 from the logit gradients)."""
    rows, inn = 13871, 768
    rng = np.random.default_rng(11)
    spread = np.exp(rng.uniform(-7, 7, (rows, 1))).astype(np.float32)  # e^±7: six decades across rows
    x = (sx * spread * rng.standard_normal((rows, inn))).astype(np.float32)
    for out in (2304, 768):
        print(f"two-piece magnitudes sx={sx} sw={sw} sdy={sdy} out={out}", flush=True)
        W = (sw * 0.05 * rng.standard_normal((out, inn))).astype(np.float32)
        dy = (sdy * spread * rng.standard_normal((rows, out))).astype(np.float32)
        w = param(ctx, "w", W)
        y_, dx_ = dev(ctx, np.zeros((rows, out), np.float32)), dev(ctx, np.zeros((rows, inn), np.float32))
        xd, dyd = dev(ctx, x), dev(ctx, dy)
        laya.linear(w, None, xd, rows, y_)
        laya.linear_backward(w, None, xd, dyd, rows, dx_)
        dW = np.zeros((out, inn)); db = np.zeros(out)
        dx_ref = oracle.linear_backward(x, dy, W, True, dW, db, double=True)
        y_ref = oracle.linear(x, W, None, double=True)
        tol = 1e-6 * (rows / 2048) ** 0.5
        for ref, got in ((y_ref, y_.numpy()), (dx_ref, dx_.numpy()), (dW, w.gradient.numpy())):
            if not np.any(ref):
                assert not np.any(got)
            else:
                assert rel_l2(ref, got) < tol
        # Row by row: y and dX rows are outputs in their own right. A row 2^-k below its operand's largest keeps
        # ≈ 2^(k-39) relative error (its fp16 pieces turn subnormal); here the rows span ≈ 2^20.
        for what, ref, got in (("y", y_ref, y_.numpy()), ("dx", dx_ref, dx_.numpy())):
            if not np.any(ref):
                continue
            num = np.linalg.norm(ref - got.astype(np.float64), axis=1)
            den = np.maximum(np.linalg.norm(ref, axis=1), 1e-300)
            worst = float((num / den).max())
            print(f"  {what}: worst row relative error {worst:.2e} over rows spanning "
                  f"{float(den.max() / den.min()):.1e}", flush=True)
            assert worst < 2e-5, (what, worst)


def test_two_piece_products_propagate_non_finite_values(ctx):
    """An infinity or NaN in an operand reaches the outputs it reaches in fp32 arithmetic: the rows (dX,
    y) and columns (dW) that touch it are non-finite, every other output is finite and accurate (the
    operand scales come from the finite magnitudes only)."""
    rows, inn, out = 13871, 768, 2304
    rng = np.random.default_rng(12)
    x = rng.standard_normal((rows, inn)).astype(np.float32)
    W = (0.05 * rng.standard_normal((out, inn))).astype(np.float32)
    dy = rng.standard_normal((rows, out)).astype(np.float32)
    x[100, 5] = np.inf
    dy[200, 7] = np.nan
    w = param(ctx, "w", W)
    y_, dx_ = dev(ctx, np.zeros((rows, out), np.float32)), dev(ctx, np.zeros((rows, inn), np.float32))
    xd, dyd = dev(ctx, x), dev(ctx, dy)
    laya.linear(w, None, xd, rows, y_)
    laya.linear_backward(w, None, xd, dyd, rows, dx_)
    y, dx, g = y_.numpy(), dx_.numpy(), w.gradient.numpy()
    bad_y = ~np.isfinite(y).all(axis=1)
    assert bad_y[100] and bad_y.sum() == 1
    bad_dx = ~np.isfinite(dx).all(axis=1)
    assert bad_dx[200] and bad_dx.sum() == 1
    assert not np.isfinite(g[7]).any() and not np.isfinite(g[:, 5]).any()
    ok = np.ones(rows, bool); ok[100] = False
    assert rel_l2(oracle.linear(x[ok], W, None, double=True), y[ok]) < 1e-6
    okd = np.ones(rows, bool); okd[200] = False
    x0, dy0 = x.copy(), dy.copy()
    x0[100] = 0; dy0[200] = 0
    dW = np.zeros((out, inn)); db = np.zeros(out)
    dx_ref = oracle.linear_backward(x0, dy0, W, True, dW, db, double=True)
    assert rel_l2(dx_ref[okd], dx[okd]) < 1e-6
    # dW off row 7 and column 5 sums finite terms only (the poisoned tokens' other entries are finite):
    # the fp64 reference with just the two poisoned entries cleared.
    xc, dyc = x.copy(), dy.copy()
    xc[100, 5] = 0; dyc[200, 7] = 0
    dWc = np.zeros((out, inn)); dbc = np.zeros(out)
    oracle.linear_backward(xc, dyc, W, False, dWc, dbc, double=True)
    keep = np.ones((out, inn), bool); keep[7] = False; keep[:, 5] = False
    assert rel_l2(dWc[keep], g[keep]) < 1e-6 * (rows / 2048) ** 0.5


@pytest.mark.parametrize("rows,inn,out,with_bias", [(512, 768, 768, True), (200, 2304, 768, False)])
def test_linear_in_place_residual_with_split_k(ctx, rows, inn, out, with_bias):
    """y = x·Wᵀ + b + y with the residual being the output itself, on grids small enough (24 and 12 tiles)
    that the product splits K and a reduce applies bias and residual."""
    print(f"linear in-place residual rows={rows} in={inn} out={out}", flush=True)
    rng = np.random.default_rng(rows + inn)
    x = rng.standard_normal((rows, inn)).astype(np.float32)
    W = (0.05 * rng.standard_normal((out, inn))).astype(np.float32)
    b = rng.standard_normal(out).astype(np.float32)
    y0 = rng.standard_normal((rows, out)).astype(np.float32)
    w, bias = param(ctx, "w", W), (param(ctx, "b", b) if with_bias else None)
    yd = dev(ctx, y0)
    laya.linear(w, bias, dev(ctx, x), rows, yd, residual=yd)
    ref = oracle.linear(x, W, b if with_bias else None, double=True) + y0
    assert rel_l2(ref, yd.numpy()) < 1e-6


@pytest.mark.parametrize("rows,inn,out", [(4100, 64, 96), (1500, 256, 132)])
def test_linear_backward_one_product(ctx, rows, inn, out):
    """dW alone (split-K partials over a ragged last slice) and dx alone (frozen weight)."""
    print(f"linear one-product rows={rows} in={inn} out={out}", flush=True)
    rng = np.random.default_rng(rows * 7 + inn)
    x = rng.standard_normal((rows, inn)).astype(np.float32)
    W = (0.05 * rng.standard_normal((out, inn))).astype(np.float32)
    dy = rng.standard_normal((rows, out)).astype(np.float32)
    dW = np.zeros((out, inn)); db = np.zeros(out)
    dx_ref = oracle.linear_backward(x, dy, W, True, dW, db, double=True)
    xd, dyd = dev(ctx, x), dev(ctx, dy)
    w = param(ctx, "w", W)
    laya.linear_backward(w, None, xd, dyd, rows, None)
    assert rel_l2(dW, w.gradient.numpy()) < 1e-6
    frozen = param(ctx, "wf", W, trainable=False)
    dx_ = dev(ctx, np.zeros((rows, inn), np.float32))
    laya.linear_backward(frozen, None, xd, dyd, rows, dx_)
    assert rel_l2(dx_ref, dx_.numpy()) < 1e-6


@pytest.mark.parametrize("rows,n,with_bias,saved", [(33, 128, False, True), (513, 768, True, True),
                                                    (200, 768, False, False), (7, 1024, True, False)])
def test_layernorm_forward_and_backward(ctx, rows, n, with_bias, saved):
    print(f"layernorm rows={rows} n={n}", flush=True)
    rng = np.random.default_rng(rows * n)
    x = (2 + 3 * rng.standard_normal((rows, n))).astype(np.float32)
    g = (1 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    bb = rng.standard_normal(n).astype(np.float32) if with_bias else None
    dy = rng.standard_normal((rows, n)).astype(np.float32)
    dx0 = rng.standard_normal((rows, n)).astype(np.float32)
    w = param(ctx, "g", g)
    bias = param(ctx, "b", bb) if with_bias else None
    xd, yd = dev(ctx, x), dev(ctx, np.zeros_like(x))
    mean, rstd = dev(ctx, np.zeros(rows, np.float32)), dev(ctx, np.zeros(rows, np.float32))
    laya.layer_norm(xd, rows, n, w, bias, 1e-5, yd, mean, rstd)
    assert rel_l2(oracle.layernorm(x, g, bb, 1e-5, double=True), yd.numpy()) < 1e-6
    dxd = dev(ctx, dx0)
    laya.layer_norm_backward(xd, rows, n, w, bias, 1e-5, dev(ctx, dy), dxd, mean if saved else None,
                             rstd if saved else None)
    dx_ref = dx0.astype(np.float64).copy()
    dg = np.zeros(n)
    dbeta = np.zeros(n) if with_bias else None
    oracle.layernorm_backward(x, g, 1e-5, dy, dx_ref, dg, dbeta, double=True)
    assert rel_l2(dx_ref, dxd.numpy()) < 1e-5
    assert rel_l2(dg, w.gradient.numpy()) < 1e-5
    if with_bias:
        assert rel_l2(dbeta, bias.gradient.numpy()) < 1e-5


def test_gelu_and_geglu(ctx):
    rng = np.random.default_rng(3)
    rows, inter = 129, 1152
    wide = (2 * rng.standard_normal((rows, 2 * inter))).astype(np.float32)
    dact = rng.standard_normal((rows, inter)).astype(np.float32)
    wd, ad, dwd = dev(ctx, wide), dev(ctx, np.zeros((rows, inter), np.float32)), dev(ctx, np.zeros_like(wide))
    laya.geglu(ctx, wd, rows, inter, ad)
    assert rel_l2(oracle.geglu(wide, double=True), ad.numpy()) < 1e-6
    laya.geglu_backward(ctx, wd, dev(ctx, dact), rows, inter, dwd)
    assert rel_l2(oracle.geglu_backward(wide, dact, double=True), dwd.numpy()) < 1e-6
    u = (3 * rng.standard_normal(1000)).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    gd = dev(ctx, g)
    laya.gelu_backward(ctx, dev(ctx, u), gd)
    assert rel_l2(oracle.gelu_backward(u, g, double=True), gd.numpy()) < 1e-6
    yd = dev(ctx, u)
    laya.gelu(ctx, yd)
    assert rel_l2(oracle.gelu(u, double=True), yd.numpy()) < 1e-6


@pytest.mark.parametrize("p,seed", [(0.1, 12345), (0.3, 2 ** 63 + 17), (0.5, 0)])
def test_dropout_is_bit_exact(ctx, p, seed):
    rng = np.random.default_rng(1)
    v = rng.standard_normal(100_003).astype(np.float32)
    d = dev(ctx, v)
    laya.dropout(ctx, d, v.size, p, seed)
    got = d.numpy()
    ref = oracle.dropout(v, p, seed)
    np.testing.assert_array_equal(got == 0, ref == 0)
    np.testing.assert_array_equal(got, ref)
    assert laya.uniform(seed, 7) == oracle.uniform(seed, 7)
    assert laya.mix(seed, 9) == oracle.mix(seed, 9)


ATTENTION_CASES = [
    # (head_dim, heads, lengths, half_window, theta, dropout)
    (32, 4, [21, 13, 9], 4, 160000.0, 0.0),
    (64, 12, [300, 129, 64, 1, 200], 64, 10000.0, 0.0),
    (64, 12, [300, 129, 64, 1, 200], -1, 160000.0, 0.0),
    (64, 2, [77, 5, 130], -1, 0.0, 0.1),
    (64, 12, [512, 400], 64, 10000.0, 0.0),
    (32, 2, [40, 200], 8, 10000.0, 0.3),
    # Long-context shapes (2 × 8192, global θ 160000 and sliding ±64 θ 10000): RoPE positions to 8191,
    # the dropout index's 21-bit key field near its top, and 64 query blocks per segment.
    (64, 1, [8192, 8192], -1, 160000.0, 0.0),
    (64, 2, [8192, 8192], 64, 10000.0, 0.0),
    (64, 1, [8192], -1, 0.0, 0.1),
]


@pytest.mark.parametrize("policy", ["fp32", "fp32-split3", "fp32-mfma"])
@pytest.mark.parametrize("hd,heads,lengths,hw,theta,p", ATTENTION_CASES)
def test_attention_forward_and_backward(ctx, hd, heads, lengths, hw, theta, p, policy):
    """Every fp32 implementation at the fp64 oracle's result to 1e-5: for head_dim 64 two-piece fp16
    products of scaled operands (the default) or three-piece bf16 splits on the 16-bit matrix cores, else
    (and under fp32-mfma) the fp32 matrix cores."""
    print(f"attention hd={hd} heads={heads} lengths={lengths} hw={hw} theta={theta} p={p} {policy}", flush=True)
    ctx.set_matmul_precision(policy)
    rng = np.random.default_rng(hd * 1000 + sum(lengths))
    hidden = hd * heads
    T = sum(lengths)
    qkv = rng.standard_normal((T, 3 * hidden)).astype(np.float32)
    dctx = rng.standard_normal((T, hidden)).astype(np.float32)
    scale = laya.default_scale(hd)
    seed = 987654321
    segs = laya.Segments(ctx, lengths)
    rot = laya.Rotary(ctx, hd, theta, max(lengths)) if theta > 0 else None
    shape = laya.AttentionShape(hidden, heads, scale, hw, rot, p, seed)
    qd = dev(ctx, qkv)
    cd = dev(ctx, np.zeros((T, hidden), np.float32))
    lse = dev(ctx, np.zeros(T * heads, np.float32))
    laya.attention_forward(qd, segs, shape, cd, lse)
    ref = oracle.attention_forward(qkv, lengths, heads, scale, hw, theta, p, seed, double=True)
    assert rel_l2(ref, cd.numpy()) < 1e-5
    dq = dev(ctx, np.zeros_like(qkv))
    dcd = dev(ctx, dctx)
    laya.attention_backward(qd, segs, shape, dcd, dq, context=cd, lse=lse)
    dref = oracle.attention_backward(qkv, dctx, lengths, heads, scale, hw, theta, p, seed, double=True)
    got = dq.numpy()
    for part, sl in (("q", slice(0, hidden)), ("k", slice(hidden, 2 * hidden)), ("v", slice(2 * hidden, None))):
        assert rel_l2(dref[:, sl], got[:, sl]) < 1e-5, part
    # The reference's signature (Ops.AttentionBackward carries no forward outputs): the row statistics are
    # recomputed by the same kernels, so the result is the same to the bit.
    dq2 = dev(ctx, np.zeros_like(qkv))
    laya.attention_backward(qd, segs, shape, dcd, dq2)
    np.testing.assert_array_equal(got, dq2.numpy())
    ctx.set_matmul_precision("fp32")


def test_attention_over_many_segments(ctx):
    """40,000 segments of 1–6 tokens and a few of 100–300, in shuffled order: more than 2¹⁵ segments, so the
    launch's block list (longest segments first) carries segment indices past 32767, and most workgroups
    are single short segments. The default two-piece products against the fp64 oracle to 1e-5, forward and
    backward."""
    rng = np.random.default_rng(40000)
    lengths = [int(v) for v in rng.integers(1, 7, 40000)]
    for i in rng.choice(40000, 8, replace=False):
        lengths[i] = int(rng.integers(100, 301))
    heads, hd = 2, 64
    hidden, T = heads * hd, sum(lengths)
    print(f"attention over {len(lengths)} segments, {T} rows", flush=True)
    qkv = rng.standard_normal((T, 3 * hidden)).astype(np.float32)
    dctx = rng.standard_normal((T, hidden)).astype(np.float32)
    scale = laya.default_scale(hd)
    segs = laya.Segments(ctx, lengths)
    rot = laya.Rotary(ctx, hd, 10000.0, max(lengths))
    shape = laya.AttentionShape(hidden, heads, scale, -1, rot, 0.0, 0)
    qd = dev(ctx, qkv)
    cd = dev(ctx, np.zeros((T, hidden), np.float32))
    lse = dev(ctx, np.zeros(T * heads, np.float32))
    laya.attention_forward(qd, segs, shape, cd, lse)
    assert rel_l2(oracle.attention_forward(qkv, lengths, heads, scale, -1, 10000.0, 0.0, 0, double=True),
                  cd.numpy()) < 1e-5
    dq = dev(ctx, np.zeros_like(qkv))
    laya.attention_backward(qd, segs, shape, dev(ctx, dctx), dq, context=cd, lse=lse)
    dref = oracle.attention_backward(qkv, dctx, lengths, heads, scale, -1, 10000.0, 0.0, 0, double=True)
    got = dq.numpy()
    for part, sl in (("q", slice(0, hidden)), ("k", slice(hidden, 2 * hidden)), ("v", slice(2 * hidden, None))):
        assert rel_l2(dref[:, sl], got[:, sl]) < 1e-5, part


def test_operand_magnitude_ring_keeps_each_products_words():
    """Products whose callers keep no magnitude words (the per-op entry points) measure their operands into
    the context's ring of word groups, one operand after the other. A fresh context, one attention forward
    (one measurement) to set the parity, then 130 identical linears (two measurements each) put a product's
    first measurement on every odd ring position, the wrap included; a second attention forward shifts them
    onto the even ones. Every product equals the first bit for bit: recycling the ring never clears a word
    that a pending product still reads."""
    from laya_amd.device import Context
    c = Context(0)
    try:
        rng = np.random.default_rng(128)
        rows, inn, out = 200, 64, 128
        x = rng.standard_normal((rows, inn)).astype(np.float32)
        W = (0.05 * rng.standard_normal((out, inn))).astype(np.float32)
        w, xd = laya.Parameter(c, "w", W, False), dev(c, x)
        qkv = dev(c, rng.standard_normal((16, 3 * 64)).astype(np.float32))
        segs = laya.Segments(c, [16])
        shape = laya.AttentionShape(64, 1, laya.default_scale(64), -1, None, 0.0, 0)
        first = None
        for parity in range(2):
            laya.attention_forward(qkv, segs, shape, dev(c, np.zeros((16, 64), np.float32)),
                                   dev(c, np.zeros(16, np.float32)))
            for i in range(130):
                y = dev(c, np.zeros((rows, out), np.float32))
                laya.linear(w, None, xd, rows, y)
                got = y.numpy()
                if first is None:
                    first = got
                    assert rel_l2(x.astype(np.float64) @ W.astype(np.float64).T, got) < 1e-6
                np.testing.assert_array_equal(got, first, err_msg=f"parity {parity}, product {i}")
    finally:
        c.close()


def test_attention_is_deterministic(ctx):
    rng = np.random.default_rng(5)
    lengths, heads, hd = [384, 100], 12, 64
    hidden, T = heads * hd, 484
    qkv = rng.standard_normal((T, 3 * hidden)).astype(np.float32)
    dctx = rng.standard_normal((T, hidden)).astype(np.float32)
    segs = laya.Segments(ctx, lengths)
    rot = laya.Rotary(ctx, hd, 160000.0, 512)
    shape = laya.AttentionShape(hidden, heads, laya.default_scale(hd), -1, rot, 0.0, 0)
    outs = []
    for _ in range(2):
        qd, cd = dev(ctx, qkv), dev(ctx, np.zeros((T, hidden), np.float32))
        lse, dq = dev(ctx, np.zeros(T * heads, np.float32)), dev(ctx, np.zeros_like(qkv))
        laya.attention_forward(qd, segs, shape, cd, lse)
        laya.attention_backward(qd, segs, shape, dev(ctx, dctx), dq, context=cd, lse=lse)
        outs.append((cd.numpy(), dq.numpy()))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])


def test_embedding_scatter_is_in_token_order(ctx):
    rng = np.random.default_rng(11)
    vocab, hidden, n = 500, 64, 4000
    ranks = np.arange(1, vocab + 1) ** -1.1
    ids = rng.choice(vocab, size=n, p=ranks / ranks.sum()).astype(np.int32)
    d = rng.standard_normal((n, hidden)).astype(np.float32)
    g0 = rng.standard_normal((vocab, hidden)).astype(np.float32)
    gd = dev(ctx, g0)
    laya.embedding_backward(ctx, ids, dev(ctx, d), hidden, gd, vocab)
    ref = g0.copy()
    for t in range(n):  # serial, token order (TrainableDecisionModel.cs:544-547)
        ref[ids[t]] += d[t]
    np.testing.assert_array_equal(ref, gd.numpy())


def test_embedding_plan_rejects_out_of_vocabulary_ids():
    from laya_amd._native import LayaOutOfRangeError
    with pytest.raises(LayaOutOfRangeError):
        laya.embedding_plan(np.array([1, 2, 97], np.int32), 97)


def test_row_gather_and_scatter(ctx):
    rng = np.random.default_rng(2)
    src = rng.standard_normal((50, 33)).astype(np.float32)
    rows = np.array([3, 0, 0, 49, 3, 7], np.int32)
    out = dev(ctx, np.zeros((6, 33), np.float32))
    laya.gather_rows(ctx, dev(ctx, src), dev(ctx, rows), 6, 33, out)
    np.testing.assert_array_equal(out.numpy(), src[rows])
    dst0 = rng.standard_normal((50, 33)).astype(np.float32)
    dd = dev(ctx, dst0)
    add = rng.standard_normal((6, 33)).astype(np.float32)
    laya.scatter_add_rows(ctx, dev(ctx, add), dev(ctx, rows), 6, 33, dd)
    ref = dst0.copy()
    for r in range(6):
        ref[rows[r]] += add[r]
    np.testing.assert_array_equal(ref, dd.numpy())


def test_softmax_cross_entropy_gradient(ctx):
    rng = np.random.default_rng(4)
    ks = np.array([8, 4, 2, 5], np.int32)
    logits = rng.standard_normal(ks.sum()).astype(np.float32)
    targets = np.concatenate([np.eye(k, dtype=np.float32)[rng.integers(k)] for k in ks])
    off = np.concatenate([[0], np.cumsum(ks)]).astype(np.int32)
    g = dev(ctx, np.zeros_like(logits))
    loss = dev(ctx, np.zeros(1, np.float32))
    laya.softmax_ce_backward(ctx, dev(ctx, logits), dev(ctx, targets), dev(ctx, off), len(ks), 1.0, 4.0, g, loss)
    ce, gref = oracle.cross_entropy(ks, logits, targets, 1.0, 4.0)
    np.testing.assert_allclose(g.numpy(), gref, rtol=1e-5, atol=1e-7)
    assert abs(loss.numpy()[0] - ce) < 1e-5


def test_adamw_and_clip_match_the_oracle(ctx):
    import ctypes
    from laya_amd._native import check, lib
    rng = np.random.default_rng(9)
    n = 10_000
    p = rng.standard_normal(n).astype(np.float32)
    g = (3 * rng.standard_normal(n)).astype(np.float32)
    pd, gd = dev(ctx, p), dev(ctx, g)
    md, vd = dev(ctx, np.zeros(n, np.float32)), dev(ctx, np.zeros(n, np.float32))
    norm, coef = dev(ctx, np.zeros(2, np.float32)), dev(ctx, np.zeros(1, np.float32))
    check(lib().laya_grad_norm(ctx.handle, gd.ptr, n, 1.0, norm.ptr, coef.ptr))
    nrm = norm.numpy().view(np.float64)[0]
    assert abs(nrm - np.sqrt((g.astype(np.float64) ** 2).sum())) < 1e-9 * nrm
    gc = g.copy()
    oracle.clip([gc], 1.0)
    begin = (ctypes.c_size_t * 2)(0, 6000)
    end = (ctypes.c_size_t * 2)(6000, n)
    lr = (ctypes.c_double * 2)(1e-3, 1e-4)
    pr, mr, vr = p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for step in (1, 2, 3):
        check(lib().laya_adamw(ctx.handle, pd.ptr, gd.ptr, md.ptr, vd.ptr, 2, begin, end, lr, 0.9, 0.999, 1e-8, 0.01,
                               step, coef.ptr, 0))
        oracle.adamw_tensor(pr[:6000], gc[:6000], mr[:6000], vr[:6000], 1e-3, step)
        a, b, c = pr[6000:].copy(), mr[6000:].copy(), vr[6000:].copy()
        oracle.adamw_tensor(a, gc[6000:].copy(), b, c, 1e-4, step)
        pr[6000:], mr[6000:], vr[6000:] = a, b, c
    assert rel_l2(pr, pd.numpy()) < 1e-6
    assert rel_l2(mr, md.numpy()) < 1e-6
    assert rel_l2(vr, vd.numpy()) < 1e-6


def _device_f64(ctx, a):
    """A float64 array on the device (DeviceArray holds 4-byte elements: twice as many)."""
    from laya_amd.device import DeviceArray
    a = np.ascontiguousarray(a, np.float64)
    d = DeviceArray(ctx, (2 * max(a.size, 1),), np.float32, zero=False)
    if a.size:
        d.upload(a.view(np.float32))
    return d


def _rlcd_on_device(ctx, ks, qtypes, logits, targets, draws, sigma, **kw):
    offsets = np.concatenate([[0], np.cumsum(ks)]).astype(np.int32)
    return laya.rlcd_objective(ctx, dev(ctx, logits), dev(ctx, targets), dev(ctx, offsets),
                               dev(ctx, np.asarray(qtypes, np.int32)), ks, _device_f64(ctx, draws),
                               len(draws) // len(logits), sigma, **kw)


def test_rlcd_objective_matches_the_notebook_fixture(ctx):
    """The reference's objective golden values (the notebook's loss terms and logit gradient)."""
    from fixtures import objective_fixture
    fx = objective_fixture()
    ks = fx["ks"]
    logits = np.concatenate(fx["logits"]).astype(np.float32)
    target = np.concatenate(fx["target"]).astype(np.float32)
    draws = np.concatenate([np.concatenate(g) for g in fx["draws"]])
    (loss, policy, ce, reward), grad = _rlcd_on_device(ctx, ks, fx["qtypes"], logits, target, draws, fx["sigma"])
    assert abs(ce - fx["loss_ce"]) < 1e-5
    assert abs(policy - fx["loss_rl"]) < 1e-4
    assert abs(reward - fx["reward_mean"]) < 1e-4
    assert abs(loss - fx["loss"]) < 1e-4
    np.testing.assert_allclose(grad.numpy()[:logits.size], np.concatenate(fx["grad"]), atol=1e-4)


def test_rlcd_objective_matches_the_oracle_at_batch_size(ctx):
    """32 items cycling choice K = 8 / score K = 4 / noul K = 2 plus one 64-option item, G = 4, soft targets,
    σ 0.4, weights off their defaults, gradient scale 1/4 (accumulation)."""
    rng = np.random.default_rng(8)
    ks = [8, 4, 2] * 11 + [64]
    qtypes = [0, 1, 2] * 11 + [1]
    logits = rng.standard_normal(sum(ks)).astype(np.float32)
    targets = np.concatenate([rng.dirichlet(np.ones(k)) for k in ks]).astype(np.float32)
    G = 4
    draws = rng.standard_normal(G * sum(ks))
    kw = dict(spherical_weight=0.6, rps_weight=0.8, ce_weight=0.5, scale=0.25)
    (loss, policy, ce, reward), grad = _rlcd_on_device(ctx, ks, qtypes, logits, targets, draws, 0.4, **kw)
    out, g = oracle.rlcd(ks, qtypes, logits, targets, draws, 0.4, spherical=0.6, rps=0.8, ce_weight=0.5, scale=0.25)
    # fp32 softmax on both sides; device and host exp may differ by an ulp.
    np.testing.assert_allclose([loss, policy, ce, reward], out, rtol=1e-5, atol=1e-6)
    assert rel_l2(g, grad.numpy()[:logits.size]) < 1e-5
