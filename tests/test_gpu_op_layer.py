"""The per-op C-ABI as a drop-in: one encoder layer composed from op entry points only, in the order
TrainableDecisionModel runs them, against the same composition of the oracle's fp64 ops.

A C# host that re-points `Ops` at the library runs exactly this sequence
(TrainableDecisionModel.cs:361-414 forward, 551-603 backward): LayerNorm, Linear, AttentionForward,
Linear, Add, LayerNorm, Linear, GeGLU, Linear, Add; then LinearBackward (dx overwritten), the GeGLU
backward, LinearBackward, LayerNormBackward (dx added), LinearBackward, AttentionBackward with no forward
outputs (the reference's signature), LinearBackward and the first LayerNormBackward. Also Rotary.Apply
on its own."""
import numpy as np
import pytest

import laya_amd.ops as laya
import oracle
from fixtures import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from laya_amd.device import Context
    print("op-layer tests: creating context on device 0", flush=True)
    c = Context(0)
    yield c
    c.close()


def _dev(ctx, a):
    from laya_amd.device import DeviceArray
    return DeviceArray.from_numpy(ctx, np.ascontiguousarray(a, np.float32))


def _zeros(ctx, shape):
    from laya_amd.device import DeviceArray
    return DeviceArray(ctx, shape)


def _host_layer(x, P, lengths, heads, hw, theta, first, dout, eps):
    """The same layer in fp64 on the oracle's ops: returns the output, dx and the parameter gradients."""
    f = dict(double=True)
    T, d = x.shape
    scale = laya.default_scale(d // heads)
    normed = x if first else oracle.layernorm(x, P["attn_norm"], None, eps, **f)
    qkv = oracle.linear(normed, P["Wqkv"], **f)
    context = oracle.attention_forward(qkv, lengths, heads, scale, hw, theta, **f)
    residual = oracle.linear(context, P["Wo"], **f) + x
    mlp_normed = oracle.layernorm(residual, P["mlp_norm"], None, eps, **f)
    wide = oracle.linear(mlp_normed, P["Wi"], **f)
    act = oracle.geglu(wide, **f)
    out = oracle.linear(act, P["MlpWo"], **f) + residual
    G = {k: np.zeros(v.shape) for k, v in P.items()}
    d_res = np.array(dout, np.float64)
    d_act = oracle.linear_backward(act, dout, P["MlpWo"], dW=G["MlpWo"], **f)
    d_wide = oracle.geglu_backward(wide, d_act, **f)
    d_mn = oracle.linear_backward(mlp_normed, d_wide, P["Wi"], dW=G["Wi"], **f)
    oracle.layernorm_backward(residual, P["mlp_norm"], eps, d_mn, d_res, dgamma=G["mlp_norm"], **f)
    d_ctx = oracle.linear_backward(context, d_res, P["Wo"], dW=G["Wo"], **f)
    d_qkv = oracle.attention_backward(qkv, d_ctx, lengths, heads, scale, hw, theta, **f)
    d_n = oracle.linear_backward(normed, d_qkv, P["Wqkv"], dW=G["Wqkv"], **f)
    dx = d_res
    if first:
        dx += d_n
    else:
        oracle.layernorm_backward(x, P["attn_norm"], eps, d_n, dx, dgamma=G["attn_norm"], **f)
    return out, dx, G


@pytest.mark.parametrize("kind", ["layer0-global", "sliding"])
def test_one_encoder_layer_from_op_entry_points(ctx, kind):
    print(f"op-level encoder layer: {kind}", flush=True)
    d, heads, inter, eps = 768, 12, 1152, 1e-5
    first = kind == "layer0-global"
    hw, theta = (-1, 160000.0) if first else (64, 10000.0)
    lengths = [300, 129, 64, 17]
    T = sum(lengths)
    rng = np.random.default_rng(17 if first else 18)
    x = rng.standard_normal((T, d)).astype(np.float32)
    dout = rng.standard_normal((T, d)).astype(np.float32)
    P = {"attn_norm": (1 + 0.2 * rng.standard_normal(d)).astype(np.float32),
         "Wqkv": (0.05 * rng.standard_normal((3 * d, d))).astype(np.float32),
         "Wo": (0.05 * rng.standard_normal((d, d))).astype(np.float32),
         "mlp_norm": (1 + 0.2 * rng.standard_normal(d)).astype(np.float32),
         "Wi": (0.05 * rng.standard_normal((2 * inter, d))).astype(np.float32),
         "MlpWo": (0.05 * rng.standard_normal((d, inter))).astype(np.float32)}
    if first:
        del P["attn_norm"]
    W = {k: laya.Parameter(ctx, k, v) for k, v in P.items()}

    # ---- forward (TrainableDecisionModel.cs:361-414)
    segs = laya.Segments(ctx, lengths)
    rot = laya.Rotary(ctx, d // heads, theta, max(lengths))
    shape = laya.AttentionShape(d, heads, laya.default_scale(d // heads), hw, rot, 0.0, 0)
    xd = _dev(ctx, x)
    if first:
        normed = xd
    else:
        normed = _zeros(ctx, (T, d))
        laya.layer_norm(xd, T, d, W["attn_norm"], None, eps, normed)
    qkv = _zeros(ctx, (T, 3 * d))
    laya.linear(W["Wqkv"], None, normed, T, qkv)
    context, lse = _zeros(ctx, (T, d)), _zeros(ctx, (T * heads,))
    laya.attention_forward(qkv, segs, shape, context, lse)
    residual = _zeros(ctx, (T, d))
    laya.linear(W["Wo"], None, context, T, residual)
    laya.add(ctx, residual, xd)
    mlp_normed = _zeros(ctx, (T, d))
    laya.layer_norm(residual, T, d, W["mlp_norm"], None, eps, mlp_normed)
    wide = _zeros(ctx, (T, 2 * inter))
    laya.linear(W["Wi"], None, mlp_normed, T, wide)
    act = _zeros(ctx, (T, inter))
    laya.geglu(ctx, wide, T, inter, act)
    out = _zeros(ctx, (T, d))
    laya.linear(W["MlpWo"], None, act, T, out)
    laya.add(ctx, out, residual)

    # ---- backward (TrainableDecisionModel.cs:551-603)
    d_out = _dev(ctx, dout)
    d_res = _dev(ctx, dout)  # dOutput.Clone()
    d_act = _zeros(ctx, (T, inter))
    laya.linear_backward(W["MlpWo"], None, act, d_out, T, d_act)
    d_wide = _zeros(ctx, (T, 2 * inter))
    laya.geglu_backward(ctx, wide, d_act, T, inter, d_wide)
    d_mn = _zeros(ctx, (T, d))
    laya.linear_backward(W["Wi"], None, mlp_normed, d_wide, T, d_mn)
    laya.layer_norm_backward(residual, T, d, W["mlp_norm"], None, eps, d_mn, d_res)
    d_ctx = _zeros(ctx, (T, d))
    laya.linear_backward(W["Wo"], None, context, d_res, T, d_ctx)
    d_qkv = _zeros(ctx, (T, 3 * d))
    laya.attention_backward(qkv, segs, shape, d_ctx, d_qkv)
    d_n = _zeros(ctx, (T, d))
    laya.linear_backward(W["Wqkv"], None, normed, d_qkv, T, d_n)
    if first:
        laya.add(ctx, d_res, d_n)
    else:
        laya.layer_norm_backward(xd, T, d, W["attn_norm"], None, eps, d_n, d_res)

    ref_out, dx, G = _host_layer(x, P, lengths, heads, hw, theta, first, dout, eps)
    assert rel_l2(ref_out, out.numpy()) < 1e-5, "output"
    assert rel_l2(dx, d_res.numpy()) < 1e-5, "dx"
    for k in P:
        assert rel_l2(G[k], W[k].gradient.numpy()) < 1e-5, k
    for obj in (segs, rot):
        obj.close()


def test_rotary_apply_matches_the_oracle(ctx):
    """Rotary.Apply (Ops.cs:489-503) on rows at arbitrary positions, forward and inverse: the oracle's
    rotation in fp32 and fp64, norms kept, and inverse ∘ forward = identity."""
    from laya_amd.device import DeviceArray
    rng = np.random.default_rng(23)
    for hd, theta in ((64, 160000.0), (64, 10000.0), (32, 10000.0)):
        rows = 700
        vec = rng.standard_normal((rows, hd)).astype(np.float32)
        pos = rng.integers(0, 8192, rows).astype(np.int32)
        pos[:3] = [0, 1, 8191]
        rot = laya.Rotary(ctx, hd, theta, 8192)
        v = _dev(ctx, vec)
        pd = DeviceArray.from_numpy(ctx, pos)
        rot.apply(v, rows, pd, inverse=False)
        got = v.numpy()
        ref64 = np.stack([oracle.rotary_apply(theta, vec[i], int(pos[i]), double=True) for i in range(rows)])
        ref32 = np.stack([oracle.rotary_apply(theta, vec[i], int(pos[i])) for i in range(rows)])
        assert rel_l2(ref64, got) < 1e-6
        assert rel_l2(ref32, got) < 1e-6
        np.testing.assert_array_equal(got[0], vec[0])  # position 0 is the identity
        np.testing.assert_allclose(np.linalg.norm(got, axis=1), np.linalg.norm(vec, axis=1), rtol=1e-5)
        rot.apply(v, rows, pd, inverse=True)
        assert rel_l2(vec, v.numpy()) < 1e-6
        rot.close()


def test_whole_step_from_op_entry_points_matches_the_oracle_and_the_model_driver(ctx):
    """The whole training step composed from op entry points only (laya_amd.opmodel: what a host re-pointing
    Ops runs, TrainableDecisionModel.cs:248-640 over Ops.cs), at ModernBERT-base widths with 3 encoder layers,
    the two-layer head with dropout 0.1 and the scorer, on a batch of five ragged items. Every gradient against
    the fp64 oracle at max(1e-4, 4 × the fp32 oracle's error), and the weights after a full step (soft CE,
    clip, AdamW) equal to the reference's clip and AdamW formulas applied to the op path's own gradients."""
    from helpers import fixture_params, mid_config, mixed_batch
    from laya_amd.opmodel import OpBatch, OpLevelModel
    mc = mid_config(layers=3)
    o = oracle.OracleModel(mc)
    params = fixture_params(o.shapes, 23)
    batch = mixed_batch(np.random.default_rng(24), [300, 200, 129, 64, 17], mc.encoder.vocab_size)
    rng = np.random.default_rng(25)
    targets = np.concatenate([np.eye(k, dtype=np.float32)[rng.integers(k)] for k in batch.n_options])
    seed, scale = 7, float(batch.n_items)
    om = OpLevelModel(mc, {n: params[n] for n in o.names}, ctx)
    ob = OpBatch(ctx, batch, targets, mc.encoder.vocab_size)
    logits = om.forward(ob, seed, training=True).numpy()
    _, g = oracle.cross_entropy(batch.n_options, logits, targets, 1.0, scale)
    from laya_amd.device import DeviceArray
    gd = DeviceArray.from_numpy(ctx, g)
    om.backward(gd)
    o64 = oracle.OracleModel(mc, double=True)
    for ref in (o, o64):
        ref.set_params(params)
        ref.set_head_dropout(0.1)
        ref.forward(batch, training=True, keep_tape=True, seed=seed)
        ref.backward(g)
    assert rel_l2(o64.forward(batch, training=True, keep_tape=False, seed=seed), logits) < 1e-5
    worst = 0.0
    for name in o.names:
        if not o64.has_grad(name):
            continue
        exact = o64.grad(name)
        bar = max(1e-4, 4 * rel_l2(exact, o.grad(name)))
        r = rel_l2(exact, om.grad(name))
        assert r < bar, (name, r, bar)
        if bar == 1e-4:
            worst = max(worst, r)
    print(f"op-level step: worst gradient rel-L2 vs fp64 {worst:.2e}", flush=True)
    # The rest of the step on the op path: the device soft-CE gradient, then ClipByGlobalNorm and AdamW.Step,
    # against the reference's formulas applied on the host to the same gradients.
    om.zero_gradients()
    logits = om.forward(ob, seed, training=True)
    dl = DeviceArray(ctx, (batch.n_markers,))
    laya.softmax_ce_backward(ctx, logits, ob.targets, ob.offsets, batch.n_items, 1.0, scale, dl)
    assert np.abs(dl.numpy() - g).max() <= 1e-6 * max(1.0, np.abs(g).max())
    om.backward(dl)
    trained = [n for n in o.names if o64.has_grad(n)]
    grads = {n: om.grad(n) for n in trained}
    clipped = {n: grads[n].copy() for n in trained}
    oracle.clip(list(clipped.values()), 1.0)
    lr = 1e-3
    om.clip_and_step(1.0, lr, lr)
    for name in o.names:
        w = params[name].astype(np.float32).reshape(-1).copy()
        if name != "temperature":
            gr = clipped[name].reshape(-1) if name in clipped else np.zeros_like(w)
            oracle.adamw_tensor(w, np.ascontiguousarray(gr), np.zeros_like(w), np.zeros_like(w), lr, 1)
        assert np.abs(om.param(name).reshape(-1) - w).max() <= 1e-6 * max(1.0, np.abs(w).max()), name
    assert not np.any(om.grad("scorer.1.weight"))  # the step cleared the gradients
    ob.close()
    om.close()


def test_op_path_magnitude_words_change_nothing(ctx):
    """A binding that keeps the encoder operands' magnitude words (the _w entry points: producers fill them, the
    products read them instead of measuring) computes the same step as one that keeps none: each group holds
    the same largest magnitude a measuring pass would find, so the scales, the products and every gradient
    agree bit for bit (ModernBERT-base widths, 3 encoder layers, the head and scorer, five ragged items)."""
    from helpers import fixture_params, mid_config, mixed_batch
    from laya_amd.device import DeviceArray
    from laya_amd.opmodel import OpBatch, OpLevelModel
    mc = mid_config(layers=3)
    o = oracle.OracleModel(mc)
    params = fixture_params(o.shapes, 31)
    batch = mixed_batch(np.random.default_rng(32), [300, 200, 129, 64, 17], mc.encoder.vocab_size)
    rng = np.random.default_rng(33)
    targets = np.concatenate([np.eye(k, dtype=np.float32)[rng.integers(k)] for k in batch.n_options])
    runs = []
    for words in (False, True):
        om = OpLevelModel(mc, {n: params[n] for n in o.names}, ctx)
        om.carry_words = words
        ob = OpBatch(ctx, batch, targets, mc.encoder.vocab_size)
        logits = om.forward(ob, 9, training=True)
        dl = DeviceArray(ctx, (batch.n_markers,))
        laya.softmax_ce_backward(ctx, logits, ob.targets, ob.offsets, batch.n_items, 1.0, float(batch.n_items), dl)
        om.backward(dl)
        runs.append((logits.numpy(), {n: om.grad(n) for n in o.names if o.has_grad(n)}))
        ob.close()
        om.close()
    (l0, g0), (l1, g1) = runs
    np.testing.assert_array_equal(l0, l1)
    for n in g0:
        np.testing.assert_array_equal(g0[n], g1[n], err_msg=n)
