"""Model-level parity on the GPU: the reference's golden fixture, and the oracle at ModernBERT-base
widths, through the model driver of the C-ABI.

Bar (fp32): relative L2 ≤ 1e-4 per gradient tensor, and the reference test's own
max|Δ|/max|g| < 1e-4 on the golden fixture (TrainingGradientTests.cs:58-85).
"""
import numpy as np
import pytest

import oracle
from fixtures import max_rel, rel_l2, tiny_batch, tiny_config, tiny_grads, tiny_params, TINY
from helpers import mid_config, mixed_batch, random_params

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from laya_amd.device import Context
    print("GPU model tests: creating context on device 0", flush=True)
    c = Context(0)
    yield c
    c.close()


def test_tiny_fixture_logits_and_every_gradient(ctx):
    from laya_amd.model import TrainableDecisionModel
    print("model: training-tiny fixture", flush=True)
    m = TrainableDecisionModel.from_directory(TINY, ctx)
    m.set_trainable_encoder_layers(None)
    batch, coeff, torch_logits = tiny_batch()
    logits = m.forward(batch, training=False)
    assert np.abs(logits - torch_logits).max() < 1e-4
    m.backward(coeff)
    grads = tiny_grads()
    for name, expected in grads.items():
        got = m.grad(name)
        assert max_rel(expected, got) < 1e-4, name
        assert rel_l2(expected, got) < 1e-4, name
    for name in m.names:
        if name.startswith("act_head."):
            assert not np.any(m.grad(name))


def test_tiny_freezing_the_encoder(ctx):
    from laya_amd.model import TrainableDecisionModel
    m = TrainableDecisionModel.from_directory(TINY, ctx)
    m.set_trainable_encoder_layers(1)
    batch, coeff, _ = tiny_batch()
    m.forward(batch)
    m.backward(coeff)
    assert not m.has_grad("encoder.layers.0.attn.Wqkv.weight")
    assert not m.has_grad("encoder.embeddings.tok_embeddings.weight")
    assert m.has_grad("encoder.layers.3.attn.Wqkv.weight")
    expected = tiny_grads()["encoder.layers.3.mlp.Wi.weight"]
    assert rel_l2(expected, m.grad("encoder.layers.3.mlp.Wi.weight")) < 1e-4


@pytest.mark.parametrize("dropout", [0.0, 0.3])
def test_tiny_training_mode_matches_the_oracle(ctx, dropout):
    """Training mode regenerates the same counter-RNG masks as the oracle (bit-exact integer work),
    so GPU and oracle gradients agree to fp32 rounding."""
    from laya_amd.model import TrainableDecisionModel
    m = TrainableDecisionModel.from_directory(TINY, ctx)
    m.head_dropout = dropout
    o = oracle.OracleModel(tiny_config())
    o.set_params(tiny_params())
    o.set_trainable_encoder_layers(None)
    o.set_head_dropout(dropout)
    batch, coeff, _ = tiny_batch()
    seed = 12345
    lg = m.forward(batch, training=True, seed=seed)
    lo = o.forward(batch, training=True, keep_tape=True, seed=seed)
    assert np.abs(lg - lo).max() < 1e-5
    m.backward(coeff)
    o.backward(coeff)
    for name in m.names:
        if name == "temperature" or name.startswith("act_head"):
            continue
        assert rel_l2(o.grad(name), m.grad(name)) < 1e-4, name


def _mid_case(layers=3, lengths=(300, 200, 129, 64, 17), seed=0, std=0.02):
    mc = mid_config(layers=layers)
    o = oracle.OracleModel(mc)
    params = random_params(o.shapes, seed, std=std)
    rng = np.random.default_rng(seed + 1)
    batch = mixed_batch(rng, list(lengths), mc.encoder.vocab_size)
    return mc, o, params, batch


def test_modernbert_base_width_gradients_match_the_oracle(ctx):
    """d = 768, 12 heads × 64, GeGLU 1152, 3 layers (global θ 160000, then sliding ±64 θ 10000),
    5 ragged segments (longer and shorter than the window), head dropout 0.1 in training mode.

    The head's ReLU makes the gradient discontinuous: a pre-activation within fp32 rounding of zero
    can flip between any two fp32 implementations. So each tensor is held to the exact (fp64 oracle)
    result at max(1e-4, 4 × the error of the reference-faithful fp32 oracle itself)."""
    from laya_amd.model import TrainableDecisionModel
    print("model: d=768, 3 layers (global, sliding, sliding), 5 ragged segments", flush=True)
    mc, o, params, batch = _mid_case()
    o64 = oracle.OracleModel(mc, double=True)
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    m.head_dropout = 0.1
    rng = np.random.default_rng(7)
    dlogits = rng.standard_normal(batch.n_markers).astype(np.float32)
    for ref in (o, o64):
        ref.set_params(params)
        ref.set_head_dropout(0.1)
        ref.forward(batch, training=True, keep_tape=True, seed=99)
        ref.backward(dlogits)
    lg = m.forward(batch, training=True, seed=99)
    assert rel_l2(o64.forward(batch, training=True, keep_tape=False, seed=99), lg) < 1e-5
    m.backward(dlogits)
    worst = 0.0
    for name in m.names:
        if name == "temperature" or name.startswith("act_head"):
            continue
        exact = o64.grad(name)
        bar = max(1e-4, 4 * rel_l2(exact, o.grad(name)))
        r = rel_l2(exact, m.grad(name))
        worst = max(worst, r)
        assert r < bar, (name, r, bar)
    print(f"worst relative L2 vs fp64 over {len(m.names)} tensors: {worst:.2e}", flush=True)


def test_wide_tile_forward_matches_the_oracle(ctx):
    """4448 tokens at d = 768: the QKV projection (RoPE in its epilogue, no bias: qkv's magnitude is a bound
    folded in before the epilogue) runs on 256 × 256 tiles and the GeGLU input projection with GeGLU in its
    epilogue (both asserted from the live profile); the logits match the fp64 oracle to 1e-5, and every gradient
    of a backward that reads those activations (attention reads qkv's magnitude word) is within max(1e-4, 4 ×
    the fp32 oracle's error) of fp64."""
    from laya_amd.model import TrainableDecisionModel
    print("model: d=768, 1 global layer, 4448 tokens", flush=True)
    mc, o, params, batch = _mid_case(layers=1, lengths=(2048, 1500, 900))
    o64 = oracle.OracleModel(mc, double=True)
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    dlogits = np.random.default_rng(6).standard_normal(batch.n_markers).astype(np.float32)
    for ref in (o, o64):
        ref.set_params(params)
        ref.forward(batch, training=False, keep_tape=True)
        ref.backward(dlogits)
    ctx.profile_begin()
    lg = m.forward(batch, training=False)
    prof = ctx.profile_end()
    assert prof.get("gemm_nt_h2w", {}).get("launches", 0) >= 2, sorted(prof)
    assert any(k.startswith("gemm_nt_geglu_") for k in prof) and "geglu_fwd" not in prof, sorted(prof)
    assert rel_l2(o64.forward(batch, training=False, keep_tape=False), lg) < 1e-5
    m.backward(dlogits)
    worst = 0.0
    for name in m.names:
        if name == "temperature" or name.startswith("act_head"):
            continue
        exact = o64.grad(name)
        bar = max(1e-4, 4 * rel_l2(exact, o.grad(name)))
        r = rel_l2(exact, m.grad(name))
        worst = max(worst, r)
        assert r < bar, (name, r, bar)
    print(f"worst relative L2 vs fp64 over {len(m.names)} tensors: {worst:.2e}", flush=True)


def test_biased_encoder_on_wide_tiles_gradients_match_the_oracle(ctx):
    """ModernBERT's optional biases (attention_bias, mlp_bias, norm_bias: ModernBertConfig) at 4448 tokens,
    d = 768, one global layer: the QKV projection (bias, then RoPE, in its epilogue) takes 256 × 256 tiles, the
    GeGLU input projection has bias, then GeGLU, in its epilogue, and qkv's magnitude for the two-piece
    attention is measured after the biased product. Logits to 1e-5 and every gradient to max(1e-4, 4 × the
    fp32 oracle's error) of fp64."""
    from laya_amd.model import TrainableDecisionModel
    print("model: d=768, 1 global layer with biases, 4448 tokens", flush=True)
    mc = mid_config(layers=1)
    mc.encoder.attention_bias = mc.encoder.mlp_bias = mc.encoder.norm_bias = True
    o = oracle.OracleModel(mc)
    params = random_params(o.shapes, 3, std=0.02)
    batch = mixed_batch(np.random.default_rng(4), [2048, 1500, 900], mc.encoder.vocab_size)
    o64 = oracle.OracleModel(mc, double=True)
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    assert any(n.endswith("attn.Wqkv.bias") for n in m.names), m.names
    dlogits = np.random.default_rng(5).standard_normal(batch.n_markers).astype(np.float32)
    for ref in (o, o64):
        ref.set_params(params)
        ref.forward(batch, training=True, keep_tape=True, seed=11)
        ref.backward(dlogits)
    ctx.profile_begin()
    lg = m.forward(batch, training=True, seed=11)
    prof = ctx.profile_end()
    assert prof.get("gemm_nt_h2w", {}).get("launches", 0) >= 2, sorted(prof)
    assert any(k.startswith("gemm_nt_geglu_") for k in prof) and "geglu_fwd" not in prof, sorted(prof)
    assert rel_l2(o64.forward(batch, training=True, keep_tape=False, seed=11), lg) < 1e-5
    m.backward(dlogits)
    worst = 0.0
    for name in m.names:
        if name == "temperature" or name.startswith("act_head"):
            continue
        exact = o64.grad(name)
        bar = max(1e-4, 4 * rel_l2(exact, o.grad(name)))
        r = rel_l2(exact, m.grad(name))
        worst = max(worst, r)
        assert r < bar, (name, r, bar)
    print(f"worst relative L2 vs fp64 over {len(m.names)} tensors: {worst:.2e}", flush=True)


@pytest.mark.parametrize("inter,lengths", [(1100, (2048, 1500, 900)), (1000, (2000, 2000, 1500, 1500))])
def test_geglu_fused_product_on_partial_tiles_matches_the_oracle(ctx, inter, lengths):
    """The GeGLU input product with GeGLU in its epilogue where neither its rows nor its output columns fill the
    last tile: GeGLU widths of 1100 and 1000 (128-column tiles end part-way), with mlp_bias, at 4448 and 7000
    tokens (the 192 x 256 and the 256 x 256 kernels on 256 CUs). Logits to 1e-5 and every gradient (the backward reads
    GeGLU's stored input and output) to max(1e-4, 4 × the fp32 oracle's error) of fp64."""
    from laya_amd.model import TrainableDecisionModel
    print(f"model: d=768, 1 global layer, GeGLU {inter}, {sum(lengths)} tokens", flush=True)
    mc = mid_config(layers=1, inter=inter)
    mc.encoder.mlp_bias = True
    o = oracle.OracleModel(mc)
    params = random_params(o.shapes, 7, std=0.02)
    batch = mixed_batch(np.random.default_rng(8), list(lengths), mc.encoder.vocab_size)
    o64 = oracle.OracleModel(mc, double=True)
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    dlogits = np.random.default_rng(9).standard_normal(batch.n_markers).astype(np.float32)
    for ref in (o, o64):
        ref.set_params(params)
        ref.forward(batch, training=True, keep_tape=True, seed=13)
        ref.backward(dlogits)
    ctx.profile_begin()
    lg = m.forward(batch, training=True, seed=13)
    prof = ctx.profile_end()
    fused = sorted(k for k in prof if k.startswith("gemm_nt_geglu_"))
    print(f"fused GeGLU products: {fused}", flush=True)
    assert fused and "geglu_fwd" not in prof, sorted(prof)
    assert rel_l2(o64.forward(batch, training=True, keep_tape=False, seed=13), lg) < 1e-5
    m.backward(dlogits)
    worst = 0.0
    for name in m.names:
        if name == "temperature" or name.startswith("act_head"):
            continue
        exact = o64.grad(name)
        bar = max(1e-4, 4 * rel_l2(exact, o.grad(name)))
        r = rel_l2(exact, m.grad(name))
        worst = max(worst, r)
        assert r < bar, (name, r, bar)
    print(f"worst relative L2 vs fp64 over {len(m.names)} tensors: {worst:.2e}", flush=True)
    m.close()


def test_full_train_step_matches_the_oracle(ctx):
    """fwd → soft-CE gradient → bwd → clip → AdamW (Trainer.cs:131-144). The gradients of the forward and
    backward are held directly to the fp64 oracle (max(1e-4, 4 × the fp32 oracle's error)); then the fused
    train_step, run from the same weights, must leave exactly the weights that the reference's clip and AdamW
    formulas (AdamW.cs:29-73, 103-130) give when applied on the host to those GPU gradients.

    The logit gradient of the separate backward is the device's soft-CE kernel's (the fused step's own), held
    to the oracle's at fp32 rounding: the two exponentials (the device's expf and the host's) may differ in the
    last bit, and AdamW's first step, g / (|g| + ε), turns a last-bit difference in a gradient within a few ε
    of zero into a visible weight difference."""
    from laya_amd.device import DeviceArray
    from laya_amd.model import TrainableDecisionModel
    import laya_amd.ops as laya
    mc, o, params, batch = _mid_case(layers=2, lengths=(150, 90, 33))
    o64 = oracle.OracleModel(mc, double=True)
    rng = np.random.default_rng(3)
    targets = np.concatenate([np.eye(k, dtype=np.float32)[rng.integers(k)] for k in batch.n_options])
    seed, lr, scale = 5, 3e-3, float(batch.n_items)
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    lg = m.forward(batch, training=True, seed=seed)
    ce, g = oracle.cross_entropy(batch.n_options, lg, targets, 1.0, scale)
    offsets = np.concatenate([[0], np.cumsum(batch.n_options)]).astype(np.int32)
    gd = DeviceArray.from_numpy(ctx, np.zeros_like(lg))
    laya.softmax_ce_backward(ctx, DeviceArray.from_numpy(ctx, lg), DeviceArray.from_numpy(ctx, targets),
                             DeviceArray.from_numpy(ctx, offsets), len(batch.n_options), 1.0, scale, gd)
    g_device = gd.numpy()
    assert np.abs(g_device - g).max() <= 4 * np.finfo(np.float32).eps * np.abs(g).max()
    m.backward(g_device)
    for ref in (o, o64):
        ref.set_params(params)
        ref.forward(batch, training=True, keep_tape=True, seed=seed)
        ref.backward(g)
    trained = [name for name in m.names if m.has_grad(name)]
    assert trained == [name for name in m.names if o64.has_grad(name)]
    grads = {}
    for name in trained:
        exact, grads[name] = o64.grad(name), m.grad(name)
        if name == "scorer.3.bias":
            # Σ of the soft-CE gradient over every option, exactly 0: rounding noise of that sum, which no
            # relative error describes.
            noise = 8 * np.finfo(np.float32).eps * np.abs(g_device).sum()
            assert np.abs(grads[name] - exact).max() <= noise, (name, grads[name], exact, noise)
            continue
        bar = max(1e-4, 4 * rel_l2(exact, o.grad(name)))
        assert rel_l2(exact, grads[name]) < bar, (name, rel_l2(exact, grads[name]), bar)
    m.close()
    # The fused step from the same weights.
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    loss_gpu = m.train_step(batch, targets, seed, loss_scale=scale, max_norm=1.0, lr_encoder=lr, lr_head=lr,
                            want_loss=True)
    assert abs(loss_gpu - ce) < 1e-5 * max(1.0, abs(ce))
    clipped = {name: grads[name].copy() for name in trained}
    oracle.clip(list(clipped.values()), 1.0)  # scales the copies in place
    for name in m.names:
        w = params[name].astype(np.float32).reshape(-1).copy()
        if m.trainable(name):
            gr = clipped[name].reshape(-1) if name in clipped else np.zeros_like(w)
            oracle.adamw_tensor(w, np.ascontiguousarray(gr), np.zeros_like(w), np.zeros_like(w), lr, 1)
        got = m.param(name).reshape(-1)
        if name == "scorer.3.bias":
            # Σ over an item's options of the soft-CE gradient is exactly 0, so this bias's gradient is rounding
            # noise on either side and Adam's first step moves it by up to lr in either direction.
            assert np.abs(got - params[name].reshape(-1)).max() <= lr * 1.01
            continue
        assert np.abs(got - w).max() <= 1e-6 * max(1.0, np.abs(w).max()), name
    # The step cleared the gradients.
    assert not np.any(m.grad("scorer.1.weight"))
    m.close()


def test_full_modernbert_base_step_at_4x128_matches_the_oracle(ctx):
    """The CPU-runnable configuration at full model size: ModernBERT-base (22 layers, vocab 50368,
    164M parameters) plus the decision head, 4 sequences × 128 tokens without padding, ids U[0, 50368),
    one choice head with K = 5 per item, labels U[0, 5), mean CE, head dropout 0.1, weights N(0, 0.02).

    Every gradient before the clip is held to the fp64 oracle at max(1e-4, 4 × the fp32 oracle's own
    distance), and to the reference's max|Δ|/max|g| < 1e-4 (TrainingGradientTests.cs:58-85); then the
    clip and AdamW step on both sides give the same weights."""
    from laya_amd.batch import Batch
    from laya_amd.config import modernbert_base
    from laya_amd.model import TrainableDecisionModel
    print("model: ModernBERT-base 22 layers, 4 x 128 tokens, gradients and one step", flush=True)
    mc = modernbert_base()
    o = oracle.OracleModel(mc)
    params = random_params(o.shapes, 11, std=0.02)
    rng = np.random.default_rng(12)
    n, L, K = 4, 128, 5
    batch = Batch(lengths=np.full(n, L, np.int32), tokens=rng.integers(0, 50368, n * L).astype(np.int32),
                  n_options=np.full(n, K, np.int32), markers=np.tile(1 + 2 * np.arange(K), n).astype(np.int32),
                  qtypes=np.zeros(n, np.int32))
    targets = np.concatenate([np.eye(K, dtype=np.float32)[rng.integers(K)] for _ in range(n)])
    seed, lr = 21, 1e-3
    o64 = oracle.OracleModel(mc, double=True)
    for r in (o64, o):
        r.set_params(params)
        r.set_head_dropout(0.1)
    logits64 = o64.forward(batch, training=True, keep_tape=True, seed=seed)
    ce, g = oracle.cross_entropy(batch.n_options, logits64.astype(np.float32), targets, 1.0, 1.0)
    o64.backward(g)
    o.forward(batch, training=True, keep_tape=True, seed=seed)
    o.backward(g)
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    m.head_dropout = 0.1
    lg = m.forward(batch, training=True, seed=seed)
    assert np.abs(lg - logits64).max() < 1e-5
    m.backward(g)
    worst = (0.0, "")
    for name in m.names:
        assert m.has_grad(name) == o64.has_grad(name), name
        if not m.has_grad(name):
            continue
        exact, got = o64.grad(name), m.grad(name)
        bar = max(1e-4, 4 * rel_l2(exact, o.grad(name)))
        r = rel_l2(exact, got)
        assert r < bar, (name, r, bar)
        # The reference's metric, with the same floor: an exact gradient that is rounding noise (the output
        # bias's: softmax gradients sum to zero per item) is noise in every fp32 implementation.
        mbar = max(1e-4, 4 * max_rel(exact, o.grad(name)))
        assert max_rel(exact, got) < mbar, (name, max_rel(exact, got), mbar)
        if bar == 1e-4:
            worst = max(worst, (r, name))
    print(f"4 x 128: worst gradient rel-L2 vs fp64 {worst[0]:.2e} ({worst[1]}) among the tensors whose fp32-oracle "
          "error is below 2.5e-5", flush=True)
    # Clip and AdamW (Trainer.cs:138-141) on the GPU's own gradients, against the reference's formulas
    # applied on the host to those same gradients: the step's arithmetic, separated from the gradient
    # comparison above (Adam's first step moves each weight by ≈ ±lr whatever the gradient's size, so a
    # gradient that is rounding noise on both sides, such as the output bias's, has no stable sign).
    trained = [name for name in m.names if m.has_grad(name)]
    grads = {name: m.grad(name) for name in trained}
    norm_gpu = m.clip_grad_norm(1.0)
    norm_host = oracle.clip([grads[name] for name in trained], 1.0)
    assert abs(norm_gpu - norm_host) < 1e-9 * norm_host
    m.adamw_step(lr, lr)
    for name in m.names:
        w = params[name].astype(np.float32).reshape(-1).copy()
        if m.trainable(name):
            g = grads[name].reshape(-1) if name in grads else np.zeros_like(w)
            oracle.adamw_tensor(w, np.ascontiguousarray(g), np.zeros_like(w), np.zeros_like(w), lr, 1)
        got = m.param(name).reshape(-1)
        assert np.abs(got - w).max() <= 1e-6 * max(1.0, np.abs(w).max()), name
    m.close()


def test_gradients_are_bitwise_deterministic(ctx):
    from laya_amd.model import TrainableDecisionModel
    mc, o, params, batch = _mid_case(layers=2, lengths=(256, 100))
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    d = np.random.default_rng(1).standard_normal(batch.n_markers).astype(np.float32)
    runs = []
    for _ in range(2):
        m.zero_gradients()
        m.forward(batch, training=True, seed=4)
        m.backward(d)
        runs.append({n: m.grad(n) for n in ("encoder.layers.0.attn.Wqkv.weight", "encoder.embeddings.norm.weight",
                                             "encoder.embeddings.tok_embeddings.weight", "type_emb.weight")})
    for n in runs[0]:
        np.testing.assert_array_equal(runs[0][n], runs[1][n])


def test_out_of_vocabulary_token_is_rejected_before_any_math(ctx):
    from laya_amd._native import LayaOutOfRangeError
    from laya_amd.batch import Batch
    from laya_amd.model import TrainableDecisionModel
    m = TrainableDecisionModel.from_directory(TINY, ctx)
    bad = Batch(lengths=np.array([3], np.int32), tokens=np.array([1, 97, 2], np.int32),
                n_options=np.array([1], np.int32), markers=np.array([0], np.int32), qtypes=np.array([0], np.int32))
    with pytest.raises(LayaOutOfRangeError):
        m.forward(bad)


def test_staged_batches_train_exactly_like_batches_passed_by_value(ctx):
    """A staged batch (validated and uploaded once) gives the same step as the batch passed by value:
    same kernels on the same inputs, so identical losses and weights; two staged batches alternate;
    a released slot is refused; staging validates like train_step."""
    from laya_amd._native import LayaOutOfRangeError
    from laya_amd.batch import Batch
    from laya_amd.model import TrainableDecisionModel
    mc, o, params, batch = _mid_case(layers=2, lengths=(150, 90, 33))
    _, _, _, batch2 = _mid_case(layers=2, lengths=(64, 200), seed=3)
    rng = np.random.default_rng(3)
    t1 = np.concatenate([np.eye(k, dtype=np.float32)[rng.integers(k)] for k in batch.n_options])
    t2 = np.concatenate([np.eye(k, dtype=np.float32)[rng.integers(k)] for k in batch2.n_options])
    a = TrainableDecisionModel(mc, ctx)
    b = TrainableDecisionModel(mc, ctx)
    a.set_params(params)
    b.set_params(params)
    s1, s2 = b.stage_batch(batch, t1), b.stage_batch(batch2, t2)
    kw = dict(max_norm=1.0, lr_encoder=1e-3, lr_head=1e-3)
    for seed, (bt, tt, slot) in enumerate([(batch, t1, s1), (batch2, t2, s2), (batch, t1, s1)]):
        la = a.train_step(bt, tt, seed, loss_scale=float(bt.n_items), want_loss=True, **kw)
        lb = b.train_step_staged(slot, seed, loss_scale=float(bt.n_items), want_loss=True, **kw)
        assert la == lb
    for name in a.names:
        np.testing.assert_array_equal(a.param(name), b.param(name))
    b.release_batch(s1)
    with pytest.raises(ValueError):
        b.train_step_staged(s1, 0)
    bad = Batch(lengths=np.array([3], np.int32), tokens=np.array([1, mc.encoder.vocab_size, 2], np.int32),
                n_options=np.array([1], np.int32), markers=np.array([0], np.int32), qtypes=np.array([0], np.int32))
    with pytest.raises(LayaOutOfRangeError):
        b.stage_batch(bad, np.ones(1, np.float32))
    b.release_batch(s2)


def test_rlcd_step_on_the_device_matches_the_host_objective(ctx):
    """Forward → RLCD objective on the device → backward from the device gradient gives the gradients of
    forward → the oracle's objective on the host logits → backward (Trainer.cs:134-137)."""
    from laya_amd.model import TrainableDecisionModel
    mc, o, params, batch = _mid_case(layers=2, lengths=(150, 90, 33))
    rng = np.random.default_rng(4)
    targets = np.concatenate([rng.dirichlet(np.ones(k)) for k in batch.n_options]).astype(np.float32)
    draws = rng.standard_normal((4, batch.n_markers))
    a = TrainableDecisionModel(mc, ctx)
    b = TrainableDecisionModel(mc, ctx)
    a.set_params(params)
    b.set_params(params)
    logits = a.forward(batch, training=True, seed=6)
    losses = a.objective_rlcd(targets, draws, 0.3, scale=0.5)
    a.backward_from_objective()
    b.forward(batch, training=True, seed=6)
    out, g = oracle.rlcd(batch.n_options, batch.qtypes, logits, targets, draws.reshape(-1), 0.3, scale=0.5)
    np.testing.assert_allclose(losses, out, rtol=1e-5, atol=1e-6)
    b.backward(g)
    for name in a.names:
        if b.has_grad(name):
            # The output bias gradient is Σ dlogits, exactly 0 (softmax gradients sum to zero per item):
            # both sides hold rounding noise there, hence the absolute floor.
            want, got = b.grad(name), a.grad(name)
            assert np.linalg.norm(got - want) <= 1e-5 * np.linalg.norm(want) + 1e-6, name


def _clear_of_the_relu(params, mc, seed):
    """Moves every head linear1 bias to ±5 × the RMS of its product (random sign per unit): no ReLU input
    then lies anywhere near zero, while the ReLU still masks about half the units.

    The head's ReLU is the model's one discontinuity. With ~10⁶ ReLU inputs drawn around zero, a few lie
    within fp32 rounding of it, and any two fp32 implementations (the reference-faithful fp32 oracle
    included) land some on different sides now and then, which moves every gradient below by up to ~1e-3
    (measured: 1–3 of 8 seeds for each implementation). Away from zero the step is a smooth function of the
    inputs and fp32 implementations agree to their rounding."""
    rng = np.random.default_rng(seed + 100)
    scale = 5.0 * 0.02 * np.sqrt(mc.encoder.hidden_size)  # weights N(0, 0.02) on unit-scale normed inputs
    for j in range(mc.head_layers):
        name = f"head.layers.{j}.linear1.bias"
        params[name] = (scale * rng.choice([-1.0, 1.0], params[name].shape)).astype(np.float32)
    return params


def _large_shape_case(ctx, mc, trainable, lengths, seed, zipf=0.0):
    """One training-mode forward/backward (head dropout 0.1) of a checkpoint-sized shape on the GPU and on the
    oracle (fp64 = exact, and fp32), weights N(0, 0.02) with non-trivial norms and the head ReLU's inputs
    clear of zero. Each gradient is held to the reference test's tolerance (TrainingGradientTests.cs:205-214:
    max|Δ|/max|g| < 1e-3, cosine > 0.99999) and to the fp32 bar, rel-L2 ≤ max(1e-4, 4 × the fp32 oracle's)."""
    from laya_amd.batch import synthetic_batch
    from laya_amd.model import TrainableDecisionModel
    o32 = oracle.OracleModel(mc)
    params = _clear_of_the_relu(random_params(o32.shapes, seed, std=0.02), mc, seed)
    rng = np.random.default_rng(seed + 1)
    opts = [(8, 4, 2)[i % 3] for i in range(len(lengths))]
    batch = synthetic_batch(rng, lengths, opts, [i % 3 for i in range(len(lengths))], mc.encoder.vocab_size, zipf)
    dlogits = rng.standard_normal(batch.n_markers).astype(np.float32)
    o64 = oracle.OracleModel(mc, double=True)
    for r in (o32, o64):
        r.set_params(params)
        r.set_head_dropout(0.1)
        r.set_trainable_encoder_layers(trainable)
        logits_o = r.forward(batch, training=True, keep_tape=True, seed=seed)
        r.backward(dlogits)
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    m.head_dropout = 0.1
    m.set_trainable_encoder_layers(trainable)
    logits_m = m.forward(batch, training=True, seed=seed)
    m.backward(dlogits)
    assert np.abs(logits_o - logits_m).max() < 1e-3
    checked, worst = 0, (0.0, "")
    for name in m.names:
        assert m.has_grad(name) == o64.has_grad(name), name
        if not m.has_grad(name) or name == "scorer.3.bias":
            continue
        exact, ref32, got = o64.grad(name), o32.grad(name), m.grad(name)
        cos = float(np.dot(exact.ravel(), got.ravel().astype(np.float64)) /
                    max(np.linalg.norm(exact) * np.linalg.norm(got), 1e-300))
        assert cos > 0.99999, (name, cos)
        assert max_rel(exact, got) < 1e-3, (name, max_rel(exact, got))
        e = rel_l2(exact, got)
        assert e < max(1e-4, 4 * rel_l2(exact, ref32)), (name, e)
        worst = max(worst, (e, name))
        checked += 1
    print(f"worst gradient rel-L2 {worst[0]:.1e} ({worst[1]})", flush=True)
    m.close()
    return checked


def test_modernbert_large_gradients_match_the_oracle(ctx):
    """The English / TypedDecisions checkpoint shape (ModernBERT-large: 28 layers, d 1024, 16 heads,
    GeGLU 2624, 421M parameters with the head), all layers trainable, 2 sequences of 160 and 96 tokens."""
    from laya_amd.config import modernbert_large
    print("model: ModernBERT-large 28 layers, 2 sequences", flush=True)
    n = _large_shape_case(ctx, modernbert_large(), None, [160, 96], 71)
    assert n >= 195  # 28 layers × 6 tensors (layer 0: 5), embeddings, final norm, head, scorer


def test_partial_training_of_the_top_layers_at_large_shape(ctx):
    """SetTrainableEncoderLayers(4) (TrainableDecisionModel.cs:206-231) on the large shape: only the top
    four layers, the final norm and the head get gradients, and those match the oracle."""
    from laya_amd.config import modernbert_large
    print("model: ModernBERT-large, top 4 layers trainable", flush=True)
    n = _large_shape_case(ctx, modernbert_large(), 4, [140, 70, 33], 72)
    assert 30 < n < 100


def test_mmbert_base_gradients_match_the_oracle(ctx):
    """The Multilingual checkpoint shape (mmBERT-base: ModernBERT-base widths, 256,000-token vocabulary),
    Zipf(1.1) ids so embedding rows repeat."""
    from laya_amd.config import mmbert_base
    print("model: mmBERT-base 22 layers, vocab 256000", flush=True)
    _large_shape_case(ctx, mmbert_base(), None, [120, 64, 40], 73, zipf=1.1)


def test_readout_matches_the_oracle_on_the_fixture(ctx):
    """DecisionModel.ReadOut on the device (DecisionModel.cs:170-226): with the fixture's trained scorer and act
    head, the option logits, the four calibration features and the action probabilities of every item match
    the oracle's read-out (fp64) to fp32 rounding; decide() = eval forward + read-out."""
    from laya_amd.model import TrainableDecisionModel
    m = TrainableDecisionModel.from_directory(TINY, ctx)
    batch, _, torch_logits = tiny_batch()
    o = oracle.OracleModel(tiny_config(), double=True)
    o.set_params(tiny_params())
    o.forward(batch, training=False)
    probs_o, feats_o, _ = o.readout()
    m.forward(batch, training=False)
    logits, probs, feats = m.readout()
    np.testing.assert_allclose(np.concatenate(logits), torch_logits, atol=1e-4)
    np.testing.assert_allclose(feats, feats_o, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(probs, probs_o, rtol=1e-5, atol=1e-6)
    out = m.decide(batch)
    assert len(out) == batch.n_items
    for i, (lg, p) in enumerate(out):
        np.testing.assert_array_equal(lg, logits[i])
        np.testing.assert_array_equal(p, probs[i])
    m.close()


def test_readout_at_modernbert_base_width(ctx):
    """d = 768 (act-head input 772, hidden 256), items with K = 8, 4, 2 and 1 option, random weights, after a
    training-mode forward (the read-out takes whatever the last forward left)."""
    from laya_amd.batch import synthetic_batch
    from laya_amd.model import TrainableDecisionModel
    mc = mid_config(layers=2)
    o = oracle.OracleModel(mc)
    params = random_params(o.shapes, 31, std=0.05)
    rng = np.random.default_rng(32)
    batch = synthetic_batch(rng, [120, 77, 40, 9, 33], [8, 4, 2, 1, 3], [0, 1, 2, 0, 1], mc.encoder.vocab_size)
    o64 = oracle.OracleModel(mc, double=True)
    o64.set_params(params)
    o64.forward(batch, training=True, seed=5)
    probs_o, feats_o, _ = o64.readout()
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    m.forward(batch, training=True, seed=5)
    logits, probs, feats = m.readout()
    # Against fp64 the forward's own fp32 error (≈ 1e-6 of the logits) carries through; the margin top1 − top2
    # is a difference of two probabilities, hence the absolute bar.
    np.testing.assert_allclose(feats, feats_o, atol=1e-5)
    np.testing.assert_allclose(probs, probs_o, atol=1e-5)
    # The feature arithmetic itself, on the device's own logits, to fp32 rounding.
    for i, lg in enumerate(logits):
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        k = max(2, len(lg))
        srt = np.sort(p)[::-1]
        want = [srt[0], srt[0] - (srt[1] if len(lg) > 1 else 0.0),
                -np.sum(p * np.log(np.maximum(p, 1e-9))) / np.log(k), k / 255.0]
        np.testing.assert_allclose(feats[i], want, atol=2e-7)
    assert feats[3, 2] == 0.0 and abs(feats[3, 0] - 1.0) < 1e-7  # K = 1: p = 1, entropy 0
    m.close()


def test_readout_act_head_wiring_in_closed_form(ctx):
    """The device read-out against closed forms (tests/helpers.closed_form_readout_case; the same case pins the
    oracle in tests/test_oracle_readout.py): the act head wired to pass one input slot through GELU, so
    log(p0/p1) = GELU(slot value) for pooled columns of h[start] and the four features in order."""
    from scipy.special import erf

    from helpers import READOUT_SLOTS, act_head_selecting, closed_form_readout_case
    from laya_amd.model import TrainableDecisionModel
    mc, params, batch, expected = closed_form_readout_case()
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    m.forward(batch, training=False)
    for slot in READOUT_SLOTS:
        m.set_params(act_head_selecting(params, slot))
        _, probs, feats = m.readout()
        got = np.log(probs[:, 0].astype(np.float64) / probs[:, 1])
        x = expected[:, slot]
        np.testing.assert_allclose(got, 0.5 * x * (1.0 + erf(x / np.sqrt(2.0))), atol=2e-6, err_msg=f"slot {slot}")
    np.testing.assert_allclose(feats, expected[:, 64:], atol=1e-6)
    m.close()


def test_backward_keeps_precision_for_items_with_tiny_logit_gradients(ctx):
    """An item whose logit gradients sit 1e-9 below the others' (a confidently right item under a summed CE):
    every activation-gradient row of that item is ≈1e-9 of the largest, below what a two-piece product's
    tensor-wide scale represents to fp32 precision. The backward sees the span in the logit gradients and runs
    its products on three-piece splits; the embedding-gradient rows of tokens only that item holds (tiny, and
    outputs of the dX chain) then match fp64 row by row to 1e-4, and every gradient to the usual bar. With the
    span removed the two-piece products run again."""
    from helpers import fixture_params
    from laya_amd.batch import Batch
    from laya_amd.model import TrainableDecisionModel
    mc = mid_config(layers=2)
    o = oracle.OracleModel(mc)
    params = fixture_params(o.shapes, 17)
    rng = np.random.default_rng(18)
    lengths = [200, 150, 90]
    opts = [8, 4, 2]
    # The last item's tokens come from ids [900, 1000), the others' from [0, 900).
    tokens = np.concatenate([rng.integers(0, 900, 200), rng.integers(0, 900, 150), rng.integers(900, 1000, 90)])
    batch = Batch(lengths=np.array(lengths, np.int32), tokens=tokens.astype(np.int32),
                  n_options=np.array(opts, np.int32),
                  markers=np.concatenate([1 + 2 * np.arange(k) for k in opts]).astype(np.int32),
                  qtypes=np.array([0, 1, 2], np.int32))
    dl = rng.standard_normal(batch.n_markers).astype(np.float32)
    dl[-2:] *= np.float32(1e-9)
    o64 = oracle.OracleModel(mc, double=True)
    for ref in (o, o64):
        ref.set_params(params)
        ref.forward(batch, training=False, keep_tape=True)
        ref.backward(dl)
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    m.forward(batch, training=False)
    ctx.profile_begin()
    m.backward(dl)
    prof = ctx.profile_end()
    assert m.backward_fell_back
    assert not any(k.endswith(("_h2w", "_h2t", "_h2")) and k.startswith(("gemm_bwd", "attention_bwd"))
                   for k in prof), sorted(prof)
    emb = "encoder.embeddings.tok_embeddings.weight"
    exact, got = o64.grad(emb), m.grad(emb)
    only_small = np.unique(tokens[-90:])
    num = np.linalg.norm(exact[only_small] - got[only_small], axis=1)
    den = np.linalg.norm(exact[only_small], axis=1)
    assert den.max() < 1e-6 * np.linalg.norm(exact[:900], axis=1).max()  # the rows really are tiny
    print(f"tiny item's embedding rows: worst row relative error {float((num / den).max()):.2e}", flush=True)
    assert (num / den).max() < 1e-4
    for name in m.names:
        if name == "temperature" or name.startswith("act_head"):
            continue
        e = o64.grad(name)
        bar = max(1e-4, 4 * rel_l2(e, o.grad(name)))
        assert rel_l2(e, m.grad(name)) < bar, name
    m.zero_gradients()
    dl2 = rng.standard_normal(batch.n_markers).astype(np.float32)
    m.backward(dl2)
    assert not m.backward_fell_back
    m.close()


def test_adamw_step_folds_the_weights_magnitudes_exactly(ctx):
    """The AdamW step folds each updated product weight's max|w| into its magnitude word, so the next forward
    measures nothing: its logits and gradients are bitwise those of a forward that measured the same weights
    afresh (the weights written back unchanged from the host, which clears every word)."""
    from laya_amd.model import TrainableDecisionModel
    mc, o, params, batch = _mid_case(layers=2, lengths=(150, 90, 33))
    m = TrainableDecisionModel(mc, ctx)
    m.set_params(params)
    rng = np.random.default_rng(9)
    targets = np.concatenate([np.eye(k, dtype=np.float32)[rng.integers(k)] for k in batch.n_options])
    d = rng.standard_normal(batch.n_markers).astype(np.float32)
    for step in range(2):
        m.train_step(batch, targets, 40 + step, loss_scale=float(batch.n_items), lr_encoder=1e-3, lr_head=1e-3)
    ctx.profile_begin()
    folded = m.forward(batch, training=True, seed=3)
    prof_folded = ctx.profile_end()
    m.zero_gradients()
    m.backward(d)
    g_folded = {n: m.grad(n) for n in m.names if m.has_grad(n)}
    m.set_params({n: m.param(n) for n in m.names})  # unchanged values; the words are measured again
    m.zero_gradients()
    ctx.profile_begin()
    measured = m.forward(batch, training=True, seed=3)
    prof_measured = ctx.profile_end()
    m.backward(d)
    # The forward after the step skips the one launch that measures every weight.
    launches = lambda p: p.get("absmax", {}).get("launches", 0)  # noqa: E731
    assert launches(prof_folded) == launches(prof_measured) - 1, (prof_folded.get("absmax"), prof_measured["absmax"])
    np.testing.assert_array_equal(folded, measured)
    for n, g in g_folded.items():
        np.testing.assert_array_equal(g, m.grad(n), err_msg=n)
    m.close()
