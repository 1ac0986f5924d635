"""Layer checkpointing (TrainableDecisionModel.cs:61-64): the encoder layers keep only their inputs from
forward to backward and are recomputed, one at a time, just before their backward.

The recompute runs the same kernels on the same inputs, so the gradients must be bitwise those of the mode
that keeps every activation; the arena must shrink by the internals of every layer but one; and the
automatic mode must switch to recomputing when keeping everything would exceed the context's cap."""
import numpy as np
import pytest

from helpers import mid_config, mixed_batch, random_params

pytestmark = pytest.mark.gpu

LENGTHS = [300, 129, 64, 17, 211, 96]


@pytest.fixture(scope="module")
def ctx():
    from laya_amd.device import Context
    print("checkpointing tests: creating context on device 0", flush=True)
    c = Context(0)
    yield c
    c.close()


def _model(ctx, layers=4):
    from laya_amd.model import TrainableDecisionModel
    cfg = mid_config(layers=layers)
    m = TrainableDecisionModel(cfg, ctx)
    m.set_params(random_params(m.shapes, 31, std=0.03))
    return m, cfg


def _step(m, batch, d, mode, trainable=None):
    m.layer_checkpointing = mode
    m.set_trainable_encoder_layers(trainable)
    m.zero_gradients()
    logits = m.forward(batch, training=True, seed=9)
    m.backward(d)
    # After the backward every workspace of the step has grown to its size: the rest is the arena.
    return logits, {n: m.grad(n) for n in m.names if m.has_grad(n)}, m.ctx.memory_in_use()


@pytest.mark.parametrize("trainable", [None, 2])
def test_recomputed_layers_give_bitwise_the_same_gradients(ctx, trainable):
    print(f"checkpointing: keep vs recompute, trainable encoder layers {trainable}", flush=True)
    m, cfg = _model(ctx)
    batch = mixed_batch(np.random.default_rng(4), LENGTHS, cfg.encoder.vocab_size)
    d = np.random.default_rng(5).standard_normal(batch.n_markers).astype(np.float32)
    l0, g0, use0 = _step(m, batch, d, m.CHECKPOINT_KEEP, trainable)
    assert not m.recomputing
    l1, g1, use1 = _step(m, batch, d, m.CHECKPOINT_RECOMPUTE, trainable)
    assert m.recomputing and m.layer_checkpointing == m.CHECKPOINT_RECOMPUTE
    np.testing.assert_array_equal(l0, l1)
    assert sorted(g0) == sorted(g1)
    for n in g0:
        np.testing.assert_array_equal(g0[n], g1[n], err_msg=n)
    # A layer's internals per token: 7 rows of d floats (normed, qkv, context, residual, MLP input), 3 of the
    # intermediate width (wide, act), 4 LayerNorm statistics and one log-sum-exp per head.
    T, dm, inter, H = batch.n_tokens, cfg.encoder.hidden_size, cfg.encoder.intermediate_size, \
        cfg.encoder.num_attention_heads
    internals = 4 * T * (7 * dm + 3 * inter + 4 + H)
    assert use0 - use1 >= (cfg.encoder.num_hidden_layers - 1) * internals * 0.95, (use0, use1, internals)
    m.close()


def test_automatic_mode_recomputes_only_when_the_arena_would_not_fit(ctx):
    print("checkpointing: automatic mode under a memory cap", flush=True)
    m, cfg = _model(ctx)
    batch = mixed_batch(np.random.default_rng(6), LENGTHS, cfg.encoder.vocab_size)
    d = np.random.default_rng(7).standard_normal(batch.n_markers).astype(np.float32)
    assert m.layer_checkpointing == m.CHECKPOINT_AUTO
    _, g_full, _ = _step(m, batch, d, m.CHECKPOINT_AUTO)
    assert not m.recomputing  # no cap: everything is kept
    _, _, use_rc = _step(m, batch, d, m.CHECKPOINT_RECOMPUTE)
    _, _, use_full = _step(m, batch, d, m.CHECKPOINT_KEEP)
    assert use_full > use_rc
    # Between the two: the full arena no longer fits, the recomputing one does.
    ctx.set_memory_cap(use_rc + (use_full - use_rc) // 2)
    try:
        _, g_auto, _ = _step(m, batch, d, m.CHECKPOINT_AUTO)
        assert m.recomputing
        for n in g_full:
            np.testing.assert_array_equal(g_full[n], g_auto[n], err_msg=n)
        # Keeping everything under the same cap is refused with the context's memory error.
        from laya_amd._native import LayaError
        m.layer_checkpointing = m.CHECKPOINT_KEEP
        with pytest.raises(LayaError):
            m.forward(batch, training=True, seed=9)
    finally:
        ctx.set_memory_cap(0)
    m.close()


def test_the_mode_is_checked(ctx):
    from laya_amd._native import LayaError
    m, _ = _model(ctx, layers=1)
    with pytest.raises(LayaError):
        m.layer_checkpointing = 3
    m.layer_checkpointing = True
    assert m.layer_checkpointing == m.CHECKPOINT_RECOMPUTE
    m.close()
