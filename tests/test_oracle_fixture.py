"""The oracle against the reference's own golden vectors.

Ports TrainingGradientTests.cs (LogitsMatchPyTorch 44-56, EveryGradientMatchesPyTorch 58-85,
FreezingTheEncoderLeavesItsGradientsEmpty 87-106) and the objective / optimizer closed values of
TrainingTests.cs (19-83). These pin the oracle before it is trusted as the GPU checker.
"""
import numpy as np
import pytest

import oracle
from fixtures import max_rel, objective_fixture, rel_l2, tiny_batch, tiny_config, tiny_grads, tiny_params


def _run(double, trainable=None):
    m = oracle.OracleModel(tiny_config(), double=double)
    m.set_params(tiny_params())
    m.set_trainable_encoder_layers(trainable)
    batch, coeff, _ = tiny_batch()
    logits = m.forward(batch, training=False, keep_tape=True)
    m.backward(coeff)
    return m, logits


@pytest.mark.parametrize("double", [False, True])
def test_logits_match_pytorch(double):
    _, logits = _run(double)
    _, _, torch_logits = tiny_batch()
    assert np.abs(logits - torch_logits).max() < 1e-4


@pytest.mark.parametrize("double", [False, True])
def test_every_gradient_matches_pytorch(double):
    m, _ = _run(double)
    grads = tiny_grads()
    assert len(grads) == 57
    for name, expected in grads.items():
        actual = m.grad(name)
        assert max_rel(expected, actual) < 1e-4, name
        assert rel_l2(expected, actual) < 1e-4, name
    for name in m.names:
        if name.startswith("act_head."):
            assert not m.has_grad(name) or not np.any(m.grad(name))


def test_freezing_the_encoder_leaves_its_gradients_empty():
    m, _ = _run(False, trainable=1)
    assert not m.has_grad("encoder.layers.0.attn.Wqkv.weight")
    assert not m.has_grad("encoder.embeddings.tok_embeddings.weight")
    assert m.has_grad("encoder.layers.3.attn.Wqkv.weight")
    full, _ = _run(False)
    np.testing.assert_allclose(m.grad("encoder.layers.3.mlp.Wi.weight"), full.grad("encoder.layers.3.mlp.Wi.weight"),
                               atol=1e-6)


def test_objective_matches_the_notebook_loss_and_gradient():
    fx = objective_fixture()
    ks = fx["ks"]
    logits = np.concatenate(fx["logits"])
    target = np.concatenate(fx["target"])
    draws = np.concatenate([np.concatenate(g) for g in fx["draws"]])
    out, grad = oracle.rlcd(ks, fx["qtypes"], logits, target, draws, fx["sigma"])
    loss, policy, ce, reward = out
    assert abs(ce - fx["loss_ce"]) < 1e-5
    assert abs(policy - fx["loss_rl"]) < 1e-4
    assert abs(reward - fx["reward_mean"]) < 1e-4
    np.testing.assert_allclose(grad, np.concatenate(fx["grad"]), atol=1e-4)
    # The CE-only path (no groups) is the same soft cross-entropy term.
    ce2, g2 = oracle.cross_entropy(ks, logits, target)
    assert abs(ce2 - fx["loss_ce"]) < 1e-5
    # Its gradient is pinned two ways. (1) The objective is linear in its term weights, so the fixture's full
    # gradient minus the policy-only gradient (ce_weight 0) is the CE gradient.
    _, g_policy = oracle.rlcd(ks, fx["qtypes"], logits, target, draws, fx["sigma"], ce_weight=0.0)
    np.testing.assert_allclose(g2, np.concatenate(fx["grad"]) - g_policy, atol=1e-4)
    # (2) Central differences of the CE value, itself pinned to the fixture above.
    h = 1e-2
    for i in range(len(logits)):
        up, dn = logits.copy(), logits.copy()
        up[i] += h
        dn[i] -= h
        fd = (oracle.cross_entropy(ks, up, target)[0] - oracle.cross_entropy(ks, dn, target)[0]) / (2 * h)
        assert abs(fd - g2[i]) < 2e-4, (i, fd, g2[i])


def test_adamw_and_cosine_match_pytorch_closed_values():
    # TrainingTests.cs:46-70: torch.optim.AdamW(lr=0.1, wd=0.01) + CosineAnnealingLR(T_max=3, eta_min=1e-6).
    p = np.array([0.5, -1.0, 2.0, 0.0], np.float32)
    m = np.zeros(4, np.float32)
    v = np.zeros(4, np.float32)
    grads = [[0.1, -0.2, 0.3, 0.0], [0.5, 0.5, -0.5, 0.0], [-0.3, 0.1, 0.2, 1.0]]
    expected = [[0.39950001, -0.89900005, 1.898, 0.0], [0.3346217, -0.93149203, 1.91859365, 0.0],
                [0.32829964, -0.94257891, 1.9182955, -0.01597082]]
    lr = 0.1
    for step in range(3):
        g = np.array(grads[step], np.float32)
        oracle.adamw_tensor(p, g, m, v, lr, step + 1)
        np.testing.assert_allclose(p, expected[step], atol=1e-5)
        lr = 1e-6 + (0.1 - 1e-6) * (1 + np.cos(np.pi * (step + 1) / 3)) / 2


def test_clipping_scales_to_the_maximum_norm():
    # TrainingTests.cs:72-83.
    a = np.array([3.0, 0.0], np.float32)
    b = np.array([4.0], np.float32)
    assert abs(oracle.clip([a, b], 1.0) - 5.0) < 1e-6
    assert abs(a[0] - 0.6) < 1e-5 and abs(b[0] - 0.8) < 1e-5
    c = np.array([0.3, 0.4], np.float32)
    assert abs(oracle.clip([c], 1.0) - 0.5) < 1e-6
    np.testing.assert_array_equal(c, np.array([0.3, 0.4], np.float32))
