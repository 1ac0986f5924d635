"""The fine-tuning loop, checkpoints and resume on the GPU, against the same loop run on the oracle.

The reference loop (Trainer.cs:111-168) is restated below over the oracle model, with the same item
order, dropout seeds and Gaussian draws (the System.Random restatement, pinned by known answers in the
host tests), so the device trainer and the oracle see identical inputs at every micro-step.
"""
import json
import os

import numpy as np
import pytest

import oracle
from fixtures import TINY, rel_l2, tiny_config, tiny_params

pytestmark = pytest.mark.gpu

trainer_mod = pytest.importorskip("laya_amd.trainer")


@pytest.fixture(scope="module")
def ctx():
    from laya_amd.device import Context
    print("GPU trainer tests: creating context on device 0", flush=True)
    c = Context(0)
    yield c
    c.close()


def _items(n, seed=3):
    from laya_amd.batch import TrainingItem
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        length = int(rng.integers(12, 40))  # markers reach position 9
        k = [2, 4, 3, 5][i % 4]
        ids = rng.integers(3, 97, length).astype(np.int32)
        markers = np.array([1 + 2 * o for o in range(k)], np.int32)
        out.append(TrainingItem(ids, markers, i % 3, rng.dirichlet(np.ones(k)).astype(np.float32)))
    return out


def _draws(noise, groups, n):
    from laya_amd.netrandom import gaussian
    return np.array([[gaussian(noise) for _ in range(n)] for _ in range(groups)], np.float64).reshape(groups, n)


def oracle_train(o, items, double=False):
    """Trainer.Train's loop (Trainer.cs:111-168) on the oracle model, training only (no calibration)."""
    from laya_amd.batch import Batch
    from laya_amd.netrandom import DotNetRandom, trainer_shuffle
    from laya_amd.trainer import CosineSchedule
    om = oracle.OracleModel(tiny_config(), double=double)
    om.set_params(tiny_params())
    om.set_trainable_encoder_layers(o.trainable_encoder_layers)
    om.set_head_dropout(o.head_dropout)
    total = len(items) // (o.micro_batch * o.gradient_accumulation) * o.epochs
    schedule = CosineSchedule([o.encoder_learning_rate, o.head_learning_rate], max(1, total), o.minimum_learning_rate)
    order, micro, steps, epoch_loss = list(items), 0, 0, []
    for epoch in range(o.epochs):
        trainer_shuffle(order, DotNetRandom(o.seed + epoch))
        noise = DotNetRandom(o.seed * 7919 + epoch)
        sigma = o.sigma_start + (o.sigma_end - o.sigma_start) * epoch / max(1, o.epochs - 1)
        om.zero_grad()
        acc, loss_sum, batches = 0, 0.0, 0
        for start in range(0, len(order), o.micro_batch):
            chunk = order[start:start + o.micro_batch]
            batch = Batch.from_items(chunk)
            logits = om.forward(batch, training=True, seed=oracle.mix(o.seed, micro + 1))
            targets = np.concatenate([c.target for c in chunk]).astype(np.float32)
            out, g = oracle.rlcd(batch.n_options, batch.qtypes, logits, targets,
                                 _draws(noise, o.group_size, batch.n_markers).reshape(-1), sigma,
                                 spherical=o.spherical_weight, rps=o.rps_weight, ce_weight=o.cross_entropy_weight,
                                 scale=1.0 / o.gradient_accumulation)
            om.backward(g)
            acc += 1
            micro += 1
            if acc % o.gradient_accumulation == 0 or start + o.micro_batch >= len(order):
                om.clip(o.max_gradient_norm)
                om.adamw(schedule.rates[0], schedule.rates[1], weight_decay=o.weight_decay)
                schedule.step()
                om.zero_grad()
                steps += 1
            loss_sum += out[0]
            batches += 1
        epoch_loss.append(loss_sum / batches)
    return om, steps, epoch_loss


# Directions whose exact gradient is zero, so both implementations hold rounding noise there and AdamW
# turns it into ±lr steps of arbitrary sign: they are bounded, not compared.
#  - the output bias: its gradient is Σ over options of the logit gradient, and softmax cross-entropy
#    and the zero-mean noise both sum to zero per item;
#  - the key third of the head attention's in_proj bias: it adds q·b_k to a whole row of scores, which
#    softmax ignores.
def _noise_only(name, size):
    mask = np.zeros(size, bool)
    if name == "scorer.3.bias":
        mask[:] = True
    elif name.endswith("self_attn.in_proj_bias"):
        mask[size // 3:2 * size // 3] = True
    return mask


def _compare_trained(names, got, want, init, steps, lr, exact=None):
    """Trained weights against the fp32 oracle's: the fp32 bar (rel-L2 1e-4) on the weights, and on the
    updates (weights − initial) max(2e-3, 4 × the fp32 oracle's own deviation from the fp64 oracle ``exact``),
    since Adam divides each gradient by its own magnitude and so amplifies rounding in small elements."""
    for name in names:
        if name == "temperature":
            continue
        g, w, i0 = (np.asarray(a, np.float64).reshape(-1) for a in (got[name], want[name], init[name]))
        noise = _noise_only(name, g.size)
        assert np.all(np.abs(g - i0)[noise] <= steps * lr * 1.01 + 1e-7), name
        keep = ~noise
        g, w, i0 = g[keep], w[keep], i0[keep]
        assert rel_l2(w, g) < 1e-4, name
        if np.linalg.norm(w - i0) > 0:
            bar = 2e-3
            if exact is not None:
                e = np.asarray(exact[name], np.float64).reshape(-1)[keep]
                bar = max(bar, 4 * rel_l2(e - i0, w - i0))
            assert rel_l2(w - i0, g - i0) < bar, (name, rel_l2(w - i0, g - i0), bar)


def test_trainer_matches_the_oracle_loop(ctx, tmp_path):
    """Two epochs over 10 items: micro-batches of 2 with accumulation 2 (a step after 2, 4 and the last
    micro-batch of each epoch), RLCD with 4 groups, clipping, two learning rates under the cosine schedule,
    head dropout, σ annealed; then calibration and the saved checkpoint."""
    from laya_amd.trainer import Trainer, TrainerOptions
    from laya_amd.safetensors_io import SafetensorsFile
    items = _items(10)
    o = TrainerOptions(epochs=2, micro_batch=2, gradient_accumulation=2, encoder_learning_rate=1e-3,
                       head_learning_rate=3e-3, max_gradient_norm=0.5, seed=7, log_every=1)
    seen = []
    report = Trainer(o, progress=seen.append, ctx=ctx).train(TINY, items, str(tmp_path / "out"))
    om, steps, epoch_loss = oracle_train(o, items)
    om64, _, _ = oracle_train(o, items, double=True)
    assert report.optimizer_steps == steps == 6 and report.micro_steps == 10
    np.testing.assert_allclose(report.epoch_loss, epoch_loss, rtol=1e-4)
    st = SafetensorsFile(str(tmp_path / "out" / "model.safetensors"))
    init = tiny_params()
    got = {n: st.read_float32(n) for n in st.entries}
    want = {n: om.param(n) for n in st.entries if n != "temperature"}
    _compare_trained(want.keys(), got, want, init, steps, 3e-3, {n: om64.param(n) for n in want})
    with open(tmp_path / "out" / "rl_agent_config.json") as f:
        cfg = json.load(f)
    assert cfg["training"]["updates"] == 6 and cfg["training"]["epochs_completed"] == 2
    assert len(cfg["temperature"]) == 3 and cfg["fine_tuned"] is True
    assert os.path.exists(tmp_path / "out" / "encoder" / "config.json")
    # A rolling checkpoint after the first epoch (not after the last), with its loop state.
    with open(tmp_path / "out" / "checkpoint_latest" / "checkpoint_meta.json") as f:
        assert json.load(f)["epoch"] == 1
    assert any(p.message and "epoch 2/2 done" in p.message for p in seen)


def test_resumed_training_equals_uninterrupted_training(ctx, tmp_path):
    """Three epochs straight, against two epochs, a cancellation, and a resume from checkpoint_latest:
    the final weights and the per-epoch losses are bit-identical."""
    from laya_amd.trainer import Trainer, TrainerOptions
    from laya_amd.safetensors_io import SafetensorsFile
    items = _items(8, seed=5)
    o = TrainerOptions(epochs=3, micro_batch=2, gradient_accumulation=2, encoder_learning_rate=1e-3,
                       head_learning_rate=1e-3, seed=11)
    straight = Trainer(o, ctx=ctx).train(TINY, items, str(tmp_path / "a"))
    calls = []

    def stop_in_third_epoch():
        calls.append(1)
        return len(calls) > 8  # 4 micro-batches per epoch

    with pytest.raises(InterruptedError):
        Trainer(o, ctx=ctx).train(TINY, items, str(tmp_path / "b"), should_stop=stop_in_third_epoch)
    resumed = Trainer(o, ctx=ctx).train(TINY, items, str(tmp_path / "b"), resume=True)
    assert resumed.optimizer_steps == straight.optimizer_steps == 6
    assert resumed.micro_steps == straight.micro_steps == 12
    assert resumed.epoch_loss == straight.epoch_loss
    a = SafetensorsFile(str(tmp_path / "a" / "model.safetensors"))
    b = SafetensorsFile(str(tmp_path / "b" / "model.safetensors"))
    for name in a.entries:
        np.testing.assert_array_equal(a.read_float32(name), b.read_float32(name), err_msg=name)


def test_a_saved_checkpoint_reloads_exactly(ctx, tmp_path):
    """TrainingTests.cs:155-207: items and noise from System.Random(9), two AdamW steps at 1e-3 (one group,
    no clipping), save, reload: the reloaded model's logits equal the trained model's, every tensor keeps
    its dtype, scorer.1.weight moved. The two steps also match the oracle."""
    from laya_amd.batch import Batch, TrainingItem
    from laya_amd.model import TrainableDecisionModel
    from laya_amd.netrandom import DotNetRandom
    from laya_amd.safetensors_io import SafetensorsFile
    r = DotNetRandom(9)
    items = []
    for i in range(4):
        ids = np.array([r.next_range(3, 97) for _ in range(10 + 3 * i)], np.int32)
        k = 2 + i % 3
        target = np.array([r.next_double() for _ in range(k)], np.float32)
        total = np.float32(0)
        for v in target:
            total = np.float32(total + v)
        items.append(TrainingItem(ids, np.array([1 + 2 * o for o in range(k)], np.int32), i % 3,
                                  (target / total).astype(np.float32)))
    batch = Batch.from_items(items)
    targets = np.concatenate([i.target for i in items])
    model = TrainableDecisionModel.from_directory(TINY, ctx)
    model.set_trainable_encoder_layers(None)
    om = oracle.OracleModel(tiny_config())
    om.set_params(tiny_params())
    om.set_head_dropout(0.1)
    for step in range(2):
        draws = _draws(r, 4, batch.n_markers)
        model.forward(batch, training=True, seed=step, want_logits=False)
        model.objective_rlcd(targets, draws, 0.4)
        model.backward_from_objective()
        model.adamw_step(1e-3, 1e-3)
        model.zero_gradients()
        logits = om.forward(batch, training=True, seed=step)
        _, g = oracle.rlcd(batch.n_options, batch.qtypes, logits, targets, draws.reshape(-1), 0.4)
        om.backward(g)
        om.adamw(1e-3, 1e-3)
        om.zero_grad()
    expected = model.forward(batch, training=False)
    with open(os.path.join(TINY, "rl_agent_config.json")) as f:
        config = json.load(f)
    out = str(tmp_path / "saved")
    model.save(out, TINY, config)
    reloaded = TrainableDecisionModel.from_directory(out, ctx)
    np.testing.assert_array_equal(reloaded.forward(batch, training=False), expected)
    original, saved = SafetensorsFile(os.path.join(TINY, "model.safetensors")), SafetensorsFile(
        os.path.join(out, "model.safetensors"))
    assert sorted(original.entries) == sorted(saved.entries)
    assert all(saved.dtype(n) == original.dtype(n) for n in saved.entries)
    assert saved.names_in_file_order() == original.names_in_file_order()
    assert not np.array_equal(original.read_float32("scorer.1.weight"), saved.read_float32("scorer.1.weight"))
    init = tiny_params()
    got = {n: saved.read_float32(n) for n in saved.entries}
    want = {n: om.param(n) for n in saved.entries if n != "temperature"}
    _compare_trained(want.keys(), got, want, init, 2, 1e-3)
    reloaded.close()
    model.close()


def test_bf16_checkpoints_keep_their_dtype_and_resume_from_master_weights(ctx, tmp_path):
    """A checkpoint stored in BF16 is written back in BF16 (round to nearest even) and its optimizer state
    carries fp32 master weights and both moments, so training continues from the exact state."""
    import shutil
    from laya_amd.batch import Batch
    from laya_amd.model import TrainableDecisionModel
    from laya_amd.safetensors_io import SafetensorsFile, write
    src = tmp_path / "bf16"
    shutil.copytree(TINY, src)
    st = SafetensorsFile(os.path.join(TINY, "model.safetensors"))
    write(str(src / "model.safetensors"),
          [(n, st.shape(n), st.read_float32(n), "BF16" if "weight" in n and n != "temperature" else "F32")
           for n in st.names_in_file_order()])
    items = _items(4, seed=9)
    batch = Batch.from_items(items)
    targets = np.concatenate([i.target for i in items])
    a = TrainableDecisionModel.from_directory(str(src), ctx)
    draws = np.random.default_rng(1).standard_normal((4, batch.n_markers))

    def step(m, seed):
        m.forward(batch, training=True, seed=seed, want_logits=False)
        m.objective_rlcd(targets, draws, 0.3)
        m.backward_from_objective()
        m.clip_grad_norm(1.0)
        m.adamw_step(1e-3, 1e-3)
        m.zero_gradients()

    step(a, 1)
    with open(os.path.join(TINY, "rl_agent_config.json")) as f:
        config = json.load(f)
    a.save(str(tmp_path / "ck"), str(src), config)
    a.save_optimizer_state(str(tmp_path / "ck" / "opt.safetensors"))
    saved = SafetensorsFile(str(tmp_path / "ck" / "model.safetensors"))
    w = a.param("scorer.1.weight")
    bits = w.view(np.uint32)
    rne = (((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    np.testing.assert_array_equal(saved.read_float32("scorer.1.weight"), rne)
    assert saved.dtype("scorer.1.weight") == "BF16" and saved.dtype("scorer.1.bias") == "F32"
    b = TrainableDecisionModel.from_directory(str(tmp_path / "ck"), ctx)
    b.load_optimizer_state(str(tmp_path / "ck" / "opt.safetensors"))
    assert b.steps == a.steps == 1
    step(a, 2)
    step(b, 2)
    for name in a.names:
        np.testing.assert_array_equal(a.param(name), b.param(name), err_msg=name)
    a.close()
    b.close()


def test_zero_groups_is_the_cross_entropy_objective(ctx):
    """GroupSize 0: no policy term, mean reward 0/0 (NaN); the gradient is the soft cross-entropy's."""
    from laya_amd import ops as laya
    from laya_amd.device import DeviceArray
    rng = np.random.default_rng(2)
    ks = [8, 4, 2, 5]
    logits = rng.standard_normal(sum(ks)).astype(np.float32)
    targets = np.concatenate([rng.dirichlet(np.ones(k)) for k in ks]).astype(np.float32)
    offsets = np.concatenate([[0], np.cumsum(ks)]).astype(np.int32)
    dev = lambda a: DeviceArray.from_numpy(ctx, np.asarray(a))
    (loss, policy, ce, reward), grad = laya.rlcd_objective(
        ctx, dev(logits), dev(targets), dev(offsets), dev(np.array([0, 1, 2, 0], np.int32)), ks,
        DeviceArray(ctx, (2,)), 0, 0.0, scale=0.5)
    want_ce, want_g = oracle.cross_entropy(ks, logits, targets, scale=0.5)
    assert policy == 0.0 and np.isnan(reward)
    assert loss == pytest.approx(ce) and ce == pytest.approx(want_ce, rel=1e-5)
    assert rel_l2(want_g, grad.numpy()[:logits.size]) < 1e-5
