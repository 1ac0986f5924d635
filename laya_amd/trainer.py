"""The fine-tuning loop on the GPU: ``Trainer.Train`` (src/StructuredDecisions.Laya.Training/Trainer.cs:79-180)
over the device model.

The loop is the reference's: per epoch the item order is shuffled in place with ``System.Random(seed +
epoch)`` and the objective's noise comes from ``System.Random(seed·7919 + epoch)`` (both reproduced draw
for draw by ``netrandom``); σ is annealed linearly over epochs; every micro-batch runs forward (training
mode, dropout seed ``Mix(seed, microStep + 1)``), the RLCD objective with gradient scale
1/accumulation, and backward; every ``gradient_accumulation`` micro-batches, and after the last one of
an epoch, the gradients are clipped to ``max_gradient_norm``, AdamW steps with the encoder/head learning
rates, the cosine schedule advances and the gradients are zeroed. After the last epoch the temperatures
are fitted on a calibration sample and the checkpoint is written.

What moves to the device: the forward, the objective (loss terms and logit gradient are computed next
to the logits; only the four loss values come back), the backward, clipping and AdamW. The host draws
the Gaussian noise (a few hundred values per micro-batch) and builds the batch tables.

Beyond the reference: the rolling ``checkpoint_latest`` also holds the optimizer state (both Adam moments,
the step count, fp32 master copies of tensors stored in a narrower dtype) and the loop position, so
``train(..., resume=True)`` continues a run exactly where its last completed epoch left it (the reference
cannot resume, TODO.md:74).
"""
from __future__ import annotations

import json
import math
import os
import shutil
import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import numpy as np

from .batch import Batch, TrainingItem
from .calibration import CalibrationSample, TemperatureFit, fit as fit_temperatures
from .device import Context
from .model import TrainableDecisionModel
from .netrandom import DotNetRandom, gaussian, trainer_shuffle
from .ops import mix

ROLLING = "checkpoint_latest"
STATE_FILE = "training_state.json"
STATE_TENSORS = "training_state.safetensors"


def _int32(v: int) -> int:
    """C#'s unchecked 32-bit int arithmetic."""
    return (int(v) + 2 ** 31) % 2 ** 32 - 2 ** 31


@dataclass
class TrainerOptions:
    """TrainerOptions (Trainer.cs:16-58), same names in snake case and the same defaults."""
    epochs: int = 4
    micro_batch: int = 8
    gradient_accumulation: int = 4
    group_size: int = 4
    encoder_learning_rate: float = 2.5e-5
    head_learning_rate: float = 1.0e-4
    minimum_learning_rate: float = 1e-6
    weight_decay: float = 0.01
    max_gradient_norm: float = 1.0
    sigma_start: float = 0.4
    sigma_end: float = 0.1
    spherical_weight: float = 0.75
    rps_weight: float = 1.0
    cross_entropy_weight: float = 1.0
    head_dropout: float = 0.1
    trainable_encoder_layers: Optional[int] = None
    seed: int = 42
    max_steps: Optional[int] = None
    calibration_stride: int = 15
    calibration_maximum: int = 400
    minimum_bucket_samples: int = 30
    rolling_checkpoint: bool = True
    model_name: str = "laya-fine-tuned"
    log_every: int = 50


@dataclass
class TrainingProgress:
    epoch: int
    epochs: int
    micro_step: int
    optimizer_step: int
    loss: float
    mean_reward: float
    learning_rate: float
    sigma: float
    elapsed: float
    message: Optional[str] = None


@dataclass
class TrainingReport:
    optimizer_steps: int
    micro_steps: int
    epoch_loss: List[float]
    temperatures: TemperatureFit
    elapsed: float
    output_directory: str
    trainable_parameters: int


class CosineSchedule:
    """CosineSchedule (AdamW.cs:80-94): after step t, rate = min + (base − min)(1 + cos(π t / T)) / 2."""

    def __init__(self, base_rates: Sequence[float], total_steps: int, minimum: float = 1e-6, step: int = 0):
        self.base = list(base_rates)
        self.total = max(1, int(total_steps))
        self.minimum = minimum
        self.t = step
        self.rates = list(self.base) if step == 0 else [self.at(b, step) for b in self.base]

    def at(self, base: float, step: int) -> float:
        return self.minimum + (base - self.minimum) * (1 + math.cos(math.pi * step / self.total)) / 2

    def step(self) -> None:
        self.t += 1
        self.rates = [self.at(b, self.t) for b in self.base]


def calibration_sample(items: Sequence[TrainingItem], options: TrainerOptions) -> List[TrainingItem]:
    """Trainer.CalibrationSample (Trainer.cs:191-197): ⌈n / stride⌉ items (at most the maximum), drawn by
    shuffling the indices with System.Random(seed), kept in item order."""
    stride = max(1, options.calibration_stride)
    count = min(options.calibration_maximum, (len(items) + options.calibration_stride - 1) // stride)
    indices = list(range(len(items)))
    DotNetRandom(options.seed).shuffle_span(indices)
    return [items[i] for i in sorted(indices[:count])]


def calibrate(model: TrainableDecisionModel, items: Sequence[TrainingItem],
              minimum_bucket_samples: int = 30) -> TemperatureFit:
    """Trainer.Calibrate (Trainer.cs:200-211): eval-mode forward in chunks of 16, then the fit."""
    samples = []
    for start in range(0, len(items), 16):
        chunk = list(items[start:start + 16])
        batch = Batch.from_items(chunk)
        logits = batch.split(model.forward(batch, training=False))
        for item, z in zip(chunk, logits):
            samples.append(CalibrationSample(item.question_type, np.array(z, np.float32),
                                             np.asarray(item.target, np.float32)))
    return fit_temperatures(samples, minimum_bucket_samples)


def write_temperatures(config: dict, fit: TemperatureFit) -> None:
    """Trainer.WriteTemperatures (Trainer.cs:233-240): the buckets are replaced, never merged."""
    config["temperature"] = [float(t) for t in fit.by_type]
    config["temperature_by_options"] = {k: float(v) for k, v in fit.by_bucket.items()}


def recalibrate(directory: str, items: Sequence[TrainingItem], minimum_bucket_samples: int = 30,
                ctx: Optional[Context] = None) -> TemperatureFit:
    """Trainer.Recalibrate (Trainer.cs:221-231): refits a checkpoint's temperatures in place."""
    model = TrainableDecisionModel.from_directory(directory, ctx)
    try:
        fit = calibrate(model, items, minimum_bucket_samples)
    finally:
        model.close()
    path = os.path.join(directory, "rl_agent_config.json")
    with open(path) as f:
        config = json.load(f)
    write_temperatures(config, fit)
    with open(path, "w") as f:
        json.dump(config, f, indent=2)
    return fit


def build_config(source_directory: str, o: TrainerOptions, fit: Optional[TemperatureFit], max_length: Optional[int],
                 head_max_length: Optional[int], steps: int, epochs: int, elapsed: float) -> dict:
    """Trainer.BuildConfig (Trainer.cs:255-275): the source's rl_agent_config.json, unknown keys kept,
    with what training changed."""
    with open(os.path.join(source_directory, "rl_agent_config.json")) as f:
        config = json.load(f)
    if max_length is not None:
        config["max_len"] = int(max_length)
    if head_max_length is not None:
        config["head_max_len"] = int(head_max_length)
    config["fine_tuned"] = True
    config["model_name"] = o.model_name
    if fit is not None:
        write_temperatures(config, fit)
    config["training"] = {
        "updates": steps,
        "epochs_completed": epochs,
        "hours": round(elapsed / 3600.0, 2),
        "world_size": 1,
        "fine_tuned_from_checkpoint": True,
        "trainer": "laya_amd (MI355X)",
        "trainable_encoder_layers": o.trainable_encoder_layers,
    }
    return config


@dataclass
class _LoopState:
    """Where the loop is, at an epoch boundary: what a resumed run needs besides the model."""
    next_epoch: int = 0
    micro_step: int = 0
    epoch_loss: List[float] = field(default_factory=list)
    elapsed: float = 0.0


_STAGING, _RETIRED = ".new", ".old"


def _fsync_tree(path: str) -> None:
    """Flushes every file under `path`, then every directory (deepest first), to stable storage."""
    for root, dirs, files in os.walk(path, topdown=False):
        for name in files:
            fd = os.open(os.path.join(root, name), os.O_RDONLY)
            try:
                os.fsync(fd)
            finally:
                os.close(fd)
        _fsync_dir(root)


def _fsync_dir(path: str) -> None:
    fd = os.open(path, os.O_RDONLY)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def _state_complete(directory: str) -> bool:
    """A checkpoint directory counts as complete when its loop state (written last) parses."""
    try:
        with open(os.path.join(directory, STATE_FILE)) as f:
            json.load(f)
        return True
    except (OSError, ValueError):
        return False


def _swap_in(staging: str, rolling: str) -> None:
    """Replaces `rolling` by the complete checkpoint in `staging` with two renames. The staged files are on
    stable storage before the renames, and the renames before the retired copy is removed, so a power loss at
    any point leaves a complete checkpoint under `rolling` or `rolling.old`."""
    retired = rolling + _RETIRED
    parent = os.path.dirname(os.path.abspath(rolling))
    _fsync_tree(staging)
    shutil.rmtree(retired, ignore_errors=True)
    if os.path.exists(rolling):
        os.rename(rolling, retired)
    os.rename(staging, rolling)
    _fsync_dir(parent)
    shutil.rmtree(retired, ignore_errors=True)
    _fsync_dir(parent)


def _recover_rolling(rolling: str) -> None:
    """Finishes a swap an interruption cut short: a staged checkpoint whose loop state was written and parses
    is complete and wins; otherwise the retired one is restored. A rolling checkpoint whose loop state does not
    parse is replaced by the retired one when that exists."""
    staging, retired = rolling + _STAGING, rolling + _RETIRED
    if os.path.exists(rolling):
        if not _state_complete(rolling) and _state_complete(retired):
            shutil.rmtree(rolling)
            os.rename(retired, rolling)
        return
    if _state_complete(staging):
        os.rename(staging, rolling)
    elif os.path.exists(retired):
        os.rename(retired, rolling)


class Trainer:
    """Trainer (Trainer.cs:73-180) on one GPU."""

    def __init__(self, options: Optional[TrainerOptions] = None,
                 progress: Optional[Callable[[TrainingProgress], None]] = None, ctx: Optional[Context] = None):
        self.options = options or TrainerOptions()
        self.progress = progress
        self.ctx = ctx

    def _report(self, p: TrainingProgress) -> None:
        if self.progress is not None:
            self.progress(p)

    def train(self, source_directory: str, items: Sequence[TrainingItem], output_directory: str,
              calibration_items: Optional[Sequence[TrainingItem]] = None, max_length: Optional[int] = None,
              head_max_length: Optional[int] = None, resume: bool = False,
              should_stop: Optional[Callable[[], bool]] = None) -> TrainingReport:
        """Trainer.Train. ``resume`` continues from ``output_directory/checkpoint_latest`` when that holds
        a loop state; ``should_stop`` is polled before every micro-batch (the cancellation token) and
        raises ``InterruptedError`` when it returns true."""
        if len(items) == 0:
            raise ValueError("no training items.")
        o = self.options
        if o.micro_batch < 1 or o.gradient_accumulation < 1 or o.group_size < 0:
            raise ValueError("micro_batch and gradient_accumulation must be positive, group_size non-negative")
        clock = time.perf_counter()
        rolling = os.path.join(output_directory, ROLLING)
        state = _LoopState()
        load_from = source_directory
        if resume:
            _recover_rolling(rolling)
        if resume and os.path.exists(os.path.join(rolling, STATE_FILE)):
            with open(os.path.join(rolling, STATE_FILE)) as f:
                saved = json.load(f)
            state = _LoopState(saved["next_epoch"], saved["micro_step"], list(saved["epoch_loss"]),
                               float(saved["elapsed"]))
            load_from = rolling

        model = TrainableDecisionModel.from_directory(load_from, self.ctx)
        try:
            return self._train(model, source_directory, items, output_directory, calibration_items, max_length,
                               head_max_length, state, load_from != source_directory, clock, should_stop)
        finally:
            model.close()

    def _train(self, model, source_directory, items, output_directory, calibration_items, max_length,
               head_max_length, state: _LoopState, resumed: bool, clock: float, should_stop) -> TrainingReport:
        o = self.options
        model.set_trainable_encoder_layers(o.trainable_encoder_layers)
        model.head_dropout = o.head_dropout
        rolling = os.path.join(output_directory, ROLLING)
        if resumed:
            model.load_optimizer_state(os.path.join(rolling, STATE_TENSORS))
        elapsed = lambda: state.elapsed + time.perf_counter() - clock
        self._report(TrainingProgress(0, o.epochs, 0, 0, 0, 0, 0, 0, elapsed(),
                                      f"loaded {model.parameter_count / 1e6:.0f}M parameters, "
                                      f"{model.trainable_parameter_count / 1e6:.1f}M trainable; {len(items)} items"))

        total_updates = len(items) // (o.micro_batch * o.gradient_accumulation) * o.epochs
        schedule = CosineSchedule([o.encoder_learning_rate, o.head_learning_rate], max(1, total_updates),
                                  o.minimum_learning_rate, step=model.steps)
        order = list(items)
        for epoch in range(state.next_epoch):  # the order is shuffled in place, epoch after epoch
            trainer_shuffle(order, DotNetRandom(_int32(o.seed + epoch)))
        micro_step = state.micro_step
        epoch_loss = list(state.epoch_loss)
        stop = o.max_steps is not None and model.steps >= o.max_steps
        for epoch in range(state.next_epoch, o.epochs):
            if stop:
                break
            trainer_shuffle(order, DotNetRandom(_int32(o.seed + epoch)))
            noise = DotNetRandom(_int32(o.seed * 7919 + epoch))
            progress = epoch / max(1, o.epochs - 1)
            sigma = o.sigma_start + (o.sigma_end - o.sigma_start) * progress
            loss_sum, batches, accumulated = 0.0, 0, 0
            model.zero_gradients()
            for start in range(0, len(order), o.micro_batch):
                if should_stop is not None and should_stop():
                    raise InterruptedError("training cancelled")
                chunk = order[start:start + o.micro_batch]
                seed = mix(o.seed & (2 ** 64 - 1), micro_step + 1)
                batch = Batch.from_items(chunk)
                model.forward(batch, training=True, seed=seed, want_logits=False)
                draws = np.array([[gaussian(noise) for _ in range(batch.n_markers)] for _ in range(o.group_size)],
                                 np.float64).reshape(o.group_size, batch.n_markers)
                targets = np.concatenate([np.asarray(i.target, np.float32) for i in chunk])
                loss, _, _, reward = model.objective_rlcd(targets, draws, sigma, o.spherical_weight, o.rps_weight,
                                                          o.cross_entropy_weight, 1.0 / o.gradient_accumulation)
                model.backward_from_objective()
                accumulated += 1
                micro_step += 1
                if accumulated % o.gradient_accumulation == 0 or start + o.micro_batch >= len(order):
                    model.clip_grad_norm(o.max_gradient_norm)
                    model.adamw_step(schedule.rates[0], schedule.rates[1], weight_decay=o.weight_decay)
                    schedule.step()
                    model.zero_gradients()
                    if o.max_steps is not None and model.steps >= o.max_steps:
                        stop = True
                loss_sum += loss
                batches += 1
                if batches % o.log_every == 0 or stop:
                    self._report(TrainingProgress(epoch + 1, o.epochs, batches, model.steps, loss, reward,
                                                  schedule.rates[-1], sigma, elapsed()))
                if stop:
                    break
            average = loss_sum / max(1, batches)
            epoch_loss.append(average)
            self._report(TrainingProgress(epoch + 1, o.epochs, batches, model.steps, average, 0, schedule.rates[-1],
                                          sigma, elapsed(), f"epoch {epoch + 1}/{o.epochs} done, average loss "
                                          f"{average:.4f}"))
            if o.rolling_checkpoint and not stop and epoch + 1 < o.epochs:
                # The whole checkpoint is written into a sibling directory, the loop state last, and only
                # then swapped in: an interruption never leaves weights of one epoch beside the loop state
                # and moments of another.
                staging = rolling + _STAGING
                shutil.rmtree(staging, ignore_errors=True)
                model.save(staging, source_directory, build_config(source_directory, o, None, max_length,
                                                                   head_max_length, model.steps, epoch + 1, elapsed()))
                with open(os.path.join(staging, "checkpoint_meta.json"), "w") as f:
                    json.dump({"epoch": epoch + 1, "total_epochs": o.epochs, "avg_loss": average}, f, indent=2)
                model.save_optimizer_state(os.path.join(staging, STATE_TENSORS))
                with open(os.path.join(staging, STATE_FILE), "w") as f:
                    json.dump({"next_epoch": epoch + 1, "micro_step": micro_step, "epoch_loss": epoch_loss,
                               "elapsed": elapsed(), "optimizer_steps": model.steps}, f, indent=2)
                _swap_in(staging, rolling)

        calibration = list(calibration_items) if calibration_items is not None else calibration_sample(items, o)
        fit = calibrate(model, calibration, o.minimum_bucket_samples)
        self._report(TrainingProgress(o.epochs, o.epochs, 0, model.steps, 0, 0, 0, 0, elapsed(),
                                      f"calibrated on {len(calibration)} items: {fit.describe()}"))
        model.save(output_directory, source_directory, build_config(source_directory, o, fit, max_length,
                                                                    head_max_length, model.steps, len(epoch_loss),
                                                                    elapsed()))
        return TrainingReport(model.steps, micro_step, epoch_loss, fit, elapsed(), output_directory,
                              model.trainable_parameter_count)

