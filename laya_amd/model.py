"""The trainable decision model on the GPU, mirroring the reference's ``TrainableDecisionModel``
(src/StructuredDecisions.Laya.Training/TrainableDecisionModel.cs) over liblaya_hip's model driver.

Parameters, gradients and optimizer moments live in device arenas; the forward keeps every
activation the backward needs in HBM (no per-layer recompute); only token ids, segment tables and
marker rows go in, and logits come out (dlogits go back in).
"""
from __future__ import annotations

import ctypes
import json
import os
import shutil
from typing import Dict, List, Optional, Sequence

import numpy as np

from ._native import ERR_MISSING, ERR_NOT_FINITE, BatchC, LayaMissingError, ModelConfigC, check, lib
from .batch import Batch, TrainingItem
from .config import ModelConfig
from .device import Context
from .safetensors_io import SafetensorsFile
from .safetensors_io import write as write_safetensors


def _config_struct(mc: ModelConfig):
    e = mc.encoder
    kinds = (ctypes.c_int * max(1, e.num_hidden_layers))(*e.layer_kinds)
    c = ModelConfigC(vocab=e.vocab_size, hidden=e.hidden_size, intermediate=e.intermediate_size,
                     layers=e.num_hidden_layers, heads=e.num_attention_heads, local_attention=e.local_attention,
                     global_every=e.global_attn_every_n_layers, layer_kinds=kinds,
                     theta_global=e.global_rope_theta, theta_local=e.local_rope_theta, norm_eps=e.norm_eps,
                     norm_bias=int(e.norm_bias), attention_bias=int(e.attention_bias), mlp_bias=int(e.mlp_bias),
                     head_layers=mc.head_layers, head_ff=mc.head_ff, n_act=mc.n_act)
    return c, kinds


class _BatchArgs:
    """Keeps the host arrays of a batch alive while the C struct points into them."""

    def __init__(self, batch: Batch):
        self.arrays = [np.ascontiguousarray(a, dtype=np.int32) for a in
                       (batch.lengths, batch.tokens, batch.n_options, batch.markers, batch.qtypes)]
        self.struct = BatchC(batch.n_items, *[a.ctypes.data for a in self.arrays])


def synthetic_params(shapes: Dict[str, tuple], seed: int = 0, std: float = 0.02) -> Dict[str, np.ndarray]:
    """A host-side random init of the kind ``TrainableDecisionModel.synthetic`` makes on the device: N(0, std)
    matrices and embeddings, unit LayerNorm weights (and the frozen temperatures), zero biases. Each tensor
    draws from its own generator keyed by (seed, name), so a CPU restatement of the model fed the same shapes
    gets the same values."""
    import zlib
    ones = ("norm.weight", "norm1.weight", "norm2.weight", "scorer.0.weight")
    out = {}
    for name, shape in shapes.items():
        if name == "temperature" or name.endswith(ones):
            out[name] = np.ones(shape, np.float32)
        elif name.endswith("bias"):
            out[name] = np.zeros(shape, np.float32)
        else:
            rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
            out[name] = (std * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
    return out


def _as_batch(items) -> Batch:
    if isinstance(items, Batch):
        return items
    return Batch.from_items(list(items))


class TrainableDecisionModel:
    def __init__(self, config: ModelConfig, ctx: Optional[Context] = None):
        self.config = config
        self.ctx = ctx or Context(0)
        cs, self._kinds = _config_struct(config)
        h = ctypes.c_void_p()
        check(lib().laya_model_create(self.ctx.handle, ctypes.byref(cs), ctypes.byref(h)))
        self.handle = h.value
        self.ctx.register(self)
        n = ctypes.c_int()
        check(lib().laya_model_num_params(self.handle, ctypes.byref(n)))
        self.names: List[str] = []
        self.shapes: Dict[str, tuple] = {}
        self.index: Dict[str, int] = {}
        for i in range(n.value):
            name = ctypes.c_char_p()
            ndim = ctypes.c_int()
            dims = (ctypes.c_int * 4)()
            off, numel, tr = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int()
            check(lib().laya_model_param_info(self.handle, i, ctypes.byref(name), ctypes.byref(ndim), dims,
                                              ctypes.byref(off), ctypes.byref(numel), ctypes.byref(tr)))
            nm = name.value.decode()
            self.names.append(nm)
            self.shapes[nm] = tuple(dims[k] for k in range(ndim.value))
            self.index[nm] = i
        self._batch: Optional[Batch] = None
        self._head_dropout = 0.1
        # What Save writes back (TrainableDecisionModel.cs:649-661): the source's tensors in file order,
        # each in the dtype it was stored in; tensors the model does not use are kept as read.
        self.stored_dtypes: Dict[str, str] = {n: "F32" for n in self.names}
        self.file_order: List[str] = list(self.names)
        self.extra_tensors: Dict[str, np.ndarray] = {}

    def close(self) -> None:
        if getattr(self, "handle", None) and getattr(self.ctx, "handle", None):
            lib().laya_model_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------------ construction / IO

    @classmethod
    def from_directory(cls, directory: str, ctx: Optional[Context] = None) -> "TrainableDecisionModel":
        """TrainableDecisionModel.FromDirectory (TrainableDecisionModel.cs:191-197)."""
        model = cls(ModelConfig.from_directory(directory), ctx)
        st = SafetensorsFile(os.path.join(directory, "model.safetensors"))
        for name in model.names:
            if name not in st.entries:
                if name == "temperature":
                    continue
                # InvalidDataException of TrainableDecisionModel.cs:184-186: the same status the C-ABI
                # gives a lookup of a tensor the model does not have.
                raise LayaMissingError(ERR_MISSING, f"the checkpoint has no '{name}' tensor; is it a laya "
                                                    "decision model?")
            model.set_param(name, st.read_float32(name))
        model.file_order = st.names_in_file_order()
        model.stored_dtypes = {n: st.dtype(n) for n in model.file_order}
        model.extra_tensors = {n: st.read_float32(n) for n in model.file_order if n not in model.index}
        return model

    def save(self, directory: str, source_directory: str, config: dict) -> None:
        """TrainableDecisionModel.Save (TrainableDecisionModel.cs:649-661): model.safetensors with every
        tensor in its stored dtype (BF16 rounds to nearest even), the source's encoder/ and tokenizer/
        copied, and ``config`` as rl_agent_config.json."""
        os.makedirs(directory, exist_ok=True)
        tensors = []
        for name in self.file_order:
            values = self.extra_tensors[name] if name in self.extra_tensors else self.param(name)
            dtype = self.stored_dtypes.get(name, "F32")
            tensors.append((name, tuple(values.shape), values, dtype if dtype in ("F32", "F16", "BF16") else "F32"))
        write_safetensors(os.path.join(directory, "model.safetensors"), tensors)
        for sub, required in (("encoder", True), ("tokenizer", False)):
            src, dst = os.path.join(source_directory, sub), os.path.join(directory, sub)
            if not os.path.isdir(src):
                if required:
                    raise FileNotFoundError(f"{src}: the source checkpoint has no {sub} directory")
                continue
            if os.path.abspath(src) != os.path.abspath(dst):
                shutil.copytree(src, dst, dirs_exist_ok=True)
        with open(os.path.join(directory, "rl_agent_config.json"), "w") as f:
            json.dump(config, f, indent=2)

    # Optimizer state (the reference trainer cannot resume, TODO.md:74; its AdamW keeps these per
    # parameter, AdamW.cs:24): both moments of every trainable tensor and the step count.
    def optimizer_state(self) -> Dict[str, tuple]:
        out = {}
        for name in self.names:
            if not self.trainable(name):
                continue
            m1 = np.empty(self.shapes[name], np.float32)
            m2 = np.empty(self.shapes[name], np.float32)
            check(lib().laya_model_get_moments(self.handle, self.index[name], m1.ctypes.data, m2.ctypes.data))
            out[name] = (m1, m2)
        return out

    def save_optimizer_state(self, path: str) -> None:
        """Writes the moments as F32 tensors 'exp_avg.<name>' / 'exp_avg_sq.<name>', an F32 master copy
        'master.<name>' of every tensor the checkpoint stores in a narrower dtype (so a resumed run starts
        from the exact weights, not their rounding), and the step count in a JSON side file."""
        tensors = []
        for name, (m1, m2) in self.optimizer_state().items():
            tensors.append(("exp_avg." + name, m1.shape, m1, "F32"))
            tensors.append(("exp_avg_sq." + name, m2.shape, m2, "F32"))
        for name in self.names:
            if self.stored_dtypes.get(name, "F32") != "F32":
                values = self.param(name)
                tensors.append(("master." + name, values.shape, values, "F32"))
        write_safetensors(path, tensors)
        with open(path + ".json", "w") as f:
            json.dump({"steps": self.steps}, f)

    def load_optimizer_state(self, path: str) -> None:
        """Restores what save_optimizer_state wrote: master weights, moments and the step count."""
        st = SafetensorsFile(path)
        with open(path + ".json") as f:
            steps = int(json.load(f)["steps"])
        for name in self.names:
            if ("master." + name) in st.entries:
                self.set_param(name, st.read_float32("master." + name))
            if ("exp_avg." + name) in st.entries:
                m1 = np.ascontiguousarray(st.read_float32("exp_avg." + name), np.float32)
                m2 = np.ascontiguousarray(st.read_float32("exp_avg_sq." + name), np.float32)
                if m1.shape != self.shapes[name] or m2.shape != self.shapes[name]:
                    raise ValueError(f"{path}: optimizer state of '{name}' has shape {m1.shape}")
                check(lib().laya_model_set_moments(self.handle, self.index[name], m1.ctypes.data, m2.ctypes.data))
        check(lib().laya_model_set_steps(self.handle, steps))

    @classmethod
    def synthetic(cls, config: ModelConfig, seed: int = 0, std: float = 0.02,
                  ctx: Optional[Context] = None) -> "TrainableDecisionModel":
        """Random init on the device: N(0, std) matrices, unit norm weights, zero biases."""
        model = cls(config, ctx)
        check(lib().laya_model_init_random(model.handle, seed & (2 ** 64 - 1), std))
        return model

    def set_param(self, name: str, values: np.ndarray) -> None:
        a = np.ascontiguousarray(values, np.float32).reshape(-1)
        if a.size != int(np.prod(self.shapes[name])):
            raise ValueError(f"{name}: {a.size} values for shape {self.shapes[name]}")
        check(lib().laya_model_set_param(self.handle, self.index[name], a.ctypes.data))

    def set_params(self, params: Dict[str, np.ndarray]) -> None:
        for name in self.names:
            if name in params:
                self.set_param(name, params[name])

    def param(self, name: str) -> np.ndarray:
        out = np.empty(self.shapes[name], np.float32)
        check(lib().laya_model_get_param(self.handle, self.index[name], out.ctypes.data))
        return out

    def grad(self, name: str) -> np.ndarray:
        out = np.empty(self.shapes[name], np.float32)
        check(lib().laya_model_get_grad(self.handle, self.index[name], out.ctypes.data))
        return out

    def _head_activation(self, layer: int, which: int):
        dev, n = ctypes.c_void_p(), ctypes.c_size_t()
        check(lib().laya_model_head_activation(self.handle, int(layer), int(which), ctypes.byref(dev),
                                               ctypes.byref(n)))
        return dev.value, n.value

    def head_activation(self, layer: int, which: str = "linear1") -> np.ndarray:
        """The last forward's saved head feed-forward activation of head layer `layer`, [tokens, head_ff]:
        "linear1" is linear1's output (the ReLU's input), "relu" the ReLU-dropout output whose sign is the
        mask the backward applies."""
        dev, n = self._head_activation(layer, {"linear1": 0, "relu": 1}[which])
        out = np.empty(n, np.float32)
        check(lib().laya_download(self.ctx.handle, out.ctypes.data, dev, out.nbytes))
        return out.reshape(-1, self.config.head_ff)

    def set_head_activation(self, layer: int, which: str, values: np.ndarray) -> None:
        """Overwrites a saved head activation (see head_activation) before the backward reads it: tests use
        it to put the ReLU decisions of ties within rounding of zero where the exact computation puts them."""
        dev, n = self._head_activation(layer, {"linear1": 0, "relu": 1}[which])
        a = np.ascontiguousarray(values, np.float32).reshape(-1)
        if a.size != n:
            raise ValueError(f"head activation: {a.size} values for {n}")
        check(lib().laya_upload(self.ctx.handle, dev, a.ctypes.data, a.nbytes))

    def has_grad(self, name: str) -> bool:
        v = ctypes.c_int()
        check(lib().laya_model_has_grad(self.handle, self.index[name], ctypes.byref(v)))
        return bool(v.value)

    def trainable(self, name: str) -> bool:
        tr = ctypes.c_int()
        check(lib().laya_model_param_info(self.handle, self.index[name], None, None, None, None, None,
                                          ctypes.byref(tr)))
        return bool(tr.value)

    @property
    def parameter_count(self) -> int:
        return sum(int(np.prod(s)) for n, s in self.shapes.items() if n != "temperature")

    @property
    def trainable_parameter_count(self) -> int:
        return sum(int(np.prod(s)) for n, s in self.shapes.items() if self.trainable(n))

    # ------------------------------------------------------------------------ training

    def set_trainable_encoder_layers(self, n: Optional[int]) -> None:
        check(lib().laya_model_set_trainable_encoder_layers(self.handle, -1 if n is None else int(n)))

    @property
    def head_dropout(self) -> float:
        return self._head_dropout

    @head_dropout.setter
    def head_dropout(self, p: float) -> None:
        check(lib().laya_model_set_head_dropout(self.handle, float(p)))
        self._head_dropout = float(p)

    CHECKPOINT_KEEP, CHECKPOINT_RECOMPUTE, CHECKPOINT_AUTO = 0, 1, 2

    @property
    def layer_checkpointing(self) -> int:
        """Layer checkpointing (TrainableDecisionModel.cs:61-64, where every layer is always checkpointed):
        0 keeps every encoder activation, 1 recomputes each encoder layer before its backward, 2 (default)
        recomputes only when keeping everything would not fit. Gradients are bitwise the same."""
        mode = ctypes.c_int()
        check(lib().laya_model_layer_checkpointing(self.handle, ctypes.byref(mode), None))
        return mode.value

    @layer_checkpointing.setter
    def layer_checkpointing(self, mode) -> None:
        if isinstance(mode, bool):
            mode = self.CHECKPOINT_RECOMPUTE if mode else self.CHECKPOINT_KEEP
        check(lib().laya_model_set_layer_checkpointing(self.handle, int(mode)))

    def set_bf16_weights(self, on: bool = True) -> None:
        """bf16 weights (PackedMatrixBf16's semantics, PackedMatrixBf16.cs:7-21): every matrix product reads each
        weight rounded to bf16 and widened back to fp32; activations stay fp32 and the fp32 weights stay the
        masters AdamW updates. Takes effect at the next forward."""
        check(lib().laya_model_set_bf16_weights(self.handle, int(bool(on))))

    def set_bf16_copies(self, on: bool) -> None:
        """Keep bf16 copies of the weights (updated by AdamW) and of the saved activations for the bf16
        products while the context's precision policy has any (the default), or drop them; same results."""
        check(lib().laya_model_set_bf16_copies(self.handle, 1 if on else 0))

    def param_bf16(self, name: str) -> np.ndarray:
        """The bf16 copy of a parameter, as float32 values (exactly representable)."""
        bits = np.zeros(int(np.prod(self.shapes[name])), np.uint16)
        check(lib().laya_model_get_param_bf16(self.handle, self.index[name], bits.ctypes.data))
        return (bits.astype(np.uint32) << 16).view(np.float32).reshape(self.shapes[name])

    @property
    def recomputing(self) -> bool:
        """Whether the current activation arena recomputes encoder layers in backward."""
        r = ctypes.c_int()
        check(lib().laya_model_layer_checkpointing(self.handle, None, ctypes.byref(r)))
        return bool(r.value)

    def forward(self, items, training: bool = False, seed: int = 0, want_logits: bool = True):
        """Forward (TrainableDecisionModel.cs:248-353): returns the per-option logits, concatenated."""
        batch = _as_batch(items)
        args = _BatchArgs(batch)
        logits = np.zeros(max(1, batch.n_markers), np.float32) if want_logits else None
        check(lib().laya_model_forward(self.handle, ctypes.byref(args.struct), int(training),
                                       seed & (2 ** 64 - 1), None if logits is None else logits.ctypes.data))
        self._batch = batch
        return None if logits is None else logits[:batch.n_markers]

    def readout(self):
        """DecisionModel.ReadOut (DecisionModel.cs:170-226) for every item of the last forward, on the device:
        (per-item option logits, action probabilities [items, n_act], calibration features [items, 4] =
        top1, top1 − top2, normalised entropy, K/255)."""
        if self._batch is None:
            raise RuntimeError("readout: run forward first")
        b = self._batch
        na = self.shapes["act_head.2.bias"][0]
        logits = np.zeros(max(1, b.n_markers), np.float32)
        probs = np.zeros((b.n_items, na), np.float32)
        feats = np.zeros((b.n_items, 4), np.float32)
        check(lib().laya_model_readout(self.handle, logits.ctypes.data, probs.ctypes.data, feats.ctypes.data))
        offs = np.concatenate([[0], np.cumsum(b.n_options)])
        return [logits[offs[i]:offs[i + 1]] for i in range(b.n_items)], probs, feats

    def decide(self, items):
        """DecisionModel.Forward (DecisionModel.cs:128-169) for a batch: the eval-mode forward and the read-out;
        returns (option logits, action probabilities) per item, as DecisionOutput holds them."""
        self.forward(items, training=False, want_logits=False)
        logits, probs, _ = self.readout()
        return [(lg, probs[i]) for i, lg in enumerate(logits)]

    def backward(self, logit_gradients) -> None:
        """Backward (TrainableDecisionModel.cs:479-549): per-option dL/dlogit, concatenated or per item."""
        if isinstance(logit_gradients, (list, tuple)):
            logit_gradients = np.concatenate([np.asarray(g, np.float32).reshape(-1) for g in logit_gradients])
        d = np.ascontiguousarray(logit_gradients, np.float32)
        check(lib().laya_model_backward(self.handle, d.ctypes.data))

    @property
    def backward_fell_back(self) -> bool:
        """Whether the last backward ran its products on three-piece splits because the items' logit gradients
        spanned more than 2^14 (two-piece products would lose precision on the smallest items' rows)."""
        v = ctypes.c_int()
        check(lib().laya_model_backward_fallback(self.handle, ctypes.byref(v)))
        return bool(v.value)

    def objective_rlcd(self, targets, draws, sigma: float, spherical_weight: float = 0.75, rps_weight: float = 1.0,
                       ce_weight: float = 1.0, scale: float = 1.0) -> tuple:
        """RlcdObjective.Compute on the last forward's logits, on the device (RlcdObjective.cs:57-155):
        targets [Σ n_options], draws [groups][Σ n_options] standard normal (None or zero groups: the
        cross-entropy term alone). The logit gradient stays on the device for backward_from_objective.
        Returns (loss, policy, cross-entropy, mean reward)."""
        t = np.ascontiguousarray(targets, np.float32).reshape(-1)
        z = np.zeros((0, t.size)) if draws is None else np.ascontiguousarray(draws, np.float64)
        groups = z.shape[0] if z.ndim > 1 else z.size // max(1, t.size)
        if z.size != groups * t.size:
            raise ValueError(f"draws: {z.size} values for {groups} groups of {t.size} options")
        out = np.zeros(4, np.float64)
        check(lib().laya_model_objective_rlcd(self.handle, t.ctypes.data, z.ctypes.data, groups, sigma,
                                              spherical_weight, rps_weight, ce_weight, scale, out.ctypes.data))
        return tuple(float(v) for v in out)

    def backward_from_objective(self) -> None:
        """Backward from the logit gradient objective_rlcd left on the device."""
        check(lib().laya_model_backward_from_objective(self.handle))

    def zero_gradients(self) -> None:
        check(lib().laya_model_zero_grad(self.handle))

    def clip_grad_norm(self, max_norm: float) -> float:
        """Gradients.ClipByGlobalNorm (AdamW.cs:103-130); the scaling is applied by the next AdamW step.
        Like the reference it returns a NaN or infinite norm and leaves such gradients unscaled;
        ``check_gradients_finite`` turns that case into an exception."""
        v = ctypes.c_double()
        rc = lib().laya_model_clip_grad_norm(self.handle, float(max_norm), ctypes.byref(v))
        if rc != ERR_NOT_FINITE:
            check(rc)
        return v.value

    def check_gradients_finite(self) -> None:
        """Raises LayaNotFiniteError when the last gradient norm (an explicit clip, or the one inside
        train_step) met a NaN or infinite gradient."""
        check(lib().laya_model_grad_norm_status(self.handle))

    def adamw_step(self, lr_encoder: float, lr_head: float, beta1: float = 0.9, beta2: float = 0.999,
                   eps: float = 1e-8, weight_decay: float = 0.01) -> None:
        check(lib().laya_model_adamw_step(self.handle, lr_encoder, lr_head, beta1, beta2, eps, weight_decay))

    @property
    def steps(self) -> int:
        v = ctypes.c_int()
        check(lib().laya_model_steps(self.handle, ctypes.byref(v)))
        return v.value

    def train_step(self, batch: Batch, targets: np.ndarray, seed: int, ce_weight: float = 1.0,
                   loss_scale: float = 1.0, max_norm: float = 1.0, lr_encoder: float = 3e-5, lr_head: float = 3e-5,
                   beta1: float = 0.9, beta2: float = 0.999, eps: float = 1e-8, weight_decay: float = 0.01,
                   want_loss: bool = False, _args: Optional[_BatchArgs] = None) -> Optional[float]:
        """One micro-step with GradAccum = 1 (Trainer.cs:131-144), CE objective on the device."""
        args = _args or _BatchArgs(batch)
        t = np.ascontiguousarray(targets, np.float32)
        loss = ctypes.c_float()
        check(lib().laya_model_train_step(self.handle, ctypes.byref(args.struct), t.ctypes.data, ce_weight,
                                          loss_scale, seed & (2 ** 64 - 1), max_norm, lr_encoder, lr_head, beta1,
                                          beta2, eps, weight_decay, ctypes.byref(loss) if want_loss else None))
        return float(loss.value) if want_loss else None

    def batch_args(self, batch: Batch) -> _BatchArgs:
        return _BatchArgs(batch)

    def stage_batch(self, batch: Batch, targets: np.ndarray) -> int:
        """Validates and uploads a batch and its soft-CE targets once; returns the slot train_step_staged
        takes. The checks and errors are train_step's."""
        args = _BatchArgs(batch)
        t = np.ascontiguousarray(targets, np.float32)
        slot = ctypes.c_int()
        check(lib().laya_model_stage_batch(self.handle, ctypes.byref(args.struct), t.ctypes.data, ctypes.byref(slot)))
        return slot.value

    def train_step_staged(self, slot: int, seed: int, ce_weight: float = 1.0, loss_scale: float = 1.0,
                          max_norm: float = 1.0, lr_encoder: float = 3e-5, lr_head: float = 3e-5, beta1: float = 0.9,
                          beta2: float = 0.999, eps: float = 1e-8, weight_decay: float = 0.01,
                          want_loss: bool = False) -> Optional[float]:
        """train_step on a staged batch: every input is already in device memory."""
        loss = ctypes.c_float()
        check(lib().laya_model_train_step_staged(self.handle, slot, ce_weight, loss_scale, seed & (2 ** 64 - 1),
                                                 max_norm, lr_encoder, lr_head, beta1, beta2, eps, weight_decay,
                                                 ctypes.byref(loss) if want_loss else None))
        return float(loss.value) if want_loss else None

    def release_batch(self, slot: int) -> None:
        check(lib().laya_model_release_batch(self.handle, slot))
