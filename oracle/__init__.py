"""Oracle bindings — test infrastructure only.

ctypes bindings over ``oracle/liblaya_oracle.so``, the C++ restatement of the reference's C# CPU
fine-tuning path (see ``laya_oracle.cpp``). Only ``tests/``, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` import this package, and only as the checker or the timed CPU
baseline; the product library never loads it.

Parity status of each restated function is recorded next to its tests: every function here is
pinned by the reference's golden fixture (tests/golden/training-tiny), by closed forms, or by
fp64 autograd / finite differences.
"""
from __future__ import annotations

import ctypes
import os
from typing import Dict, List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblaya_oracle.so")
_lib = None

c_int, c_long, c_float, c_double, c_u64 = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_double, ctypes.c_uint64
P = ctypes.c_void_p


class OrcConfig(ctypes.Structure):
    _fields_ = [("vocab", c_int), ("hidden", c_int), ("intermediate", c_int), ("layers", c_int), ("heads", c_int),
                ("local_attention", c_int), ("global_every", c_int), ("layer_kinds", ctypes.POINTER(c_int)),
                ("theta_global", c_double), ("theta_local", c_double), ("norm_eps", c_float),
                ("norm_bias", c_int), ("attention_bias", c_int), ("mlp_bias", c_int),
                ("head_layers", c_int), ("head_ff", c_int), ("n_act", c_int)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_last_error.restype = ctypes.c_char_p
        L.orc_model_create.restype = P
        L.orc_model_create.argtypes = [ctypes.POINTER(OrcConfig), c_int]
        for name in ["orc_model_destroy", "orc_model_zero_grad"]:
            getattr(L, name).argtypes = [P]
            getattr(L, name).restype = None
        L.orc_model_num_params.argtypes = [P]
        L.orc_model_param_name.argtypes = [P, c_int]
        L.orc_model_param_name.restype = ctypes.c_char_p
        L.orc_model_param_ndim.argtypes = [P, c_int]
        L.orc_model_param_dim.argtypes = [P, c_int, c_int]
        L.orc_model_param_numel.argtypes = [P, c_int]
        L.orc_model_param_numel.restype = c_long
        L.orc_model_param_trainable.argtypes = [P, c_int]
        L.orc_model_has_grad.argtypes = [P, c_int]
        L.orc_model_set_param.argtypes = [P, c_int, P]
        L.orc_model_get_param.argtypes = [P, c_int, P]
        L.orc_model_get_grad.argtypes = [P, c_int, P]
        L.orc_model_set_trainable_encoder_layers.argtypes = [P, c_int]
        L.orc_model_set_head_dropout.argtypes = [P, c_float]
        L.orc_model_forward.argtypes = [P, c_int, P, P, P, P, P, c_int, c_int, c_u64, P]
        L.orc_model_backward.argtypes = [P, P]
        L.orc_model_readout.argtypes = [P, P, P, P]
        L.orc_model_clip.argtypes = [P, c_double]
        L.orc_model_clip.restype = c_double
        L.orc_model_adamw.argtypes = [P, c_double, c_double, c_double, c_double, c_double, c_double]
        L.orc_model_adamw.restype = None
        L.orc_model_steps.argtypes = [P]
        L.orc_model_set_capture_head.argtypes = [P, c_int]
        L.orc_model_set_capture_head.restype = None
        L.orc_model_head_preactivation.argtypes = [P, c_int, P]
        L.orc_model_head_preactivation.restype = c_long
        L.orc_set_threads.argtypes = [c_int]
        L.orc_set_threads.restype = c_int
        L.orc_uniform.argtypes = [c_u64, c_u64]
        L.orc_uniform.restype = c_float
        L.orc_mix.argtypes = [c_u64, c_u64]
        L.orc_mix.restype = c_u64
        L.orc_exp_f32.argtypes = [c_float]
        L.orc_exp_f32.restype = c_float
        L.orc_erf_f32.argtypes = [c_float]
        L.orc_erf_f32.restype = c_float
        for s in ("f32", "f64"):
            getattr(L, f"orc_gemm_{s}").argtypes = [c_int, c_int, c_int, P, c_long, c_long, P, c_long, c_long, P,
                                                      c_long, c_int]
            getattr(L, f"orc_linear_{s}").argtypes = [P, c_int, c_int, P, c_int, P, P]
            getattr(L, f"orc_linear_backward_{s}").argtypes = [P, P, c_int, c_int, c_int, P, P, P, P]
            getattr(L, f"orc_layernorm_{s}").argtypes = [P, c_int, c_int, P, P, c_float, P]
            getattr(L, f"orc_layernorm_backward_{s}").argtypes = [P, c_int, c_int, P, c_float, P, P, P, P]
            getattr(L, f"orc_gelu_{s}").argtypes = [P, c_long]
            getattr(L, f"orc_gelu_backward_{s}").argtypes = [P, P, c_long]
            getattr(L, f"orc_geglu_{s}").argtypes = [P, c_int, c_int, P]
            getattr(L, f"orc_geglu_backward_{s}").argtypes = [P, P, c_int, c_int, P]
            getattr(L, f"orc_dropout_{s}").argtypes = [P, c_long, c_float, c_u64]
            getattr(L, f"orc_rotary_apply_{s}").argtypes = [c_double, c_int, P, c_int, c_int]
            getattr(L, f"orc_attention_forward_{s}").argtypes = [P, c_int, P, P, c_int, c_int, c_float, c_int,
                                                                   c_double, c_float, c_u64, P]
            getattr(L, f"orc_attention_backward_{s}").argtypes = [P, c_int, P, P, c_int, c_int, c_float, c_int,
                                                                    c_double, c_float, c_u64, P, P]
            getattr(L, f"orc_adamw_tensor_{s}").argtypes = [P, P, P, P, c_long, c_double, c_double, c_double,
                                                              c_double, c_double, c_int]
        L.orc_clip_f32.argtypes = [c_int, P, P, c_double]
        L.orc_clip_f32.restype = c_double
        L.orc_cross_entropy.argtypes = [c_int, P, P, P, c_double, c_double, P]
        L.orc_cross_entropy.restype = c_double
        L.orc_rlcd.argtypes = [c_int, P, P, P, P, c_int, P, c_double, c_double, c_double, c_double, c_double, P, P]
        L.orc_proper_reward.argtypes = [c_int, P, P, c_int, c_double, c_double]
        L.orc_proper_reward.restype = c_double
        _lib = L
    return _lib


def ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _ftype(double: bool):
    return (np.float64, "f64") if double else (np.float32, "f32")


def make_config(mc) -> (OrcConfig, object):
    """OrcConfig from a ``laya_amd.config.ModelConfig``; returns the struct and the kinds buffer."""
    e = mc.encoder
    kinds = (c_int * e.num_hidden_layers)(*e.layer_kinds)
    cfg = OrcConfig(vocab=e.vocab_size, hidden=e.hidden_size, intermediate=e.intermediate_size,
                    layers=e.num_hidden_layers, heads=e.num_attention_heads, local_attention=e.local_attention,
                    global_every=e.global_attn_every_n_layers, layer_kinds=kinds,
                    theta_global=e.global_rope_theta, theta_local=e.local_rope_theta, norm_eps=e.norm_eps,
                    norm_bias=int(e.norm_bias), attention_bias=int(e.attention_bias), mlp_bias=int(e.mlp_bias),
                    head_layers=mc.head_layers, head_ff=mc.head_ff, n_act=mc.n_act)
    return cfg, kinds


class OracleModel:
    """The reference ``TrainableDecisionModel`` + ``AdamW`` + ``Gradients`` restated on the CPU."""

    def __init__(self, mc, double: bool = False):
        self.mc = mc
        self.double = double
        L = lib()
        cfg, kinds = make_config(mc)
        self._h = L.orc_model_create(ctypes.byref(cfg), int(double))
        if not self._h:
            raise RuntimeError(L.orc_last_error().decode())
        n = L.orc_model_num_params(self._h)
        self.names: List[str] = []
        self.shapes: Dict[str, tuple] = {}
        for i in range(n):
            name = L.orc_model_param_name(self._h, i).decode()
            shape = tuple(L.orc_model_param_dim(self._h, i, d) for d in range(L.orc_model_param_ndim(self._h, i)))
            self.names.append(name)
            self.shapes[name] = shape
        self.index = {nm: i for i, nm in enumerate(self.names)}

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_model_destroy(self._h)
            self._h = None

    def set_params(self, params: Dict[str, np.ndarray]) -> None:
        for name in self.names:
            if name not in params:
                raise KeyError(f"missing parameter '{name}'")
            a = np.ascontiguousarray(params[name], dtype=np.float32).reshape(-1)
            if a.size != int(np.prod(self.shapes[name])):
                raise ValueError(f"{name}: size {a.size} vs shape {self.shapes[name]}")
            lib().orc_model_set_param(self._h, self.index[name], ptr(a))

    def param(self, name: str) -> np.ndarray:
        out = np.zeros(int(np.prod(self.shapes[name])), np.float64)
        lib().orc_model_get_param(self._h, self.index[name], ptr(out))
        return out.reshape(self.shapes[name])

    def grad(self, name: str) -> np.ndarray:
        out = np.zeros(int(np.prod(self.shapes[name])), np.float64)
        lib().orc_model_get_grad(self._h, self.index[name], ptr(out))
        return out.reshape(self.shapes[name])

    def has_grad(self, name: str) -> bool:
        return bool(lib().orc_model_has_grad(self._h, self.index[name]))

    def trainable(self, name: str) -> bool:
        return bool(lib().orc_model_param_trainable(self._h, self.index[name]))

    def set_trainable_encoder_layers(self, n: Optional[int]) -> None:
        lib().orc_model_set_trainable_encoder_layers(self._h, -1 if n is None else int(n))

    def set_head_dropout(self, p: float) -> None:
        lib().orc_model_set_head_dropout(self._h, float(p))

    def forward(self, batch, training: bool = False, keep_tape: bool = True, seed: int = 0) -> np.ndarray:
        logits = np.zeros(batch.n_markers, np.float64)
        a = [np.ascontiguousarray(x, dtype=np.int32) for x in
             (batch.lengths, batch.tokens, batch.n_options, batch.markers, batch.qtypes)]
        rc = lib().orc_model_forward(self._h, batch.n_items, *[ptr(x) for x in a], int(training), int(keep_tape),
                                     ctypes.c_uint64(seed & (2**64 - 1)), ptr(logits))
        if rc != 0:
            raise RuntimeError(lib().orc_last_error().decode())
        self._last_opts = np.asarray(batch.n_options)
        return logits

    def backward(self, dlogits: np.ndarray) -> None:
        d = np.ascontiguousarray(dlogits, dtype=np.float32)
        if lib().orc_model_backward(self._h, ptr(d)) != 0:
            raise RuntimeError(lib().orc_last_error().decode())

    def readout(self):
        """DecisionModel.ReadOut on the last forward: (action probabilities [items, n_act], features
        [items, 4] = top1, top1 − top2, normalised entropy, K/255, pooled rows [items, d])."""
        n = len(self._last_opts)
        na = self.shapes["act_head.2.bias"][0]
        probs = np.zeros((n, na), np.float32)
        feats = np.zeros((n, 4), np.float32)
        pooled = np.zeros((n, self.shapes["type_emb.weight"][1]), np.float64)
        if lib().orc_model_readout(self._h, ptr(probs), ptr(feats), ptr(pooled)) != 0:
            raise RuntimeError(lib().orc_last_error().decode())
        return probs, feats, pooled

    def zero_grad(self) -> None:
        lib().orc_model_zero_grad(self._h)

    def capture_head_preactivations(self, on: bool = True) -> None:
        """Keep each head layer's linear1 output (the ReLU's input) of the forwards that follow."""
        lib().orc_model_set_capture_head(self._h, int(on))

    def head_preactivation(self, layer: int) -> np.ndarray:
        """Head layer `layer`'s linear1 output of the last forward, [tokens, head_ff], in double."""
        n = lib().orc_model_head_preactivation(self._h, int(layer), None)
        if n < 0:
            raise RuntimeError("no head pre-activations kept (call capture_head_preactivations first)")
        out = np.empty(n, np.float64)
        lib().orc_model_head_preactivation(self._h, int(layer), ptr(out))
        return out.reshape(-1, self.mc.head_ff)

    def clip(self, max_norm: float) -> float:
        return lib().orc_model_clip(self._h, float(max_norm))

    def adamw(self, lr_encoder: float, lr_head: float, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01):
        lib().orc_model_adamw(self._h, lr_encoder, lr_head, beta1, beta2, eps, weight_decay)


# ------------------------------------------------------------------------------------ op wrappers

def set_threads(n: int) -> int:
    """OpenMP threads of the oracle's later calls; returns the previous count."""
    return lib().orc_set_threads(int(n))


def uniform(seed: int, index: int) -> float:
    return lib().orc_uniform(seed & (2**64 - 1), index & (2**64 - 1))


def mix(seed: int, salt: int) -> int:
    return lib().orc_mix(seed & (2**64 - 1), salt & (2**64 - 1))


def linear(x, W, b=None, double=False):
    ft, s = _ftype(double)
    x = np.ascontiguousarray(x, ft)
    W = np.ascontiguousarray(W, ft)
    b = None if b is None else np.ascontiguousarray(b, ft)
    rows, inn = x.shape
    out = W.shape[0]
    y = np.zeros((rows, out), ft)
    getattr(lib(), f"orc_linear_{s}")(ptr(x), rows, inn, ptr(W), out, ptr(b), ptr(y))
    return y


def linear_backward(x, dy, W, want_dx=True, dW=None, db=None, double=False):
    ft, s = _ftype(double)
    x, dy, W = (np.ascontiguousarray(a, ft) for a in (x, dy, W))
    rows, inn = x.shape
    out = W.shape[0]
    dx = np.zeros((rows, inn), ft) if want_dx else None
    getattr(lib(), f"orc_linear_backward_{s}")(ptr(x), ptr(dy), rows, inn, out, ptr(W), ptr(dx), ptr(dW), ptr(db))
    return dx


def layernorm(x, w, b, eps, double=False):
    ft, s = _ftype(double)
    x, w = np.ascontiguousarray(x, ft), np.ascontiguousarray(w, ft)
    b = None if b is None else np.ascontiguousarray(b, ft)
    y = np.zeros_like(x)
    getattr(lib(), f"orc_layernorm_{s}")(ptr(x), x.shape[0], x.shape[1], ptr(w), ptr(b), eps, ptr(y))
    return y


def layernorm_backward(x, w, eps, dy, dx, dgamma=None, dbeta=None, double=False):
    ft, s = _ftype(double)
    x, w, dy = (np.ascontiguousarray(a, ft) for a in (x, w, dy))
    getattr(lib(), f"orc_layernorm_backward_{s}")(ptr(x), x.shape[0], x.shape[1], ptr(w), eps, ptr(dy), ptr(dx),
                                                   ptr(dgamma), ptr(dbeta))


def gelu(x, double=False):
    ft, s = _ftype(double)
    y = np.array(x, dtype=ft, copy=True).reshape(-1)
    getattr(lib(), f"orc_gelu_{s}")(ptr(y), y.size)
    return y.reshape(np.shape(x))


def gelu_backward(u, grad, double=False):
    ft, s = _ftype(double)
    u = np.ascontiguousarray(u, ft).reshape(-1)
    g = np.array(grad, dtype=ft, copy=True).reshape(-1)
    getattr(lib(), f"orc_gelu_backward_{s}")(ptr(u), ptr(g), g.size)
    return g.reshape(np.shape(grad))


def geglu(wide, double=False):
    ft, s = _ftype(double)
    wide = np.ascontiguousarray(wide, ft)
    rows, two_i = wide.shape
    act = np.zeros((rows, two_i // 2), ft)
    getattr(lib(), f"orc_geglu_{s}")(ptr(wide), rows, two_i // 2, ptr(act))
    return act


def geglu_backward(wide, dact, double=False):
    ft, s = _ftype(double)
    wide, dact = np.ascontiguousarray(wide, ft), np.ascontiguousarray(dact, ft)
    dwide = np.zeros_like(wide)
    getattr(lib(), f"orc_geglu_backward_{s}")(ptr(wide), ptr(dact), wide.shape[0], wide.shape[1] // 2, ptr(dwide))
    return dwide


def dropout(values, p, seed, double=False):
    ft, s = _ftype(double)
    v = np.array(values, dtype=ft, copy=True).reshape(-1)
    getattr(lib(), f"orc_dropout_{s}")(ptr(v), v.size, float(p), seed & (2**64 - 1))
    return v.reshape(np.shape(values))


def rotary_apply(theta, vec, position, inverse=False, double=False):
    ft, s = _ftype(double)
    v = np.array(vec, dtype=ft, copy=True)
    getattr(lib(), f"orc_rotary_apply_{s}")(theta, v.size, ptr(v), position, int(inverse))
    return v


def _segs(lengths):
    lengths = np.asarray(lengths, np.int32)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int32)
    return starts, lengths


def attention_forward(qkv, lengths, heads, scale, half_window=-1, theta=0.0, dropout=0.0, seed=0, double=False):
    ft, s = _ftype(double)
    qkv = np.ascontiguousarray(qkv, ft)
    hidden = qkv.shape[1] // 3
    starts, lengths = _segs(lengths)
    ctx = np.zeros((qkv.shape[0], hidden), ft)
    getattr(lib(), f"orc_attention_forward_{s}")(ptr(qkv), len(lengths), ptr(starts), ptr(lengths), hidden, heads,
                                                  scale, half_window, theta, dropout, seed & (2**64 - 1), ptr(ctx))
    return ctx


def attention_backward(qkv, dctx, lengths, heads, scale, half_window=-1, theta=0.0, dropout=0.0, seed=0,
                       double=False):
    ft, s = _ftype(double)
    qkv, dctx = np.ascontiguousarray(qkv, ft), np.ascontiguousarray(dctx, ft)
    hidden = qkv.shape[1] // 3
    starts, lengths = _segs(lengths)
    dqkv = np.zeros_like(qkv)
    getattr(lib(), f"orc_attention_backward_{s}")(ptr(qkv), len(lengths), ptr(starts), ptr(lengths), hidden, heads,
                                                   scale, half_window, theta, dropout, seed & (2**64 - 1), ptr(dctx),
                                                   ptr(dqkv))
    return dqkv


def adamw_tensor(p, g, m, v, lr, step, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, double=False):
    ft, s = _ftype(double)
    getattr(lib(), f"orc_adamw_tensor_{s}")(ptr(p), ptr(g), ptr(m), ptr(v), p.size, lr, beta1, beta2, eps,
                                             weight_decay, step)


def clip(grads, max_norm):
    """ClipByGlobalNorm over a list of fp32 arrays (scaled in place); returns the norm."""
    arr = (ctypes.c_void_p * len(grads))(*[g.ctypes.data for g in grads])
    lens = np.array([g.size for g in grads], np.int64)
    return lib().orc_clip_f32(len(grads), arr, ptr(lens), max_norm)


def cross_entropy(n_options, logits, targets, ce_weight=1.0, scale=1.0):
    n_options = np.ascontiguousarray(n_options, np.int32)
    logits = np.ascontiguousarray(logits, np.float32)
    targets = np.ascontiguousarray(targets, np.float32)
    g = np.zeros_like(logits)
    ce = lib().orc_cross_entropy(len(n_options), ptr(n_options), ptr(logits), ptr(targets), ce_weight, scale, ptr(g))
    return ce, g


def rlcd(n_options, qtypes, logits, targets, draws, sigma, spherical=0.75, rps=1.0, ce_weight=1.0, scale=1.0):
    n_options = np.ascontiguousarray(n_options, np.int32)
    qtypes = np.ascontiguousarray(qtypes, np.int32)
    logits = np.ascontiguousarray(logits, np.float32)
    targets = np.ascontiguousarray(targets, np.float32)
    draws = np.ascontiguousarray(draws, np.float64)
    groups = draws.size // max(1, logits.size)
    g = np.zeros_like(logits)
    out = np.zeros(4, np.float64)
    lib().orc_rlcd(len(n_options), ptr(n_options), ptr(qtypes), ptr(logits), ptr(targets), groups, ptr(draws),
                   sigma, spherical, rps, ce_weight, scale, ptr(g), ptr(out))
    return out, g
