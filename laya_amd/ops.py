"""The differentiable op surface, mirroring the reference's ``Ops``
(src/StructuredDecisions.Laya.Training/Ops.cs:17-504) over device arrays.

Same names, argument meaning and conventions: a forward writes its output; ``linear_backward``
OVERWRITES its input gradient; every other backward ADDS into its input gradient; parameter
gradients always ACCUMULATE (Ops.cs:8-16). Each call is one C-ABI entry point of liblaya_hip.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from ._native import check, lib, ptr
from .device import Context, DeviceArray


class Parameter:
    """Parameter.cs:14-70: device values plus a lazily allocated, accumulating device gradient."""

    def __init__(self, ctx: Context, name: str, data: np.ndarray, trainable: bool = True):
        self.ctx = ctx
        self.name = name
        self.shape = tuple(np.shape(data))
        self.data = DeviceArray.from_numpy(ctx, np.asarray(data, np.float32))
        self.trainable = trainable
        self._grad: Optional[DeviceArray] = None

    @property
    def gradient(self) -> Optional[DeviceArray]:
        return self._grad

    def gradient_buffer(self) -> DeviceArray:
        if self._grad is None:
            self._grad = DeviceArray(self.ctx, self.shape)
        return self._grad

    def zero_gradient(self) -> None:
        if self._grad is not None:
            self._grad.fill(0.0)


def _h(ctx: Context):
    return ctx.handle


# Operand magnitude words (laya_hip.h: LAYA_AMAX_WORDS): a group of uint32 device words a binding may keep
# beside a buffer. The functions below take them as keyword arguments: an output's group receives the largest
# finite magnitude of what the call writes, and an input's group stands for that input in place of a measuring
# pass, while nothing else has written the input since the group was filled.
AMAX_WORDS = 1024


def magnitude_words(ctx: Context) -> DeviceArray:
    """A magnitude word group on the device (zeroed)."""
    return DeviceArray.from_numpy(ctx, np.zeros(AMAX_WORDS, np.uint32))


def measure_words(ctx: Context, x: DeviceArray, words: DeviceArray) -> None:
    """Fill `words` with max|x| over x's finite elements (laya_amax)."""
    check(lib().laya_amax(_h(ctx), x.ptr, x.size, words.ptr))


# ----------------------------------------------------------------------------------- linear

def linear(weight: Parameter, bias: Optional[Parameter], x: DeviceArray, rows: int, y: DeviceArray,
           residual: Optional[DeviceArray] = None, x_words: Optional[DeviceArray] = None,
           y_words: Optional[DeviceArray] = None) -> None:
    """Ops.Linear (Ops.cs:22-27): y = x·Wᵀ + b (+ residual, the skip add fused into the epilogue)."""
    out, inn = weight.shape
    b = None if bias is None else bias.data.ptr
    if x_words is None and y_words is None:
        check(lib().laya_linear_fwd(_h(weight.ctx), x.ptr, rows, inn, weight.data.ptr, out, b, ptr(residual), y.ptr))
    else:
        check(lib().laya_linear_fwd_w(_h(weight.ctx), x.ptr, rows, inn, weight.data.ptr, out, b, ptr(residual), y.ptr,
                                      ptr(x_words), None, ptr(y_words)))


def linear_backward(weight: Parameter, bias: Optional[Parameter], x: DeviceArray, dy: DeviceArray, rows: int,
                    dx: Optional[DeviceArray], x_words: Optional[DeviceArray] = None,
                    dy_words: Optional[DeviceArray] = None, dx_words: Optional[DeviceArray] = None) -> None:
    """Ops.LinearBackward (Ops.cs:33-69): dx = dy·W (overwritten), dW += dyᵀ·x, db += Σ dy."""
    out, inn = weight.shape
    dW = weight.gradient_buffer().ptr if weight.trainable else None
    db = bias.gradient_buffer().ptr if (bias is not None and bias.trainable) else None
    if x_words is None and dy_words is None and dx_words is None:
        check(lib().laya_linear_bwd(_h(weight.ctx), x.ptr, dy.ptr, rows, inn, out, weight.data.ptr, ptr(dx), dW, db))
    else:
        check(lib().laya_linear_bwd_w(_h(weight.ctx), x.ptr, dy.ptr, rows, inn, out, weight.data.ptr, ptr(dx), dW, db,
                                      ptr(x_words), ptr(dy_words), None, ptr(dx_words)))


# ------------------------------------------------------------------------------- layer norm

def layer_norm(x: DeviceArray, rows: int, n: int, weight: Parameter, bias: Optional[Parameter], epsilon: float,
               y: DeviceArray, mean: Optional[DeviceArray] = None, rstd: Optional[DeviceArray] = None,
               y_words: Optional[DeviceArray] = None) -> None:
    """Ops.LayerNorm (Ops.cs:103-110); optionally keeps the row statistics for the backward."""
    b = None if bias is None else bias.data.ptr
    if y_words is None:
        check(lib().laya_layernorm_fwd(_h(weight.ctx), x.ptr, rows, n, weight.data.ptr, b, epsilon, y.ptr, ptr(mean),
                                       ptr(rstd)))
    else:
        check(lib().laya_layernorm_fwd_w(_h(weight.ctx), x.ptr, rows, n, weight.data.ptr, b, epsilon, y.ptr,
                                         ptr(mean), ptr(rstd), y_words.ptr))


def layer_norm_backward(x: DeviceArray, rows: int, n: int, weight: Parameter, bias: Optional[Parameter],
                        epsilon: float, dy: DeviceArray, dx: DeviceArray, mean: Optional[DeviceArray] = None,
                        rstd: Optional[DeviceArray] = None, dx_words: Optional[DeviceArray] = None) -> None:
    """Ops.LayerNormBackward (Ops.cs:117-186): dx += …, dγ += Σ dy·x̂, dβ += Σ dy."""
    dg = weight.gradient_buffer().ptr if weight.trainable else None
    dbeta = bias.gradient_buffer().ptr if (bias is not None and bias.trainable) else None
    if dx_words is None:
        check(lib().laya_layernorm_bwd(_h(weight.ctx), x.ptr, rows, n, weight.data.ptr, epsilon, dy.ptr, dx.ptr, dg,
                                       dbeta, ptr(mean), ptr(rstd)))
    else:
        check(lib().laya_layernorm_bwd_w(_h(weight.ctx), x.ptr, rows, n, weight.data.ptr, epsilon, dy.ptr, dx.ptr,
                                         dg, dbeta, ptr(mean), ptr(rstd), dx_words.ptr))


# ------------------------------------------------------------------------------ activations

def gelu(ctx: Context, x: DeviceArray, y: Optional[DeviceArray] = None) -> None:
    """SimdOps.Gelu (SimdOps.cs:305-323), exact erf GELU (in place when y is None)."""
    check(lib().laya_gelu_fwd(_h(ctx), x.ptr, x.size, (y or x).ptr))


def gelu_backward(ctx: Context, u: DeviceArray, grad: DeviceArray) -> None:
    """Ops.GeluBackward (Ops.cs:194-218): grad *= Φ(u) + u·φ(u)."""
    check(lib().laya_gelu_bwd(_h(ctx), u.ptr, grad.ptr, grad.size))


def geglu(ctx: Context, wide: DeviceArray, rows: int, intermediate: int, act: DeviceArray,
          act_words: Optional[DeviceArray] = None) -> None:
    if act_words is None:
        check(lib().laya_geglu_fwd(_h(ctx), wide.ptr, rows, intermediate, act.ptr))
    else:
        check(lib().laya_geglu_fwd_w(_h(ctx), wide.ptr, rows, intermediate, act.ptr, act_words.ptr))


def geglu_backward(ctx: Context, wide: DeviceArray, dact: DeviceArray, rows: int, intermediate: int,
                   dwide: DeviceArray, dwide_words: Optional[DeviceArray] = None) -> None:
    if dwide_words is None:
        check(lib().laya_geglu_bwd(_h(ctx), wide.ptr, dact.ptr, rows, intermediate, dwide.ptr))
    else:
        check(lib().laya_geglu_bwd_w(_h(ctx), wide.ptr, dact.ptr, rows, intermediate, dwide.ptr, dwide_words.ptr))


def add(ctx: Context, dst: DeviceArray, src: DeviceArray) -> None:
    """SimdOps.Add (SimdOps.cs:84-93): dst += src (the residual adds of TrainableDecisionModel.cs:385, 402)."""
    if dst.size != src.size:
        raise ValueError(f"add: {dst.size} and {src.size} elements")
    check(lib().laya_add(_h(ctx), dst.ptr, src.ptr, dst.size))


# ---------------------------------------------------------------------------------- dropout

def uniform(seed: int, index: int) -> float:
    """Ops.Uniform (Ops.cs:227-234)."""
    return lib().laya_uniform(seed & (2 ** 64 - 1), index & (2 ** 64 - 1))


def mix(seed: int, salt: int) -> int:
    """Ops.Mix (Ops.cs:236-241)."""
    return lib().laya_mix(seed & (2 ** 64 - 1), salt & (2 ** 64 - 1))


def dropout(ctx: Context, values: DeviceArray, length: int, probability: float, seed: int) -> None:
    """Ops.Dropout (Ops.cs:244-258), in place; its own backward."""
    if probability <= 0:
        return
    check(lib().laya_dropout(_h(ctx), values.ptr, length, probability, seed & (2 ** 64 - 1)))


# -------------------------------------------------------------------------------- attention

class Rotary:
    """Rotary (Ops.cs:446-504): device cos/sin tables built in double, rounded to float."""

    def __init__(self, ctx: Context, head_dim: int, theta: float, positions: int = 1024):
        import ctypes
        self.ctx = ctx
        self.head_dim = head_dim
        self.theta = theta
        h = ctypes.c_void_p()
        check(lib().laya_rotary_create(_h(ctx), head_dim, float(theta), max(1, positions), ctypes.byref(h)))
        self.handle = h.value
        self.positions = max(1, positions)
        ctx.register(self)

    def close(self) -> None:
        if getattr(self, "handle", None) and getattr(self.ctx, "handle", None):
            lib().laya_rotary_destroy(self.ctx.handle, self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def ensure(self, positions: int) -> None:
        if positions > self.positions:
            self.close()
            self.__init__(self.ctx, self.head_dim, self.theta, max(positions, 2 * self.positions))

    def apply(self, vec: DeviceArray, rows: int, positions: DeviceArray, inverse: bool) -> None:
        check(lib().laya_rotary_apply(_h(self.ctx), self.handle, vec.ptr, rows, positions.ptr, int(inverse)))


@dataclass
class AttentionShape:
    """Ops.AttentionShape (Ops.cs:263-267). half_window < 0 (or None) means no window."""
    hidden: int
    heads: int
    scale: float
    half_window: Optional[int]
    rotary: Optional[Rotary]
    dropout: float
    seed: int

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


class Segments:
    """The concatenated items of a batch (ModernBertEncoder.Segment), uploaded once as a laya_segments
    handle that every attention call of the batch shares."""

    def __init__(self, ctx: Context, lengths: Sequence[int], starts: Optional[Sequence[int]] = None):
        import ctypes
        lengths = np.ascontiguousarray(lengths, np.int32)
        self.ctx = ctx
        self.lengths = lengths
        if starts is None:
            starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]) if len(lengths) else np.zeros(0)
        self.starts = np.ascontiguousarray(starts, np.int32)
        self.count = len(lengths)
        self.max_len = int(lengths.max()) if len(lengths) else 0
        self.rows = int((self.starts + lengths).max()) if len(lengths) else 0
        h = ctypes.c_void_p()
        check(lib().laya_segments_create(_h(ctx), self.starts.ctypes.data, lengths.ctypes.data, self.count,
                                         ctypes.byref(h)))
        self.handle = h.value
        ctx.register(self)

    def close(self) -> None:
        if getattr(self, "handle", None) and getattr(self.ctx, "handle", None):
            lib().laya_segments_destroy(self.ctx.handle, self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _hw(shape: AttentionShape) -> int:
    return -1 if shape.half_window is None or shape.half_window < 0 else int(shape.half_window)


def attention_forward(qkv: DeviceArray, segments: Segments, shape: AttentionShape, context: DeviceArray,
                      lse: DeviceArray, qkv_words: Optional[DeviceArray] = None,
                      context_words: Optional[DeviceArray] = None) -> None:
    """Ops.AttentionForward (Ops.cs:275-277); also writes the row log-sum-exp the backward may reuse."""
    if shape.rotary is not None:
        shape.rotary.ensure(segments.max_len)
    args = (_h(qkv.ctx), qkv.ptr, segments.handle, shape.hidden, shape.heads, shape.scale, _hw(shape),
            None if shape.rotary is None else shape.rotary.handle, shape.dropout, shape.seed & (2 ** 64 - 1),
            context.ptr, lse.ptr)
    if qkv_words is None and context_words is None:
        check(lib().laya_attention_fwd(*args))
    else:
        check(lib().laya_attention_fwd_w(*args, ptr(qkv_words), ptr(context_words)))


def attention_backward(qkv: DeviceArray, segments: Segments, shape: AttentionShape, dcontext: DeviceArray,
                       dqkv: DeviceArray, context: Optional[DeviceArray] = None,
                       lse: Optional[DeviceArray] = None, qkv_words: Optional[DeviceArray] = None,
                       dcontext_words: Optional[DeviceArray] = None,
                       dqkv_words: Optional[DeviceArray] = None) -> None:
    """Ops.AttentionBackward (Ops.cs:280-282): dq, dk, dv written (not added) into dqkv. The forward's
    context and lse are reused when given; without them the row statistics are recomputed, as the
    reference recomputes each row's softmax."""
    if shape.rotary is not None:
        shape.rotary.ensure(segments.max_len)
    args = (_h(qkv.ctx), qkv.ptr, segments.handle, shape.hidden, shape.heads, shape.scale, _hw(shape),
            None if shape.rotary is None else shape.rotary.handle, shape.dropout, shape.seed & (2 ** 64 - 1),
            ptr(context), ptr(lse), dcontext.ptr, dqkv.ptr)
    if qkv_words is None and dcontext_words is None and dqkv_words is None:
        check(lib().laya_attention_bwd(*args))
    else:
        check(lib().laya_attention_bwd_w(*args, ptr(qkv_words), ptr(dcontext_words), ptr(dqkv_words)))


def default_scale(head_dim: int) -> float:
    """1/√d_h as the reference computes it in float (TrainableDecisionModel.cs:417)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


# ------------------------------------------------------------------ rows, embeddings, objective

def gather_rows(ctx: Context, src: DeviceArray, rows: DeviceArray, n: int, width: int, dst: DeviceArray) -> None:
    check(lib().laya_gather_rows(_h(ctx), src.ptr, rows.ptr, n, width, dst.ptr))


def scatter_add_rows(ctx: Context, src: DeviceArray, rows: DeviceArray, n: int, width: int, dst: DeviceArray) -> None:
    check(lib().laya_scatter_add_rows(_h(ctx), src.ptr, rows.ptr, n, width, dst.ptr))


def type_embedding(ctx: Context, states: DeviceArray, qtype_of_row: DeviceArray, rows: int, width: int,
                   table: Parameter) -> None:
    """TrainableDecisionModel.cs:300-304: each row gets its item's question-type vector added."""
    check(lib().laya_type_embedding_fwd(_h(ctx), states.ptr, qtype_of_row.ptr, rows, width, table.data.ptr))


def type_embedding_backward(ctx: Context, dstates: DeviceArray, qtype_of_row: DeviceArray, rows: int, width: int,
                            table: Parameter) -> None:
    """TrainableDecisionModel.cs:512-521: the type vectors' gradient, Σ of their rows' gradients."""
    if table.trainable:
        check(lib().laya_type_embedding_bwd(_h(ctx), dstates.ptr, qtype_of_row.ptr, rows, width,
                                            table.gradient_buffer().ptr))


def embedding_plan(ids: np.ndarray, vocab: int):
    """Token positions stably sorted by id, the unique ids and their run offsets."""
    import ctypes
    ids = np.ascontiguousarray(ids, np.int32)
    n = ids.size
    sorted_pos = np.zeros(max(n, 1), np.int32)
    unique = np.zeros(max(n, 1), np.int32)
    offsets = np.zeros(n + 1, np.int32)
    nu = ctypes.c_int()
    check(lib().laya_embedding_plan(ids.ctypes.data, n, vocab, sorted_pos.ctypes.data, unique.ctypes.data,
                                    offsets.ctypes.data, ctypes.byref(nu)))
    return sorted_pos[:n], unique[:nu.value], offsets[:nu.value + 1]


def embedding_backward(ctx: Context, ids: np.ndarray, d: DeviceArray, hidden: int, grad: DeviceArray,
                       vocab: int) -> None:
    """grad[id] += Σ d[t] over that id's tokens, in token order (TrainableDecisionModel.cs:543-547)."""
    sp, un, off = embedding_plan(ids, vocab)
    if un.size == 0:
        return
    a, b, c = (DeviceArray.from_numpy(ctx, x) for x in (sp, un, off))
    check(lib().laya_embedding_bwd(_h(ctx), a.ptr, b.ptr, c.ptr, un.size, d.ptr, hidden, grad.ptr))
    ctx.sync()


def softmax_ce_backward(ctx: Context, logits: DeviceArray, targets: DeviceArray, option_offsets: DeviceArray,
                        n_items: int, ce_weight: float, scale: float, grad: DeviceArray,
                        loss: Optional[DeviceArray] = None) -> None:
    check(lib().laya_softmax_ce_bwd(_h(ctx), logits.ptr, targets.ptr, option_offsets.ptr, n_items, ce_weight, scale,
                                    grad.ptr, ptr(loss)))


def rlcd_objective(ctx: Context, logits: DeviceArray, targets: DeviceArray, option_offsets: DeviceArray,
                   qtypes: DeviceArray, n_options, draws: DeviceArray, groups: int, sigma: float,
                   spherical_weight: float = 0.75, rps_weight: float = 1.0, ce_weight: float = 1.0,
                   scale: float = 1.0, grad: Optional[DeviceArray] = None) -> tuple:
    """RlcdObjective.Compute (RlcdObjective.cs:57-155) with supplied standard-normal draws
    [groups][Σ n_options] (a float64 device array), on the device. Returns (losses, grad): losses =
    (total, policy, cross-entropy, mean reward), grad the scaled logit gradient (device)."""
    n_options = np.asarray(n_options, np.int64)
    total, longest = int(n_options.sum()), int(n_options.max()) if n_options.size else 0
    grad = grad or DeviceArray(ctx, (max(total, 1),))
    losses = DeviceArray(ctx, (8,))  # four doubles
    check(lib().laya_rlcd_objective(_h(ctx), logits.ptr, targets.ptr, option_offsets.ptr, qtypes.ptr, len(n_options),
                                    total, longest, groups, draws.ptr, sigma, spherical_weight, rps_weight, ce_weight,
                                    scale, grad.ptr, losses.ptr))
    out = np.zeros(4, np.float64)
    check(lib().laya_download(_h(ctx), out.ctypes.data, losses.ptr, 32))
    losses.free()
    return tuple(float(v) for v in out), grad


def layer_norm_eps_default() -> float:
    return 1e-5


def attention_scale(hidden: int, heads: int) -> float:
    return 1.0 / math.sqrt(hidden // heads)
