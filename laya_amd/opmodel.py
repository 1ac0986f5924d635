"""A training step of the decision model composed from the per-op entry points alone.

This is what a host that keeps the reference's autograd and re-points ``Ops`` (Ops.cs:17-439) at
liblaya_hip runs: ``TrainableDecisionModel.Forward`` (TrainableDecisionModel.cs:248-353, with
EncoderLayerForward 361-414 and HeadLayerForward 428-468), the soft cross-entropy gradient
(RlcdObjective.cs:139-150), ``Backward`` (479-549, EncoderLayerBackward 551-603, HeadLayerBackward 605-640),
``Gradients.ClipByGlobalNorm`` and ``AdamW.Step`` (AdamW.cs:29-73, 103-130), each op one C-ABI call
(laya_amd.ops) on device arrays the host owns. Parameters, gradients and both moments are views into four
flat arenas (one allocation each, in the checkpoint's tensor order), so the clip and the optimizer run over
them as the model driver's do. Every op recomputes what the op surface does not carry between calls: the
linears measure their operands' magnitudes at each call and attention rotates a copy of q and k. The host
keeps each attention forward's context and LSE beside its qkv and hands them to the backward, as the C#
binding does (``Ops.AttentionBackward`` carries neither; without them the backward reruns the row statistics).

The model driver (laya_amd.model.TrainableDecisionModel) runs the same step with its own fusions; the two
are compared in the tests and timed side by side by ``bench.py --per-op``.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional

import numpy as np

from . import ops as laya
from ._native import check, lib
from .batch import Batch
from .config import ModelConfig
from .device import Context, DeviceArray


class _View:
    """A device array inside an arena (the op wrappers read .ptr, .size, .ctx)."""

    def __init__(self, ctx: Context, ptr: int, shape):
        self.ctx = ctx
        self.ptr = ptr
        self.shape = tuple(int(s) for s in shape)
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = 4 * self.size

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, np.float32)
        check(lib().laya_download(self.ctx.handle, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def fill(self, value: float) -> None:
        check(lib().laya_fill(self.ctx.handle, self.ptr, float(value), self.size))


class _Param:
    """Parameter.cs's surface for the op wrappers: values and gradient as arena views."""

    def __init__(self, ctx: Context, name: str, shape, data: _View, grad: _View, trainable: bool):
        self.ctx, self.name, self.shape = ctx, name, tuple(shape)
        self.data, self._grad, self.trainable = data, grad, trainable

    @property
    def gradient(self):
        return self._grad

    def gradient_buffer(self):
        return self._grad


class _Scratch:
    """Activation buffers sized for the largest batch seen; views of the current batch's rows."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.arrays: Dict[str, DeviceArray] = {}

    def get(self, key: str, shape) -> _View:
        n = int(np.prod(shape))
        a = self.arrays.get(key)
        if a is None or a.size < n:
            if a is not None:
                a.free()
            a = DeviceArray(self.ctx, (max(n, 4),), zero=False)
            self.arrays[key] = a
        return _View(self.ctx, a.ptr, shape)

    def free(self) -> None:
        for a in self.arrays.values():
            a.free()
        self.arrays.clear()


class OpBatch:
    """A batch's device tables for the op-level step (uploaded once, before the step)."""

    def __init__(self, ctx: Context, batch: Batch, targets: np.ndarray, vocab: int):
        self.batch = batch
        self.T, self.n_items, self.n_markers = batch.n_tokens, batch.n_items, batch.n_markers
        self.segments = laya.Segments(ctx, batch.lengths, batch.starts())
        self.tokens_host = np.ascontiguousarray(batch.tokens, np.int32)
        if self.tokens_host.size and (self.tokens_host.min() < 0 or self.tokens_host.max() >= vocab):
            raise IndexError("a token id is outside the vocabulary")
        self.tokens = DeviceArray.from_numpy(ctx, self.tokens_host)
        self.marker_rows = DeviceArray.from_numpy(ctx, batch.marker_rows())
        self.row_type = DeviceArray.from_numpy(ctx, np.repeat(batch.qtypes, batch.lengths).astype(np.int32))
        offsets = np.concatenate([[0], np.cumsum(batch.n_options)]).astype(np.int32)
        self.offsets = DeviceArray.from_numpy(ctx, offsets)
        self.targets = DeviceArray.from_numpy(ctx, np.ascontiguousarray(targets, np.float32))
        sp, un, off = laya.embedding_plan(self.tokens_host, vocab)
        self.plan = (DeviceArray.from_numpy(ctx, sp), DeviceArray.from_numpy(ctx, un),
                     DeviceArray.from_numpy(ctx, off), int(un.size))

    def close(self) -> None:
        self.segments.close()
        for a in (self.tokens, self.marker_rows, self.row_type, self.offsets, self.targets, *self.plan[:3]):
            a.free()


class OpLevelModel:
    """TrainableDecisionModel over the per-op C-ABI. `params` maps every parameter name, in the checkpoint's
    order, to its values; `temperature` is frozen and the act head gets no gradient (it is still decayed)."""

    def __init__(self, config: ModelConfig, params: Dict[str, np.ndarray], ctx: Context):
        self.config, self.ctx = config, ctx
        self.names: List[str] = list(params)
        self.shapes = {n: tuple(np.shape(v)) for n, v in params.items()}
        off, self.offsets = 0, {}
        for n in self.names:
            self.offsets[n] = off
            off += (int(np.prod(self.shapes[n])) + 63) // 64 * 64  # 256-byte aligned tensors
        self.total = off
        self.arena = {k: DeviceArray(ctx, (self.total,)) for k in ("P", "G", "M1", "M2")}
        self.p: Dict[str, _Param] = {}
        for n in self.names:
            o, shape = self.offsets[n], self.shapes[n]
            self.p[n] = _Param(ctx, n, shape, _View(ctx, self.arena["P"].ptr + 4 * o, shape),
                               _View(ctx, self.arena["G"].ptr + 4 * o, shape), n != "temperature")
            a = np.ascontiguousarray(params[n], np.float32)
            check(lib().laya_upload(ctx.handle, self.p[n].data.ptr, a.ctypes.data, a.nbytes))
        # AdamW's two groups (Trainer.cs:96-100): the encoder's tensors, then the rest; temperature last, frozen.
        self.encoder_end = min(self.offsets[n] for n in self.names if not n.startswith("encoder."))
        self.head_end = self.offsets["temperature"] if "temperature" in self.offsets else self.total
        self.steps = 0
        self.head_dropout = 0.1
        self.carry_attention_state = True
        # The operands' magnitude word groups, kept beside the encoder's buffers the host writes through the
        # per-op calls (laya_hip.h's _w variants): the products read them instead of measuring (False: every
        # product measures its operands, as a binding without them does).
        self.carry_words = True
        self._words: Dict[str, DeviceArray] = {}
        self._dout_words_valid = False
        self.rot_global = laya.Rotary(ctx, config.encoder.head_dim, config.encoder.global_rope_theta, 1024)
        self.rot_local = laya.Rotary(ctx, config.encoder.head_dim, config.encoder.local_rope_theta, 1024)
        self.s = _Scratch(ctx)
        self.norm = DeviceArray(ctx, (4,))  # the clip's norm (double) and coefficient (float)

    def close(self) -> None:
        self.s.free()
        for w in self._words.values():
            w.free()
        self._words.clear()
        for a in self.arena.values():
            a.free()
        self.norm.free()
        self.rot_global.close()
        self.rot_local.close()

    def grad(self, name: str) -> np.ndarray:
        return self.p[name].gradient.numpy()

    def param(self, name: str) -> np.ndarray:
        return self.p[name].data.numpy()

    def zero_gradients(self) -> None:
        self.arena["G"].fill(0.0)

    # ------------------------------------------------------------------------------------------ forward

    def _enc(self, l: int, what: str) -> _Param:
        return self.p.get(f"encoder.layers.{l}.{what}")

    def _head(self, j: int, what: str) -> _Param:
        return self.p.get(f"head.layers.{j}.{what}")

    def _w(self, key: str) -> Optional[DeviceArray]:
        """The magnitude word group kept for buffer `key`, or None when words are not carried."""
        if not self.carry_words:
            return None
        if key not in self._words:
            self._words[key] = laya.magnitude_words(self.ctx)
        return self._words[key]

    def _salt(self, seed: int, layer: int, site: int) -> int:
        return laya.mix(seed, layer * 16 + site + 1)  # TrainableDecisionModel.cs:426

    def forward(self, b: OpBatch, seed: int, training: bool = True) -> _View:
        ctx, cfg, s = self.ctx, self.config, self.s
        e = cfg.encoder
        T, d, I, ff = b.T, cfg.hidden, e.intermediate_size, cfg.head_ff
        eps = e.norm_eps
        self.b, self.seed, self.training = b, seed, training
        p = self.head_dropout if training else 0.0
        # Embeddings (TrainableDecisionModel.cs:277-285)
        emb = s.get("emb", (T, d))
        check(lib().laya_embedding_fwd(ctx.handle, b.tokens.ptr, T, self.p["encoder.embeddings.tok_embeddings.weight"]
                                       .data.ptr, e.vocab_size, d, emb.ptr, None))
        x = s.get("x0", (T, d))
        laya.layer_norm(emb, T, d, self.p["encoder.embeddings.norm.weight"], self.p.get("encoder.embeddings.norm.bias"),
                        eps, x, s.get("emb_mean", (T,)), s.get("emb_rstd", (T,)), y_words=self._w("x0"))
        for l in range(e.num_hidden_layers):
            x = self._encoder_layer(l, x)
        fin = s.get("final", (T, d))
        laya.layer_norm(x, T, d, self.p["encoder.final_norm.weight"], self.p.get("encoder.final_norm.bias"), eps, fin,
                        s.get("fin_mean", (T,)), s.get("fin_rstd", (T,)))
        laya.type_embedding(ctx, fin, b.row_type, T, d, self.p["type_emb.weight"])
        self.enc_out = x
        h = fin
        for j in range(cfg.head_layers):
            h = self._head_layer(j, h, p, seed)
        # Scorer at the option markers (TrainableDecisionModel.cs:313-323)
        M = b.n_markers
        s_in, s_norm, s_pre, s_act = (s.get(k, (M, d)) for k in ("s_in", "s_norm", "s_pre", "s_act"))
        laya.gather_rows(ctx, h, b.marker_rows, M, d, s_in)
        laya.layer_norm(s_in, M, d, self.p["scorer.0.weight"], self.p["scorer.0.bias"], 1e-5, s_norm,
                        s.get("s_mean", (M,)), s.get("s_rstd", (M,)))
        laya.linear(self.p["scorer.1.weight"], self.p["scorer.1.bias"], s_norm, M, s_pre)
        laya.gelu(ctx, s_pre, s_act)
        logits = s.get("logits", (M,))
        laya.linear(self.p["scorer.3.weight"], self.p["scorer.3.bias"], s_act, M, logits)
        self.head_out = h
        return logits

    def _attention_shape(self, kind: int) -> laya.AttentionShape:
        e = self.config.encoder
        rot = self.rot_global if kind == 0 else self.rot_local
        return laya.AttentionShape(e.hidden_size, e.num_attention_heads, laya.default_scale(e.head_dim),
                                   e.sliding_half_window if kind == 1 else -1, rot, 0.0, 0)

    def _head_shape(self, j: int, p: float, seed: int) -> laya.AttentionShape:
        d = self.config.hidden
        heads = self.config.head_heads
        return laya.AttentionShape(d, heads, laya.default_scale(d // heads), -1, None, p, self._salt(seed, j, 0))

    def _encoder_layer(self, l: int, x: _View) -> _View:
        """EncoderLayerForward (TrainableDecisionModel.cs:361-414)."""
        ctx, s, b = self.ctx, self.s, self.b
        T, d, I = b.T, self.config.hidden, self.config.encoder.intermediate_size
        eps = self.config.encoder.norm_eps
        g = lambda k, shape: s.get(f"e{l}.{k}", shape)  # noqa: E731
        norm = self._enc(l, "attn_norm.weight")
        w = lambda k: self._w(f"e{l}.{k}")  # noqa: E731
        if norm is None:
            normed, wn = x, (self._w("x0") if l == 0 else None)  # layer 0: nn.Identity
        else:
            normed, wn = g("normed", (T, d)), w("normed")
            laya.layer_norm(x, T, d, norm, self._enc(l, "attn_norm.bias"), eps, normed, g("mean1", (T,)),
                            g("rstd1", (T,)), y_words=wn)
        qkv = g("qkv", (T, 3 * d))
        laya.linear(self._enc(l, "attn.Wqkv.weight"), self._enc(l, "attn.Wqkv.bias"), normed, T, qkv, x_words=wn)
        context, lse = g("ctx", (T, d)), g("lse", (T * self.config.encoder.num_attention_heads,))
        # (q and k are rotated into a copy that measures itself: qkv's own words would go unread)
        laya.attention_forward(qkv, b.segments, self._attention_shape(self.config.encoder.layer_kinds[l]), context, lse,
                               context_words=w("ctx"))
        res = g("res", (T, d))
        laya.linear(self._enc(l, "attn.Wo.weight"), self._enc(l, "attn.Wo.bias"), context, T, res, residual=x,
                    x_words=w("ctx"))
        mlpn = g("mlpn", (T, d))
        laya.layer_norm(res, T, d, self._enc(l, "mlp_norm.weight"), self._enc(l, "mlp_norm.bias"), eps, mlpn,
                        g("mean2", (T,)), g("rstd2", (T,)), y_words=w("mlpn"))
        wide = g("wide", (T, 2 * I))
        laya.linear(self._enc(l, "mlp.Wi.weight"), self._enc(l, "mlp.Wi.bias"), mlpn, T, wide, x_words=w("mlpn"))
        act = g("act", (T, I))
        laya.geglu(ctx, wide, T, I, act, act_words=w("act"))
        out = g("out", (T, d))
        laya.linear(self._enc(l, "mlp.Wo.weight"), self._enc(l, "mlp.Wo.bias"), act, T, out, residual=res,
                    x_words=w("act"))
        return out

    def _head_layer(self, j: int, x: _View, p: float, seed: int) -> _View:
        """HeadLayerForward (TrainableDecisionModel.cs:428-468): nn.TransformerEncoderLayer, post-norm, ReLU."""
        ctx, s, b = self.ctx, self.s, self.b
        T, d, ff = b.T, self.config.hidden, self.config.head_ff
        g = lambda k, shape: s.get(f"h{j}.{k}", shape)  # noqa: E731
        n1 = g("n1", (T, d))
        laya.layer_norm(x, T, d, self._head(j, "norm1.weight"), self._head(j, "norm1.bias"), 1e-5, n1,
                        g("mean1", (T,)), g("rstd1", (T,)))
        qkv = g("qkv", (T, 3 * d))
        laya.linear(self._head(j, "self_attn.in_proj_weight"), self._head(j, "self_attn.in_proj_bias"), n1, T, qkv)
        context, lse = g("ctx", (T, d)), g("lse", (T * self.config.head_heads,))
        laya.attention_forward(qkv, b.segments, self._head_shape(j, p, seed), context, lse)
        res = g("res", (T, d))
        if p > 0:
            laya.linear(self._head(j, "self_attn.out_proj.weight"), self._head(j, "self_attn.out_proj.bias"), context,
                        T, res)
            laya.dropout(ctx, res, T * d, p, self._salt(seed, j, 1))
            laya.add(ctx, res, x)
        else:
            laya.linear(self._head(j, "self_attn.out_proj.weight"), self._head(j, "self_attn.out_proj.bias"), context,
                        T, res, residual=x)
        n2 = g("n2", (T, d))
        laya.layer_norm(res, T, d, self._head(j, "norm2.weight"), self._head(j, "norm2.bias"), 1e-5, n2,
                        g("mean2", (T,)), g("rstd2", (T,)))
        wide, drop = g("wide", (T, ff)), g("drop", (T, ff))
        laya.linear(self._head(j, "linear1.weight"), self._head(j, "linear1.bias"), n2, T, wide)
        check(lib().laya_relu_dropout_fwd(ctx.handle, wide.ptr, T * ff, p, self._salt(seed, j, 2) & (2 ** 64 - 1),
                                          drop.ptr))
        out = g("out", (T, d))
        if p > 0:
            laya.linear(self._head(j, "linear2.weight"), self._head(j, "linear2.bias"), drop, T, out)
            laya.dropout(ctx, out, T * d, p, self._salt(seed, j, 3))
            laya.add(ctx, out, res)
        else:
            laya.linear(self._head(j, "linear2.weight"), self._head(j, "linear2.bias"), drop, T, out, residual=res)
        return out

    # ----------------------------------------------------------------------------------------- backward

    def backward(self, dlogits: _View) -> None:
        """Backward (TrainableDecisionModel.cs:479-549) from dL/dlogits on the device."""
        ctx, s, b, cfg = self.ctx, self.s, self.b, self.config
        e = cfg.encoder
        T, d, M = b.T, cfg.hidden, b.n_markers
        eps = e.norm_eps
        # Scorer (484-504)
        ds_act, ds_norm = s.get("ds_act", (M, d)), s.get("ds_norm", (M, d))
        laya.linear_backward(self.p["scorer.3.weight"], self.p["scorer.3.bias"], s.get("s_act", (M, d)), dlogits, M,
                             ds_act)
        laya.gelu_backward(ctx, s.get("s_pre", (M, d)), ds_act)
        laya.linear_backward(self.p["scorer.1.weight"], self.p["scorer.1.bias"], s.get("s_norm", (M, d)), ds_act, M,
                             ds_norm)
        ds_mark = s.get("ds_mark", (M, d))
        ds_mark.fill(0.0)
        laya.layer_norm_backward(s.get("s_in", (M, d)), M, d, self.p["scorer.0.weight"], self.p["scorer.0.bias"], 1e-5,
                                 ds_norm, ds_mark, s.get("s_mean", (M,)), s.get("s_rstd", (M,)))
        dstates = s.get("dstates", (T, d))
        dstates.fill(0.0)
        laya.scatter_add_rows(ctx, ds_mark, b.marker_rows, M, d, dstates)
        for j in reversed(range(cfg.head_layers)):
            dstates = self._head_layer_backward(j, dstates)
        # Type embedding (512-521), final norm (523-531)
        laya.type_embedding_backward(ctx, dstates, b.row_type, T, d, self.p["type_emb.weight"])
        dx = s.get("dx_a", (T, d))
        dx.fill(0.0)
        laya.layer_norm_backward(self.enc_out, T, d, self.p["encoder.final_norm.weight"],
                                 self.p.get("encoder.final_norm.bias"), eps, dstates, dx, s.get("fin_mean", (T,)),
                                 s.get("fin_rstd", (T,)), dx_words=self._w("dout"))
        self._dout_words_valid = True
        for l in reversed(range(e.num_hidden_layers)):
            dx = self._encoder_layer_backward(l, dx)
        # Embedding norm and the token-order scatter (538-548)
        demb = s.get("demb", (T, d))
        demb.fill(0.0)
        laya.layer_norm_backward(s.get("emb", (T, d)), T, d, self.p["encoder.embeddings.norm.weight"],
                                 self.p.get("encoder.embeddings.norm.bias"), eps, dx, demb, s.get("emb_mean", (T,)),
                                 s.get("emb_rstd", (T,)))
        sp, un, off, nu = b.plan
        if nu:
            check(lib().laya_embedding_bwd(ctx.handle, sp.ptr, un.ptr, off.ptr, nu, demb.ptr, d,
                                           self.p["encoder.embeddings.tok_embeddings.weight"].gradient.ptr))

    def _encoder_layer_backward(self, l: int, dout: _View) -> _View:
        """EncoderLayerBackward (TrainableDecisionModel.cs:551-603); dout becomes the layer's input gradient."""
        ctx, s, b = self.ctx, self.s, self.b
        T, d, I = b.T, self.config.hidden, self.config.encoder.intermediate_size
        eps = self.config.encoder.norm_eps
        g = lambda k, shape: s.get(f"e{l}.{k}", shape)  # noqa: E731
        w = lambda k: self._w(f"e{l}.{k}")  # noqa: E731
        # dout's words while the last write to dout was a call that filled them
        wdo = self._w("dout") if self._dout_words_valid else None
        d_act, d_wide, d_n = s.get("d_act", (T, I)), s.get("d_wide", (T, 2 * I)), s.get("d_n", (T, d))
        laya.linear_backward(self._enc(l, "mlp.Wo.weight"), self._enc(l, "mlp.Wo.bias"), g("act", (T, I)), dout, T,
                             d_act, x_words=w("act"), dy_words=wdo)
        laya.geglu_backward(ctx, g("wide", (T, 2 * I)), d_act, T, I, d_wide, dwide_words=self._w("d_wide"))
        laya.linear_backward(self._enc(l, "mlp.Wi.weight"), self._enc(l, "mlp.Wi.bias"), g("mlpn", (T, d)), d_wide, T,
                             d_n, x_words=w("mlpn"), dy_words=self._w("d_wide"))
        laya.layer_norm_backward(g("res", (T, d)), T, d, self._enc(l, "mlp_norm.weight"), self._enc(l, "mlp_norm.bias"),
                                 eps, d_n, dout, g("mean2", (T,)), g("rstd2", (T,)), dx_words=self._w("dout"))
        wdo = self._w("dout")
        d_ctx, d_qkv = s.get("d_ctx", (T, d)), s.get("d_qkv", (T, 3 * d))
        laya.linear_backward(self._enc(l, "attn.Wo.weight"), self._enc(l, "attn.Wo.bias"), g("ctx", (T, d)), dout, T,
                             d_ctx, x_words=w("ctx"), dy_words=wdo, dx_words=self._w("d_ctx"))
        laya.attention_backward(g("qkv", (T, 3 * d)), b.segments,
                                self._attention_shape(self.config.encoder.layer_kinds[l]), d_ctx, d_qkv,
                                *self._saved(g, T, d, self.config.encoder.num_attention_heads),
                                dcontext_words=self._w("d_ctx"), dqkv_words=self._w("d_qkv"))
        norm = self._enc(l, "attn_norm.weight")
        if norm is None:
            x_in = self.s.get("x0", (T, d)) if l == 0 else s.get(f"e{l - 1}.out", (T, d))
            laya.linear_backward(self._enc(l, "attn.Wqkv.weight"), self._enc(l, "attn.Wqkv.bias"), x_in, d_qkv, T, d_n,
                                 x_words=self._w("x0") if l == 0 else None, dy_words=self._w("d_qkv"))
            laya.add(ctx, dout, d_n)
            self._dout_words_valid = False  # a plain add: dout's words no longer describe it
        else:
            laya.linear_backward(self._enc(l, "attn.Wqkv.weight"), self._enc(l, "attn.Wqkv.bias"), g("normed", (T, d)),
                                 d_qkv, T, d_n, x_words=w("normed"), dy_words=self._w("d_qkv"))
            x_in = self.s.get("x0", (T, d)) if l == 0 else s.get(f"e{l - 1}.out", (T, d))
            laya.layer_norm_backward(x_in, T, d, norm, self._enc(l, "attn_norm.bias"), eps, d_n, dout,
                                     g("mean1", (T,)), g("rstd1", (T,)), dx_words=self._w("dout"))
            self._dout_words_valid = True
        return dout

    def _head_layer_backward(self, j: int, dout: _View) -> _View:
        """HeadLayerBackward (TrainableDecisionModel.cs:605-640); dout becomes the layer's input gradient."""
        ctx, s, b = self.ctx, self.s, self.b
        T, d, ff = b.T, self.config.hidden, self.config.head_ff
        p = self.head_dropout if self.training else 0.0
        seed = self.seed
        g = lambda k, shape: s.get(f"h{j}.{k}", shape)  # noqa: E731
        x_in = s.get("final", (T, d)) if j == 0 else s.get(f"h{j - 1}.out", (T, d))
        dy = dout
        if p > 0:
            dy = s.get("hdy", (T, d))  # dOutput.Clone(), then its dropout (TrainableDecisionModel.cs:611-613)
            laya.add(ctx, self._zeroed(dy), dout)
            laya.dropout(ctx, dy, T * d, p, self._salt(seed, j, 3))
        d_drop = s.get("d_drop", (T, ff))
        laya.linear_backward(self._head(j, "linear2.weight"), self._head(j, "linear2.bias"), g("drop", (T, ff)), dy, T,
                             d_drop)
        check(lib().laya_relu_dropout_bwd(ctx.handle, g("wide", (T, ff)).ptr, d_drop.ptr, T * ff, p,
                                          self._salt(seed, j, 2) & (2 ** 64 - 1)))
        d_n = s.get("d_n", (T, d))
        laya.linear_backward(self._head(j, "linear1.weight"), self._head(j, "linear1.bias"), g("n2", (T, d)), d_drop, T,
                             d_n)
        laya.layer_norm_backward(g("res", (T, d)), T, d, self._head(j, "norm2.weight"), self._head(j, "norm2.bias"),
                                 1e-5, d_n, dout, g("mean2", (T,)), g("rstd2", (T,)))
        datt = dout
        if p > 0:
            datt = s.get("hdatt", (T, d))
            laya.add(ctx, self._zeroed(datt), dout)
            laya.dropout(ctx, datt, T * d, p, self._salt(seed, j, 1))
        d_ctx, d_qkv = s.get("d_ctx", (T, d)), s.get("d_qkv", (T, 3 * d))
        laya.linear_backward(self._head(j, "self_attn.out_proj.weight"), self._head(j, "self_attn.out_proj.bias"),
                             g("ctx", (T, d)), datt, T, d_ctx)
        laya.attention_backward(g("qkv", (T, 3 * d)), b.segments, self._head_shape(j, p, seed), d_ctx, d_qkv,
                                *self._saved(g, T, d, self.config.head_heads))
        laya.linear_backward(self._head(j, "self_attn.in_proj_weight"), self._head(j, "self_attn.in_proj_bias"),
                             g("n1", (T, d)), d_qkv, T, d_n)
        laya.layer_norm_backward(x_in, T, d, self._head(j, "norm1.weight"), self._head(j, "norm1.bias"), 1e-5, d_n,
                                 dout, g("mean1", (T,)), g("rstd1", (T,)))
        return dout

    def _saved(self, g, T: int, d: int, heads: int):
        """The attention forward's context and LSE, which the host keeps beside the qkv it ran on and hands to the
        backward (Ops.AttentionBackward's signature carries neither; without them the backward recomputes the
        row statistics). None, None when the host does not keep them (carry_attention_state = False)."""
        if not self.carry_attention_state:
            return None, None
        return g("ctx", (T, d)), g("lse", (T * heads,))

    @staticmethod
    def _zeroed(v: _View) -> _View:
        v.fill(0.0)
        return v

    # -------------------------------------------------------------------------------------- the step

    def train_step(self, b: OpBatch, seed: int, ce_weight: float = 1.0, loss_scale: float = 1.0,
                   max_norm: float = 1.0, lr_encoder: float = 3e-5, lr_head: float = 3e-5, beta1: float = 0.9,
                   beta2: float = 0.999, eps: float = 1e-8, weight_decay: float = 0.01) -> None:
        """One micro-step with GradAccum = 1 (Trainer.cs:131-144): forward, the soft-CE gradient, backward,
        ClipByGlobalNorm, AdamW.Step, ZeroGradients."""
        ctx = self.ctx
        logits = self.forward(b, seed, training=True)
        dl = self.s.get("dlogits", (b.n_markers,))
        laya.softmax_ce_backward(ctx, logits, b.targets, b.offsets, b.n_items, ce_weight, loss_scale, dl)
        self.backward(dl)
        self.clip_and_step(max_norm, lr_encoder, lr_head, beta1, beta2, eps, weight_decay)

    def clip_and_step(self, max_norm: float, lr_encoder: float, lr_head: float, beta1: float = 0.9,
                      beta2: float = 0.999, eps: float = 1e-8, weight_decay: float = 0.01) -> None:
        ctx = self.ctx
        G = self.arena["G"]
        check(lib().laya_grad_norm(ctx.handle, G.ptr, self.head_end, max_norm, self.norm.ptr, self.norm.ptr + 8))
        self.steps += 1
        begin = (ctypes.c_size_t * 2)(0, self.encoder_end)
        end = (ctypes.c_size_t * 2)(self.encoder_end, self.head_end)
        lr = (ctypes.c_double * 2)(lr_encoder, lr_head)
        check(lib().laya_adamw(ctx.handle, self.arena["P"].ptr, G.ptr, self.arena["M1"].ptr, self.arena["M2"].ptr, 2,
                               begin, end, lr, beta1, beta2, eps, weight_decay, self.steps, self.norm.ptr + 8, 1))
