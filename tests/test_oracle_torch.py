"""Pins the oracle's hand-written backward with autograd: an independent PyTorch float64 formulation of the
same forward (dense per-segment attention with an explicit window mask, torch's layer_norm, erf GELU, the
counter-RNG dropout masks recomputed in numpy) is differentiated by torch.autograd on the CPU and compared
with the fp64 oracle's gradients, at ModernBERT-base widths with sliding windows shorter than the segments.
"""
import math

import numpy as np
import pytest

import oracle
from fixtures import rel_l2, tiny_batch, tiny_config, tiny_params
from helpers import mid_config, mixed_batch, random_params

torch = pytest.importorskip("torch")

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def np_uniform(seed: int, idx: np.ndarray) -> np.ndarray:
    """Ops.Uniform (Ops.cs:227-234), vectorised over uint64 indices (wrapping arithmetic)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (idx.astype(np.uint64) + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return (z >> np.uint64(40)).astype(np.float64) / float(1 << 24)


def mix(seed: int, salt: int) -> int:
    m = (1 << 64) - 1
    z = seed ^ ((salt * 0xD1B54A32D192ED03 + 0x8CB92BA72F3D8DD7) & m)
    z = ((z ^ (z >> 33)) * 0xFF51AFD7ED558CCD) & m
    return z ^ (z >> 33)


def salt(seed, layer, site):
    return mix(seed, layer * 16 + site + 1)


def keep_scale(p):
    pf = float(np.float32(p))
    return 1.0 / (1.0 - pf)


def dropout_mask(shape, p, seed):
    if p <= 0:
        return None
    u = np_uniform(seed, np.arange(int(np.prod(shape)), dtype=np.uint64)).reshape(shape)
    return torch.tensor(np.where(u < np.float32(p), 0.0, keep_scale(p)))


def attention(qkv, starts, lengths, heads, scale, hw, theta, p, seed):
    T, h3 = qkv.shape
    hidden = h3 // 3
    d = hidden // heads
    out = torch.zeros((T, hidden), dtype=torch.float64)
    pieces = []
    for s, L in zip(starts, lengths):
        rows = []
        for h in range(heads):
            q = qkv[s:s + L, h * d:(h + 1) * d]
            k = qkv[s:s + L, hidden + h * d:hidden + (h + 1) * d]
            v = qkv[s:s + L, 2 * hidden + h * d:2 * hidden + (h + 1) * d]
            if theta > 0:
                i = torch.arange(d // 2, dtype=torch.float64)
                ang = torch.arange(L, dtype=torch.float64)[:, None] * (1.0 / theta ** (2.0 * i / d))[None, :]
                c, sn = torch.cos(ang), torch.sin(ang)

                def rot(m):
                    a, b = m[:, :d // 2], m[:, d // 2:]
                    return torch.cat([a * c - b * sn, b * c + a * sn], 1)
                q, k = rot(q), rot(k)
            S = scale * (q @ k.T)
            if hw >= 0:
                t = torch.arange(L)
                S = S.masked_fill((t[:, None] - t[None, :]).abs() > hw, float("-inf"))
            P = torch.softmax(S, 1)
            if p > 0:
                row = (np.arange(L, dtype=np.uint64) + np.uint64(s))[:, None]
                key = np.arange(L, dtype=np.uint64)[None, :]
                idx = (np.uint64(h) << np.uint64(42)) | (row << np.uint64(21)) | key
                u = np_uniform(seed, idx)
                P = P * torch.tensor(np.where(u < np.float32(p), 0.0, keep_scale(p)))
            rows.append(P @ v)
        pieces.append(torch.cat(rows, 1))
    return torch.cat(pieces, 0)


def gelu(x):
    return 0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0)))


def torch_forward(mc, P, batch, training, seed, head_dropout):
    e = mc.encoder
    d, I, ff = e.hidden_size, e.intermediate_size, mc.head_ff
    ln = torch.nn.functional.layer_norm
    lengths = [int(x) for x in batch.lengths]
    starts = [int(x) for x in batch.starts()]
    tokens = torch.tensor(batch.tokens.astype(np.int64))
    x = P["encoder.embeddings.tok_embeddings.weight"][tokens]
    x = ln(x, (d,), P["encoder.embeddings.norm.weight"], None, e.norm_eps)
    hd = d // e.num_attention_heads
    for l in range(e.num_hidden_layers):
        pre = f"encoder.layers.{l}."
        normed = x if l == 0 else ln(x, (d,), P[pre + "attn_norm.weight"], None, e.norm_eps)
        qkv = normed @ P[pre + "attn.Wqkv.weight"].T
        sliding = e.layer_kinds[l] == 1
        ctx = attention(qkv, starts, lengths, e.num_attention_heads, 1.0 / math.sqrt(hd),
                        e.local_attention // 2 if sliding else -1,
                        e.local_rope_theta if sliding else e.global_rope_theta, 0.0, 0)
        res = x + ctx @ P[pre + "attn.Wo.weight"].T
        mn = ln(res, (d,), P[pre + "mlp_norm.weight"], None, e.norm_eps)
        wide = mn @ P[pre + "mlp.Wi.weight"].T
        x = res + (gelu(wide[:, :I]) * wide[:, I:]) @ P[pre + "mlp.Wo.weight"].T
    x = ln(x, (d,), P["encoder.final_norm.weight"], None, e.norm_eps)
    qt = torch.tensor(np.repeat(batch.qtypes, batch.lengths).astype(np.int64))
    x = x + P["type_emb.weight"][qt]
    p = head_dropout if training else 0.0
    hh = max(1, d // 64)
    for j in range(mc.head_layers):
        pre = f"head.layers.{j}."
        n1 = ln(x, (d,), P[pre + "norm1.weight"], P[pre + "norm1.bias"], 1e-5)
        qkv = n1 @ P[pre + "self_attn.in_proj_weight"].T + P[pre + "self_attn.in_proj_bias"]
        ctx = attention(qkv, starts, lengths, hh, 1.0 / math.sqrt(d // hh), -1, 0.0, p, salt(seed, j, 0))
        att = ctx @ P[pre + "self_attn.out_proj.weight"].T + P[pre + "self_attn.out_proj.bias"]
        m1 = dropout_mask(att.shape, p, salt(seed, j, 1))
        res = x + (att * m1 if m1 is not None else att)
        n2 = ln(res, (d,), P[pre + "norm2.weight"], P[pre + "norm2.bias"], 1e-5)
        wide = torch.relu(n2 @ P[pre + "linear1.weight"].T + P[pre + "linear1.bias"])
        m2 = dropout_mask(wide.shape, p, salt(seed, j, 2))
        wide = wide * m2 if m2 is not None else wide
        out = wide @ P[pre + "linear2.weight"].T + P[pre + "linear2.bias"]
        m3 = dropout_mask(out.shape, p, salt(seed, j, 3))
        x = res + (out * m3 if m3 is not None else out)
    rows = torch.tensor(batch.marker_rows().astype(np.int64))
    m = x[rows]
    m = ln(m, (d,), P["scorer.0.weight"], P["scorer.0.bias"], 1e-5)
    m = gelu(m @ P["scorer.1.weight"].T + P["scorer.1.bias"])
    return (m @ P["scorer.3.weight"].T + P["scorer.3.bias"])[:, 0]


def compare(mc, params, batch, coeff, training, seed, dropout, bar):
    o = oracle.OracleModel(mc, double=True)
    o.set_params(params)
    o.set_head_dropout(dropout)
    lo = o.forward(batch, training=training, keep_tape=True, seed=seed)
    o.backward(coeff)
    P = {n: torch.tensor(v.astype(np.float64), requires_grad=True) for n, v in params.items()}
    logits = torch_forward(mc, P, batch, training, seed, dropout)
    (logits * torch.tensor(coeff.astype(np.float64))).sum().backward()
    assert np.abs(logits.detach().numpy() - lo).max() < 1e-10
    worst = 0.0
    for name, t in P.items():
        if name.startswith("act_head") or name == "temperature":
            continue
        g = t.grad.numpy() if t.grad is not None else np.zeros(t.shape)
        r = rel_l2(g, o.grad(name)) if np.any(g) else float(np.abs(o.grad(name)).max())
        worst = max(worst, r)
        assert r < bar, (name, r)
    return worst


@pytest.mark.parametrize("training,dropout", [(False, 0.0), (True, 0.3)])
def test_tiny_fixture_backward_against_autograd(training, dropout):
    batch, coeff, _ = tiny_batch()
    compare(tiny_config(), tiny_params(), batch, coeff, training, 12345, dropout, 1e-9)


@pytest.mark.slow
def test_modernbert_base_width_backward_against_autograd():
    mc = mid_config(layers=3)
    o = oracle.OracleModel(mc)
    params = random_params(o.shapes, 0, std=0.02)
    batch = mixed_batch(np.random.default_rng(1), [300, 200, 129, 64, 17], mc.encoder.vocab_size)
    coeff = np.random.default_rng(7).standard_normal(batch.n_markers).astype(np.float32)
    compare(mc, params, batch, coeff, True, 99, 0.1, 1e-9)
