"""Pins the oracle's functions with what the mathematics fixes: closed forms, invariants, brute force,
and central finite differences of the fp64 model in training mode (dropout on).

Ports NumericsTests.cs (GELU values 156-167, exp vs library 169-182, erf values 210-220, LayerNorm formula
110-127, RoPE invariants 343-369, GEMM triple loops 46-72) and DropoutGradientsMatchFiniteDifferences
(TrainingGradientTests.cs:108-161).
"""
import math

import numpy as np
import pytest

import oracle
from fixtures import tiny_batch, tiny_config, tiny_params

MASK64 = (1 << 64) - 1


def splitmix_uniform(seed: int, index: int) -> float:
    """Ops.Uniform (Ops.cs:227-234) in Python integers."""
    z = (seed + (index + 1) * 0x9E3779B97F4A7C15) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    z ^= z >> 31
    return (z >> 40) / float(1 << 24)


def mix(seed: int, salt: int) -> int:
    z = seed ^ ((salt * 0xD1B54A32D192ED03 + 0x8CB92BA72F3D8DD7) & MASK64)
    z = ((z ^ (z >> 33)) * 0xFF51AFD7ED558CCD) & MASK64
    return z ^ (z >> 33)


def test_counter_rng_is_bit_exact():
    for seed in (0, 1, 12345, 2 ** 63 + 5, MASK64):
        for idx in (0, 1, 7, 1 << 21, (3 << 42) | (17 << 21) | 5, MASK64 - 1):
            assert oracle.uniform(seed, idx) == splitmix_uniform(seed, idx)
        assert oracle.mix(seed, 9) == mix(seed, 9)


def test_dropout_mask_follows_the_counter_rng():
    v = np.arange(1, 2001, dtype=np.float32)
    out = oracle.dropout(v, 0.3, 42)
    keep = np.array([splitmix_uniform(42, i) >= 0.3 for i in range(v.size)])
    np.testing.assert_array_equal(out == 0, ~keep)
    np.testing.assert_array_equal(out[keep], v[keep] * np.float32(1 / np.float32(0.7)))


def test_exp_and_erf_match_the_library():
    xs = np.linspace(-20, 20, 4001, dtype=np.float32)
    e = np.array([oracle.lib().orc_exp_f32(float(x)) for x in xs], np.float64)
    np.testing.assert_allclose(e, np.exp(xs.astype(np.float64)), rtol=4e-7)
    xs = np.linspace(-7, 7, 2801, dtype=np.float32)
    erf = np.array([oracle.lib().orc_erf_f32(float(x)) for x in xs], np.float64)
    ref = np.array([math.erf(float(x)) for x in xs])
    assert np.abs(erf - ref).max() < 3e-7


def test_gelu_known_values():
    # exact GELU x·Φ(x): NumericsTests.cs:156-167 uses these points.
    for double in (False, True):
        g = oracle.gelu(np.array([-3.0, -1.0, -0.5, 0.0, 0.5, 1.0, 3.0]), double=double)
        ref = [x * 0.5 * (1 + math.erf(x / math.sqrt(2))) for x in (-3.0, -1.0, -0.5, 0.0, 0.5, 1.0, 3.0)]
        np.testing.assert_allclose(g, ref, atol=1e-6)
    u = np.linspace(-5, 5, 101)
    h = 1e-6
    num = (oracle.gelu(u + h, double=True) - oracle.gelu(u - h, double=True)) / (2 * h)
    np.testing.assert_allclose(oracle.gelu_backward(u, np.ones_like(u), double=True), num, atol=1e-8)


def test_layernorm_formula():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((17, 96)) * 3 + 1
    w, b = rng.standard_normal(96), rng.standard_normal(96)
    mu = x.mean(1, keepdims=True)
    var = ((x - mu) ** 2).mean(1, keepdims=True)  # biased
    ref = (x - mu) / np.sqrt(var + 1e-5) * w + b
    np.testing.assert_allclose(oracle.layernorm(x, w, b, 1e-5, double=True), ref, rtol=1e-12, atol=1e-12)


def test_layernorm_backward_is_the_adjoint():
    rng = np.random.default_rng(1)
    x, w, dy = rng.standard_normal((5, 40)), rng.standard_normal(40), rng.standard_normal((5, 40))
    dx = np.zeros_like(x)
    dg = np.zeros(40)
    oracle.layernorm_backward(x, w, 1e-5, dy, dx, dg, None, double=True)
    h = 1e-6
    for (r, c) in [(0, 0), (2, 17), (4, 39)]:
        xp, xm = x.copy(), x.copy()
        xp[r, c] += h
        xm[r, c] -= h
        num = ((oracle.layernorm(xp, w, None, 1e-5, True) - oracle.layernorm(xm, w, None, 1e-5, True)) * dy).sum()
        assert abs(num / (2 * h) - dx[r, c]) < 1e-7
    np.testing.assert_allclose(dg, (dy * oracle.layernorm(x, np.ones(40), None, 1e-5, True)).sum(0), rtol=1e-12)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 13, 5), (37, 130, 96), (200, 17, 300)])
def test_gemm_against_a_triple_loop(M, N, K):
    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((M, K))
    B = rng.standard_normal((K, N))
    for trans_a in (False, True):
        a = np.ascontiguousarray(A.T if trans_a else A)
        sam, sak = (1, M) if trans_a else (K, 1)
        C = np.zeros((M, N))
        oracle.lib().orc_gemm_f64(M, N, K, oracle.ptr(a), sam, sak, oracle.ptr(B), N, 1, oracle.ptr(C), N, 0)
        ref = np.array([[sum(A[i, k] * B[k, j] for k in range(K)) for j in range(N)] for i in range(M)])
        np.testing.assert_allclose(C, ref, rtol=1e-12, atol=1e-12)


def test_rotary_invariants():
    rng = np.random.default_rng(2)
    v = rng.standard_normal(64)
    for theta in (10000.0, 160000.0):
        np.testing.assert_allclose(oracle.rotary_apply(theta, v, 0, double=True), v, rtol=0, atol=0)
        for pos in (1, 17, 511, 8191):
            r = oracle.rotary_apply(theta, v, pos, double=True)
            assert abs(np.linalg.norm(r) - np.linalg.norm(v)) < 1e-12
            np.testing.assert_allclose(oracle.rotary_apply(theta, r, pos, inverse=True, double=True), v, atol=1e-12)
            # rotate-half by θ_i = pos·theta^(-2i/d): [a, b] → [a c − b s, b c + a s]
            i = np.arange(32)
            ang = pos * theta ** (-2.0 * i / 64)
            ref = np.concatenate([v[:32] * np.cos(ang) - v[32:] * np.sin(ang), v[32:] * np.cos(ang) + v[:32] * np.sin(ang)])
            np.testing.assert_allclose(r, ref, atol=1e-12)


def naive_attention(qkv, lengths, heads, scale, hw, theta):
    """Dense per-segment attention with an explicit window mask (an independent formulation)."""
    T, H3 = qkv.shape
    hidden = H3 // 3
    d = hidden // heads
    out = np.zeros((T, hidden))
    start = 0
    for L in lengths:
        for h in range(heads):
            q = qkv[start:start + L, h * d:(h + 1) * d].copy()
            k = qkv[start:start + L, hidden + h * d:hidden + (h + 1) * d].copy()
            v = qkv[start:start + L, 2 * hidden + h * d:2 * hidden + (h + 1) * d]
            if theta > 0:
                i = np.arange(d // 2)
                ang = np.arange(L)[:, None] * theta ** (-2.0 * i / d)[None, :]
                c, s = np.cos(ang), np.sin(ang)
                for m in (q, k):
                    a, b = m[:, :d // 2].copy(), m[:, d // 2:].copy()
                    m[:, :d // 2], m[:, d // 2:] = a * c - b * s, b * c + a * s
            S = scale * q @ k.T
            if hw >= 0:
                t = np.arange(L)
                S[np.abs(t[:, None] - t[None, :]) > hw] = -np.inf
            P = np.exp(S - S.max(1, keepdims=True))
            P /= P.sum(1, keepdims=True)
            out[start:start + L, h * d:(h + 1) * d] = P @ v
        start += L
    return out


@pytest.mark.parametrize("lengths,heads,hw,theta", [([21, 13, 9], 4, 4, 160000.0), ([40, 1, 70], 2, -1, 0.0),
                                                    ([130, 64], 2, 64, 10000.0)])
def test_attention_forward_against_dense_masked_attention(lengths, heads, hw, theta):
    rng = np.random.default_rng(sum(lengths))
    hidden = 32 * heads
    qkv = rng.standard_normal((sum(lengths), 3 * hidden))
    scale = float(np.float32(0.17))  # the scale crosses the ABI as a float
    got = oracle.attention_forward(qkv, lengths, heads, scale, hw, theta, double=True)
    np.testing.assert_allclose(got, naive_attention(qkv, lengths, heads, scale, hw, theta), atol=1e-12)


def test_attention_backward_against_finite_differences():
    rng = np.random.default_rng(3)
    lengths, heads, hw, theta, p, seed = [9, 6], 2, 2, 10000.0, 0.3, 77
    qkv = rng.standard_normal((15, 3 * 32))
    dctx = rng.standard_normal((15, 32))
    g = oracle.attention_backward(qkv, dctx, lengths, heads, 0.25, hw, theta, p, seed, double=True)
    h = 1e-6
    for idx in [(0, 0), (3, 20), (8, 40), (10, 70), (14, 95), (5, 33)]:
        a, b = qkv.copy(), qkv.copy()
        a[idx] += h
        b[idx] -= h
        fa = (oracle.attention_forward(a, lengths, heads, 0.25, hw, theta, p, seed, True) * dctx).sum()
        fb = (oracle.attention_forward(b, lengths, heads, 0.25, hw, theta, p, seed, True) * dctx).sum()
        assert abs((fa - fb) / (2 * h) - g[idx]) < 1e-7, idx


def test_dropout_gradients_match_finite_differences():
    """TrainingGradientTests.cs:108-161 in fp64: dropout 0.3, the same seed regenerates the same masks."""
    mc = tiny_config()
    params = tiny_params()
    m = oracle.OracleModel(mc, double=True)
    m.set_params(params)
    m.set_head_dropout(0.3)
    batch, coeff, _ = tiny_batch()
    seed = 12345

    def loss():
        return float((m.forward(batch, training=True, keep_tape=False, seed=seed) * coeff).sum())

    m.forward(batch, training=True, keep_tape=True, seed=seed)
    m.backward(coeff)
    h = 1e-4
    for name in ["head.layers.0.linear1.weight", "head.layers.1.self_attn.in_proj_weight",
                 "head.layers.0.self_attn.out_proj.bias", "encoder.layers.3.mlp.Wi.weight", "scorer.1.weight",
                 "encoder.embeddings.tok_embeddings.weight", "type_emb.weight"]:
        g = m.grad(name).reshape(-1)
        base = params[name].astype(np.float32).reshape(-1).copy()
        for index in np.argsort(-np.abs(g))[:3]:
            p = base.copy()
            p[index] += h
            m.set_params({**params, name: p.reshape(params[name].shape)})
            plus = loss()
            p[index] = base[index] - h
            m.set_params({**params, name: p.reshape(params[name].shape)})
            minus = loss()
            m.set_params(params)
            # set_params rounds to float32: use the realised step.
            step = (np.float32(base[index] + h) - np.float32(base[index] - h))
            num = (plus - minus) / float(step)
            # The reference allows 5 %; fp64 leaves only the rare ReLU kink crossed by a ±h step.
            assert abs(num - g[index]) <= 2e-3 * abs(g[index]) + 1e-8, (name, index, num, g[index])
