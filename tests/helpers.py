"""Shared test helpers: seeded parameters and model shapes."""
import numpy as np

from laya_amd.batch import synthetic_batch
from laya_amd.config import EncoderConfig, ModelConfig


def random_params(shapes: dict, seed: int, std: float = 0.08) -> dict:
    """Every tensor non-trivial (norm weights 1 + 0.2·N(0,1), the rest std·N(0,1)), as the reference's
    fixture generator does (tools/dump_training_reference.py:51-56)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in shapes.items():
        if len(shape) == 1 and "norm" in name and name.endswith("weight") or name.startswith("scorer.0.weight"):
            out[name] = (1.0 + 0.2 * rng.standard_normal(shape)).astype(np.float32)
        elif name == "temperature":
            out[name] = np.ones(shape, np.float32)
        else:
            out[name] = (std * rng.standard_normal(shape)).astype(np.float32)
    return out


def mid_config(layers: int = 3, hidden: int = 768, heads: int = 12, inter: int = 1152, vocab: int = 1000,
               window: int = 128, head_layers: int = 2) -> ModelConfig:
    """ModernBERT-base widths at a few layers: global first, then sliding (θ 160000 / 10000)."""
    enc = EncoderConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
                        num_attention_heads=heads, local_attention=window, global_attn_every_n_layers=3)
    return ModelConfig(encoder=enc, head_layers=head_layers, n_act=2)


def mixed_batch(rng, lengths, vocab, options=(8, 4, 2)):
    n = len(lengths)
    opts = [min(options[i % len(options)], max(1, (lengths[i] - 1) // 2)) for i in range(n)]
    qtypes = [i % 3 for i in range(n)]
    return synthetic_batch(rng, lengths, opts, qtypes, vocab)


def fixture_params(shapes: dict, seed: int, std: float = 0.02) -> dict:
    """Parameters of the full-size parity fixtures: each tensor from its own generator keyed by (seed, name),
    so the draw does not depend on the order the shapes are listed in. Norm weights and the scorer's norm
    1 + 0.2·N(0,1) (so γ errors show), biases and the rest std·N(0,1), temperature 1.

    The head's linear1 biases are ±5 × the RMS of their product (random sign per unit) instead: the
    head's ReLU is the model's one discontinuity, and with ~10⁸ of its inputs drawn around zero a few lie
    within fp32 rounding of it, so any two fp32 implementations may put one on different sides and move
    every gradient below it by ~1e-4 (measured: one such unit moved head layer 1's gradients by 3e-4
    between two fp32 GPU paths that agree to 1e-5 on other dropout seeds and to 3e-6 with the biases
    moved). Away from zero the step is smooth, and the ReLU still masks about half the units."""
    import zlib
    out = {}
    for name, shape in shapes.items():
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        if name == "temperature":
            out[name] = np.ones(shape, np.float32)
        elif name.startswith("head.layers.") and name.endswith(".linear1.bias"):
            fan_in = shapes[name[:-len("bias")] + "weight"][1]
            out[name] = (5.0 * std * np.sqrt(fan_in) * rng.choice([-1.0, 1.0], shape)).astype(np.float32)
        elif len(shape) == 1 and "norm" in name and name.endswith("weight") or name.startswith("scorer.0.weight"):
            out[name] = (1.0 + 0.2 * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
        else:
            out[name] = (std * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
    return out


def closed_form_readout_case():
    """A model whose read-out inputs are known in closed form, to pin DecisionModel.ReadOut's wiring
    (DecisionModel.cs:170-227) without repeating its formulas: no encoder or head layers, so the final states
    are final_norm(emb_norm(E[id])) + type_emb[qtype]; every embedding row holds ±A (32 of each sign over
    d = 64, mean exactly zero), so both LayerNorms give ±c with c closed-form, and column 0's sign is + only for
    even ids, which only each item's first token has. The scorer's output weight is zero, so every item's
    option logits are equal (uniform probabilities: top1 = 1/K, margin 0, normalised entropy 1 for K ≥ 2;
    K = 1 gives top1 1, margin 1, entropy 0). Returns (config, params, batch, expected) where expected[i] is
    item i's act-head input [h[start], top1, top1 − top2, entropy, max(2, K)/255] in float64."""
    from laya_amd.batch import Batch
    d, vocab, A, eps = 64, 16, 0.5, 1e-5
    enc = EncoderConfig(vocab_size=vocab, hidden_size=d, intermediate_size=32, num_hidden_layers=0,
                        num_attention_heads=1, norm_eps=eps)
    mc = ModelConfig(encoder=enc, head_layers=0, n_act=2)
    rng = np.random.default_rng(77)
    signs = np.empty((vocab, d))
    for v in range(vocab):
        first = 1.0 if v % 2 == 0 else -1.0
        rest = np.array([1.0] * (32 - (first > 0)) + [-1.0] * (32 - (first < 0)))
        signs[v] = np.concatenate([[first], rng.permutation(rest)])
    assert np.all(signs.sum(axis=1) == 0)
    type_emb = np.array([[0.1 * (q + 1) * (-1) ** c + 0.01 * c for c in range(d)] for q in range(3)])
    params = {"encoder.embeddings.tok_embeddings.weight": (A * signs).astype(np.float32),
              "encoder.embeddings.norm.weight": np.ones(d, np.float32),
              "encoder.final_norm.weight": np.ones(d, np.float32),
              "type_emb.weight": type_emb.astype(np.float32),
              "scorer.0.weight": np.ones(d, np.float32), "scorer.0.bias": np.zeros(d, np.float32),
              "scorer.1.weight": (0.05 * rng.standard_normal((d, d))).astype(np.float32),
              "scorer.1.bias": np.zeros(d, np.float32),
              "scorer.3.weight": np.zeros((1, d), np.float32), "scorer.3.bias": np.full(1, 0.3, np.float32),
              "act_head.0.weight": np.zeros((256, d + 4), np.float32), "act_head.0.bias": np.zeros(256, np.float32),
              "act_head.2.weight": np.zeros((2, 256), np.float32), "act_head.2.bias": np.zeros(2, np.float32),
              "temperature": np.ones(3, np.float32)}
    # Items: lengths, option counts, question types; the first token has an even id, the rest odd ids.
    lengths, opts, qtypes = [5, 7, 4, 9], [1, 2, 3, 5], [0, 1, 2, 0]
    tokens, markers = [], []
    for i, (L, K) in enumerate(zip(lengths, opts)):
        tokens += [2 * (i % 8)] + [2 * ((i + j) % 8) + 1 for j in range(1, L)]
        markers += [min(L - 1, 1 + 2 * k) for k in range(K)]
    batch = Batch(lengths=np.array(lengths, np.int32), tokens=np.array(tokens, np.int32),
                  n_options=np.array(opts, np.int32), markers=np.array(markers, np.int32),
                  qtypes=np.array(qtypes, np.int32))
    y = A / np.sqrt(A * A + eps)          # emb_norm of ±A: mean 0, variance A²
    c = y / np.sqrt(y * y + eps)           # final_norm of ±y
    expected = []
    off = 0
    for i, (L, K) in enumerate(zip(lengths, opts)):
        h = c * signs[tokens[off]] + type_emb[qtypes[i]]
        off += L
        feats = [1.0, 1.0, 0.0] if K == 1 else [1.0 / K, 0.0, 1.0]
        expected.append(np.concatenate([h, feats, [max(2, K) / 255.0]]))
    return mc, params, batch, np.array(expected)


def act_head_selecting(params: dict, slot: int) -> dict:
    """The act head wired so that action logit 0 is GELU(input[slot]) and action logit 1 is GELU(0) = 0: hidden
    unit 0 reads input `slot` alone, the other units read nothing, and the output layer is the identity on the
    first two units."""
    p = dict(params)
    w1 = np.zeros_like(params["act_head.0.weight"])
    w1[0, slot] = 1.0
    w2 = np.zeros_like(params["act_head.2.weight"])
    w2[0, 0] = w2[1, 1] = 1.0
    p["act_head.0.weight"], p["act_head.2.weight"] = w1, w2
    return p


# Input slots the closed-form read-out tests select: pooled columns (the first, two others, the last) and the
# four calibration features in order.
READOUT_SLOTS = [0, 1, 17, 63, 64, 65, 66, 67]
