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
