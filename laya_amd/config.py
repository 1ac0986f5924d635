"""Model configuration: the parts of ``encoder/config.json`` and ``rl_agent_config.json`` the
fine-tuning path needs.

Mirrors ``ModernBertConfig.FromJson`` (src/StructuredDecisions.Laya/Models/ModernBertConfig.cs:60-117)
and ``LayaConfig.Load`` (ModernBertConfig.cs:146-183), including their defaults, so a checkpoint
directory the reference trains from configures this library the same way.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from typing import List, Optional

GLOBAL, SLIDING = 0, 1


@dataclass
class EncoderConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    norm_eps: float = 1e-5
    norm_bias: bool = False
    attention_bias: bool = False
    mlp_bias: bool = False
    local_attention: int = 128
    global_attn_every_n_layers: int = 3
    global_rope_theta: float = 160000.0
    local_rope_theta: float = 10000.0
    max_position_embeddings: int = 8192
    layer_kinds: List[int] = field(default_factory=list)

    def __post_init__(self):
        if not self.layer_kinds:
            n = self.global_attn_every_n_layers
            self.layer_kinds = [GLOBAL if i % n == 0 else SLIDING for i in range(self.num_hidden_layers)]

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def sliding_half_window(self) -> int:
        """A sliding layer's token sees [i - w, i + w] (ModernBertConfig.cs:51)."""
        return self.local_attention // 2

    @classmethod
    def from_json(cls, root: dict) -> "EncoderConfig":
        layers = int(root["num_hidden_layers"])
        every = int(root.get("global_attn_every_n_layers", 3))
        kinds: List[int] = []
        if isinstance(root.get("layer_types"), list):
            kinds = [SLIDING if t == "sliding_attention" else GLOBAL for t in root["layer_types"][:layers]]
            kinds += [GLOBAL] * (layers - len(kinds))
        g_theta, l_theta = 160000.0, 10000.0
        rope = root.get("rope_parameters")
        if isinstance(rope, dict):
            if "rope_theta" in rope.get("full_attention", {}):
                g_theta = float(rope["full_attention"]["rope_theta"])
            if "rope_theta" in rope.get("sliding_attention", {}):
                l_theta = float(rope["sliding_attention"]["rope_theta"])
        if "global_rope_theta" in root:
            g_theta = float(root["global_rope_theta"])
        if "local_rope_theta" in root:
            l_theta = float(root["local_rope_theta"])
        return cls(
            vocab_size=int(root["vocab_size"]),
            hidden_size=int(root["hidden_size"]),
            intermediate_size=int(root["intermediate_size"]),
            num_hidden_layers=layers,
            num_attention_heads=int(root["num_attention_heads"]),
            norm_eps=float(root.get("norm_eps", 1e-5)),
            norm_bias=bool(root.get("norm_bias", False)),
            attention_bias=bool(root.get("attention_bias", False)),
            mlp_bias=bool(root.get("mlp_bias", False)),
            local_attention=int(root.get("local_attention", 128)),
            global_attn_every_n_layers=every,
            global_rope_theta=g_theta,
            local_rope_theta=l_theta,
            max_position_embeddings=int(root.get("max_position_embeddings", 8192)),
            layer_kinds=kinds,
        )

    @classmethod
    def load(cls, path: str) -> "EncoderConfig":
        with open(path) as f:
            return cls.from_json(json.load(f))


@dataclass
class LayaConfig:
    head_layers: int = 2
    max_len: int = 512
    head_max_len: int = 192
    act_costs: dict = field(default_factory=dict)
    temperature: List[float] = field(default_factory=lambda: [1.0, 1.0, 1.0])

    @property
    def action_count(self) -> int:
        return len(self.act_costs) + 1

    @classmethod
    def load(cls, path: str) -> "LayaConfig":
        with open(path) as f:
            root = json.load(f)
        return cls(
            head_layers=int(root.get("head_layers", 2)),
            max_len=int(root.get("max_len", 512)),
            head_max_len=int(root.get("head_max_len", 192)),
            act_costs=dict(root.get("act_costs", {})),
            temperature=list(root.get("temperature", [1.0, 1.0, 1.0])),
        )


@dataclass
class ModelConfig:
    """Encoder + decision head, as ``TrainableDecisionModel`` builds it
    (src/StructuredDecisions.Laya.Training/TrainableDecisionModel.cs:105-182): the head has
    ``max(1, d/64)`` heads and a ``4·d`` ReLU feed-forward (.reference/laya/common.py:96-98)."""

    encoder: EncoderConfig
    head_layers: int = 2
    n_act: int = 2

    @property
    def hidden(self) -> int:
        return self.encoder.hidden_size

    @property
    def head_heads(self) -> int:
        return max(1, self.hidden // 64)

    @property
    def head_ff(self) -> int:
        return 4 * self.hidden

    @classmethod
    def from_directory(cls, directory: str) -> "ModelConfig":
        enc = EncoderConfig.load(os.path.join(directory, "encoder", "config.json"))
        laya = LayaConfig.load(os.path.join(directory, "rl_agent_config.json"))
        return cls(encoder=enc, head_layers=laya.head_layers, n_act=laya.action_count)


def modernbert_base(layers: Optional[int] = None) -> ModelConfig:
    """ModernBERT-base shape: 22 layers, d 768, 12 heads × 64, GeGLU intermediate 1152, vocab 50368,
    every third layer global (θ 160000), the rest sliding window 128 (θ 10000), bias-free norms."""
    enc = EncoderConfig(vocab_size=50368, hidden_size=768, intermediate_size=1152,
                        num_hidden_layers=22 if layers is None else layers, num_attention_heads=12,
                        local_attention=128, global_attn_every_n_layers=3)
    return ModelConfig(encoder=enc, head_layers=2, n_act=2)


def modernbert_large(layers: Optional[int] = None) -> ModelConfig:
    """ModernBERT-large shape (the reference's English and TypedDecisions checkpoints, 421M parameters with
    the head): 28 layers, d 1024, 16 heads × 64, GeGLU intermediate 2624, vocab 50368, every third layer
    global (θ 160000), the rest sliding window 128 (θ 10000)."""
    enc = EncoderConfig(vocab_size=50368, hidden_size=1024, intermediate_size=2624,
                        num_hidden_layers=28 if layers is None else layers, num_attention_heads=16,
                        local_attention=128, global_attn_every_n_layers=3)
    return ModelConfig(encoder=enc, head_layers=2, n_act=2)


def mmbert_base(layers: Optional[int] = None) -> ModelConfig:
    """mmBERT-base shape (the reference's Multilingual checkpoint): ModernBERT-base widths with a
    256,000-token vocabulary."""
    enc = EncoderConfig(vocab_size=256000, hidden_size=768, intermediate_size=1152,
                        num_hidden_layers=22 if layers is None else layers, num_attention_heads=12,
                        local_attention=128, global_attn_every_n_layers=3)
    return ModelConfig(encoder=enc, head_layers=2, n_act=2)
