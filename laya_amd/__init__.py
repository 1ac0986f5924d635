"""laya_amd: an MI355X-native (gfx950) fine-tuning step for the Laya ModernBERT decision model.

The compute runs in ``liblaya_hip.so``, a C-ABI library of hand-written HIP kernels (declared in
``include/laya_hip.h``). This package is its host-side mirror of the reference's C# surface:
``ops`` mirrors ``Ops``, ``model`` mirrors ``TrainableDecisionModel``, ``training`` mirrors
``AdamW`` / ``CosineSchedule`` / ``Gradients`` / ``RlcdObjective``.
"""
from .config import EncoderConfig, LayaConfig, ModelConfig, modernbert_base  # noqa: F401
from .batch import Batch, TrainingItem  # noqa: F401
