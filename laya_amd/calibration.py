"""Post-training temperature scaling, as the reference trainer runs it after its last epoch.

``fit_one`` / ``fit`` follow TemperatureFitting.FitOne / Fit
(src/StructuredDecisions.Laya.Training/TemperatureFitting.cs:35-101): the temperature T minimising the
soft cross-entropy −mean Σ t·log softmax(z / T), found by an 80-step golden-section search over log T in
[log 0.02, log 50]; types with no samples get 1.2, fits on fewer than 10 samples return 1.0, and every
fit is clamped to [0.5, 5] (NaN → 1) as Calibration.ClampTemperature (Calibration.cs:15-24) does.
Buckets are "type:size" with size 2 / 3-5 / 6-10 / 11+ (Questions.cs:38-42).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Sequence

import numpy as np

MISSING_TYPE_TEMPERATURE = 1.2
MINIMUM_SAMPLES = 10
TEMPERATURE_MIN, TEMPERATURE_MAX = 0.5, 5.0
QUESTION_TYPES = ("choice", "score", "noul")


@dataclass
class CalibrationSample:
    question_type: int
    logits: np.ndarray
    target: np.ndarray


@dataclass
class TemperatureFit:
    by_type: List[float]
    by_bucket: Dict[str, float] = field(default_factory=dict)
    samples_per_bucket: Dict[str, int] = field(default_factory=dict)

    def describe(self) -> str:
        """Trainer.Describe (Trainer.cs:213-215)."""
        buckets = ", ".join(f"{k}={v:.3f} (n={self.samples_per_bucket[k]})" for k, v in self.by_bucket.items())
        return (f"choice {self.by_type[0]:.3f}, score {self.by_type[1]:.3f}, noul {self.by_type[2]:.3f}; "
                f"buckets {buckets}")


def _f32(v: float) -> float:
    return float(np.float32(v))


def clamp_temperature(t: float, lo: float = TEMPERATURE_MIN, hi: float = TEMPERATURE_MAX) -> float:
    t = _f32(t)
    return min(max(t, lo), hi) if math.isfinite(t) else 1.0


def question_type_name(qtype: int) -> str:
    return QUESTION_TYPES[qtype] if qtype in (0, 1) else "noul"


def temperature_bucket(qtype: int, options: int) -> str:
    size = "2" if options <= 2 else "3-5" if options <= 5 else "6-10" if options <= 10 else "11+"
    return f"{question_type_name(qtype)}:{size}"


def _objective(samples: Sequence[CalibrationSample], log_t: float) -> float:
    t = math.exp(log_t)
    total = 0.0
    for s in samples:
        z = np.asarray(s.logits, np.float32).astype(np.float64)
        scaled = z / t
        mx = float(np.max(scaled))
        log_sum = mx + math.log(float(np.sum(np.exp(scaled - mx))))
        total -= float(np.sum(np.asarray(s.target, np.float32).astype(np.float64) * (scaled - log_sum)))
    return total / len(samples)


def fit_one(samples: Sequence[CalibrationSample]) -> float:
    """TemperatureFitting.FitOne: golden-section search over log T (an fp32 result)."""
    if len(samples) < MINIMUM_SAMPLES:
        return 1.0
    low, high = math.log(0.02), math.log(50.0)
    ratio = (math.sqrt(5.0) - 1.0) / 2.0
    a, b = high - ratio * (high - low), low + ratio * (high - low)
    fa, fb = _objective(samples, a), _objective(samples, b)
    iteration = 0
    while iteration < 80 and high - low > 1e-7:
        if fa < fb:
            high, b, fb = b, a, fa
            a = high - ratio * (high - low)
            fa = _objective(samples, a)
        else:
            low, a, fa = a, b, fb
            b = low + ratio * (high - low)
            fb = _objective(samples, b)
        iteration += 1
    return _f32(math.exp((low + high) / 2.0))


def fit(samples: Sequence[CalibrationSample], minimum_bucket_samples: int = 30) -> TemperatureFit:
    """TemperatureFitting.Fit: every type, and every bucket with enough samples."""
    by_type = []
    for qtype in range(3):
        selected = [s for s in samples if s.question_type == qtype]
        by_type.append(_f32(MISSING_TYPE_TEMPERATURE) if not selected else clamp_temperature(fit_one(selected)))
    groups: Dict[str, List[CalibrationSample]] = {}
    for s in samples:  # first-appearance order, as LINQ GroupBy keeps it
        groups.setdefault(temperature_bucket(s.question_type, len(s.logits)), []).append(s)
    by_bucket, counts = {}, {}
    for key, group in groups.items():
        counts[key] = len(group)
        if len(group) >= minimum_bucket_samples:
            by_bucket[key] = clamp_temperature(fit_one(group))
    return TemperatureFit(by_type, by_bucket, counts)
