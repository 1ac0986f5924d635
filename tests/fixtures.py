"""Loaders for the reference's golden fixture (tests/golden/training-tiny, copied from the
reference's tests/StructuredDecisions.Tests/Fixtures/training-tiny, written by PyTorch autograd in
tools/dump_training_reference.py:37-99)."""
import json
import os

import numpy as np

from laya_amd.batch import Batch, TrainingItem
from laya_amd.config import ModelConfig
from laya_amd.safetensors_io import SafetensorsFile

TINY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "training-tiny")


def tiny_config() -> ModelConfig:
    return ModelConfig.from_directory(TINY)


def tiny_params() -> dict:
    st = SafetensorsFile(os.path.join(TINY, "model.safetensors"))
    return {n: st.read_float32(n) for n in st.entries}


def tiny_grads() -> dict:
    st = SafetensorsFile(os.path.join(TINY, "grads.safetensors"))
    return {n: st.read_float32(n) for n in st.entries}


def tiny_batch():
    """(batch, coeff = dL/dlogits, torch logits) of batch.json (TrainingGradientTests.cs:22-31)."""
    with open(os.path.join(TINY, "batch.json")) as f:
        b = json.load(f)
    items = [TrainingItem(np.array(i["ids"]), np.array(i["markers"]), i["qtype"], np.zeros(len(i["markers"])))
             for i in b["items"]]
    coeff = np.concatenate([i["coeff"] for i in b["items"]]).astype(np.float32)
    logits = np.concatenate([i["logits"] for i in b["items"]]).astype(np.float64)
    return Batch.from_items(items), coeff, logits


def objective_fixture() -> dict:
    with open(os.path.join(TINY, "objective.json")) as f:
        return json.load(f)


def max_rel(expected, actual) -> float:
    """The reference test's metric: max|Δ| / max|g| (TrainingGradientTests.cs:69-77)."""
    e = np.asarray(expected, np.float64)
    a = np.asarray(actual, np.float64)
    return float(np.abs(e - a).max() / max(np.abs(e).max(), 1e-12)) if e.size else 0.0


def rel_l2(expected, actual) -> float:
    e = np.asarray(expected, np.float64).reshape(-1)
    a = np.asarray(actual, np.float64).reshape(-1)
    return float(np.linalg.norm(e - a) / max(np.linalg.norm(e), 1e-30)) if e.size else 0.0
