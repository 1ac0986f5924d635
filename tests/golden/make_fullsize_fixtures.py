"""Writes the full-size parity fixtures of the GPU tests in tests/test_gpu_fullsize.py.

    python tests/golden/make_fullsize_fixtures.py b32x512      # ~10 min on 8 cores
    python tests/golden/make_fullsize_fixtures.py b2x8192      # ~1 h on 8 cores

For one workload (ModernBERT-base, 22 layers, plus the decision head, the first batch bench.py draws for
it) the oracle runs one training-mode forward (head dropout 0.1) and backward in fp64 (the exact
result) and in fp32 (the reference's own arithmetic), from parameters made by helpers.fixture_params.
The logit gradient is the workload's cross-entropy gradient of the fp64 logits. Stored, per parameter
with a gradient: a count sketch of the fp64 gradient (tests/sketch.py), its 64 largest-magnitude
entries and their positions, its max |g|, and the fp32 oracle's relative L2 distance from it (the
bar's floor: two fp32 implementations may differ by that much). Also the fp64 logits and the logit
gradient. The GPU test regenerates the parameters and the batch, runs the same step, and compares
sketches.

Whole gradients of 164M parameters do not fit a fixture; sketches of them do (≈ 1 MB per workload).
"""
from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "tests")]

import bench  # noqa: E402
import oracle  # noqa: E402
from helpers import fixture_params  # noqa: E402
from laya_amd.config import modernbert_base  # noqa: E402
from sketch import sketch, top_entries  # noqa: E402

PARAM_SEED = 20241
STEP_SEED = 1001
HEAD_DROPOUT = 0.1


def fixture_path(workload: str) -> str:
    return os.path.join(HERE, f"fullsize_{workload}.npz")


def workload_batch(workload: str):
    """The first batch bench.py draws for the workload, its targets and its loss scale."""
    w = bench.WORKLOADS[workload]
    batch, targets = bench.make_batch(np.random.default_rng(2024), w)
    return batch, targets, (float(batch.n_items) if w["summed"] else 1.0)


def main(workload: str) -> None:
    mc = modernbert_base()
    batch, targets, scale = workload_batch(workload)
    print(f"{workload}: {batch.n_items} sequences, {batch.n_tokens} tokens", flush=True)
    out = {}
    runs = {}
    for double in (True, False):
        t0 = time.time()
        o = oracle.OracleModel(mc, double=double)
        o.set_params(fixture_params(o.shapes, PARAM_SEED))
        o.set_head_dropout(HEAD_DROPOUT)
        logits = o.forward(batch, training=True, keep_tape=True, seed=STEP_SEED)
        if double:
            _, dlogits = oracle.cross_entropy(batch.n_options, logits.astype(np.float32), targets, 1.0, scale)
            out["logits"] = logits.astype(np.float64)
            out["dlogits"] = dlogits.astype(np.float32)
        o.backward(out["dlogits"])
        runs[double] = {n: o.grad(n) for n in o.shapes if o.has_grad(n)}
        print(f"  {'fp64' if double else 'fp32'} oracle: {time.time() - t0:.0f} s", flush=True)
        del o
    names = sorted(runs[True])
    fp32_err, max_abs = [], []
    for n in names:
        e, g32 = runs[True][n].astype(np.float64).reshape(-1), runs[False][n].astype(np.float64).reshape(-1)
        fp32_err.append(float(np.linalg.norm(e - g32) / max(np.linalg.norm(e), 1e-30)))
        max_abs.append(float(np.abs(e).max()))
        out["sk/" + n] = sketch(n, e).astype(np.float32)
        out["top_i/" + n], out["top_v/" + n] = top_entries(e)
    out["names"] = np.array(names)
    out["fp32_err"] = np.array(fp32_err)
    out["max_abs"] = np.array(max_abs)
    out["meta"] = np.array([PARAM_SEED, STEP_SEED, batch.n_tokens, batch.n_items], np.int64)
    np.savez(fixture_path(workload), **out)
    worst = int(np.argmax(fp32_err))
    print(f"wrote {fixture_path(workload)}: {len(names)} gradients, fp32 oracle worst rel-L2 "
          f"{fp32_err[worst]:.2e} ({names[worst]})", flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "b32x512")
