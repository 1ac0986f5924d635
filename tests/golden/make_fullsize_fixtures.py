"""Writes the full-size parity fixtures of the GPU tests in tests/test_gpu_fullsize.py.

    python tests/golden/make_fullsize_fixtures.py b32x512              # ~10 min on 8 cores
    python tests/golden/make_fullsize_fixtures.py b2x8192              # ~1 h on 8 cores
    python tests/golden/make_fullsize_fixtures.py b32x512 --bench-init # bench.py's own parameters and step

For one workload (ModernBERT-base, 22 layers, plus the decision head, the first batch bench.py draws for
it) the oracle runs one training-mode forward (head dropout 0.1) and backward in fp64 (the exact
result) and in fp32 (the reference's own arithmetic). The parameters come from helpers.fixture_params
(γ = 1 + 0.2·N(0,1) so γ errors show, head linear1 biases away from the ReLU's kink), or, with
--bench-init, from laya_amd.model.synthetic_params with bench.py's seed (N(0, 0.02) matrices, γ = 1,
zero biases: exactly what bench.py times) and bench.py's first step seed.
The logit gradient is the workload's cross-entropy gradient of the fp64 logits. Stored, per parameter
with a gradient: a count sketch of the fp64 gradient (tests/sketch.py), its 64 largest-magnitude
entries and their positions, its max |g|, and the fp32 oracle's relative L2 distance from it (the
bar's floor: two fp32 implementations may differ by that much). Also the fp64 logits and the logit
gradient. The GPU test regenerates the parameters and the batch, runs the same step, and compares
sketches.

The head's ReLU is the model's one discontinuity. For each head layer the fixture also keeps the exact
linear1 outputs (the ReLU's inputs) that lie within TIE_WIDTH × their RMS of zero, with their positions,
and a SHA-256 of the exact sign bits of every other position (packed, the tie positions cleared): a
GPU run whose own sign bits, tie positions cleared, hash the same agrees with the exact computation on
every ReLU decision outside the ties, and its tie values can be compared one by one.

Whole gradients of 164M parameters do not fit a fixture; sketches of them do (≈ 1 MB per workload).
"""
from __future__ import annotations

import hashlib
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
from laya_amd.model import synthetic_params  # noqa: E402
from sketch import sketch, top_entries  # noqa: E402

PARAM_SEED = 20241
STEP_SEED = 1001
HEAD_DROPOUT = 0.1
# What bench.py runs: its parameter seed and the seed of its first step (bench.py: seed = 1000 + i).
BENCH_PARAM_SEED = bench.PARAM_SEED
BENCH_STEP_SEED = bench.STEP_SEED0
# Head ReLU inputs closer to zero than this fraction of their layer's RMS count as ties.
TIE_WIDTH = 1e-4


def fixture_path(workload: str, bench_init: bool = False) -> str:
    return os.path.join(HERE, f"fullsize_{workload}{'_bench_init' if bench_init else ''}.npz")


def workload_batch(workload: str):
    """The first batch bench.py draws for the workload, its targets and its loss scale."""
    w = bench.WORKLOADS[workload]
    batch, targets = bench.make_batch(np.random.default_rng(2024), w)
    return batch, targets, (float(batch.n_items) if w["summed"] else 1.0)


def params_for(shapes, bench_init: bool):
    return synthetic_params(shapes, BENCH_PARAM_SEED) if bench_init else fixture_params(shapes, PARAM_SEED)


def sign_digest(h: np.ndarray, ties: np.ndarray) -> str:
    """SHA-256 of the packed sign bits (h > 0) of a flat array, the positions `ties` cleared."""
    bits = np.asarray(h).reshape(-1) > 0
    bits[ties] = False
    return hashlib.sha256(np.packbits(bits).tobytes()).hexdigest()


def main(workload: str, bench_init: bool) -> None:
    mc = modernbert_base()
    batch, targets, scale = workload_batch(workload)
    step_seed = BENCH_STEP_SEED if bench_init else STEP_SEED
    print(f"{workload}{' (bench init)' if bench_init else ''}: {batch.n_items} sequences, {batch.n_tokens} tokens",
          flush=True)
    out = {}
    runs, pre = {}, {}
    for double in (True, False):
        t0 = time.time()
        o = oracle.OracleModel(mc, double=double)
        o.set_params(params_for(o.shapes, bench_init))
        o.set_head_dropout(HEAD_DROPOUT)
        o.capture_head_preactivations(True)
        logits = o.forward(batch, training=True, keep_tape=True, seed=step_seed)
        pre[double] = [o.head_preactivation(j).reshape(-1) for j in range(mc.head_layers)]
        if double:
            _, dlogits = oracle.cross_entropy(batch.n_options, logits.astype(np.float32), targets, 1.0, scale)
            out["logits"] = logits.astype(np.float64)
            out["dlogits"] = dlogits.astype(np.float32)
        o.capture_head_preactivations(False)
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
    for j, h in enumerate(pre[True]):
        rms = float(np.sqrt(np.mean(h * h)))
        ties = np.flatnonzero(np.abs(h) < TIE_WIDTH * rms).astype(np.int64)
        out[f"relu{j}/rms"] = np.array(rms)
        out[f"relu{j}/tie_i"] = ties
        out[f"relu{j}/tie_v"] = h[ties]
        out[f"relu{j}/digest"] = np.array(sign_digest(h, ties))
        flips32 = int(np.count_nonzero((pre[False][j] > 0) != (h > 0)))
        out[f"relu{j}/fp32_flips"] = np.array(flips32)
        print(f"  head layer {j}: ReLU input RMS {rms:.4f}, {ties.size} ties within {TIE_WIDTH:g} × RMS, the fp32 "
              f"oracle decides {flips32} differently from fp64", flush=True)
    out["names"] = np.array(names)
    out["fp32_err"] = np.array(fp32_err)
    out["max_abs"] = np.array(max_abs)
    out["meta"] = np.array([BENCH_PARAM_SEED if bench_init else PARAM_SEED, step_seed, batch.n_tokens,
                            batch.n_items], np.int64)
    path = fixture_path(workload, bench_init)
    np.savez(path, **out)
    worst = int(np.argmax(fp32_err))
    print(f"wrote {path}: {len(names)} gradients, fp32 oracle worst rel-L2 "
          f"{fp32_err[worst]:.2e} ({names[worst]})", flush=True)


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    main(args[0] if args else "b32x512", "--bench-init" in sys.argv[1:])
