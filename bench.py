"""Fine-tuning throughput of the Laya ModernBERT decision model on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--workload NAME]

A step is one full optimizer step over one synthetic batch: forward, the decision head's soft
cross-entropy gradient, backward, global-norm clip and AdamW (fwd+bwd+AdamW), all on the device.
Workload: ModernBERT-base (22 layers, d 768, 12 heads × 64, GeGLU 1152, vocab 50368, every third
layer global, the rest a 128-token sliding window) plus the two-layer decision head, fp32, batch
32 × seq 512 with a trailing-padding fraction U[0, 0.3] per sequence (padding is never computed:
sequences are packed), items cycling choice K=8 / score K=4 / noul K=2, summed cross-entropy,
AdamW lr 3e-5 wd 0.01, clip 1.0, head dropout 0.1. Weights N(0, 0.02) from a fixed seed
(laya_amd.model.synthetic_params), unit LayerNorm weights, zero biases.

`--workload` selects another shape (batch 4 × 128; batch 32 × 1024 and a packed Zipf batch of 64
sequences with bf16 weights and the backward products on bf16 operands; batch 2 × 8192); the default is the
one above.

Prints one JSON line. `value` counts real (unpadded) tokens per second over the timed steps, with
every input already resident; `roofline` describes the kernel with the largest share of device
time, measured live with HIP events on the library's stream during a second pass over the same
batches (so the events never sit inside the timed steps); `cpu_baseline` times the C++ oracle
(the reference algorithm restated, per-layer recompute included) on a bounded sample of the same
workload on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fine-tune tokens/sec (fwd+bwd+AdamW), 1 MI355X; bwd MFMA util % & HBM GB/s"
PEAK_FP32_MFMA = 157.3e12
PEAK_HBM = 8.0e12
# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE and calibrated against a
# copy-like kernel of known size (the commands and the calibration sit in
# profiles/gemm_bwd_pair_h2w_hbm_traffic_b32x512.md, and for the three-piece kernel in
# profiles/gemm_bwd_pair_x6w_hbm_traffic_b32x512.md). Counters cannot be read from inside the process, so
# the figure is carried here per (workload, kernel) it was measured on and is reported only when that kernel
# is the dominant one of that workload; any other case reports null.
MEASURED_TRAFFIC = {("b32x512", "gemm_bwd_pair_x6w"): 0.865e9,
                    ("b32x512", "gemm_bwd_pair_h2w"): 0.852e9}


PEAK_BF16_MFMA = 2.5e15
# The parameters (laya_amd.model.synthetic_params with this seed) and the seed of timed step i (STEP_SEED0 + i,
# warm-up steps first): tests/golden/make_fullsize_fixtures.py --bench-init reruns the first step on the oracle.
PARAM_SEED = 42
STEP_SEED0 = 1000


def mfma_peaks(name: str):
    """(peak in algorithmic fp32 flops/s, 16-bit MFMA issues per algorithmic flop) of a matrix-core kernel.

    Kernels named *_x6 / *_x6w / *_x6t compute fp32 products from exact three-piece bf16 splits: six bf16
    MFMA products per fp32 one, so their fp32-equivalent peak is the bf16 peak over six. *_h2w / *_h2t
    compute them from two-piece fp16 splits of power-of-two-scaled operands: three fp16 MFMA products per
    fp32 one (fp16 and bf16 share the 2.5 PFLOP/s dense peak), peak over three; *_h2b1 / *_h2b1w / *_h2b1t
    the same with bf16-valued weights, which are one fp16 piece: two products, peak over two. *_bf16 /
    *_bf16w run bf16 operands (one product each). The rest run the fp32 matrix cores."""
    base = name[:-1] if name.endswith(("_x6w", "_x6t", "_bf16w", "_h2w", "_h2t", "_h2q", "_h2b1w",
                                       "_h2b1t")) else name
    if base.endswith("_x6"):
        return PEAK_BF16_MFMA / 6, 6.0
    if base.endswith("_h2b1"):
        return PEAK_BF16_MFMA / 2, 2.0
    if base.endswith("_h2"):
        return PEAK_BF16_MFMA / 3, 3.0
    if base.endswith("_bf16"):
        return PEAK_BF16_MFMA, 1.0
    return PEAK_FP32_MFMA, 0.0


def mfma_summary(prof: dict, names) -> dict:
    """Algorithmic TFLOP/s of a group of kernels, its fraction of the group's fp32-equivalent peak, and
    the fraction of the bf16 matrix-core pipe the hardware products keep busy (the same denominator for
    GEMMs and attention)."""
    ks = [(n, prof[n]) for n in names if n in prof and prof[n]["flops"]]
    if not ks:
        return {}
    flops = sum(k["flops"] for _, k in ks)
    sec = sum(k["ms"] for _, k in ks) / 1e3
    peak_time = sum(k["flops"] / mfma_peaks(n)[0] for n, k in ks)
    out = {"tflops": round(flops / sec / 1e12, 1), "frac_of_peak": round(peak_time / sec, 4)}
    bf16_ops = sum(k["flops"] * mfma_peaks(n)[1] for n, k in ks)
    if bf16_ops:
        out["bf16_pipe_frac"] = round(bf16_ops / sec / PEAK_BF16_MFMA, 4)
    return out

# The workloads: batch shape, heads, loss scaling (summed CE multiplies the mean by the item count) and
# the precision of the matrix products. b32x512 is the headline configuration.
WORKLOADS = {
    "b4x128": dict(desc="batch 4 x seq 128, no padding, one choice head K=5, mean CE", batch=4, seq=128, pad=0.0,
                   heads="choice5", summed=False, matmul="fp32"),
    "b32x512": dict(desc="batch 32 x seq 512, trailing padding U[0,0.3], heads choice8/score4/noul2, summed CE",
                    batch=32, seq=512, pad=0.3, heads="mixed", summed=True, matmul="fp32"),
    "b32x1024-bf16": dict(desc="batch 32 x seq 1024, no padding, heads choice8/score4/noul2, summed CE, bf16 weights "
                               "(the forward's fp32-accurate products read them rounded to bf16), backward products "
                               "on bf16 operands (fp32 master weights, accumulation, softmax and LayerNorm statistics)",
                          batch=32, seq=1024, pad=0.0, heads="mixed", summed=True, matmul="bf16-backward",
                          bf16_weights=True),
    "b2x8192": dict(desc="batch 2 x seq 8192, no padding, one choice head K=5, mean CE", batch=2, seq=8192, pad=0.0,
                    heads="choice5", summed=False, matmul="fp32"),
    "packed64-zipf-bf16": dict(desc="64 sequences of lengths U[16,2048] packed without padding, ids Zipf(1.1), heads "
                                    "choice8/score4/noul2, summed CE, bf16 weights, backward products on bf16 "
                                    "operands",
                               batch=64, seq=2048, pad=None, heads="mixed", summed=True, matmul="bf16-backward",
                               bf16_weights=True),
}


def make_batch(rng, w, vocab=50368):
    from laya_amd.batch import Batch
    n = w["batch"]
    if w["pad"] is None:  # packed variable lengths U[16, seq]
        lengths = rng.integers(16, w["seq"] + 1, size=n).astype(np.int32)
    else:
        fractions = rng.uniform(0.0, w["pad"], size=n)
        lengths = (w["seq"] - np.floor(w["seq"] * fractions)).astype(np.int32)
    kinds = [(0, 5)] if w["heads"] == "choice5" else [(0, 8), (1, 4), (2, 2)]  # choice / score / noul
    qtypes = np.array([kinds[i % len(kinds)][0] for i in range(n)], np.int32)
    n_options = np.array([kinds[i % len(kinds)][1] for i in range(n)], np.int32)
    total = int(lengths.sum())
    if w["pad"] is None:  # Zipf(1.1) ranks over the vocabulary, rank r → id r − 1
        p = np.arange(1, vocab + 1, dtype=np.float64) ** -1.1
        tokens = rng.choice(vocab, size=total, p=p / p.sum()).astype(np.int32)
    else:
        tokens = rng.integers(0, vocab, size=total, dtype=np.int64).astype(np.int32)
    markers = np.concatenate([1 + 2 * np.arange(k) for k in n_options]).astype(np.int32)
    labels = [rng.integers(0, k) for k in n_options]
    targets = np.concatenate([np.eye(k, dtype=np.float32)[lab] for k, lab in zip(n_options, labels)])
    return Batch(lengths=lengths, tokens=tokens, n_options=n_options, markers=markers, qtypes=qtypes), targets


def _oracle_step(mc, sub, t_sub, summed: bool) -> float:
    """One full fp32 step of the oracle (forward, CE, backward with per-layer recompute, clip, AdamW) on `sub`;
    returns its wall time. The Adam moments are allocated first, as the reference's first step does."""
    import oracle
    o = oracle.OracleModel(mc)
    prng = np.random.default_rng(1)
    o.set_params({n: (np.ones(s, np.float32) if ("norm" in n and n.endswith("weight")) or n == "scorer.0.weight"
                      or n == "temperature" else
                      np.zeros(s, np.float32) if n.endswith("bias") else
                      (0.02 * prng.standard_normal(s)).astype(np.float32)) for n, s in o.shapes.items()})
    o.set_head_dropout(0.1)
    o.adamw(0.0, 0.0)
    t0 = time.perf_counter()
    logits = o.forward(sub, training=True, keep_tape=True, seed=1).astype(np.float32)
    _, g = oracle.cross_entropy(sub.n_options, logits, t_sub, 1.0, float(sub.n_items) if summed else 1.0)
    o.backward(g)
    o.clip(1.0)
    o.adamw(3e-5, 3e-5)
    return time.perf_counter() - t0


def cpu_baseline(mc, batch, targets, items: int, summed: bool, extrapolate: bool, one_thread: bool):
    """The oracle (the reference algorithm restated, fp32, OpenMP over the host cores) on the first `items`
    sequences of the batch. With `extrapolate`, the step is timed on 3- and 6-layer encoders and extrapolated
    linearly in layers to the model's depth (the long-sequence workloads, whose 22-layer CPU step would take
    minutes). With `one_thread`, the same sample is also timed on one thread."""
    import oracle
    from laya_amd.batch import Batch
    from laya_amd.config import modernbert_base
    sub = Batch(lengths=batch.lengths[:items], tokens=batch.tokens[:int(batch.lengths[:items].sum())],
                n_options=batch.n_options[:items], markers=batch.markers[:int(batch.n_options[:items].sum())],
                qtypes=batch.qtypes[:items])
    t_sub = targets[:sub.n_markers]
    layers = mc.encoder.num_hidden_layers

    def timed():
        if not extrapolate:
            return _oracle_step(mc, sub, t_sub, summed), "one full fp32 step"
        t3 = _oracle_step(modernbert_base(3), sub, t_sub, summed)
        print(f"cpu baseline: 3-layer step {t3:.1f} s", file=sys.stderr, flush=True)
        t6 = _oracle_step(modernbert_base(6), sub, t_sub, summed)
        print(f"cpu baseline: 6-layer step {t6:.1f} s", file=sys.stderr, flush=True)
        return (t3 + (t6 - t3) * (layers - 3) / 3.0,
                f"one fp32 step extrapolated linearly in layers to {layers} from 3- and 6-layer encoders "
                f"({t3:.1f} s and {t6:.1f} s)")

    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    oracle.set_threads(cores)
    dt, how = timed()
    out = {"value": sub.n_tokens / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
           "sample": f"{how} (fwd+CE+bwd with per-layer recompute+clip+AdamW over all parameters) of the first "
                     f"{items} sequences ({sub.n_tokens} real tokens) of the same batch, {dt:.1f} s"}
    if one_thread:
        oracle.set_threads(1)
        dt1, how1 = timed()
        oracle.set_threads(cores)
        out["one_thread"] = {"value": sub.n_tokens / dt1, "unit": "tokens/s", "cores": 1,
                             "sample": f"{how1} on one thread, same sample, {dt1:.1f} s"}
    return out


def per_op_rate(ctx, mc, model, batches, w, args, scale):
    """The same warm-up and timed steps composed from the per-op entry points alone (laya_amd.opmodel), from
    the benchmark's initial weights, every batch's tables uploaded before the timed region."""
    from laya_amd.model import synthetic_params
    from laya_amd.opmodel import OpBatch, OpLevelModel
    if w["matmul"] != "fp32" or w.get("bf16_weights"):
        raise SystemExit("--per-op measures the fp32 workloads")
    params = synthetic_params(model.shapes, PARAM_SEED)
    om = OpLevelModel(mc, {n: params[n] for n in model.names}, ctx)
    om.head_dropout = 0.1
    obs = [OpBatch(ctx, b, t, mc.encoder.vocab_size) for b, t in batches]
    ctx.sync()

    def step(i):
        om.train_step(obs[i], seed=STEP_SEED0 + i, ce_weight=1.0, loss_scale=scale(batches[i][0]), max_norm=1.0,
                      lr_encoder=3e-5, lr_head=3e-5, weight_decay=0.01)

    for i in range(args.warmup):
        step(i)
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + args.steps):
        step(i)
    ctx.sync()
    dt = time.perf_counter() - t0
    tokens = sum(b.n_tokens for b, _ in batches[args.warmup:])
    print(f"per-op: timed {args.steps} steps in {dt:.3f} s", file=sys.stderr, flush=True)
    # A non-finite value anywhere in a step reaches every weight through AdamW; the rate of steps on NaN data
    # (which the matrix cores run at a different clock) is no rate of this path.
    bad = [n for n in (model.names[1], model.names[len(model.names) // 2], model.names[-1])
           if not np.isfinite(om.param(n)).all()]
    if bad:
        for ob in obs:
            ob.close()
        om.close()
        raise RuntimeError(f"per-op path: {bad[0]} is not finite after the timed steps")
    if not args.no_profile:
        ctx.profile_begin()
        for i in range(args.warmup, args.warmup + args.steps):
            step(i)
        ctx.sync()
        prof = ctx.profile_end()
        total_ms = sum(k["ms"] for k in prof.values())
        for name, k in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])[:16]:
            print(f"  per-op {name:22s} {k['launches']:6d} launches {k['ms']:9.2f} ms {k['ms'] / total_ms * 100:5.1f}%",
                  file=sys.stderr)
    for ob in obs:
        ob.close()
    om.close()
    return {"value": round(tokens / dt, 1), "unit": "tokens/s", "ms_per_step": round(dt / args.steps * 1e3, 3),
            "how": "the same steps composed from the per-op C-ABI entry points (laya_amd.opmodel), one call per "
                   "Ops method in TrainableDecisionModel's order, from the same initial weights; the binding keeps "
                   "the encoder operands' magnitude words (laya_hip.h's _w variants) as it keeps attention's "
                   "context and LSE"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline leg")
    ap.add_argument("--cpu-items", type=int, default=None,
                    help="sequences in the CPU sample (default 16 for b32x512, 1 for the long-sequence workloads)")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="b32x512")
    ap.add_argument("--cpu-full", action="store_true",
                    help="time the CPU baseline at full depth even for the long-sequence workloads")
    ap.add_argument("--cpu-one-thread", action="store_true",
                    help="also time the CPU baseline's sample on one thread (always done for the headline)")
    ap.add_argument("--fp32-mfma", action="store_true",
                    help="fp32 products on the fp32 matrix cores instead of exact bf16 splits (for comparison)")
    ap.add_argument("--split3", action="store_true",
                    help="fp32 products from three-piece bf16 splits in every kernel instead of two-piece fp16 "
                         "products in the 256-wide ones (for comparison)")
    ap.add_argument("--no-profile", action="store_true", help="time without per-launch events")
    ap.add_argument("--all-bf16", action="store_true",
                    help="bf16 workloads: every product on bf16 operands (forward too: bf16 weights and activations) "
                         "instead of bf16 weights with fp32-accurate forward products (for comparison)")
    ap.add_argument("--no-bf16-copies", action="store_true",
                    help="bf16 workloads: round the fp32 weights and activations inside the products instead of "
                         "keeping bf16 copies (same results, less memory)")
    ap.add_argument("--by-value", action="store_true",
                    help="pass each batch as host arrays (laya_model_train_step: host planning and uploads inside "
                         "every step), to measure the PCIe-inclusive rate; the default stages batches first")
    ap.add_argument("--per-op", action="store_true",
                    help="also time the same steps composed from the per-op entry points alone (laya_amd.opmodel: what "
                         "a host re-pointing Ops runs), from the same initial weights, and report it beside the model "
                         "API's rate (on by default for the headline workload)")
    ap.add_argument("--no-per-op", action="store_true", help="skip the per-op leg of the headline workload")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="before the steps, run one dst += src over 2^26 floats (add_kernel: 512 MiB read, 256 MiB "
                         "written) whose HBM counters calibrate FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    from laya_amd.config import modernbert_base
    from laya_amd.device import Context
    from laya_amd.model import TrainableDecisionModel, synthetic_params

    w = WORKLOADS[args.workload]
    rng = np.random.default_rng(2024)
    mc = modernbert_base()
    batches = [make_batch(rng, w) for _ in range(args.warmup + args.steps)]
    ctx = Context(0)
    matmul = w["matmul"]
    if matmul == "fp32" and args.fp32_mfma:
        matmul = "fp32-mfma"
    elif matmul == "fp32" and args.split3:
        matmul = "fp32-split3"
    elif matmul.startswith("bf16") and args.all_bf16:
        matmul = "bf16"
    ctx.set_matmul_precision(matmul)
    cpu_items = args.cpu_items or (16 if w["seq"] <= 512 else 1)
    long_workload = w["seq"] > 512
    model = TrainableDecisionModel(mc, ctx)
    model.set_params(synthetic_params(model.shapes, PARAM_SEED))
    model.head_dropout = 0.1
    if w.get("bf16_weights") and matmul != "bf16":
        model.set_bf16_weights(True)
    if args.no_bf16_copies:
        model.set_bf16_copies(False)
    if args.traffic_probe:
        import ctypes
        from laya_amd._native import check, lib
        from laya_amd.device import DeviceArray
        n = 1 << 26
        dst, src = DeviceArray(ctx, (n,)), DeviceArray(ctx, (n,))
        check(lib().laya_add(ctx.handle, dst.ptr, src.ptr, ctypes.c_size_t(n)))
        ctx.sync()
        dst.free()
        src.free()
    # Every batch is validated, laid out and uploaded (with its targets) before timing: the timed steps
    # run on inputs already resident in HBM.
    slots = [model.stage_batch(b, t) for b, t in batches]
    ctx.sync()

    by_value = [(b, t, model.batch_args(b)) for b, t in batches] if args.by_value else None

    def scale(b):  # summed CE: the mean gradient times the item count
        return float(b.n_items) if w["summed"] else 1.0

    def step(i):
        if by_value:
            b, t, a = by_value[i]
            model.train_step(b, t, seed=STEP_SEED0 + i, ce_weight=1.0, loss_scale=scale(b), max_norm=1.0,
                             lr_encoder=3e-5, lr_head=3e-5, weight_decay=0.01, _args=a)
            return
        model.train_step_staged(slots[i], seed=STEP_SEED0 + i, ce_weight=1.0, loss_scale=scale(batches[i][0]),
                                max_norm=1.0, lr_encoder=3e-5, lr_head=3e-5, weight_decay=0.01)

    print(f"warmup {args.warmup} steps", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        step(i)
    ctx.sync()
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + args.steps):
        step(i)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    tokens = sum(b.n_tokens for b, _ in batches[args.warmup:])
    # As for the per-op leg: a rate of steps on non-finite weights is no rate of this path.
    bad = [n for n in (model.names[1], model.names[len(model.names) // 2], model.names[-1])
           if not np.isfinite(model.param(n)).all()]
    if bad:
        raise SystemExit(f"model API: {bad[0]} is not finite after the timed steps")
    prof = {}
    if not args.no_profile:
        # A separate pass over the same batches with HIP events around every launch, for the per-kernel
        # breakdown and the roofline; the events are kept out of the timed steps above.
        ctx.profile_begin()
        for i in range(args.warmup, args.warmup + args.steps):
            step(i)
        ctx.sync()
        prof = ctx.profile_end()
    loss = model.train_step_staged(slots[0], seed=7, loss_scale=scale(batches[0][0]), want_loss=True)
    print(f"timed {args.steps} steps in {elapsed:.3f} s, {tokens} real tokens, loss after {loss:.4f}",
          file=sys.stderr, flush=True)

    roofline, breakdown = None, {}
    if prof:
        total_ms = sum(k["ms"] for k in prof.values())
        for name, k in sorted(prof.items(), key=lambda kv: -kv[1]["ms"]):
            print(f"  {name:22s} {k['launches']:6d} launches {k['ms']:9.2f} ms "
                  f"{k['ms'] / total_ms * 100:5.1f}%  "
                  + (f"{k['flops'] / k['ms'] / 1e9:8.1f} TFLOP/s" if k["flops"] else
                     f"{k['bytes'] / k['ms'] / 1e6:8.1f} GB/s"), file=sys.stderr)
        name, k = max(prof.items(), key=lambda kv: kv[1]["ms"])
        per_launch_s = k["ms"] / k["launches"] / 1e3
        traffic = MEASURED_TRAFFIC.get((args.workload, name))
        if k["flops"]:
            achieved = k["flops"] / k["launches"] / per_launch_s
            peak, issue = mfma_peaks(name)
            roofline = {"bound": "mfma", "kernel": name, "achieved": round(achieved / 1e12, 2),
                        "peak": round(peak / 1e12, 1), "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                        "traffic": traffic, "avg_launch_ms": round(per_launch_s * 1e3, 4),
                        "launches": k["launches"]}
            if issue:
                roofline["bf16_pipe_frac"] = round(achieved * issue / PEAK_BF16_MFMA, 4)
                # fp32 products from pieces: the same throughput against the fp32 matrix-core peak
                roofline["vs_fp32_mfma_peak"] = round(achieved / PEAK_FP32_MFMA, 4)
        else:
            achieved = k["bytes"] / k["launches"] / per_launch_s
            roofline = {"bound": "hbm", "kernel": name, "achieved": round(achieved / 1e9, 1), "peak": 8000.0,
                        "unit": "GB/s", "frac": round(achieved / PEAK_HBM, 4), "traffic": traffic,
                        "avg_launch_ms": round(per_launch_s * 1e3, 4), "launches": k["launches"]}
        groups = {
            "bwd_gemm": [n for n in prof if n.startswith(("gemm_bwd_pair", "gemm_nn", "gemm_tn"))],
            "fwd_gemm": [n for n in prof if n.startswith("gemm_nt")],
            "attention_bwd": [n for n in prof if n.startswith(("attention_bwd_dkv", "attention_bwd_dq"))],
            "attention_fwd": [n for n in prof if n.startswith("attention_fwd")],
        }
        for g, names in groups.items():
            summ = mfma_summary(prof, names)
            if summ:
                breakdown[g] = summ
        ew = [prof[n] for n in ("layernorm_bwd", "geglu_bwd", "relu_dropout_bwd") if n in prof]
        if ew:
            b = sum(x["bytes"] for x in ew)
            ms = sum(x["ms"] for x in ew)
            breakdown["elementwise_bwd_hbm_gbs"] = round(b / (ms / 1e3) / 1e9, 1)
        hbm = {n: round(x["bytes"] / (x["ms"] / 1e3) / 1e9, 1) for n, x in prof.items() if x["bytes"] and x["ms"]}
        breakdown["hbm_gbs"] = dict(sorted(hbm.items(), key=lambda kv: -prof[kv[0]]["ms"])[:10])
        breakdown["kernel_share"] = {n: round(k["ms"] / total_ms, 4) for n, k in
                                     sorted(prof.items(), key=lambda kv: -kv[1]["ms"])[:8]}

    per_op = None
    if (args.per_op or args.workload == "b32x512") and not args.no_per_op and matmul == "fp32" and not args.by_value:
        try:
            per_op = per_op_rate(ctx, mc, model, batches, w, args, scale)
            per_op["vs_model_api"] = round(per_op["value"] / (tokens / elapsed), 4)
        except Exception as e:  # the model API's line stands on its own; say what failed
            print(f"per-op leg failed: {e}", file=sys.stderr, flush=True)
            per_op = {"error": str(e)}

    cpu = None
    if not args.no_cpu:
        print(f"cpu baseline: oracle on {cpu_items} sequences", file=sys.stderr, flush=True)
        b0, t0_ = batches[args.warmup]
        if args.workload == "b32x512":
            # All cores on 16 sequences; one thread on the first of them (≈ 10 s each).
            cpu = cpu_baseline(mc, b0, t0_, cpu_items, w["summed"], False, False)
            print("cpu baseline: one thread on 1 sequence", file=sys.stderr, flush=True)
            one = cpu_baseline(mc, b0, t0_, 1, w["summed"], False, True)
            cpu["one_thread"] = one["one_thread"]
        else:
            cpu = cpu_baseline(mc, b0, t0_, cpu_items, w["summed"], long_workload and not args.cpu_full,
                               args.cpu_one_thread)

    value = tokens / elapsed
    line = {"metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(elapsed / args.steps * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None,
            "dtype": ("fp32" if w["matmul"].startswith("fp32") else
                      "bf16 (every product on bf16 operands, fp32 accumulation)" if matmul == "bf16" else
                      "bf16 weights (fp32-accurate forward products), bf16 operands in the backward products, fp32 "
                      "accumulation"),
            "data": "synthetic",
            "config": {"workload": f"ModernBERT-base Laya encoder + decision head fine-tune step, {w['desc']}, "
                                   "AdamW lr 3e-5 wd 0.01, clip 1.0",
                       "global_batch": w["batch"], "seq_len": w["seq"], "parallelism": "none (1 GPU)",
                       "matmul_precision": {"fp32": "fp32-accurate products: two-piece fp16 splits of power-of-two-"
                                                     "scaled operands on 256-wide tiles (three fp16 MFMA products "
                                                     "each), exact three-piece bf16 splits elsewhere (six bf16 "
                                                     "MFMA products each); fp32 accumulation",
                                            "fp32-split3": "fp32 products from exact three-piece bf16 splits (six "
                                                           "bf16 MFMA products each, fp32 accumulation)",
                                            "fp32-mfma": "fp32 products on the fp32 MFMA",
                                            "bf16-backward": ("bf16 weights: the forward's fp32-accurate two-piece "
                                                              "products read each weight rounded to bf16 (fp32 "
                                                              "activations); the backward products (dX, dW) on bf16 "
                                                              "operands; fp32 accumulation and masters"
                                                              if w.get("bf16_weights") else
                                                              "fp32-accurate forward products; the backward products "
                                                              "on bf16 operands; fp32 accumulation"),
                                            "bf16": "every product on bf16 operands (weights and activations), "
                                                    "fp32 accumulation and masters"}.get(matmul, matmul),
                       "real_tokens_per_step": round(tokens / args.steps, 1),
                       "inputs": ("host arrays passed every step (PCIe-inclusive)" if args.by_value else
                                  "staged in HBM before the timed steps")},
            "roofline": roofline, "cpu_baseline": cpu, "breakdown": breakdown}
    if per_op:
        line["per_op"] = per_op
    print(json.dumps(line), flush=True)
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
