"""Benchmark: GPT-2-small-shape float32 training step through dtmi on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload (one "step"): GPT-2-small shape, float32 -- 12 layers, d_model 768,
12 heads, T = 1024, vocab 50304 (163,109,376 parameters, dtrain layout),
batch 8 sequences per replica, 4 simulated data-parallel replicas. Each
replica runs forward + backward on its own synthetic batch; gradients go
through DDP's 1 MiB buckets and the fixed-order on-device average; then the
global-norm clip at 1.0 and AdamW (lr 3e-4, betas 0.9/0.95, eps 1e-8, wd 0.1).
Weights ~N(0, 0.02) (biases 0, LayerNorm 1/0), tokens uniform over the vocab.
Everything is resident in HBM before the timed region; no host round trip
happens inside a step.

Prints one JSON line: tokens/s for the whole step (4 x 8 x 1024 tokens),
ms/step, the roofline of the dominant kernel family (the MFMA GEMMs: FLOP per
launch / average launch time measured with HIP events on the library stream
over the timed steps, against the 157.3 TFLOP/s float32 matrix peak), per-family
figures for the other kernels, and the oracle's (NumPy) speed on this
machine's host cores on a bounded sample of the same step.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "distributed-training_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "fwd+bwd+AdamW tokens/sec at GPT-2-small shape; % MFMA / % HBM roofline"
PEAK_FP32_MFMA = 157.3e12
PEAK_HBM = 8.0e12
CFG = dict(vocab=50304, ctx=1024, dim=768, heads=12, layers=12, dtype="float32")
BATCH, WORLD = 8, 4
LR, BETAS, EPS, WD, CLIP = 3e-4, (0.9, 0.95), 1e-8, 0.1, 1.0


def param_spec(c):
    C, V = c["dim"], c["vocab"]
    spec = [("tok", (V, C)), ("pos", (c["ctx"], C))]
    for i in range(c["layers"]):
        p = f"blocks.{i}."
        spec += [(p + "ln1.w", (C,)), (p + "ln1.b", (C,)), (p + "qkv.w", (C, 3 * C)), (p + "qkv.b", (3 * C,)),
                 (p + "proj.w", (C, C)), (p + "proj.b", (C,)), (p + "ln2.w", (C,)), (p + "ln2.b", (C,)),
                 (p + "fc.w", (C, 4 * C)), (p + "fc.b", (4 * C,)), (p + "out.w", (4 * C, C)), (p + "out.b", (C,))]
    return spec + [("ln.w", (C,)), ("ln.b", (C,)), ("head.w", (C, V))]


def synthetic_weights(c, seed):
    """Matrices N(0, 0.02) (float64 draw in parameter order, cast), biases 0, LayerNorm w 1, b 0."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in param_spec(c):
        if len(shape) == 2:
            out[name] = (rng.standard_normal(shape) * 0.02).astype(c["dtype"])
        elif ".ln" in "." + name and name.endswith(".w"):
            out[name] = np.ones(shape, c["dtype"])
        else:
            out[name] = np.zeros(shape, c["dtype"])
    return out


def synthetic_tokens(c, batch, seed, replicas):
    rng = np.random.default_rng(seed)
    xs, ys = [], []
    for _ in range(replicas):
        xs.append(rng.integers(0, c["vocab"], (batch, c["ctx"])))
        ys.append(rng.integers(0, c["vocab"], (batch, c["ctx"])))
    return xs, ys


def gemm_flops_per_step(c, batch, world):
    """Algorithmic FLOP of every GEMM launch of one step (forward Y = XW, dX, dW)."""
    M = batch * c["ctx"]
    C, V, L = c["dim"], c["vocab"], c["layers"]
    per_layer = 2 * M * (C * 3 * C + C * C + C * 4 * C + 4 * C * C)
    fwd = L * per_layer + 2 * M * C * V
    return world * 3 * fwd


def cpu_baseline(weights, xs, ys, seq: int):
    """The oracle (NumPy restatement of dtrain) on a bounded sample of the same
    step: one replica's forward+backward on `seq` sequences, plus the 4-replica
    bucket average, global norm, clip and AdamW over all parameters once.
    Returns tokens/s extrapolated to the full step (32 x the sampled tokens of
    forward+backward, 1 x the optimizer part)."""
    from oracle import model as OM, optim as OO
    from oracle.ddp import ddp_average

    c = OM.GPTConfig(**CFG)
    P = {k: v.copy() for k, v in weights.items()}
    t0 = time.perf_counter()
    loss, g = OM.loss_and_grads(P, c, xs[0][:seq], ys[0][:seq])
    t_fb = time.perf_counter() - t0
    names = list(P)
    glist = [g[k] for k in names]
    t1 = time.perf_counter()
    avg = ddp_average([glist] * WORLD, 4, 1.0)
    sq = OO.global_sq_norm(avg)
    s = OO.clip_scale(sq, CLIP)
    opt = OO.AdamW([P[k] for k in names], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    opt.step([x * s for x in avg])
    t_opt = time.perf_counter() - t1
    tokens_step = WORLD * BATCH * CFG["ctx"]
    full = (tokens_step / (seq * CFG["ctx"])) * t_fb + t_opt
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:  # noqa: BLE001
        threads = int(os.environ.get("OMP_NUM_THREADS", "1"))
    return {"value": round(tokens_step / full, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"oracle (NumPy) forward+backward of 1 replica x {seq} x {CFG['ctx']} tokens "
                       f"({t_fb:.1f} s) + 4-replica bucket average, clip and AdamW over 163,109,376 params "
                       f"({t_opt:.1f} s); extrapolated to the full 4 x 8 x 1024-token step")}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seq", type=int, default=2, help="sequences in the CPU baseline sample")
    ap.add_argument("--seed", type=int, default=5)
    a = ap.parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py measures one GPU: the data-parallel exchange is simulated on-device over {WORLD} replicas "
              f"and no multi-GPU path is built; --gpus {a.gpus} is not supported.", file=sys.stderr)
        return 2

    from dtmi import _lib
    from dtmi import ddp as P, nn as N, optim as O, replicas as R, train as S

    info = _lib.device_info()
    print(f"[bench] device {info['name']} ({info['num_cus']} CUs); building GPT-2-small weights", file=sys.stderr,
          flush=True)
    weights = synthetic_weights(CFG, a.seed)
    xs, ys = synthetic_tokens(CFG, BATCH, a.seed, WORLD)
    model = N.GPT(N.GPTConfig(**CFG), seed=a.seed)
    model.load_numpy(weights)
    pg = R.SimGroup(WORLD)
    ddp = P.DDP(model, pg, bucket_mb=1.0, overlap=True, algo="direct")
    opt = O.AdamW([p.data for p in model.parameters()], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    batches = [[(xs[r], ys[r])] for r in range(WORLD)]

    for i in range(a.warmup):
        res = S.step_ddp(model, ddp, opt, batches, clip=CLIP)
        print(f"[bench] warmup step {i + 1}/{a.warmup} loss {res.loss:.4f}", file=sys.stderr, flush=True)
    _lib.sync()
    _lib.timing_enable(True)
    t0 = time.perf_counter()
    for _ in range(a.steps):
        res = S.step_ddp(model, ddp, opt, batches, clip=CLIP)
    _lib.sync()
    dt = time.perf_counter() - t0
    fams = {f: _lib.timing_read(f) for f in _lib.FAM}
    _lib.timing_enable(False)
    loss = res.loss
    print(f"[bench] {a.steps} steps in {dt:.3f} s, loss {loss:.4f}", file=sys.stderr, flush=True)

    tokens = WORLD * BATCH * CFG["ctx"]
    ms_step = 1e3 * dt / a.steps
    n, ms, work = fams["gemm"]
    gemm_tflops = work / (ms * 1e-3) / 1e12 if ms else 0.0
    roofline = {"bound": "mfma", "kernel": "gemm_kernel (MFMA f32 32x32x2, Linear fwd/dX/dW)",
                "achieved": round(gemm_tflops, 2), "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                "frac": round(gemm_tflops * 1e12 / PEAK_FP32_MFMA, 4), "traffic": None,
                "launches": n, "avg_launch_ms": round(ms / max(n, 1), 4),
                "flop_per_step": gemm_flops_per_step(CFG, BATCH, WORLD)}
    kernels = {}
    for f, (cnt, fms, fwork) in fams.items():
        if not cnt:
            continue
        entry = {"launches": cnt, "ms_per_step": round(fms / a.steps, 3)}
        if f in ("gemm", "attn_fwd", "attn_bwd"):
            entry["TFLOP/s"] = round(fwork / (fms * 1e-3) / 1e12, 2)
        else:
            gbs = fwork / (fms * 1e-3) / 1e9
            entry["GB/s"] = round(gbs, 1)
            entry["hbm_frac"] = round(gbs * 1e9 / PEAK_HBM, 3)
        kernels[f] = entry

    out = {"metric": METRIC, "value": round(tokens / (ms_step * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
           "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_step, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": ("GPT-2-small-shape float32 train step: 12 layers, d_model 768, 12 heads, "
                                   "T 1024, vocab 50304, batch 8 per replica x 4 simulated replicas, 1 MiB "
                                   "buckets, fixed-order average, clip 1.0, AdamW"),
                      "global_batch": WORLD * BATCH, "seq_len": CFG["ctx"], "parallelism": "dp4-simulated",
                      "params": sum(int(np.prod(s)) for _, s in param_spec(CFG))},
           "roofline": roofline, "kernels": kernels, "loss": round(loss, 5)}
    if not a.no_cpu_baseline:
        print("[bench] CPU baseline (oracle) ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(weights, xs, ys, a.cpu_seq)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
