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
import re
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
PEAK_BF16_MFMA = 2.5e15  # dense bf16 MFMA (no sparsity)
PEAK_HBM = 8.0e12
CFG = dict(vocab=50304, ctx=1024, dim=768, heads=12, layers=12, dtype="float32")
BATCH, WORLD = 8, 4
LR, BETAS, EPS, WD, CLIP = 3e-4, (0.9, 0.95), 1e-8, 0.1, 1.0


def gemm_flops_per_step(c, batch, world):
    """Algorithmic FLOP of every GEMM launch of one step (forward Y = XW, dX, dW)."""
    M = batch * c["ctx"]
    C, V, L = c["dim"], c["vocab"], c["layers"]
    per_layer = 2 * M * (C * 3 * C + C * C + C * 4 * C + 4 * C * C)
    fwd = L * per_layer + 2 * M * C * V
    return world * 3 * fwd


def _cpu_info():
    """Host CPU model (from /proc/cpuinfo, what lscpu reports as 'Model name'),
    the cores this process may run on, and the BLAS thread count in use."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "affinity_cores": len(os.sched_getaffinity(0)), "blas_threads": _threads()}


def _median(xs):
    return sorted(xs)[len(xs) // 2]


def cpu_baseline(weights, xs, ys, seq: int):
    """The oracle (NumPy restatement of dtrain) on the host cores, on a bounded
    sample of the same step:
      - forward+backward of one replica's first `seq` sequences (default: the
        replica's whole batch, 8 x 1024 tokens): 1 warm-up, then 1 timed run,
        with the BLAS thread count the machine is configured for; and one
        sequence with 1 thread (1 warm-up, 1 timed);
      - the 4-replica bucket average (ring order), global norm, clip and
        AdamW over all 163,109,376 parameters: median of 3;
      - tokens/s extrapolated to the full step over the 4 replicas (and over
        the 8 / seq sequence groups when seq < 8), plus one optimizer pass;
      - dtrain's own published benchmark configuration (float32, dim 128, 4
        layers, 4 heads, ctx 64, batch 8, vocabulary 65) with 1 thread: median
        of 3 full steps after 1 warm-up, beside dtrain's 2,577 tokens/s
        (docs/benchmarks.md:51 of the reference, a 4-vCPU Xeon, 1 BLAS thread)."""
    from threadpoolctl import threadpool_limits

    from oracle import model as OM, optim as OO, step as OS
    from oracle.ddp import ddp_average

    c = OM.GPTConfig(**CFG)
    P = {k: v.copy() for k, v in weights.items()}
    info = _cpu_info()

    def fb(nseq):
        t0 = time.perf_counter()
        _, g = OM.loss_and_grads(P, c, xs[0][:nseq], ys[0][:nseq])
        return time.perf_counter() - t0, g

    def note(msg):
        print(f"[cpu baseline] {msg}", file=sys.stderr, flush=True)

    t_warm, _ = fb(seq)
    note(f"warm-up forward+backward of {seq} x {CFG['ctx']} tokens: {t_warm:.1f} s")
    t_fb, g = fb(seq)
    note(f"timed forward+backward: {t_fb:.1f} s")
    with threadpool_limits(limits=1):
        fb(1)
        t_fb1, _ = fb(1)
    note(f"1 sequence on 1 thread: {t_fb1:.1f} s")
    names = list(P)
    glist = [g[k] for k in names]
    del g
    opt = OO.AdamW([P[k] for k in names], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    t_opts = []
    for _ in range(3):
        t1 = time.perf_counter()
        avg = ddp_average([glist] * WORLD, 4, 1.0, "ring")
        sq = OO.global_sq_norm(avg)
        s = OO.clip_scale(sq, CLIP)
        opt.step([v * s for v in avg])
        t_opts.append(time.perf_counter() - t1)
        del avg
    t_opt = _median(t_opts)
    note(f"average + clip + AdamW: {', '.join(f'{t:.2f}' for t in t_opts)} s")
    del glist
    tokens_step = WORLD * BATCH * CFG["ctx"]
    per_step = (WORLD * BATCH / seq) * t_fb + t_opt
    per_step1 = (WORLD * BATCH) * t_fb1 + t_opt
    extrap = "the 4 replicas" if seq == BATCH else f"4 replicas x {BATCH // seq if BATCH % seq == 0 else BATCH / seq} groups"

    # dtrain's published configuration, 1 thread
    rc = OM.GPTConfig(vocab=65, ctx=64, dim=128, heads=4, layers=4, dtype="float32")
    RP = OM.dtrain_init(rc, seed=0)
    rx, ry = OM.synthetic_tokens(rc, batch=8, seed=0)
    ropt = OO.AdamW(list(RP.values()), lr=1e-3)
    with threadpool_limits(limits=1):
        rt = []
        for i in range(4):
            t0 = time.perf_counter()
            OS.single_step(RP, rc, [(rx[0], ry[0])], ropt, clip=1.0)
            if i:
                rt.append(time.perf_counter() - t0)
    ref_tps = 8 * 64 / _median(rt)
    return {"value": round(tokens_step / per_step, 2), "unit": "tokens/s", "cores": info["blas_threads"],
            "kind": "port", **info,
            "value_1_thread": round(tokens_step / per_step1, 2),
            "sample": (f"oracle (NumPy) forward+backward of 1 replica's {seq} x {CFG['ctx']} tokens: 1 timed run "
                       f"after 1 warm-up, {t_fb:.2f} s (warm-up {t_warm:.2f} s); 4-replica bucket average (ring "
                       f"order), clip and AdamW over 163,109,376 params, median of 3, {t_opt:.2f} s; extrapolated "
                       f"over {extrap} to the 4 x 8 x 1024-token step: {per_step:.1f} s. 1 thread: 1 x "
                       f"{CFG['ctx']} tokens {t_fb1:.2f} s, extrapolated over 32 sequences: {per_step1:.1f} s"),
            "reference_config_1_thread": {
                "value": round(ref_tps, 1), "unit": "tokens/s",
                "config": "float32 GPT, dim 128, 4 layers, 4 heads, ctx 64, batch 8, vocab 65 (dtrain's benchmark)",
                "sample": f"oracle full step (fwd, bwd, clip, AdamW), median of 3 after 1 warm-up, "
                          f"{_median(rt) * 1e3:.1f} ms",
                "dtrain_published": {"value": 2577, "unit": "tokens/s",
                                     "where": "docs/benchmarks.md:51, 4-vCPU Xeon 2.80 GHz, 1 BLAS thread"}}}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--warm-s", type=float, default=0.5,
                    help="least warm-up time of a microbenchmark, seconds (the GPU clock leaves idle over ~50 ms)")
    ap.add_argument("--cpu-seq", type=int, default=8,
                    help="sequences of one replica in the CPU baseline sample (8: the whole replica batch)")
    ap.add_argument("--seed", type=int, default=5)
    ap.add_argument("--workload", default="gpt2",
                    choices=["gpt2", "ln_linear", "attention", "bucket_adamw", "chargpt", "copy"],
                    help="gpt2: the headline training step; the others are the per-path microbenchmarks")
    ap.add_argument("--dtype", default="float32", choices=["float32", "float64"],
                    help="compute dtype of the microbenchmarks (the gpt2 step is float32)")
    ap.add_argument("--gemm-math", default="f32", choices=["f32", "bf16x6"],
                    help="arithmetic of the float32 GEMMs for the headline value: float32 MFMA, or operands split "
                         "exactly into three bf16 parts with the six largest partial products on the bf16 MFMA")
    ap.add_argument("--no-alt-gemm-math", action="store_true",
                    help="skip timing the same step with the other GEMM arithmetic")
    a = ap.parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py measures one GPU: the data-parallel exchange is simulated on-device over {WORLD} replicas "
              f"and no multi-GPU path is built; --gpus {a.gpus} is not supported.", file=sys.stderr)
        return 2
    if a.workload != "gpt2":
        out = MICRO[a.workload](a)
        print(json.dumps(out), flush=True)
        return 0

    from dtmi import _lib
    from dtmi import ddp as P, nn as N, optim as O, replicas as R, train as S
    from dtmi.autograd import Indices
    from dtmi.workload import synthetic_tokens, synthetic_weights

    _lib.set_gemm_math(a.gemm_math)

    info = _lib.device_info()
    print(f"[bench] device {info['name']} ({info['num_cus']} CUs); building GPT-2-small weights", file=sys.stderr,
          flush=True)
    weights = synthetic_weights(N.GPTConfig(**CFG), a.seed)
    xs, ys = synthetic_tokens(N.GPTConfig(**CFG), BATCH, a.seed, WORLD)
    model = N.GPT(N.GPTConfig(**CFG), seed=a.seed)
    model.load_numpy(weights)
    pg = R.SimGroup(WORLD)
    ddp = P.DDP(model, pg, bucket_mb=1.0, overlap=True, algo="ring")  # dtrain's default all-reduce order
    opt = O.AdamW([p.data for p in model.parameters()], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    # token ids and targets uploaded once: the timed steps copy nothing from the host
    batches = [[(Indices(xs[r]), Indices(ys[r]))] for r in range(WORLD)]

    for i in range(a.warmup):
        res = S.step_ddp(model, ddp, opt, batches, clip=CLIP)
        print(f"[bench] warmup step {i + 1}/{a.warmup} loss {res.loss:.4f}", file=sys.stderr, flush=True)

    def timed(events):
        """K steps between barriers; with events, the library also brackets
        every kernel launch with HIP events on its stream (per-family time)."""
        _lib.sync()
        _lib.timing_enable(events)
        t0 = time.perf_counter()
        for _ in range(a.steps):
            r = S.step_ddp(model, ddp, opt, batches, clip=CLIP)
        _lib.sync()
        el = time.perf_counter() - t0
        fm = {f: _lib.timing_read(f) for f in _lib.FAM} if events else None
        _lib.timing_enable(False)
        return el, fm, r

    # value / ms_per_step: K uninstrumented steps; roofline / kernels: the next
    # K steps with per-launch HIP events (which add ~10 us between launches)
    dt, _, res = timed(False)
    dt_ev, fams, res_ev = timed(True)
    loss = res.loss
    print(f"[bench] {a.steps} steps in {dt:.3f} s, loss {loss:.4f} (GEMM math {a.gemm_math}); {a.steps} more with "
          f"per-launch events in {dt_ev:.3f} s", file=sys.stderr, flush=True)
    alt = None
    if not a.no_alt_gemm_math:
        # the same step with the other GEMM arithmetic, continuing the same run;
        # a library error here is reported in the line instead of losing it
        other = "bf16x6" if a.gemm_math == "f32" else "f32"
        try:
            _lib.set_gemm_math(other)
            for _ in range(max(a.warmup, 1)):  # untimed steps in the new mode, as for the first
                S.step_ddp(model, ddp, opt, batches, clip=CLIP)
            adt, _, ares = timed(False)
            _, afams, _ = timed(True)
            an, ams, awork = afams["gemm"]
            ag = awork / (ams * 1e-3) / 1e12 if ams else 0.0
            print(f"[bench] {a.steps} steps in {adt:.3f} s, loss {ares.loss:.4f} (GEMM math {other})",
                  file=sys.stderr, flush=True)
            alt = {"gemm_math": other, "value": round(WORLD * BATCH * CFG["ctx"] / (adt / a.steps), 1),
                   "unit": "tokens/s", "ms_per_step": round(1e3 * adt / a.steps, 3), "loss": round(ares.loss, 5),
                   "gemm_ms_per_step": round(ams / a.steps, 3), "gemm_fp32_equivalent_TFLOP/s": round(ag, 2)}
            if other == "bf16x6":
                alt["gemm_mfma_frac_of_bf16_peak"] = round(6 * ag * 1e12 / PEAK_BF16_MFMA, 4)
        except RuntimeError as e:
            alt = {"gemm_math": other, "error": str(e)}
        finally:
            _lib.set_gemm_math(a.gemm_math)

    tokens = WORLD * BATCH * CFG["ctx"]
    ms_step = 1e3 * dt / a.steps
    n, ms, work = fams["gemm"]
    gemm_tflops = work / (ms * 1e-3) / 1e12 if ms else 0.0
    if a.gemm_math == "f32":
        roofline = {"bound": "mfma", "kernel": "gemm_dma_kernel (MFMA f32 32x32x2, Linear fwd/dX/dW)",
                    "achieved": round(gemm_tflops, 2), "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                    "frac": round(gemm_tflops * 1e12 / PEAK_FP32_MFMA, 4), "traffic": _profiled_traffic(),
                    "launches": n, "avg_launch_ms": round(ms / max(n, 1), 4),
                    "flop_per_step": gemm_flops_per_step(CFG, BATCH, WORLD)}
    else:
        # six bf16 MFMA products per float32 product: the matrix cores run 6x
        # the float32-equivalent FLOP, against the dense bf16 peak
        roofline = {"bound": "mfma", "kernel": ("gemm_x6_kernel (MFMA bf16 32x32x16, float32 operands split "
                                                "exactly into 3 bf16 parts, 6 partial products, Linear fwd/dX/dW)"),
                    "achieved": round(6 * gemm_tflops, 2), "peak": PEAK_BF16_MFMA / 1e12, "unit": "TFLOP/s",
                    "frac": round(6 * gemm_tflops * 1e12 / PEAK_BF16_MFMA, 4), "traffic": None,
                    "fp32_equivalent_TFLOP/s": round(gemm_tflops, 2),
                    "launches": n, "avg_launch_ms": round(ms / max(n, 1), 4),
                    "flop_per_step": gemm_flops_per_step(CFG, BATCH, WORLD)}
    kernels = {}
    for f, (cnt, fms, fwork) in fams.items():
        if not cnt:
            continue
        entry = {"launches": cnt, "ms_per_step": round(fms / a.steps, 3)}  # from the evented steps
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
                                   "buckets, ring-order average, clip 1.0, AdamW"),
                      "global_batch": WORLD * BATCH, "seq_len": CFG["ctx"], "parallelism": "dp4-simulated",
                      "params": sum(int(v.size) for v in weights.values())},
           "roofline": roofline, "kernels": kernels, "loss": round(loss, 5), "gemm_math": a.gemm_math,
           "timing_note": (f"value and ms_per_step: {a.steps} steps with no instrumentation; roofline and kernels: "
                           f"the next {a.steps} steps with HIP events around every launch "
                           f"({1e3 * dt_ev / a.steps:.1f} ms per step with the events)"),
           "gemm_math_note": ("f32: float32 MFMA (v_mfma_f32_32x32x2_f32). bf16x6: each float32 operand split "
                              "exactly into three bf16 parts, the six partial products a_i*b_j with i+j<=2 on the "
                              "bf16 MFMA (exact products, float32 accumulation; dropped terms < 2^-23 |ab|); both "
                              "pass the same float32 parity bar (rel err <= 1e-5 vs the float64 oracle)"),
           "alt_gemm_math": alt}
    if not a.no_cpu_baseline:
        print("[bench] CPU baseline (oracle) ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(weights, xs, ys, a.cpu_seq)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0



# --------------------------------------------------------------- microbenchmarks
# Per-path workloads with their own roofline line; the headline line above is
# the gpt2 step. Each times `--steps` launches after `--warmup` with the
# library's per-family HIP-event timing, so `achieved` is algorithmic work per
# launch over the average launch time of the dominant family.

def _threads():
    try:
        from threadpoolctl import threadpool_info
        return max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:  # noqa: BLE001
        return int(os.environ.get("OMP_NUM_THREADS", "1"))


def _timed(a, fn, families):
    """Wall time of `steps` uninstrumented calls, then per-family kernel time
    from `steps` more calls with HIP events around every launch. The warm-up
    is `warmup` calls and at least `--warm-s` seconds: a GPU that comes out of
    idle raises its clock over the first ~50 ms of work (the float32 attention
    backward at B 8, H 12, T 1024 takes 288 us per call over its first 20
    calls and 238 us from the second tenth of a second on), so a few short
    calls would time the ramp instead of the kernel."""
    from dtmi import _lib
    t0 = time.perf_counter()
    n = 0
    while n < a.warmup or time.perf_counter() - t0 < a.warm_s:
        fn()
        n += 1
        if n % 16 == 0:
            _lib.sync()
    _lib.sync()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        fn()
    _lib.sync()
    dt = time.perf_counter() - t0
    _lib.timing_enable(True)
    for _ in range(a.steps):
        fn()
    _lib.sync()
    fams = {f: _lib.timing_read(f) for f in families}
    _lib.timing_enable(False)
    return dt, fams


def _line(metric, value, unit, a, ms, config, roofline, cpu, extra=None):
    out = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": {"float32": "f32", "float64": "f64"}[a.dtype], "data": "synthetic", "config": config,
           "roofline": roofline, "cpu_baseline": cpu}
    if extra:
        out.update(extra)
    return out


TRAFFIC_PROFILE = ROOT / "profiles" / "gpt2_small_step_traffic.md"


def _profiled_traffic():
    """HBM-side bytes per GEMM launch of this workload, as measured with
    rocprofv3 FETCH_SIZE / WRITE_SIZE (copy-calibrated) and recorded in
    profiles/gpt2_small_step_traffic.md; None when that file is absent."""
    try:
        m = re.search(r"traffic_bytes_per_launch = (\d+)", TRAFFIC_PROFILE.read_text())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def _mfma_peak(dtype):
    return 157.3e12 if dtype == "float32" else 78.6e12


def micro_ln_linear(a):
    """LayerNorm + Linear backward, x [16384, 768], W [768, 3072]: dX, dW, db, dgamma, dbeta."""
    from dtmi import device as D, kernels as K
    M, Cin, N = 16384, 768, 3072
    dt = np.dtype(a.dtype)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((M, Cin)).astype(dt)
    W = (rng.standard_normal((Cin, N)) * 0.02).astype(dt)
    gamma = (1 + rng.standard_normal(Cin) * 0.01).astype(dt)
    beta = (rng.standard_normal(Cin) * 0.01).astype(dt)
    dY = rng.standard_normal((M, N)).astype(dt)
    dx_, dW_, dg_, db_, dY_ = D.from_numpy(x), D.from_numpy(W), D.from_numpy(gamma), D.from_numpy(beta), \
        D.from_numpy(dY)
    h, mean, rstd = K.layernorm_fwd(dx_, dg_, db_)

    def step():
        dh, dw, db = K.linear_bwd(h, dW_, dY_)
        K.layernorm_bwd(dh, dx_, dg_, mean, rstd)
    dtm, fams = _timed(a, step, ["gemm", "ln_bwd", "other"])
    n, ms, work = fams["gemm"]
    flop = 2 * 2 * M * Cin * N
    ach = work / (ms * 1e-3)
    ln_n, ln_ms, ln_work = fams["ln_bwd"]
    cpu = None
    if not a.no_cpu_baseline:
        from oracle import ops as OP
        reps, t0 = 0, time.perf_counter()
        while reps == 0 or (time.perf_counter() - t0 < 3.0 and reps < 20):
            hh, cache = OP.layer_norm_fwd(x, gamma, beta)
            gh, gW = OP.matmul_bwd(dY, hh, W)
            OP.unbroadcast(dY, (N,))
            OP.layer_norm_bwd(gh, cache, gamma)
            reps += 1
        t = (time.perf_counter() - t0) / reps
        cpu = {"value": round(flop / t / 1e9, 2), "unit": "GFLOP/s", "cores": _threads(),
               "kind": "port", **_cpu_info(), "sample": f"oracle LN forward + Linear and LN backward on all {M} "
                                                        f"rows, mean of {reps} repetitions, {t:.2f} s each"}
    return _line("LN + Linear backward GEMM throughput (dX, dW) at x[16384,768] W[768,3072]",
                 round(flop / (1e-3 * ms / a.steps) / 1e12, 2), "TFLOP/s", a, 1e3 * dtm / a.steps,
                 {"workload": f"LayerNorm + Linear backward, x [16384,768], W [768,3072], dY [16384,3072], {a.dtype}"},
                 {"bound": "mfma", "kernel": "gemm_dma_kernel", "achieved": round(ach / 1e12, 2),
                  "peak": _mfma_peak(a.dtype) / 1e12, "unit": "TFLOP/s",
                  "frac": round(ach / _mfma_peak(a.dtype), 4), "traffic": None},
                 cpu, {"ln_bwd": {"GB/s": round(ln_work / (ln_ms * 1e-3) / 1e9, 1),
                                  "ms": round(ln_ms / max(ln_n, 1), 4)}})


def micro_attention(a):
    """Causal attention backward, B 16, H 12, T 256, D 64 (forward untimed)."""
    from dtmi import device as D, kernels as K
    B, H, T, Dh = 16, 12, 256, 64
    dt = np.dtype(a.dtype)
    rng = np.random.default_rng(3)
    q, k, v, g = (rng.standard_normal((B, H, T, Dh)).astype(dt) for _ in range(4))
    dq_, dk_, dv_, dg_ = (D.from_numpy(t) for t in (q, k, v, g))
    o, rmax, rsum = K.attn_fwd(dq_, dk_, dv_)
    outs = [D.empty(q.shape, dt) for _ in range(3)]

    def step():
        K.attn_bwd(dq_, dk_, dv_, o, dg_, rmax, rsum, dq=outs[0], dk=outs[1], dv=outs[2])
    dtm, fams = _timed(a, step, ["attn_bwd"])
    n, ms, work = fams["attn_bwd"]
    ach = work / (ms * 1e-3)
    cpu = None
    if not a.no_cpu_baseline:
        from oracle import ops as OP
        bs = 4
        _, p, sc = OP.attention_fwd(q[:bs], k[:bs], v[:bs])
        runs = []
        for _ in range(4):
            t1 = time.perf_counter()
            OP.attention_bwd(g[:bs], q[:bs], k[:bs], v[:bs], p, sc)
            runs.append(time.perf_counter() - t1)
        t = _median(runs[1:])
        fl = 5 * 2 * bs * H * Dh * T * (T + 1) / 2
        cpu = {"value": round(fl / t / 1e9, 2), "unit": "GFLOP/s", "cores": _threads(), "kind": "port",
               **_cpu_info(), "sample": f"oracle causal_attention backward on {bs} of {B} batches, median of 3 "
                                        f"after 1 warm-up ({t:.3f} s), causal-exact FLOP"}
    return _line("causal attention backward throughput (5 GEMMs, causal-exact FLOP) at B16 H12 T256 D64",
                 round(ach / 1e12, 2), "TFLOP/s", a, 1e3 * dtm / a.steps,
                 {"workload": f"causal self-attention backward B=16 H=12 T=256 D=64 {a.dtype}"},
                 {"bound": "mfma", "kernel": ("attn_drow64 + attn_bwd_kvp + attn_bwd_qp (aligned float32), attn_drow64 + "
                             "attn_bwd_kv + attn_bwd_q_ds (float64)"), "achieved": round(ach / 1e12, 2),
                  "peak": _mfma_peak(a.dtype) / 1e12, "unit": "TFLOP/s",
                  "frac": round(ach / _mfma_peak(a.dtype), 4), "traffic": None}, cpu)


def micro_bucket_adamw(a):
    """124,439,808-element fixed-order 4-replica average (+ fused sum of squares),
    clip and AdamW over the full buffer, then AdamW on the 1/4 shard. Beside
    it, the same average through DDP's 1 MiB buckets: the merged launches
    DDP.finish issues, and its norm pass."""
    from dtmi import ddp as P, device as D, kernels as K, replicas as R
    from dtmi.workload import N_BUCKET_WORKLOAD, BucketParams
    n, W = N_BUCKET_WORKLOAD, 4
    dt = np.dtype(a.dtype)
    rng = np.random.default_rng(4)
    p = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)).astype(dt)
    reps = (rng.standard_normal((W, n), dtype=np.float32) * np.float32(1e-3)).astype(dt)
    m = np.abs(rng.standard_normal(n, dtype=np.float32) * np.float32(1e-4)).astype(dt)
    v = np.abs(rng.standard_normal(n, dtype=np.float32) * np.float32(1e-4)).astype(dt)
    bmodel = BucketParams(D.zeros((n,), dt))
    ddp = P.DDP(bmodel, R.SimGroup(W), bucket_mb=1.0, algo="direct")
    ddp.grads.rows.assign(reps)
    dp_, dm_, dv_, dr_ = D.from_numpy(p), D.from_numpy(m), D.from_numpy(v), ddp.grads.rows
    del reps
    g_ = D.empty((n,), dt)
    nb = K.average_blocks(n, dt)
    parts = D.empty((nb,), np.float64)
    sq, s_dev = D.empty((1,), np.float64), D.empty((1,), np.float64)
    b1t, b2t = 1 - 0.9 ** 101, 1 - 0.95 ** 101
    sh = n // 4

    def step():
        K.bucket_average(g_, dr_, W, 1.0 / W, partials=parts)
        K.sumsq_finish(parts, nb, sq)
        K.clip_scale(sq, 1.0, s_dev)
        K.adamw(dp_, g_, dm_, dv_, 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t, gscale_dev=s_dev)
        K.adamw(dp_[:sh], g_[:sh], dm_[:sh], dv_[:sh], 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t, gscale_dev=s_dev)
    dtm, fams = _timed(a, step, ["bucket_avg", "adamw", "sumsq"])
    an, ams, awork = fams["adamw"]
    bn, bms, bwork = fams["bucket_avg"]
    _, dfams = _timed(a, lambda: bmodel.hand_over(ddp), ["bucket_avg", "sumsq"])
    dn, dms, dwork = dfams["bucket_avg"]
    sn, sms, swork = dfams["sumsq"]
    total_bytes = awork + bwork
    total_ms = ams + bms
    ach = awork / (ams * 1e-3)
    cpu = None
    if not a.no_cpu_baseline:
        from oracle import optim as OO
        from oracle.ddp import fixed_order_sum
        k = n
        rr = rng.standard_normal((W, k)).astype(dt)
        runs = []
        for _ in range(3):
            pp, mm, vv = p[:k].copy(), m[:k].copy(), v[:k].copy()
            t0 = time.perf_counter()
            gg = fixed_order_sum(list(rr))
            gg *= 1.0 / W
            s = OO.clip_scale(float(np.dot(gg.astype(np.float64), gg.astype(np.float64))), 1.0)
            OO.adamw_update(pp, gg * s, mm, vv, 3e-4, 0.9, 0.95, 1e-8, 0.1, b1t, b2t)
            runs.append(time.perf_counter() - t0)
        t = _median(runs)
        cpu = {"value": round((5 + 7) * k * dt.itemsize / t / 1e9, 2), "unit": "GB/s", "cores": _threads(),
               "kind": "port", **_cpu_info(),
               "sample": f"oracle average + clip + AdamW over all {k} elements, median of 3 ({t:.2f} s)"}
    return _line("gradient bucket average + AdamW bandwidth over 124,439,808 params (4 replicas)",
                 round(total_bytes / (total_ms * 1e-3) / 1e9, 1), "GB/s", a, 1e3 * dtm / a.steps,
                 {"workload": f"124,439,808-element 4-replica fixed-order average + clip + AdamW (full + 1/4 shard) "
                              f"{a.dtype}"},
                 {"bound": "hbm", "kernel": "adamw_flat_kernel", "achieved": round(ach / 1e9, 1), "peak": 8000.0,
                  "unit": "GB/s", "frac": round(ach / 8e12, 4), "traffic": None}, cpu,
                 {"bucket_average": {"GB/s": round(bwork / (bms * 1e-3) / 1e9, 1), "ms": round(bms / max(bn, 1), 4)},
                  "bucket_average_ddp_1mib": {
                      "GB/s": round(dwork / (dms * 1e-3) / 1e9, 1), "ms": round(dms / a.steps, 4),
                      "launches": dn // a.steps, "buckets": len(ddp.buckets),
                      "norm_pass": {"GB/s": round(swork / (sms * 1e-3) / 1e9, 1), "ms": round(sms / a.steps, 4)}},
                  "adamw": {"GB/s": round(ach / 1e9, 1), "ms": round(ams / max(an, 1), 4)}})


def micro_chargpt(a):
    """The float64 char-GPT step (vocab 65, ctx 32, dim 64, 4 heads, 2 layers, batch 8)."""
    from dtmi import nn as N, optim as O, train as S
    from dtmi.workload import synthetic_weights
    a.dtype = "float64"
    c = dict(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64")
    w = synthetic_weights(N.GPTConfig(**c), 0)
    rng = np.random.default_rng(0)
    x, y = rng.integers(0, 65, (8, 32)), rng.integers(0, 65, (8, 32))
    m = N.GPT(N.GPTConfig(**c))
    m.load_numpy(w)
    opt = O.AdamW([p.data for p in m.parameters()], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)

    def step():
        S.step_single(m, opt, [[(x, y)]], clip=1.0)
    dtm, fams = _timed(a, step, ["gemm", "attn_fwd", "attn_bwd", "other"])
    ms = 1e3 * dtm / a.steps
    cpu = None
    if not a.no_cpu_baseline:
        from oracle import model as OM, optim as OO, step as OS
        oc = OM.GPTConfig(**c)
        P = {k: v.copy() for k, v in w.items()}
        oo = OO.AdamW(list(P.values()), lr=3e-4)
        t0 = time.perf_counter()
        for _ in range(5):
            OS.single_step(P, oc, [(x, y)], oo, clip=1.0)
        t = (time.perf_counter() - t0) / 5
        cpu = {"value": round(256 / t, 1), "unit": "tokens/s", "cores": _threads(), "kind": "port",
               "sample": f"oracle full step x5 ({t * 1e3:.1f} ms per step)"}
    n, gms, work = fams["gemm"]
    return _line("char-GPT float64 fwd+bwd+clip+AdamW tokens/s (launch-bound parity config)", round(256 / (ms * 1e-3), 1),
                 "tokens/s", a, ms, {"workload": "char-GPT float64 step: vocab 65, ctx 32, dim 64, 4 heads, 2 layers, "
                                                 "batch 8"},
                 {"bound": "mfma", "kernel": "gemm_dma_kernel / gemm_kernel (rows of 65 logits are not 16-byte aligned)",
                  "achieved": round(work / max(gms, 1e-9) / 1e9, 4),
                  "peak": 78.6, "unit": "TFLOP/s", "frac": round(work / max(gms, 1e-9) / 1e9 / 78.6, 6),
                  "traffic": None}, cpu)


def micro_copy(a):
    """A plain 256 MiB device-to-device copy through the flatten kernel (reads
    256 MiB, writes 256 MiB): the calibration point for HBM byte counters.
    Beside it, what other streams of the same size sustain (wall clock over
    `steps` calls, GB/s of algorithmic bytes): the elementwise scale (one read,
    one write), the runtime's own device-to-device copy, and AdamW (four reads,
    three writes) -- the measured ceilings the bandwidth kernels are held to."""
    from dtmi import _lib, device as D, kernels as K
    n = (256 << 20) // 4
    src = D.full((n,), 1.0, np.float32)
    dst = D.empty((n,), np.float32)
    dtm, fams = _timed(a, lambda: K.bucket_flatten(dst, [src], [n]), ["flatten"])
    cnt, ms, work = fams["flatten"]
    ach = work / (ms * 1e-3)

    def wall(fn, nbytes):
        for _ in range(max(a.warmup, 1)):
            fn()
        _lib.sync()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            fn()
        _lib.sync()
        return round(nbytes * a.steps / (time.perf_counter() - t0) / 1e9, 1)

    from dtmi import optim as O
    g = D.full((n,), 0.5, np.float32)
    opt = O.AdamW([dst], lr=1e-4)
    streams = {"flatten_kernel (1 read, 1 write)": wall(lambda: K.bucket_flatten(dst, [src], [n]), 8 * n),
               "scale_kernel (1 read, 1 write)": wall(lambda: K.scale(src, 1.0, out=dst), 8 * n),
               "hipMemcpyAsync device to device": wall(lambda: K.copy_into(dst, src), 8 * n),
               "adamw_flat_kernel (4 reads, 3 writes)": wall(lambda: opt.step([g]), 28 * n)}
    return _line("device copy bandwidth (256 MiB read + 256 MiB write)", round(ach / 1e9, 1), "GB/s", a,
                 1e3 * dtm / a.steps, {"workload": "flatten_kernel copy of 67,108,864 float32"},
                 {"bound": "hbm", "kernel": "flatten_kernel", "achieved": round(ach / 1e9, 1), "peak": 8000.0,
                  "unit": "GB/s", "frac": round(ach / 8e12, 4), "traffic": None}, None,
                 {"streams_GB/s": streams})


MICRO = {"ln_linear": micro_ln_linear, "attention": micro_attention, "bucket_adamw": micro_bucket_adamw,
         "chargpt": micro_chargpt, "copy": micro_copy}

if __name__ == "__main__":
    sys.exit(main())
