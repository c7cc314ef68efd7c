"""One training step of dtrain (dtrain/train.py:128-159) on one GPU.

`step_single`: `--mode single` with `--emulate-world W` (each virtual rank's
loss scaled by 1/(accum*W), leaf gradients accumulate; train.py:130-145),
then the global-norm clip and AdamW.

`step_ddp`: `--mode ddp` with W simulated replicas (each replica's loss scaled
by 1/accum; gradients through DDP buckets and the fixed-order average), then
clip and AdamW.

`step_zero`: `--mode zero` with W simulated replicas and ZeroAdamW.

The global norm, the clip factor and the optimizer all stay on the device (no
host round trip inside a step); the returned loss and gradient norm are device
scalars that `float()` reads back when they are needed. `lr_at` is dtrain's
warm-up + cosine schedule (train.py:63-69).

`main` is dtrain's training driver (train.py:31-183) with the same flags, batches
(dtmi.data.rank_batch), JSON log lines, checkpoints (dtmi.checkpoint, dtrain's
format) and resume. The ranks of `--mode ddp|zero` are `--world` simulated
replicas in this process (dtrain starts one process per rank with its
launcher); `--fail-at-step` fault injection and restarts belong to that
launcher and are not offered.

    python -m dtmi.train --mode ddp --world 4 --data input.txt --steps 100 --log run.jsonl
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import numpy as np

from .optim import clip_scale_device, grad_sq_norm


def lr_at(step: int, lr: float, warmup: int, steps: int) -> float:
    """dtrain/train.py:63-69."""
    if warmup and step < warmup:
        return lr * (step + 1) / warmup
    if not warmup:
        return lr
    t = (step - warmup) / max(1, steps - warmup)
    return lr * (0.1 + 0.9 * 0.5 * (1 + np.cos(np.pi * min(1.0, t))))


class StepResult:
    def __init__(self, losses, n_micro, world, norm, scale=1.0):
        self._losses, self._n_micro, self._world, self._norm = losses, n_micro, world, norm
        self._scale = scale

    @property
    def loss(self) -> float:
        """Mean loss as dtrain logs it (train.py:145, 160-163)."""
        per_rank = {}
        for r, l in self._losses:
            per_rank[r] = per_rank.get(r, 0.0) + float(l.numpy()) / self._n_micro
        total = 0.0
        for r in sorted(per_rank):
            total += per_rank[r]
        return total / self._world if self._world > 1 else total

    @property
    def grad_norm(self) -> float:
        return float(self._norm.numpy()[0])

    @property
    def clip_scale(self) -> float:
        """The factor the gradients were multiplied by inside AdamW."""
        s = self._scale
        return float(s.numpy()[0]) if hasattr(s, "numpy") else float(s)


def _clip(sq, clip):
    if clip:
        return clip_scale_device(sq, clip)
    s, n = clip_scale_device(sq, float("inf"))
    return 1.0, n


def step_single(model, opt, batches, clip=1.0, accum=1):
    """batches[vr][micro] = (x, y) host token arrays, one list per virtual rank."""
    params = model.parameters()
    model.zero_grad()
    vworlds = len(batches)
    n_micro = accum * vworlds
    losses = []
    for micro in range(accum):
        for vr in range(vworlds):
            x, y = batches[vr][micro]
            _, loss = model(x, y)
            (loss * (1.0 / n_micro)).backward()
            losses.append((0, loss.data))
    sq = grad_sq_norm([p.grad for p in params])
    s, norm = _clip(sq, clip)
    opt.step([p.grad for p in params], grad_scale=s)
    return StepResult(losses, n_micro, 1, norm, s)


def step_ddp(model, ddp, opt, batches, clip=1.0, accum=1):
    """batches[r][micro] = (x, y) for simulated rank r."""
    pg = ddp.pg
    params = model.parameters()
    losses = []
    for r in range(pg.world):
        with pg.replica(r):
            model.zero_grad()
            for micro in range(accum):
                x, y = batches[r][micro]
                _, loss = model(x, y)
                scaled = loss * (1.0 / accum)
                if micro < accum - 1:
                    with ddp.no_sync():
                        scaled.backward()
                else:
                    scaled.backward()
                losses.append((r, loss.data))
    ddp.finish()
    s, norm = _clip(ddp.grad_sq, clip)
    opt.step([p.grad for p in params], grad_scale=s)
    return StepResult(losses, accum, pg.world, norm, s)


def step_zero(model, zero, batches, accum=1):
    pg = zero.pg
    losses = []
    for r in range(pg.world):
        with pg.replica(r):
            model.zero_grad()
            for micro in range(accum):
                x, y = batches[r][micro]
                _, loss = model(x, y)
                (loss * (1.0 / accum)).backward()
                losses.append((r, loss.data))
    zero.step()
    return StepResult(losses, accum, pg.world, zero.last_grad_norm_device)


# ------------------------------------------------------------------ driver
def parse(argv=None):
    """dtrain/train.py:31-60, plus --world (simulated ranks for ddp / zero)."""
    ap = argparse.ArgumentParser(prog="python -m dtmi.train")
    ap.add_argument("--mode", choices=["single", "ddp", "zero"], default="single")
    ap.add_argument("--world", type=int, default=2, help="simulated ranks for --mode ddp / zero")
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--batch", type=int, default=8, help="sequences per rank per micro-step")
    ap.add_argument("--accum", type=int, default=1, help="gradient-accumulation micro-steps")
    ap.add_argument("--ctx", type=int, default=64)
    ap.add_argument("--dim", type=int, default=128)
    ap.add_argument("--heads", type=int, default=4)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--dtype", default="float32")
    ap.add_argument("--lr", type=float, default=1e-3)
    ap.add_argument("--warmup", type=int, default=0, help="linear warm-up steps, then cosine decay to lr/10")
    ap.add_argument("--wd", type=float, default=0.1)
    ap.add_argument("--clip", type=float, default=1.0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--data", default=None, help="text file")
    ap.add_argument("--emulate-world", type=int, default=1)
    ap.add_argument("--bucket-mb", type=float, default=1.0)
    ap.add_argument("--no-overlap", action="store_true")
    ap.add_argument("--algo", choices=["ring", "direct"], default="ring")
    ap.add_argument("--ckpt-dir", default=None)
    ap.add_argument("--ckpt-every", type=int, default=0)
    ap.add_argument("--resume", action="store_true", help="resume from the latest checkpoint if any")
    ap.add_argument("--stop-after", type=int, default=-1, help="stop cleanly after this many steps")
    ap.add_argument("--log", default=None)
    ap.add_argument("--save-params", default=None, help="write final parameters (.npz)")
    return ap.parse_args(argv)


def _state(model, opt=None, zero=None, rank=0):
    """One rank's checkpoint state in dtrain's layout (train.py:170-178)."""
    if zero is not None:
        sd = zero.opts[rank].state_dict()
        return {"params": zero.flat.numpy(), "t": sd["t"], "m": sd["m"][0], "v": sd["v"][0]}
    sd = opt.state_dict()
    st = {"params": np.concatenate([p.numpy().reshape(-1) for p in model.parameters()]), "t": sd["t"]}
    st.update({f"m{i}": m for i, m in enumerate(sd["m"])})
    st.update({f"v{i}": v for i, v in enumerate(sd["v"])})
    return st


def _restore(model, st, opt=None, zero=None, rank=0):
    """dtrain/train.py:100-111."""
    if zero is not None:
        zero.flat.assign(np.asarray(st["params"], dtype=zero.flat.dtype))
        zero.opts[rank].load_state_dict({"t": st["t"], "m": [st["m"]], "v": [st["v"]]})
        return
    params = model.parameters()
    off = 0
    for p in params:
        p.data.assign(st["params"][off:off + p.data.size].reshape(p.shape))
        off += p.data.size
    n = len(params)
    opt.load_state_dict({"t": st["t"], "m": [st[f"m{i}"] for i in range(n)], "v": [st[f"v{i}"] for i in range(n)]})


def main(argv=None) -> int:
    from . import checkpoint
    from .data import CharData, load_text, rank_batch
    from .ddp import DDP
    from .nn import GPT, GPTConfig
    from .optim import AdamW
    from .replicas import SimGroup
    from .zero import ZeroAdamW

    a = parse(argv)
    data = CharData(load_text(a.data))
    cfg = GPTConfig(vocab=data.vocab, ctx=a.ctx, dim=a.dim, heads=a.heads, layers=a.layers, dtype=a.dtype)
    model = GPT(cfg, seed=a.seed)
    params = model.parameters()
    world = a.world if a.mode != "single" else 1
    pg = SimGroup(world) if a.mode != "single" else None
    ddp = zero = opt = None
    if a.mode == "ddp":
        ddp = DDP(model, pg, bucket_mb=a.bucket_mb, overlap=not a.no_overlap, algo=a.algo)
        opt = AdamW([p.data for p in params], lr=a.lr, weight_decay=a.wd)
    elif a.mode == "zero":
        zero = ZeroAdamW(model, pg, max_grad_norm=a.clip, lr=a.lr, weight_decay=a.wd)
    else:
        opt = AdamW([p.data for p in params], lr=a.lr, weight_decay=a.wd)

    start = 0
    if a.resume and a.ckpt_dir and checkpoint.latest(a.ckpt_dir):
        d = checkpoint.latest(a.ckpt_dir)
        for r in range(world):
            step, st = checkpoint.load(d, r, world)
            if zero is not None or r == 0:  # DDP / single ranks hold identical state
                _restore(model, st, opt=opt, zero=zero, rank=r)
        start = step
        print(f"[dtmi] resumed from step {step}", file=sys.stderr, flush=True)

    log = open(a.log, "a") if a.log else None
    vworlds = a.emulate_world if a.mode == "single" else world
    tokens_per_step = a.batch * a.ctx * a.accum * vworlds
    try:
        for step in range(start, a.steps):
            t0 = time.perf_counter()
            lr = lr_at(step, a.lr, a.warmup, a.steps)
            if zero is not None:
                zero.opt.lr = lr
            else:
                opt.lr = lr
            batches = [[rank_batch(data.train, step, micro, a.batch, a.ctx, a.seed, r, vworlds)
                        for micro in range(a.accum)] for r in range(vworlds)]
            comm_wait = 0.0
            if ddp is not None:
                before = ddp.comm_wait_s
                res = step_ddp(model, ddp, opt, batches, clip=a.clip, accum=a.accum)
                comm_wait = ddp.comm_wait_s - before
            elif zero is not None:
                res = step_zero(model, zero, batches, accum=a.accum)
            else:
                res = step_single(model, opt, batches, clip=a.clip, accum=a.accum)
            loss, gnorm = res.loss, res.grad_norm
            dt = time.perf_counter() - t0
            if log:
                log.write(json.dumps({"step": step + 1, "lr": lr, "loss": loss, "grad_norm": gnorm, "step_s": dt,
                                      "tokens_per_s": tokens_per_step / dt, "comm_wait_s": comm_wait}) + "\n")
                log.flush()
            if a.ckpt_dir and a.ckpt_every and (step + 1) % a.ckpt_every == 0:
                checkpoint.save_group(a.ckpt_dir, step + 1,
                                      [_state(model, opt=opt, zero=zero, rank=r) for r in range(world)])
            if a.stop_after >= 0 and step + 1 >= a.stop_after:
                break
    finally:
        if log:
            log.close()
    if a.save_params:
        np.savez(a.save_params, **{n: p.numpy() for n, p in model.named_parameters()})
    if zero is not None and a.log:
        with open(a.log, "a") as f:
            f.write(json.dumps({"optimizer_state_bytes_per_rank": zero.state_bytes()}) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
