"""Write golden fixtures of dtrain's data-parallel reductions from dtrain itself:
its DDP and ZeroAdamW over its own TCP ProcessGroup, with W ranks run as
threads of this process on 127.0.0.1 (run where the dtrain source tree exists;
the fixtures are committed, so the GPU tests never need dtrain).

    python tests/golden/make_golden_ddp.py [/path/to/DISTRIBUTED-TRAINING]

dtrain_ddp_reduce.npz -- the summation order of the gradient exchange:
  - DDP (dtrain/ddp.py:73-110) with algo "ring" (comm.py:292-303, 342-372:
    chunk c of a bucket is summed starting at rank c) and "direct"
    (comm.py:374-391: rank 0 first), for W = 3 and 4, float64 and float32,
    256-byte buckets over parameters whose sizes put chunk edges inside
    parameters; every rank's gradients are drawn over 16 decades so that any
    other order changes bits. Stores the inputs and rank 0's averaged
    gradients (all ranks hold identical bits, checked here);
  - ZeroAdamW (dtrain/zero.py:46-62: ring reduce-scatter, shard r summed
    starting at rank r, *1/W, float64 norm, clip, AdamW on the shard,
    all-gather) for the same W and dtypes, with clip 1.0 and without clip
    (then AdamW sees the reduced gradients unscaled, so the parameters pin
    the reduction order bit for bit): the flat parameters after one step
    and the global norm.
dtrain_ddp_step_float64.npz -- two steps of dtrain's DDP training loop
  (train.py:128-163, --algo ring, W = 3, clip 0.5) on a tiny GPT: losses,
  norms, averaged gradients and parameters.
"""
from __future__ import annotations

import sys
import threading
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
sys.path.insert(0, str(REF))

from dtrain.autograd import Tensor  # noqa: E402
from dtrain.comm import ProcessGroup, StoreServer  # noqa: E402
from dtrain.ddp import DDP  # noqa: E402
from dtrain.nn import GPT, GPTConfig  # noqa: E402
from dtrain.optim import AdamW, clip_scale  # noqa: E402
from dtrain.zero import ZeroAdamW  # noqa: E402

SHAPES = [(7, 5), (3,), (13, 4), (1,), (33,), (6, 6), (2,), (41,)]
BUCKET_MB = 256 / (1 << 20)


def run_ranks(world, fn):
    """fn(pg) on `world` ranks (threads), each with its own ProcessGroup."""
    srv = StoreServer()
    out, errs = [None] * world, []

    def entry(r):
        try:
            pg = ProcessGroup(r, world, srv.address, timeout=60, prefix="g/")
            out[r] = fn(pg)
            pg.close()
        except BaseException as e:  # noqa: BLE001
            errs.append(e)
    ts = [threading.Thread(target=entry, args=(r,)) for r in range(world)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(120)
    srv.close()
    if errs:
        raise errs[0]
    return out


class ShapeModel:
    def __init__(self, arrays):
        self.ps = [Tensor(a.copy(), requires_grad=True) for a in arrays]

    def parameters(self):
        return self.ps


def rank_grads(world, dt, seed):
    rng = np.random.default_rng(seed)
    return [[(rng.standard_normal(s) * 10.0 ** rng.uniform(-8, 8, s)).astype(dt) for s in SHAPES]
            for _ in range(world)]


def params0(dt, seed):
    rng = np.random.default_rng(seed)
    return [(rng.standard_normal(s) * 0.5).astype(dt) for s in SHAPES]


def reduce_golden():
    out = {}
    for world in (3, 4):
        for dt in ("float64", "float32"):
            grads = rank_grads(world, dt, 100 * world + len(dt))
            p0 = params0(dt, world)
            for r in range(world):
                for i, g in enumerate(grads[r]):
                    out[f"w{world}/{dt}/g{r}/{i}"] = g
            for i, p in enumerate(p0):
                out[f"w{world}/{dt}/p0/{i}"] = p
            for algo in ("ring", "direct"):
                def ddp_fn(pg, algo=algo):
                    m = ShapeModel(p0)
                    ddp = DDP(m, pg, bucket_mb=BUCKET_MB, overlap=True, algo=algo)
                    for p, g in reversed(list(zip(m.ps, grads[pg.rank]))):
                        p.grad = g.copy()
                        ddp._on_grad(p)
                    ddp.finish()
                    return [p.grad.copy() for p in m.ps], len(ddp.buckets)
                res = run_ranks(world, ddp_fn)
                for r in range(1, world):
                    assert all(a.tobytes() == b.tobytes() for a, b in zip(res[r][0], res[0][0]))
                assert res[0][1] > 2
                for i, a in enumerate(res[0][0]):
                    out[f"w{world}/{dt}/ddp_{algo}/{i}"] = a

            for tag, clip in (("zero", 1.0), ("zero_noclip", None)):
                def zero_fn(pg, clip=clip):
                    m = ShapeModel(p0)
                    z = ZeroAdamW(m, pg, max_grad_norm=clip, lr=1e-2, weight_decay=0.1)
                    for p, g in zip(m.ps, grads[pg.rank]):
                        p.grad = g.copy()
                    z.step()
                    return z.flat.copy(), z.last_grad_norm
                res = run_ranks(world, zero_fn)
                for r in range(1, world):
                    assert res[r][0].tobytes() == res[0][0].tobytes()
                out[f"w{world}/{dt}/{tag}_flat"] = res[0][0]
                out[f"w{world}/{dt}/{tag}_norm"] = np.float64(res[0][1])
    np.savez(HERE / "dtrain_ddp_reduce.npz", **out)


def step_golden():
    world = 3
    cfg = GPTConfig(vocab=11, ctx=8, dim=16, heads=2, layers=2, dtype="float64")
    rng = np.random.default_rng(21)
    batches = [[(rng.integers(0, 11, (2, 8)), rng.integers(0, 11, (2, 8))) for _ in range(world)] for _ in range(2)]

    def fn(pg):
        model = GPT(cfg, seed=4)
        params = model.parameters()
        ddp = DDP(model, pg, bucket_mb=0.002, overlap=True, algo="ring")
        opt = AdamW([p.data for p in params], lr=3e-3, weight_decay=0.1)
        rec = {}
        for step in range(2):
            model.zero_grad()
            x, y = batches[step][pg.rank]
            _, loss = model(x, y)
            (loss * 1.0).backward()
            ddp.finish()
            sq = sum(float(np.dot(p.grad.reshape(-1).astype(np.float64), p.grad.reshape(-1).astype(np.float64)))
                     for p in params if p.grad is not None)
            s = clip_scale(sq, 0.5)
            rec[f"s{step}/grads"] = [p.grad.copy() for p in params]
            opt.step([p.grad * s for p in params])
            l = np.array([float(loss.data)])
            pg.allreduce(l)
            rec[f"s{step}/loss"] = float(l[0]) / pg.world
            rec[f"s{step}/sq"] = sq
            rec[f"s{step}/params"] = [p.data.copy() for p in params]
        return rec, [n for n, _ in model.named_parameters()]
    res = run_ranks(world, fn)
    rec, names = res[0]
    out = {}
    for step in range(2):
        for r in range(world):
            out[f"s{step}/x{r}"], out[f"s{step}/y{r}"] = batches[step][r]
        out[f"s{step}/loss"] = np.float64(rec[f"s{step}/loss"])
        out[f"s{step}/sq"] = np.float64(rec[f"s{step}/sq"])
        for n, g, p in zip(names, rec[f"s{step}/grads"], rec[f"s{step}/params"]):
            out[f"s{step}/g/{n}"] = g
            out[f"s{step}/p/{n}"] = p
    np.savez(HERE / "dtrain_ddp_step_float64.npz", **out)


if __name__ == "__main__":
    reduce_golden()
    step_golden()
    print("wrote", HERE / "dtrain_ddp_reduce.npz", HERE / "dtrain_ddp_step_float64.npz")
