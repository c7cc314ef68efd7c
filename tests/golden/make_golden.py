"""Write golden vectors from dtrain itself (run in a container that has the dtrain
source tree; the fixtures are committed, so the GPU tests never need dtrain).

    python tests/golden/make_golden.py [/path/to/DISTRIBUTED-TRAINING]

Covers the parts of the oracle that closed forms and finite differences cannot
pin bit for bit:
  - GPT initialisation draw order and per-tensor std (dtrain/nn.py:121-129);
  - a full single-process training step (forward, backward, clip, AdamW) in
    float64 and float32, with gradient accumulation over two virtual ranks
    (dtrain/train.py:128-159) -- pins dtype promotion (NumPy 2 weak scalars,
    float64 attention for float32 inputs) and the engine's accumulation;
  - AdamW in float32 over gradients spanning 1e-12..1 (weak-scalar rounding,
    dtrain/optim.py:21-33);
  - causal attention forward/backward in float32 (dtrain/autograd.py:226-247);
  - DDP bucket layout (dtrain/ddp.py:46-56) for the char-GPT and GPT-2-small
    parameter shapes, and comm.partition (dtrain/comm.py:220-226);
  - the char-GPT step at the tiny-config workload sizes as per-tensor summaries.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
REF = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
sys.path.insert(0, str(REF))
sys.path.insert(0, str(REPO))

from dtrain.autograd import Tensor, causal_attention  # noqa: E402
from dtrain.comm import partition  # noqa: E402
from dtrain.ddp import DDP  # noqa: E402
from dtrain.nn import GPT, GPTConfig  # noqa: E402
from dtrain.optim import AdamW, clip_scale  # noqa: E402

from oracle.model import GPTConfig as OCfg, param_spec, synthetic_init, synthetic_tokens  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def train_step(model, opt, batches, clip):
    """dtrain/train.py:128-159 for --mode single with len(batches) virtual ranks."""
    params = model.parameters()
    model.zero_grad()
    n_micro = len(batches)
    loss_sum = 0.0
    for x, y in batches:
        _, loss = model(x, y)
        scaled = loss * (1.0 / n_micro)
        scaled.backward()
        loss_sum += float(loss.data) / n_micro
    sq = sum(float(np.dot(p.grad.reshape(-1).astype(np.float64), p.grad.reshape(-1).astype(np.float64)))
             for p in params if p.grad is not None)
    s = clip_scale(sq, clip) if clip else 1.0
    grads = [p.grad.copy() for p in params]
    opt.step([p.grad * s if p.grad is not None else None for p in params])
    return loss_sum, sq, s, grads


def init_golden():
    out = {}
    for dt in ("float64", "float32"):
        cfg = GPTConfig(vocab=11, ctx=8, dim=16, heads=2, layers=2, dtype=dt)
        m = GPT(cfg, seed=3)
        for name, p in m.named_parameters():
            out[f"{dt}/{name}"] = p.data
    np.savez(HERE / "dtrain_init_tiny.npz", **out)


def step_golden():
    for dt in ("float64", "float32"):
        cfg = GPTConfig(vocab=11, ctx=8, dim=16, heads=2, layers=2, dtype=dt)
        m = GPT(cfg, seed=5)
        rng = np.random.default_rng(7)
        batches = [(rng.integers(0, 11, (3, 8)), rng.integers(0, 11, (3, 8))) for _ in range(2)]
        params = m.parameters()
        p0 = {n: p.data.copy() for n, p in m.named_parameters()}
        opt = AdamW([p.data for p in params], lr=3e-3, weight_decay=0.1)
        # first step clipped (large lr, clip 0.05), second unclipped
        loss1, sq1, s1, g1 = train_step(m, opt, batches, clip=0.05)
        p1 = {n: p.data.copy() for n, p in m.named_parameters()}
        loss2, sq2, s2, g2 = train_step(m, opt, batches[::-1], clip=0.0)
        out = {"x0": batches[0][0], "y0": batches[0][1], "x1": batches[1][0], "y1": batches[1][1],
               "loss1": np.float64(loss1), "sq1": np.float64(sq1), "s1": np.float64(s1),
               "loss2": np.float64(loss2), "sq2": np.float64(sq2)}
        for i, (n, _) in enumerate(m.named_parameters()):
            out[f"p0/{n}"] = p0[n]
            out[f"g1/{n}"] = g1[i]
            out[f"p1/{n}"] = p1[n]
            out[f"g2/{n}"] = g2[i]
            out[f"p2/{n}"] = params[i].data.copy()
        np.savez(HERE / f"dtrain_step_tiny_{dt}.npz", **out)


def adamw_golden():
    rng = np.random.default_rng(11)
    n = 4096
    p = (rng.standard_normal(n) * 0.05).astype(np.float32)
    out = {"p0": p.copy()}
    opt = AdamW([p], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    for k in range(3):
        g = (rng.standard_normal(n) * 10.0 ** rng.uniform(-12, 0, n)).astype(np.float32)
        out[f"g{k}"] = g
        opt.step([g])
        out[f"p{k + 1}"] = p.copy()
        out[f"m{k + 1}"] = opt.m[0].copy()
        out[f"v{k + 1}"] = opt.v[0].copy()
    np.savez(HERE / "dtrain_adamw_float32.npz", **out)


def attention_golden():
    rng = np.random.default_rng(13)
    out = {}
    for dt in ("float32", "float64"):
        q, k, v = (Tensor(rng.standard_normal((1, 2, 8, 4)).astype(dt), requires_grad=True) for _ in range(3))
        o = causal_attention(q, k, v)
        g = rng.standard_normal(o.shape).astype(dt)
        (o * Tensor(g)).sum().backward()
        out.update({f"{dt}/q": q.data, f"{dt}/k": k.data, f"{dt}/v": v.data, f"{dt}/g": g, f"{dt}/o": o.data,
                    f"{dt}/gq": q.grad, f"{dt}/gk": k.grad, f"{dt}/gv": v.grad})
    np.savez(HERE / "dtrain_attention.npz", **out)


class _LayoutPG:
    """Just enough of dtrain's ProcessGroup for DDP.__init__ (broadcast is a no-op)."""
    rank, world = 0, 4

    def broadcast(self, arr, root=0):
        return arr


class _ShapeModel:
    def __init__(self, shapes, dtype):
        self.ps = [Tensor(np.zeros(s, dtype), requires_grad=True) for s in shapes]

    def parameters(self):
        return self.ps


def layout_golden():
    out = {}
    for tag, c in (("charGPT", OCfg(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64")),
                   ("gpt2small", OCfg(vocab=50304, ctx=1024, dim=768, heads=12, layers=12, dtype="float32"))):
        shapes = [s for _, s in param_spec(c)]
        model = _ShapeModel(shapes, c.dtype)
        ddp = DDP(model, _LayoutPG(), bucket_mb=1.0, overlap=True, algo="direct")
        index = {id(p): i for i, p in enumerate(model.ps)}
        rows = []
        for bi, b in enumerate(ddp.buckets):
            for pi, p in enumerate(b.params):
                rows.append((bi, index[id(p)], b.offsets[pi], p.data.size))
        out[f"{tag}/layout"] = np.array(rows, dtype=np.int64)
        del ddp, model
    parts = []
    for n, w in ((0, 4), (1, 4), (7, 3), (110464, 4), (163109376, 4), (124439808, 4), (12345, 7)):
        parts.append([n, w] + partition(n, w) + [-1] * (8 - w))
    out["partition"] = np.array(parts, dtype=np.int64)
    np.savez(HERE / "dtrain_layout.npz", **out)


def charGPT_summary_golden():
    """The char-GPT float64 workload (vocab 65, ctx 32, dim 64, 4 heads, 2 layers,
    batch 8): N(0, 0.02) weights from oracle.synthetic_init(seed 0), tokens from
    oracle.synthetic_tokens(seed 0); one step: forward, CE backward, clip 1.0,
    AdamW(3e-4, 0.9/0.95, 1e-8, wd 0.1). Stores per-tensor summaries."""
    oc = OCfg(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64")
    P = synthetic_init(oc, seed=0)
    xs, ys = synthetic_tokens(oc, batch=8, seed=0)
    m = GPT(GPTConfig(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64"), seed=0)
    for n, p in m.named_parameters():
        p.data[...] = P[n]
    params = m.parameters()
    opt = AdamW([p.data for p in params], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    loss, sq, s, grads = train_step(m, opt, [(xs[0], ys[0])], clip=1.0)
    out = {"loss": np.float64(loss), "sq": np.float64(sq), "s": np.float64(s)}
    for i, (n, p) in enumerate(m.named_parameters()):
        g = grads[i]
        out[f"g/{n}/head"] = g.reshape(-1)[:16].copy()
        out[f"g/{n}/sum"] = np.float64(g.sum())
        out[f"g/{n}/sumsq"] = np.float64(np.dot(g.reshape(-1), g.reshape(-1)))
        out[f"g/{n}/sha256"] = np.array(sha(g))
        out[f"p/{n}/head"] = p.data.reshape(-1)[:16].copy()
        out[f"p/{n}/sha256"] = np.array(sha(p.data))
    np.savez(HERE / "dtrain_chargpt_step_summary.npz", **out)


if __name__ == "__main__":
    init_golden()
    step_golden()
    adamw_golden()
    attention_golden()
    layout_golden()
    charGPT_summary_golden()
    print("golden vectors written to", HERE)
