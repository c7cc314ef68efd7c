"""The oracle against golden vectors written from dtrain itself (CPU).

These pin the parts of the restatement that no closed form fixes bit for bit:
initialisation draw order, dtype promotion, engine accumulation, weak-scalar
rounding in float32 AdamW, the DDP bucket rule and comm.partition.
"""
import hashlib

import numpy as np
import pytest

from helpers import bits_equal
from oracle import model, ops, optim, step
from oracle.ddp import ZeroAdamW, bucket_layout, ddp_average, partition

TINY = dict(vocab=11, ctx=8, dim=16, heads=2, layers=2)


@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_init_matches_dtrain(golden, dt):
    G = golden("dtrain_init_tiny.npz")
    P = model.dtrain_init(model.GPTConfig(dtype=dt, **TINY), seed=3)
    for name, arr in P.items():
        assert bits_equal(arr, G[f"{dt}/{name}"]), name


@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_two_step_training_matches_dtrain_bit_for_bit(golden, dt):
    S = golden(f"dtrain_step_tiny_{dt}.npz")
    c = model.GPTConfig(dtype=dt, **TINY)
    names = [n for n, _ in model.param_spec(c)]
    P = {n: S[f"p0/{n}"].copy() for n in names}
    opt = optim.AdamW([P[n] for n in names], lr=3e-3, weight_decay=0.1)
    batches = [(S["x0"], S["y0"]), (S["x1"], S["y1"])]
    loss, _, g = step.single_step(P, c, batches, opt, clip=0.05, emulate_world=2)
    assert loss == float(S["loss1"])
    for i, n in enumerate(names):
        assert bits_equal(g[i], S[f"g1/{n}"]), n
        assert bits_equal(P[n], S[f"p1/{n}"]), n
    loss, _, g = step.single_step(P, c, batches[::-1], opt, clip=0.0, emulate_world=2)
    assert loss == float(S["loss2"])
    for i, n in enumerate(names):
        assert bits_equal(g[i], S[f"g2/{n}"]), n
        assert bits_equal(P[n], S[f"p2/{n}"]), n


def test_adamw_float32_weak_scalar_rounding_matches_dtrain(golden):
    G = golden("dtrain_adamw_float32.npz")
    p = G["p0"].copy()
    opt = optim.AdamW([p], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    for k in range(3):
        opt.step([G[f"g{k}"]])
        assert bits_equal(p, G[f"p{k + 1}"])
        assert bits_equal(opt.m[0], G[f"m{k + 1}"])
        assert bits_equal(opt.v[0], G[f"v{k + 1}"])


@pytest.mark.parametrize("dt", ["float32", "float64"])
def test_attention_matches_dtrain_including_float64_promotion(golden, dt):
    G = golden("dtrain_attention.npz")
    q, k, v, g = (G[f"{dt}/{s}"] for s in "qkvg")
    o, p, scale = ops.attention_fwd(q, k, v)
    assert bits_equal(o, G[f"{dt}/o"])
    gq, gk, gv = ops.attention_bwd(g, q, k, v, p, scale)
    # NumPy 2: float32 inputs produce float64 gradients (np.float64 scale)
    assert gq.dtype == np.float64
    assert bits_equal(gq, G[f"{dt}/gq"]) and bits_equal(gk, G[f"{dt}/gk"]) and bits_equal(gv, G[f"{dt}/gv"])


@pytest.mark.parametrize("tag,cfg", [
    ("charGPT", model.GPTConfig(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64")),
    ("gpt2small", model.GPTConfig(vocab=50304, ctx=1024, dim=768, heads=12, layers=12, dtype="float32")),
])
def test_bucket_layout_matches_dtrain_ddp(golden, tag, cfg):
    G = golden("dtrain_layout.npz")
    sizes = [int(np.prod(s)) for _, s in model.param_spec(cfg)]
    rows = []
    for bi, entries in enumerate(bucket_layout(sizes, np.dtype(cfg.dtype).itemsize, 1.0)):
        for i, off, n in entries:
            rows.append((bi, i, off, n))
    assert np.array_equal(np.array(rows, dtype=np.int64), G[f"{tag}/layout"])


def test_gpt2_small_layout_facts(golden):
    """163,109,376 float32 parameters in 51 buckets, the largest the 154.5 MB head."""
    c = model.GPTConfig(vocab=50304, ctx=1024, dim=768, heads=12, layers=12, dtype="float32")
    sizes = [int(np.prod(s)) for _, s in model.param_spec(c)]
    assert sum(sizes) == 163_109_376
    lay = bucket_layout(sizes, 4, 1.0)
    assert len(lay) == 51
    assert max(sum(n for _, _, n in b) for b in lay) * 4 == 154_533_888


def test_partition_matches_dtrain(golden):
    for row in golden("dtrain_layout.npz")["partition"]:
        n, w = int(row[0]), int(row[1])
        assert partition(n, w) == [int(x) for x in row[2:3 + w]]


def test_char_gpt_workload_step_matches_dtrain(golden):
    """The float64 char-GPT workload (vocab 65, ctx 32, dim 64, 4 heads, 2 layers,
    batch 8): loss, gradients and updated parameters are bit-identical to dtrain's."""
    G = golden("dtrain_chargpt_step_summary.npz")
    c = model.GPTConfig(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64")
    P = model.synthetic_init(c, seed=0)
    xs, ys = model.synthetic_tokens(c, batch=8, seed=0)
    names = list(P)
    opt = optim.AdamW([P[n] for n in names], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    loss, _, g = step.single_step(P, c, [(xs[0], ys[0])], opt, clip=1.0)
    assert loss == float(G["loss"])
    for i, n in enumerate(names):
        assert hashlib.sha256(np.ascontiguousarray(g[i]).tobytes()).hexdigest() == str(G[f"g/{n}/sha256"]), n
        assert hashlib.sha256(np.ascontiguousarray(P[n]).tobytes()).hexdigest() == str(G[f"p/{n}/sha256"]), n


# -------------------------------------------- data-parallel reduction order
SHAPES_DDP = [(7, 5), (3,), (13, 4), (1,), (33,), (6, 6), (2,), (41,)]


@pytest.mark.parametrize("world", [3, 4])
@pytest.mark.parametrize("dt", ["float64", "float32"])
@pytest.mark.parametrize("algo", ["ring", "direct"])
def test_ddp_average_matches_dtrain_ring_and_direct(golden, world, dt, algo):
    """dtrain's DDP over its own TCP ring / direct all-reduce (3 and 4 ranks,
    256-byte buckets, gradients over 16 decades): bit for bit."""
    G = golden("dtrain_ddp_reduce.npz")
    reps = [[G[f"w{world}/{dt}/g{r}/{i}"] for i in range(len(SHAPES_DDP))] for r in range(world)]
    avg = ddp_average(reps, np.dtype(dt).itemsize, 256 / (1 << 20), algo)
    for i, a in enumerate(avg):
        assert bits_equal(a, G[f"w{world}/{dt}/ddp_{algo}/{i}"]), i


@pytest.mark.parametrize("world", [3, 4])
@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_ring_and_direct_orders_differ_on_these_inputs(golden, world, dt):
    """The fixture discriminates: a restatement using the other order fails it."""
    G = golden("dtrain_ddp_reduce.npz")
    diff = sum(int(np.sum(G[f"w{world}/{dt}/ddp_ring/{i}"] != G[f"w{world}/{dt}/ddp_direct/{i}"]))
               for i in range(len(SHAPES_DDP)))
    assert diff > 0


@pytest.mark.parametrize("world", [3, 4])
@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_zero_step_matches_dtrain(golden, world, dt):
    """dtrain's ZeroAdamW (ring reduce-scatter: shard r summed from rank r;
    *1/W; norm; clip; AdamW; all-gather). Without clip the parameters after
    the step are bit-identical; with clip 1.0 they differ only through the
    last bits of the BLAS-order float64 norm (within 1e-12)."""
    G = golden("dtrain_ddp_reduce.npz")
    p0 = [G[f"w{world}/{dt}/p0/{i}"] for i in range(len(SHAPES_DDP))]
    flats = [np.concatenate([G[f"w{world}/{dt}/g{r}/{i}"].reshape(-1) for i in range(len(SHAPES_DDP))])
             for r in range(world)]
    for tag, clip in (("zero_noclip", None), ("zero", 1.0)):
        z = ZeroAdamW([p.copy() for p in p0], world, max_grad_norm=clip, lr=1e-2, weight_decay=0.1)
        z.step(flats)
        ref = G[f"w{world}/{dt}/{tag}_flat"]
        assert abs(z.last_grad_norm - float(G[f"w{world}/{dt}/{tag}_norm"])) <= 1e-14 * z.last_grad_norm
        if clip is None:
            assert bits_equal(z.flat, ref)
        else:
            assert np.max(np.abs(z.flat - ref)) <= 1e-6 * np.max(np.abs(ref))


def test_ddp_ring_training_step_matches_dtrain(golden):
    """Two steps of dtrain's DDP training loop (--algo ring, 3 ranks, clip 0.5,
    float64 tiny GPT): loss, averaged gradients and parameters bit for bit."""
    S = golden("dtrain_ddp_step_float64.npz")
    c = model.GPTConfig(dtype="float64", **TINY)
    P = model.dtrain_init(c, seed=4)
    names = list(P)
    opt = optim.AdamW([P[n] for n in names], lr=3e-3, weight_decay=0.1)
    for s in range(2):
        batches = [(S[f"s{s}/x{r}"], S[f"s{s}/y{r}"]) for r in range(3)]
        loss, gnorm, avg = step.ddp_step(P, c, batches, opt, clip=0.5, bucket_mb=0.002, algo="ring")
        assert loss == float(S[f"s{s}/loss"])
        assert gnorm == float(np.sqrt(S[f"s{s}/sq"]))
        for i, n in enumerate(names):
            assert bits_equal(avg[i], S[f"s{s}/g/{n}"]), (s, n)
            assert bits_equal(P[n], S[f"s{s}/p/{n}"]), (s, n)
