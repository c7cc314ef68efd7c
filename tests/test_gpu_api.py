"""dtrain's Python API on the device (dtmi.autograd / nn / optim / ddp / zero)
against the oracle, on identical inputs. The cases follow dtrain's own tests
(tests/test_autograd.py, tests/test_training.py equivalences,
tests/test_torch_crosscheck.py AdamW) with the GPU result compared to the
oracle instead of finite differences.

Bar: float64 normwise relative error <= 1e-12, float32 <= 1e-5; float64 AdamW
and fixed-order average bit-exact; identical bits on repeated runs.
"""
import numpy as np
import pytest

from helpers import bits_equal, rel_err
from oracle import model as OM, ops, optim as OO, step as OS
from oracle.ddp import ZeroAdamW as OZero

pytestmark = pytest.mark.gpu
TOL = {np.float64: 1e-12, np.float32: 1e-5}
rng = np.random.default_rng(0)


def _api():
    from dtmi import autograd as A, nn as N, optim as O, ddp as P, zero as Z, replicas as R, train as S
    return A, N, O, P, Z, R, S


def grad_of(fn_dev, fn_ref_bwd, *arrays):
    """(out * w).sum().backward() on the device vs the oracle backward with g = w."""
    A = _api()[0]
    xs = [A.Tensor(a, requires_grad=True) for a in arrays]
    out = fn_dev(*xs)
    w = rng.standard_normal(out.shape)
    (out * A.Tensor(w)).sum().backward()
    ref = fn_ref_bwd(w, *arrays)
    for x, r in zip(xs, ref):
        assert x.grad is not None
        assert rel_err(x.grad.numpy(), r) <= 1e-12


def test_elementwise_and_broadcast(dev):
    grad_of(lambda a, b: a + b, lambda g, a, b: ops.add_bwd(g, a.shape, b.shape), rng.standard_normal((3, 4)),
            rng.standard_normal(4))
    grad_of(lambda a, b: a * b, lambda g, a, b: ops.mul_bwd(g, a, b), rng.standard_normal((2, 3, 4)),
            rng.standard_normal((1, 4)))
    grad_of(lambda a, b: a - b, lambda g, a, b: (ops.unbroadcast(g, a.shape), -ops.unbroadcast(g, b.shape)),
            rng.standard_normal((3, 1)), rng.standard_normal((3, 5)))


def test_matmul_batched_and_broadcast(dev):
    grad_of(lambda a, b: a @ b, lambda g, a, b: ops.matmul_bwd(g, a, b), rng.standard_normal((2, 3, 4)),
            rng.standard_normal((4, 5)))
    grad_of(lambda a, b: a @ b, lambda g, a, b: ops.matmul_bwd(g, a, b), rng.standard_normal((2, 3, 4)),
            rng.standard_normal((2, 4, 2)))


def test_reductions_reshape_transpose(dev):
    grad_of(lambda a: a.sum(axis=1), lambda g, a: (ops.sum_bwd(g, a.shape, axis=1),), rng.standard_normal((3, 4, 2)))
    grad_of(lambda a: a.mean(axis=-1, keepdims=True),
            lambda g, a: (ops.sum_bwd(g * (1.0 / 4), a.shape, axis=-1, keepdims=True),), rng.standard_normal((3, 4)))
    grad_of(lambda a: a.reshape(4, 6).transpose(1, 0), lambda g, a: (g.transpose(1, 0).reshape(a.shape),),
            rng.standard_normal((2, 3, 4)))


def test_activations(dev):
    def gb(g, x):
        _, t, c = ops.gelu_fwd(x)
        return (ops.gelu_bwd(g, x, t, c),)
    grad_of(lambda a: a.gelu(), gb, rng.standard_normal((4, 5)))
    grad_of(lambda a: a.relu(), lambda g, x: (ops.relu_bwd(g, x > 0),), rng.standard_normal((4, 5)))


def test_layer_norm_attention_embedding_ops(dev):
    A = _api()[0]

    def ln_bwd(g, x, w, b):
        _, cache = ops.layer_norm_fwd(x, w, b)
        return ops.layer_norm_bwd(g, cache, w)
    grad_of(lambda x, w, b: A.layer_norm(x, w, b), ln_bwd, rng.standard_normal((2, 3, 6)), rng.standard_normal(6),
            rng.standard_normal(6))

    def at_bwd(g, q, k, v):
        _, p, s = ops.attention_fwd(q, k, v)
        return ops.attention_bwd(g, q, k, v, p, s)
    grad_of(lambda q, k, v: A.causal_attention(q, k, v), at_bwd, *(rng.standard_normal((1, 2, 4, 3)) for _ in range(3)))
    idx = np.array([[0, 2, 2], [1, 0, 2]])
    grad_of(lambda w: A.embedding(w, idx), lambda g, w: (ops.embedding_bwd(g, w.shape, w.dtype, idx),),
            rng.standard_normal((3, 4)))


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_residual_gradient_summed_in_layernorm_pass(dev, dt):
    """z = x + layer_norm(x) @ m: x's residual gradient is pending when the
    LayerNorm backward runs, which then adds its input gradient onto it in its
    own pass. Same bits as the engine's separate sum, and the oracle's values."""
    A = _api()[0]
    r = np.random.default_rng(21)
    x0 = r.standard_normal((4, 16, 64)).astype(dt)
    w0 = (1 + 0.1 * r.standard_normal(64)).astype(dt)
    b0 = (0.1 * r.standard_normal(64)).astype(dt)
    m0 = (0.1 * r.standard_normal((64, 64))).astype(dt)
    c0 = r.standard_normal((4, 16, 64)).astype(dt)

    def run(fuse):
        x, w, b = (A.Tensor(a, requires_grad=True) for a in (x0, w0, b0))
        h = A.layer_norm(x, w, b)
        used = []
        if fuse:
            i, f = h._backward.with_addend
            h._backward.with_addend = (i, lambda g, p: used.append(f(g, p)) or used[-1])
        else:
            del h._backward.with_addend
        z = x + h @ A.Tensor(m0)
        (z * A.Tensor(c0)).sum().backward()
        assert len(used) == (1 if fuse else 0) and all(u is not None for u in used)
        return x.grad.numpy(), w.grad.numpy(), b.grad.numpy()
    fused, plain = run(True), run(False)
    for a, p in zip(fused, plain):
        assert bits_equal(a, p)
    _, cache = ops.layer_norm_fwd(x0, w0, b0)
    gx, gw, gb = ops.layer_norm_bwd(c0 @ m0.T, cache, w0)
    tol = 1e-12 if dt == np.float64 else 1e-5
    for a, ref in zip(fused, (c0 + gx, gw, gb)):
        assert rel_err(a, ref) <= tol


def test_cross_entropy(dev):
    A = _api()[0]
    t = rng.integers(0, 5, size=(2, 3))
    z = rng.standard_normal((2, 3, 5))
    x = A.Tensor(z, requires_grad=True)
    loss = A.cross_entropy(x, t)
    loss.backward()
    ref_loss, cache = ops.cross_entropy_fwd(z, t)
    assert rel_err(loss.numpy(), ref_loss) <= 1e-14
    assert rel_err(x.grad.numpy(), ops.cross_entropy_bwd(np.float64(1.0), z, t, cache)) <= 1e-13


def test_grad_ready_hook_fires_once_with_final_gradient(dev):
    """dtrain tests/test_autograd.py:103-111."""
    A = _api()[0]
    w = A.Tensor(rng.standard_normal((3, 3)), requires_grad=True)
    seen = []
    w.register_grad_ready_hook(lambda t: seen.append(t.grad.copy()))
    x = A.Tensor(rng.standard_normal((2, 3)))
    y = (x @ w) + (x @ w) * 2.0  # w used twice
    y.sum().backward()
    assert len(seen) == 1
    np.testing.assert_allclose(seen[0].numpy(), w.grad.numpy())


def test_backward_needs_scalar_or_grad(dev):
    A = _api()[0]
    x = A.Tensor(rng.standard_normal((2, 2)), requires_grad=True)
    with pytest.raises(ValueError):
        (x * 2.0).backward()


@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_gpt_init_matches_dtrain(dev, golden, dt):
    N = _api()[1]
    G = golden("dtrain_init_tiny.npz")
    m = N.GPT(N.GPTConfig(vocab=11, ctx=8, dim=16, heads=2, layers=2, dtype=dt), seed=3)
    for name, p in m.named_parameters():
        assert bits_equal(p.numpy(), G[f"{dt}/{name}"]), name


@pytest.mark.parametrize("dt", [np.float64, np.float32])
def test_full_model_gradients_match_oracle(dev, dt):
    N = _api()[1]
    c = dict(vocab=13, ctx=6, dim=16, heads=4, layers=2)
    P = OM.dtrain_init(OM.GPTConfig(dtype=np.dtype(dt).name, **c), seed=2)
    x = rng.integers(0, 13, size=(3, 6))
    y = rng.integers(0, 13, size=(3, 6))
    loss_ref, G = OM.loss_and_grads(P, OM.GPTConfig(dtype=np.dtype(dt).name, **c), x, y)
    m = N.GPT(N.GPTConfig(dtype=np.dtype(dt).name, **c), seed=2)
    _, loss = m(x, y)
    loss.backward()
    assert rel_err(loss.numpy(), loss_ref) <= TOL[dt]
    for name, p in m.named_parameters():
        assert rel_err(p.grad.numpy(), G[name]) <= TOL[dt], name


class ShadowAdam:
    """The oracle's AdamW driven by the device's own gradients and clip factor:
    the device parameters must equal it bit for bit after every step (the
    AdamW update itself is exact; only the gradients carry tolerance)."""

    def __init__(self, model, lr, wd=0.1):
        self.names = [n for n, _ in model.named_parameters()]
        self.p = {n: p.numpy() for n, p in model.named_parameters()}
        self.opt = OO.AdamW([self.p[n] for n in self.names], lr=lr, weight_decay=wd)

    def check(self, model, scale):
        grads = [p.grad.numpy() for _, p in model.named_parameters()]
        self.opt.step([g * scale for g in grads])
        for n, p in model.named_parameters():
            assert bits_equal(p.numpy(), self.p[n]), n


@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_two_training_steps_match_dtrain_golden(dev, golden, dt):
    """dtrain's own two single-process steps (emulated world 2; clip 0.05, then no clip)."""
    A, N, O, P, Z, R, S_ = _api()
    S = golden(f"dtrain_step_tiny_{dt}.npz")
    names = [n for n, _ in OM.param_spec(OM.GPTConfig(vocab=11, ctx=8, dim=16, heads=2, layers=2, dtype=dt))]
    batches = [(S["x0"], S["y0"]), (S["x1"], S["y1"])]
    m = N.GPT(N.GPTConfig(vocab=11, ctx=8, dim=16, heads=2, layers=2, dtype=dt), seed=5)
    m.load_numpy({n: S[f"p0/{n}"] for n in names})
    opt = O.AdamW([p.data for p in m.parameters()], lr=3e-3, weight_decay=0.1)
    shadow = ShadowAdam(m, 3e-3)
    tol = TOL[np.dtype(dt).type]
    res = S_.step_single(m, opt, [[b] for b in batches], clip=0.05)
    assert abs(res.loss - float(S["loss1"])) <= tol * abs(float(S["loss1"]))
    for n, p in m.named_parameters():
        assert rel_err(p.grad.numpy(), S[f"g1/{n}"]) <= tol, n
    assert abs(res.clip_scale - float(S["s1"])) <= tol * float(S["s1"])
    shadow.check(m, res.clip_scale)
    # step 2 starts from the device's step-1 parameters; AdamW turns rounding
    # noise in mathematically-zero gradients (e.g. the key bias) into O(lr)
    # parameter differences, so its reference is the oracle at those inputs
    oc = OM.GPTConfig(vocab=11, ctx=8, dim=16, heads=2, layers=2, dtype=dt)
    P1 = {n: p.numpy() for n, p in m.named_parameters()}
    loss2, _, g2 = OS.single_step(P1, oc, batches[::-1], OO.AdamW(list(P1.values()), lr=0.0), clip=0.0,
                                  emulate_world=2)
    res = S_.step_single(m, opt, [[b] for b in batches[::-1]], clip=0.0)
    assert abs(res.loss - loss2) <= tol * abs(loss2)
    for i, (n, p) in enumerate(m.named_parameters()):
        assert rel_err(p.grad.numpy(), g2[i]) <= tol, n
    shadow.check(m, 1.0)


def test_char_gpt_workload_step_float64(dev):
    """The float64 char-GPT workload (vocab 65, ctx 32, dim 64, 4 heads, 2 layers,
    batch 8; forward, CE backward, clip 1.0, AdamW): loss, gradients and norm
    within 1e-12 of the oracle (itself bit-identical to dtrain); the AdamW step
    bit-exact on those gradients."""
    A, N, O, P, Z, R, S_ = _api()
    oc = OM.GPTConfig(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64")
    Pn = OM.synthetic_init(oc, seed=0)
    xs, ys = OM.synthetic_tokens(oc, batch=8, seed=0)
    m = N.GPT(N.GPTConfig(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64"))
    m.load_numpy(Pn)
    shadow = ShadowAdam(m, 3e-4)
    opt = O.AdamW([p.data for p in m.parameters()], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    oopt = OO.AdamW([Pn[n] for n in Pn], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    res = S_.step_single(m, opt, [[(xs[0], ys[0])]], clip=1.0)
    loss, gnorm, g = OS.single_step(Pn, oc, [(xs[0], ys[0])], oopt, clip=1.0)
    assert abs(res.loss - loss) <= 1e-12 * abs(loss)
    assert abs(res.grad_norm - gnorm) <= 1e-12 * gnorm
    for i, (n, p) in enumerate(m.named_parameters()):
        assert rel_err(p.grad.numpy(), g[i]) <= 1e-12, n
    shadow.check(m, res.clip_scale)


@pytest.mark.parametrize("dt", ["float64", "float32"])
@pytest.mark.parametrize("algo", ["ring", "direct"])
def test_ddp_simulated_replicas_match_oracle(dev, dt, algo):
    """DDP over 4 simulated replicas (buckets, ring or direct order average,
    clip, AdamW), two steps: averaged gradients, norm and loss against the
    oracle's DDP step; AdamW bit-exact on the averaged gradients."""
    A, N, O, P, Z, R, S_ = _api()
    cfg = dict(vocab=17, ctx=8, dim=32, heads=4, layers=2)
    oc = OM.GPTConfig(dtype=dt, **cfg)
    xs, ys = OM.synthetic_tokens(oc, batch=3, seed=9, replicas=4)
    m = N.GPT(N.GPTConfig(dtype=dt, **cfg), seed=4)
    pg = R.SimGroup(4)
    ddp = P.DDP(m, pg, bucket_mb=0.01, algo=algo)
    assert len(ddp.buckets) > 1
    opt = O.AdamW([p.data for p in m.parameters()], lr=1e-3)
    shadow = ShadowAdam(m, 1e-3)
    tol = TOL[np.dtype(dt).type]
    for step in range(2):
        Pn = {n: p.numpy() for n, p in m.named_parameters()}  # the oracle starts from the device's parameters
        oopt = OO.AdamW([Pn[n] for n in Pn], lr=1e-3)
        res = S_.step_ddp(m, ddp, opt, [[(xs[r], ys[r])] for r in range(4)], clip=0.5)
        loss, gnorm, avg = OS.ddp_step(Pn, oc, [(xs[r], ys[r]) for r in range(4)], oopt, clip=0.5, bucket_mb=0.01,
                                       algo=algo)
        assert abs(res.loss - loss) <= tol * abs(loss)
        assert abs(res.grad_norm - gnorm) <= tol * gnorm
        for i, (n, p) in enumerate(m.named_parameters()):
            assert rel_err(p.grad.numpy(), avg[i]) <= tol, n
        shadow.check(m, res.clip_scale)


def test_bucket_size_and_overlap_do_not_change_bits(dev):
    """dtrain tests/test_training.py:75-80 asserts <= 1e-12; with the direct
    order (rank 0 first for every element) the results are bit-identical."""
    A, N, O, P, Z, R, S_ = _api()
    cfg = N.GPTConfig(vocab=17, ctx=8, dim=32, heads=4, layers=2, dtype="float64")
    oc = OM.GPTConfig(vocab=17, ctx=8, dim=32, heads=4, layers=2, dtype="float64")
    xs, ys = OM.synthetic_tokens(oc, batch=2, seed=3, replicas=4)
    finals = []
    for mb, overlap in ((0.001, True), (100.0, True), (0.01, False)):
        m = N.GPT(cfg, seed=1)
        pg = R.SimGroup(4)
        ddp = P.DDP(m, pg, bucket_mb=mb, overlap=overlap, algo="direct")
        opt = O.AdamW([p.data for p in m.parameters()], lr=1e-3)
        for _ in range(2):
            S_.step_ddp(m, ddp, opt, [[(xs[r], ys[r])] for r in range(4)])
        finals.append(m.flat.numpy())
    assert bits_equal(finals[0], finals[1]) and bits_equal(finals[0], finals[2])


def test_overlap_bucket_size_and_algorithm_do_not_change_results(dev):
    """dtrain tests/test_training.py:75-80: ring with overlap, ring without it at
    another bucket size, and direct, all within 1e-12 after three steps (the
    ring's chunk edges move with the bucket size, so bits may differ)."""
    A, N, O, P, Z, R, S_ = _api()
    cfg = N.GPTConfig(vocab=17, ctx=8, dim=32, heads=4, layers=2, dtype="float64")
    oc = OM.GPTConfig(vocab=17, ctx=8, dim=32, heads=4, layers=2, dtype="float64")
    xs, ys = OM.synthetic_tokens(oc, batch=2, seed=3, replicas=3)
    finals = []
    for mb, overlap, algo in ((1.0, True, "ring"), (0.001, False, "ring"), (1.0, True, "direct")):
        m = N.GPT(cfg, seed=1)
        pg = R.SimGroup(3)
        ddp = P.DDP(m, pg, bucket_mb=mb, overlap=overlap, algo=algo)
        opt = O.AdamW([p.data for p in m.parameters()], lr=1e-3)
        for _ in range(3):
            S_.step_ddp(m, ddp, opt, [[(xs[r], ys[r])] for r in range(3)])
        finals.append(m.flat.numpy())
    assert np.max(np.abs(finals[0] - finals[1])) <= 1e-12
    assert np.max(np.abs(finals[0] - finals[2])) <= 1e-12


def test_ddp_matches_single_process_emulated_world(dev):
    """dtrain tests/test_training.py:57-62: DDP(4) == single --emulate-world 4 to 1e-10."""
    A, N, O, P, Z, R, S_ = _api()
    cfg = N.GPTConfig(vocab=17, ctx=8, dim=32, heads=4, layers=2, dtype="float64")
    oc = OM.GPTConfig(vocab=17, ctx=8, dim=32, heads=4, layers=2, dtype="float64")
    xs, ys = OM.synthetic_tokens(oc, batch=2, seed=5, replicas=4)
    m1 = N.GPT(cfg, seed=1)
    o1 = O.AdamW([p.data for p in m1.parameters()], lr=3e-3)
    m2 = N.GPT(cfg, seed=1)
    pg = R.SimGroup(4)
    ddp = P.DDP(m2, pg)
    o2 = O.AdamW([p.data for p in m2.parameters()], lr=3e-3)
    for _ in range(3):
        S_.step_single(m1, o1, [[(xs[r], ys[r])] for r in range(4)])
        S_.step_ddp(m2, ddp, o2, [[(xs[r], ys[r])] for r in range(4)])
    assert np.max(np.abs(m1.flat.numpy() - m2.flat.numpy())) <= 1e-10


def test_gradient_accumulation_equals_larger_batch(dev):
    """dtrain tests/test_training.py:83-87: accum 2 with batch b == accum 1 with
    batch 2b (float64, DDP over 2 replicas)."""
    A, N, O, P, Z, R, S_ = _api()
    cfg = N.GPTConfig(vocab=17, ctx=8, dim=32, heads=4, layers=2, dtype="float64")
    oc = OM.GPTConfig(vocab=17, ctx=8, dim=32, heads=4, layers=2, dtype="float64")
    xs, ys = OM.synthetic_tokens(oc, batch=4, seed=6, replicas=2)
    finals = []
    for accum in (1, 2):
        m = N.GPT(cfg, seed=2)
        pg = R.SimGroup(2)
        ddp = P.DDP(m, pg)
        opt = O.AdamW([p.data for p in m.parameters()], lr=3e-3)
        b = 4 // accum
        batches = [[(xs[r][i * b:(i + 1) * b], ys[r][i * b:(i + 1) * b]) for i in range(accum)] for r in range(2)]
        S_.step_ddp(m, ddp, opt, batches, accum=accum)
        finals.append(m.flat.numpy())
    assert np.max(np.abs(finals[0] - finals[1])) <= 1e-10


@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_zero_matches_oracle_and_state_bytes(dev, dt):
    A, N, O, P, Z, R, S_ = _api()
    cfg = dict(vocab=17, ctx=8, dim=32, heads=4, layers=2)
    oc = OM.GPTConfig(dtype=dt, **cfg)
    Pn = OM.dtrain_init(oc, seed=7)
    xs, ys = OM.synthetic_tokens(oc, batch=2, seed=8, replicas=4)
    m = N.GPT(N.GPTConfig(dtype=dt, **cfg), seed=7)
    pg = R.SimGroup(4)
    z = Z.ZeroAdamW(m, pg, max_grad_norm=0.5, lr=1e-3, weight_decay=0.1)
    n = z.n
    itemsize = np.dtype(dt).itemsize
    assert z.state_bytes() == 2 * itemsize * -(-n // 4)  # dtrain tests/test_training.py:72
    names = list(Pn)
    oz = OZero([Pn[k] for k in names], 4, max_grad_norm=0.5, lr=1e-3, weight_decay=0.1)
    tol = TOL[np.dtype(dt).type]
    for _ in range(2):
        S_.step_zero(m, z, [[(xs[r], ys[r])] for r in range(4)])
        flat_grads = []
        for r in range(4):
            # the oracle's per-replica gradients, flattened in forward order
            shard = {k: oz.flat[o:o + Pn[k].size].reshape(Pn[k].shape) for k, o in
                     zip(names, np.cumsum([0] + [Pn[k].size for k in names])[:-1])}
            _, G = OM.loss_and_grads(shard, oc, xs[r], ys[r])
            flat_grads.append(np.concatenate([G[k].reshape(-1) for k in names]))
        oz.step(flat_grads)
        assert rel_err(z.flat.numpy(), oz.flat) <= tol
        assert abs(z.last_grad_norm - oz.last_grad_norm) <= tol * oz.last_grad_norm


def test_step_is_deterministic(dev):
    A, N, O, P, Z, R, S_ = _api()
    cfg = N.GPTConfig(vocab=50, ctx=64, dim=64, heads=4, layers=2, dtype="float32")
    oc = OM.GPTConfig(vocab=50, ctx=64, dim=64, heads=4, layers=2, dtype="float32")
    xs, ys = OM.synthetic_tokens(oc, batch=4, seed=1, replicas=4)
    outs = []
    for _ in range(2):
        m = N.GPT(cfg, seed=0)
        pg = R.SimGroup(4)
        ddp = P.DDP(m, pg)
        opt = O.AdamW([p.data for p in m.parameters()], lr=1e-3)
        for _ in range(2):
            S_.step_ddp(m, ddp, opt, [[(xs[r], ys[r])] for r in range(4)])
        outs.append(m.flat.numpy())
    assert bits_equal(outs[0], outs[1])


# ------------------------------------------- dtrain's data-parallel orders
SHAPES_DDP = [(7, 5), (3,), (13, 4), (1,), (33,), (6, 6), (2,), (41,)]


class _Params:
    """A model of bare parameters (dtrain's DDP/ZeroAdamW only call .parameters())."""

    def __init__(self, A, arrays):
        self.ps = [A.Tensor(a.copy(), requires_grad=True) for a in arrays]

    def parameters(self):
        return self.ps


# launch grouping of the bucket averages: dtmi.ddp.DDP's defaults (every bucket
# of these tiny models in one launch at finish()), a launch per bucket as each
# completes (MERGE_BYTES 1), and runs cut by the rank-order segment limit
MERGE = {"default": None, "per_bucket": (1, 16), "segment_limit": (1 << 30, 8)}


@pytest.mark.parametrize("merge", sorted(MERGE))
@pytest.mark.parametrize("world", [3, 4])
@pytest.mark.parametrize("dt", ["float64", "float32"])
@pytest.mark.parametrize("algo", ["ring", "direct"])
def test_ddp_average_matches_dtrain_fixture(dev, golden, monkeypatch, world, dt, algo, merge):
    """dtrain's DDP over its TCP ring / direct all-reduce (3 and 4 ranks, 256-byte
    buckets, gradients over 16 decades) bit for bit: the simulated replicas'
    gradients go through the grad-ready hooks and finish(), with the bucket
    averages launched in each of the groupings DDP can make."""
    A, N, O, P, Z, R, S_ = _api()
    from dtmi import device as D
    if MERGE[merge] is not None:
        monkeypatch.setattr(P.DDP, "MERGE_BYTES", MERGE[merge][0])
        monkeypatch.setattr(P.DDP, "MAX_SEGS", MERGE[merge][1])
    G = golden("dtrain_ddp_reduce.npz")
    n = len(SHAPES_DDP)
    m = _Params(A, [G[f"w{world}/{dt}/p0/{i}"] for i in range(n)])
    pg = R.SimGroup(world)
    ddp = P.DDP(m, pg, bucket_mb=256 / (1 << 20), overlap=True, algo=algo)
    assert len(ddp.buckets) > 2
    launches = []
    average = pg.average
    pg.average = lambda out, rows, **kw: (launches.append((len(kw.get("segments") or ()), ddp._sync)),
                                          average(out, rows, **kw))
    for r in range(world):
        with pg.replica(r):
            for i in reversed(range(n)):
                p = m.ps[i]
                p.grad = D.from_numpy(G[f"w{world}/{dt}/g{r}/{i}"])
                ddp._on_grad(p)
        if r == world - 1 and merge == "per_bucket":
            # every bucket was averaged inside the last replica's hooks
            assert len(launches) == len(ddp.buckets)
    ddp.finish()
    if algo == "direct" and merge != "per_bucket":
        assert len(launches) == 1  # one rank order: every bucket in one launch
    if algo == "ring" and merge == "segment_limit":
        assert len(launches) > 1  # 3-6 segments per bucket, at most 8 per launch
    for i, p in enumerate(m.ps):
        assert bits_equal(p.grad.numpy(), G[f"w{world}/{dt}/ddp_{algo}/{i}"]), i


@pytest.mark.parametrize("world", [3, 4])
@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_zero_matches_dtrain_fixture(dev, golden, world, dt):
    """dtrain's ZeroAdamW (ring reduce-scatter, shard r summed from rank r):
    without clip the parameters after one step are bit-identical; with clip
    1.0 the norm is within 1e-14 and the parameters within the clip factor's
    last-bit difference."""
    A, N, O, P, Z, R, S_ = _api()
    from dtmi import device as D
    G = golden("dtrain_ddp_reduce.npz")
    n = len(SHAPES_DDP)
    for tag, clip in (("zero_noclip", None), ("zero", 1.0)):
        m = _Params(A, [G[f"w{world}/{dt}/p0/{i}"] for i in range(n)])
        pg = R.SimGroup(world)
        z = Z.ZeroAdamW(m, pg, max_grad_norm=clip, lr=1e-2, weight_decay=0.1)
        for r in range(world):
            with pg.replica(r):
                for i in range(n):
                    p = m.ps[i]
                    p.grad = D.from_numpy(G[f"w{world}/{dt}/g{r}/{i}"])
                    z._on_grad(p)
        z.step()
        ref = G[f"w{world}/{dt}/{tag}_flat"]
        norm = float(G[f"w{world}/{dt}/{tag}_norm"])
        assert abs(z.last_grad_norm - norm) <= 1e-14 * norm
        if clip is None:
            assert bits_equal(z.flat.numpy(), ref)
        else:
            assert np.max(np.abs(z.flat.numpy() - ref)) <= 1e-6 * np.max(np.abs(ref))


def test_ddp_ring_training_steps_match_dtrain_fixture(dev, golden):
    """Two steps of dtrain's DDP loop (--algo ring, 3 ranks, clip 0.5, float64):
    losses, norms and averaged gradients within 1e-12, and AdamW bit-exact on
    the device's averaged gradients."""
    A, N, O, P, Z, R, S_ = _api()
    S = golden("dtrain_ddp_step_float64.npz")
    cfg = N.GPTConfig(vocab=11, ctx=8, dim=16, heads=2, layers=2, dtype="float64")
    m = N.GPT(cfg, seed=4)
    pg = R.SimGroup(3)
    ddp = P.DDP(m, pg, bucket_mb=0.002)  # dtrain's default algo: ring
    assert ddp.algo == "ring"
    opt = O.AdamW([p.data for p in m.parameters()], lr=3e-3, weight_decay=0.1)
    shadow = ShadowAdam(m, 3e-3)
    for s in range(2):
        batches = [[(S[f"s{s}/x{r}"], S[f"s{s}/y{r}"])] for r in range(3)]
        res = S_.step_ddp(m, ddp, opt, batches, clip=0.5)
        assert abs(res.loss - float(S[f"s{s}/loss"])) <= 1e-12 * abs(float(S[f"s{s}/loss"]))
        sq = float(S[f"s{s}/sq"])
        assert abs(res.grad_norm - np.sqrt(sq)) <= 1e-12 * np.sqrt(sq)
        for n, p in m.named_parameters():
            assert rel_err(p.grad.numpy(), S[f"s{s}/g/{n}"]) <= 1e-12, (s, n)
        shadow.check(m, res.clip_scale)


@pytest.mark.parametrize("dt", ["float64", "float32"])
def test_model_with_head_dimension_128_matches_oracle(dev, dt):
    """dtrain's `--dim 256 --heads 2` (head dimension 128) trains: loss and every
    gradient against the oracle."""
    N = _api()[1]
    c = dict(vocab=19, ctx=16, dim=256, heads=2, layers=1)
    P = OM.dtrain_init(OM.GPTConfig(dtype=dt, **c), seed=3)
    x = rng.integers(0, 19, size=(2, 16))
    y = rng.integers(0, 19, size=(2, 16))
    loss_ref, G = OM.loss_and_grads(P, OM.GPTConfig(dtype=dt, **c), x, y)
    m = N.GPT(N.GPTConfig(dtype=dt, **c), seed=3)
    _, loss = m(x, y)
    loss.backward()
    tol = TOL[np.dtype(dt).type]
    assert rel_err(loss.numpy(), loss_ref) <= tol
    for name, p in m.named_parameters():
        assert rel_err(p.grad.numpy(), G[name]) <= tol, name
