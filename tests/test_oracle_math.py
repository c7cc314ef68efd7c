"""The oracle against mathematics (CPU): finite differences with dtrain's own
recipe (tests/test_autograd.py:11-28 of dtrain: float64, central differences,
eps 1e-6, tolerance 1e-5), closed forms, brute-force loops, an independent
library (torch float64 autograd and torch.optim.AdamW), and the invariants
dtrain's tests assert. A few tests plant a mistake in a copy of an oracle
function and show that the check catches it.
"""
import numpy as np
import pytest

from helpers import rel_err
from oracle import model, ops, optim
from oracle.ddp import ZeroAdamW, bucket_layout, ddp_average, fixed_order_sum, partition, ring_order_sum

rng = np.random.default_rng(0)


def fd_grad(f, xs, eps=1e-6):
    """Central differences of the scalar f(*xs) w.r.t. every element of every x."""
    out = []
    for x in xs:
        num = np.zeros_like(x)
        for i in np.ndindex(x.shape):
            old = x[i]
            x[i] = old + eps
            fp = f(*xs)
            x[i] = old - eps
            fm = f(*xs)
            x[i] = old
            num[i] = (fp - fm) / (2 * eps)
        out.append(num)
    return out


def check(fwd, bwd, *shapes, tol=1e-5):
    xs = [rng.standard_normal(s) for s in shapes]
    w = rng.standard_normal(np.shape(fwd(*xs)))
    analytic = bwd(w, *xs)
    numeric = fd_grad(lambda *a: float((fwd(*a) * w).sum()), xs)
    for a, n in zip(analytic, numeric):
        np.testing.assert_allclose(a, n, rtol=tol, atol=tol)


def test_fd_broadcast_add_mul_sub():
    check(lambda a, b: a + b, lambda g, a, b: ops.add_bwd(g, a.shape, b.shape), (3, 4), (4,))
    check(lambda a, b: a * b, lambda g, a, b: ops.mul_bwd(g, a, b), (2, 3, 4), (1, 4))
    check(lambda a, b: a - b, lambda g, a, b: (ops.unbroadcast(g, a.shape), -ops.unbroadcast(g, b.shape)),
          (3, 1), (3, 5))


def test_fd_matmul_batched_and_broadcast():
    check(lambda a, b: a @ b, lambda g, a, b: ops.matmul_bwd(g, a, b), (2, 3, 4), (4, 5))
    check(lambda a, b: a @ b, lambda g, a, b: ops.matmul_bwd(g, a, b), (2, 3, 4), (2, 4, 2))


def test_fd_sum_gelu_relu():
    check(lambda a: a.sum(axis=1), lambda g, a: (ops.sum_bwd(g, a.shape, axis=1),), (3, 4, 2))

    def gb(g, x):
        _, t, c = ops.gelu_fwd(x)
        return (ops.gelu_bwd(g, x, t, c),)
    check(lambda x: ops.gelu_fwd(x)[0], gb, (4, 5))
    check(lambda x: ops.relu_fwd(x)[0], lambda g, x: (ops.relu_bwd(g, x > 0),), (4, 5))


def test_fd_layer_norm():
    def bwd(g, x, w, b):
        _, cache = ops.layer_norm_fwd(x, w, b)
        return ops.layer_norm_bwd(g, cache, w)
    check(lambda x, w, b: ops.layer_norm_fwd(x, w, b)[0], bwd, (2, 3, 6), (6,), (6,))


def test_fd_causal_attention():
    def bwd(g, q, k, v):
        _, p, scale = ops.attention_fwd(q, k, v)
        return ops.attention_bwd(g, q, k, v, p, scale)
    check(lambda q, k, v: ops.attention_fwd(q, k, v)[0], bwd, (1, 2, 4, 3), (1, 2, 4, 3), (1, 2, 4, 3))


def test_fd_embedding_repeated_indices():
    idx = np.array([[0, 2, 2], [1, 0, 2]])
    check(lambda w: ops.embedding_fwd(w, idx), lambda g, w: (ops.embedding_bwd(g, w.shape, w.dtype, idx),), (3, 4))


def test_fd_cross_entropy():
    t = rng.integers(0, 5, size=(2, 3))
    z = rng.standard_normal((2, 3, 5))
    loss, cache = ops.cross_entropy_fwd(z, t)
    g = ops.cross_entropy_bwd(np.float64(1.0), z, t, cache)
    num = fd_grad(lambda zz: float(ops.cross_entropy_fwd(zz, t)[0]), [z])[0]
    np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-8)


def test_fd_full_model_float64():
    """dtrain tests/test_autograd.py:83-100: 3 coordinates of every parameter."""
    c = model.GPTConfig(vocab=7, ctx=5, dim=8, heads=2, layers=2, dtype="float64")
    P = model.dtrain_init(c, seed=1)
    x = rng.integers(0, 7, size=(2, 5))
    y = rng.integers(0, 7, size=(2, 5))
    _, G = model.loss_and_grads(P, c, x, y)
    for name, p in P.items():
        for _ in range(3):
            i = tuple(rng.integers(0, s) for s in p.shape)
            old = p[i]
            p[i] = old + 1e-6
            fp = float(model.forward(P, c, x, y)[1])
            p[i] = old - 1e-6
            fm = float(model.forward(P, c, x, y)[1])
            p[i] = old
            assert abs(G[name][i] - (fp - fm) / 2e-6) < 1e-6, name


def test_brute_force_attention_loops():
    q, k, v = (rng.standard_normal((1, 1, 5, 3)) for _ in range(3))
    o, _, _ = ops.attention_fwd(q, k, v)
    T, D = 5, 3
    ref = np.zeros((T, D))
    for i in range(T):
        s = [sum(q[0, 0, i, d] * k[0, 0, j, d] for d in range(D)) / np.sqrt(D) for j in range(i + 1)]
        m = max(s)
        e = [np.exp(x - m) for x in s]
        for j in range(i + 1):
            ref[i] += e[j] / sum(e) * v[0, 0, j]
    np.testing.assert_allclose(o[0, 0], ref, rtol=1e-13, atol=1e-14)


def test_closed_form_cross_entropy_grad_is_softmax_minus_onehot():
    z = rng.standard_normal((6, 9))
    t = rng.integers(0, 9, 6)
    loss, cache = ops.cross_entropy_fwd(z, t)
    g = ops.cross_entropy_bwd(np.float64(1.0), z, t, cache)
    p = np.exp(z) / np.exp(z).sum(-1, keepdims=True)
    p[np.arange(6), t] -= 1
    np.testing.assert_allclose(g, p / 6, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(float(loss), -np.mean(np.log(np.exp(z[np.arange(6), t]) / np.exp(z).sum(-1))),
                               rtol=1e-13)


def test_torch_float64_autograd_agrees_on_the_full_gpt():
    torch = pytest.importorskip("torch")
    c = model.GPTConfig(vocab=13, ctx=6, dim=16, heads=4, layers=2, dtype="float64")
    P = model.dtrain_init(c, seed=2)
    x = rng.integers(0, 13, size=(3, 6))
    y = rng.integers(0, 13, size=(3, 6))
    loss, G = model.loss_and_grads(P, c, x, y)
    T = {k: torch.tensor(v, requires_grad=True) for k, v in P.items()}
    B, S, C, H = 3, 6, 16, 4

    def ln(h, w, b):
        mu = h.mean(-1, keepdim=True)
        var = ((h - mu) ** 2).mean(-1, keepdim=True)
        return (h - mu) / torch.sqrt(var + 1e-5) * w + b

    h = T["tok"][torch.tensor(x)] + T["pos"][torch.arange(S)]
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
    for i in range(c.layers):
        p = f"blocks.{i}."
        a = ln(h, T[p + "ln1.w"], T[p + "ln1.b"]) @ T[p + "qkv.w"] + T[p + "qkv.b"]
        q, k, v = a.reshape(B, S, 3, H, C // H).permute(2, 0, 3, 1, 4)
        s = (q @ k.transpose(-1, -2)) / np.sqrt(C // H)
        att = torch.softmax(s.masked_fill(mask, float("-inf")), -1) @ v
        h = h + att.permute(0, 2, 1, 3).reshape(B, S, C) @ T[p + "proj.w"] + T[p + "proj.b"]
        f = ln(h, T[p + "ln2.w"], T[p + "ln2.b"]) @ T[p + "fc.w"] + T[p + "fc.b"]
        h = h + torch.nn.functional.gelu(f, approximate="tanh") @ T[p + "out.w"] + T[p + "out.b"]
    logits = ln(h, T["ln.w"], T["ln.b"]) @ T["head.w"]
    tl = torch.nn.functional.cross_entropy(logits.reshape(-1, 13), torch.tensor(y).reshape(-1))
    tl.backward()
    assert abs(float(loss) - tl.item()) < 1e-13
    for k in P:
        assert rel_err(G[k], T[k].grad.numpy()) < 1e-11, k


def test_adamw_matches_torch_adamw():
    """dtrain tests/test_torch_crosscheck.py:96-108: <= 1e-14 after 10 steps."""
    torch = pytest.importorskip("torch")
    r = np.random.default_rng(0)
    p0 = r.standard_normal(5000)
    pd, pt = p0.copy(), torch.from_numpy(p0.copy()).requires_grad_()
    od = optim.AdamW([pd], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    ot = torch.optim.AdamW([pt], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    for _ in range(10):
        g = r.standard_normal(p0.size) * 10.0 ** r.uniform(-6, 0, p0.size)
        od.step([g])
        pt.grad = torch.from_numpy(g.copy())
        ot.step()
    assert np.max(np.abs(pd - pt.detach().numpy())) <= 1e-14


def test_clip_scale_closed_form():
    assert optim.clip_scale(0.0, 1.0) == 1.0
    assert optim.clip_scale(0.25, 1.0) == 1.0
    assert optim.clip_scale(4.0, 1.0) == 1.0 / (2.0 + 1e-6)
    assert optim.clip_scale(1.0, 1.0) == 1.0


def test_fixed_order_sum_is_rank_order_and_w2_symmetric():
    a, b, c = (rng.standard_normal(1000) for _ in range(3))
    np.testing.assert_array_equal(fixed_order_sum([a, b, c]), (a + b) + c)
    np.testing.assert_array_equal(fixed_order_sum([a, b]), fixed_order_sum([b, a]))


def test_bucket_size_does_not_change_the_average():
    """dtrain tests/test_training.py:75-80: bucket size and grouping do not change results."""
    shapes = [(7, 3), (5,), (11, 4), (2,), (9, 9)]
    reps = [[rng.standard_normal(s) for s in shapes] for _ in range(4)]
    ref = ddp_average(reps, 8, 1e-9)
    for mb in (1e-5, 1e-3, 100.0):
        for a, b in zip(ddp_average(reps, 8, mb), ref):
            np.testing.assert_array_equal(a, b)
    for a, i in zip(ref, range(len(shapes))):
        np.testing.assert_array_equal(a, fixed_order_sum([r[i] for r in reps]) * 0.25)


def test_zero_shards_equal_full_adamw_and_state_bytes():
    shapes = [(13, 5), (7,), (31,)]
    params = [rng.standard_normal(s) for s in shapes]
    W = 4
    z = ZeroAdamW([p.copy() for p in params], W, max_grad_norm=1.0, lr=1e-2)
    n = sum(p.size for p in params)
    assert z.opts[0].state_bytes() == 2 * 8 * -(-n // W)  # dtrain tests/test_training.py:72
    flat_grads = [rng.standard_normal(n) for _ in range(W)]
    z.step(flat_grads)
    g = ring_order_sum(flat_grads)  # the reduce-scatter: shard r summed from rank r
    g *= 1.0 / W
    sq = 0.0
    for r in range(W):
        lo, hi = z.bounds[r], z.bounds[r + 1]
        sq += float(np.dot(g[lo:hi], g[lo:hi]))
    full = np.concatenate([p.reshape(-1) for p in params])
    opt = optim.AdamW([full], lr=1e-2)
    opt.step([g * optim.clip_scale(sq, 1.0)])
    np.testing.assert_array_equal(z.flat, full)


def test_ring_order_sum_brute_force():
    """Chunk c of partition(n, W) summed over ranks c, c+1, ..., c-1, written
    as an explicit loop per element."""
    for W, n in ((3, 10), (4, 7), (4, 2), (5, 23)):
        parts = [rng.standard_normal(n) * 10.0 ** rng.uniform(-8, 8, n) for _ in range(W)]
        got = ring_order_sum(parts)
        b = partition(n, W)
        for i in range(n):
            c = max(j for j in range(W) if b[j] <= i and b[j + 1] > i)
            acc = parts[c][i]
            for j in range(1, W):
                acc = acc + parts[(c + j) % W][i]
            assert got[i] == acc
        assert np.array_equal(ring_order_sum(parts[:2]), fixed_order_sum(parts[:2]))


def test_planted_mistake_in_ring_order_is_caught(golden):
    """A ring that starts every chunk at rank 0 (the direct order) fails
    dtrain's ring fixture."""
    G = golden("dtrain_ddp_reduce.npz")
    reps = [[G[f"w4/float64/g{r}/{i}"] for i in range(8)] for r in range(4)]
    got = ddp_average(reps, 8, 256 / (1 << 20), "direct")
    assert not all(np.array_equal(a, G[f"w4/float64/ddp_ring/{i}"]) for i, a in enumerate(got))


def test_partition_closed_form():
    for n in (0, 1, 5, 12345):
        for w in (1, 2, 3, 4, 7):
            b = partition(n, w)
            sizes = np.diff(b)
            assert b[0] == 0 and b[-1] == n and sizes.max() - sizes.min() <= 1
            assert list(sizes) == sorted(sizes, reverse=True)


def test_bucket_layout_closes_on_reaching_the_limit():
    lay = bucket_layout([10, 10, 10, 10], 8, 160 / (1 << 20))
    assert [[i for i, _, _ in b] for b in lay] == [[3, 2], [1, 0]]


# ---------------------------------------------------------- planted mistakes
def test_planted_mistake_in_layer_norm_backward_is_caught():
    def bad_bwd(g, cache, w):
        xh, rstd, _ = cache
        n = xh.shape[-1]
        gxh = g * w
        gx = rstd * (gxh - gxh.mean(-1, keepdims=True))  # dropped term
        return gx, (g * xh).reshape(-1, n).sum(0), g.reshape(-1, n).sum(0)

    def bwd(g, x, w, b):
        _, cache = ops.layer_norm_fwd(x, w, b)
        return bad_bwd(g, cache, w)
    with pytest.raises(AssertionError):
        check(lambda x, w, b: ops.layer_norm_fwd(x, w, b)[0], bwd, (2, 3, 6), (6,), (6,))


def test_planted_mistake_in_attention_backward_is_caught():
    def bwd(g, q, k, v):
        _, p, scale = ops.attention_fwd(q, k, v)
        gv = np.swapaxes(p, -1, -2) @ g
        gp = g @ np.swapaxes(v, -1, -2)
        gs = p * (gp - (gp * p).sum(-1, keepdims=True))  # missing * scale
        return gs @ k, np.swapaxes(gs, -1, -2) @ q, gv
    with pytest.raises(AssertionError):
        check(lambda q, k, v: ops.attention_fwd(q, k, v)[0], bwd, (1, 2, 4, 3), (1, 2, 4, 3), (1, 2, 4, 3))


def test_planted_mistake_in_adamw_order_is_caught(golden):
    """Swapping the decoupled weight decay after the Adam step changes float32 bits."""
    G = golden("dtrain_adamw_float32.npz")
    p = G["p0"].copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    b1t, b2t = optim.bias_corrections(0.9, 0.95, 1)
    g = G["g0"]
    m *= 0.9
    m += (1 - 0.9) * g
    v *= 0.95
    v += (1 - 0.95) * (g * g)
    p -= 1e-3 * (m / b1t) / (np.sqrt(v / b2t) + 1e-8)
    p -= 1e-3 * (0.1 * p)
    assert not np.array_equal(p, G["p1"])
