"""Pins for the oracle functions that no golden vector covers directly (CPU):

- ops.softmax_bwd (the softmax backward inside dtrain/autograd.py:242): finite
  differences of sum(w * softmax(z)), and bit-equality with the term inside the
  golden-pinned attention backward when it is used in its place;
- ops.row_stats (the row max and row sum of the masked, scaled scores of
  dtrain/autograd.py:231-236): brute-force loops, and p = exp(s - m) / l
  against the golden-pinned attention forward;
- step.ddp_step (dtrain/ddp.py:84-110 with train.py:155-163): W = 1 equals the
  single-process step bit for bit, DDP(4) equals --emulate-world 4 to 1e-10
  (dtrain tests/test_training.py:57-62), the bucket size changes no bit
  (test_training.py:75-80).

Each check is shown to fail on a planted mistake in a copy of the function.
"""
import numpy as np
import pytest

from oracle import model, ops, optim, step
from oracle.ddp import ddp_average

rng = np.random.default_rng(17)


def fd(f, x, eps=1e-6):
    num = np.zeros_like(x)
    for i in np.ndindex(x.shape):
        old = x[i]
        x[i] = old + eps
        fp = f(x)
        x[i] = old - eps
        fm = f(x)
        x[i] = old
        num[i] = (fp - fm) / (2 * eps)
    return num


def softmax(z):
    e = np.exp(z - z.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


# ------------------------------------------------------------- softmax_bwd
def _softmax_fd_check(bwd):
    z = rng.standard_normal((3, 7))
    w = rng.standard_normal((3, 7))
    analytic = bwd(softmax(z), w)
    numeric = fd(lambda zz: float((softmax(zz) * w).sum()), z)
    np.testing.assert_allclose(analytic, numeric, rtol=1e-6, atol=1e-8)


def test_softmax_bwd_finite_differences():
    _softmax_fd_check(ops.softmax_bwd)


def test_softmax_bwd_with_masked_entries_finite_differences():
    """Causal rows: -inf scores give p = 0, and their dS is exactly 0."""
    z = rng.standard_normal((5, 5))
    mask = np.triu(np.ones((5, 5), bool), 1)
    w = rng.standard_normal((5, 5))

    def f(zz):
        return float((softmax(np.where(mask, -np.inf, zz)) * w).sum())
    ds = ops.softmax_bwd(softmax(np.where(mask, -np.inf, z)), w)
    assert np.all(ds[mask] == 0.0)
    num = fd(f, z)
    np.testing.assert_allclose(ds, num, rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("dt", ["float32", "float64"])
def test_softmax_bwd_reproduces_dtrains_attention_backward_bits(golden, dt):
    """dtrain's attention backward with its inline softmax backward replaced by
    ops.softmax_bwd gives dtrain's golden dQ and dK bit for bit."""
    G = golden("dtrain_attention.npz")
    q, k, v, g = (G[f"{dt}/{s}"] for s in "qkvg")
    _, p, scale = ops.attention_fwd(q, k, v)
    gp = g @ np.swapaxes(v, -1, -2)
    gs = ops.softmax_bwd(p, gp)
    gs *= scale
    # float32 inputs give float64 gradients under NumPy 2 (np.float64 scale)
    assert (gs @ k).tobytes() == G[f"{dt}/gq"].tobytes()
    assert (np.swapaxes(gs, -1, -2) @ q).tobytes() == G[f"{dt}/gk"].tobytes()


def test_planted_mistake_in_softmax_bwd_is_caught():
    def wrong_axis(p, dp):
        return p * (dp - (dp * p).sum(-2, keepdims=True))

    def dropped_factor(p, dp):
        return dp - (dp * p).sum(-1, keepdims=True)
    for bad in (wrong_axis, dropped_factor):
        with pytest.raises(AssertionError):
            _softmax_fd_check(bad)


# --------------------------------------------------------------- row_stats
def _brute_row_stats(q, k):
    B, H, T, D = q.shape
    m = np.zeros((B, H, T))
    l = np.zeros((B, H, T))
    for b in range(B):
        for h in range(H):
            for i in range(T):
                s = [sum(q[b, h, i, d] * k[b, h, j, d] for d in range(D)) / np.sqrt(D) for j in range(i + 1)]
                m[b, h, i] = max(s)
                l[b, h, i] = sum(np.exp(x - m[b, h, i]) for x in s)
    return m, l


def _row_stats_check(fn):
    q, k = (rng.standard_normal((2, 2, 6, 3)) for _ in range(2))
    m, l = fn(q, k)
    bm, bl = _brute_row_stats(q, k)
    np.testing.assert_allclose(m, bm, rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(l, bl, rtol=1e-13, atol=1e-14)


def test_row_stats_brute_force():
    _row_stats_check(ops.row_stats)


@pytest.mark.parametrize("dt", ["float32", "float64"])
def test_row_stats_reproduce_the_golden_pinned_probabilities(golden, dt):
    """exp(s - m) / l over the visible keys is the attention forward's p, whose
    output p @ v is dtrain's golden o (to its float32 rounding)."""
    G = golden("dtrain_attention.npz")
    q, k, v = (G[f"{dt}/{s}"] for s in "qkv")
    o, p, scale = ops.attention_fwd(q, k, v)
    assert o.tobytes() == G[f"{dt}/o"].tobytes()
    m, l = ops.row_stats(q, k)
    T = q.shape[-2]
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
    np.testing.assert_allclose(np.exp(s - m[..., None]) / l[..., None], p, rtol=1e-14, atol=1e-16)


def test_planted_mistake_in_row_stats_is_caught():
    def unmasked(q, k):
        s = (q @ np.swapaxes(k, -1, -2)) / np.sqrt(q.shape[-1])
        m = s.max(-1)
        return m, np.exp(s - m[..., None]).sum(-1)

    def unscaled(q, k):
        T = q.shape[-2]
        s = q @ np.swapaxes(k, -1, -2)
        s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
        m = s.max(-1)
        return m, np.exp(s - m[..., None]).sum(-1)
    for bad in (unmasked, unscaled):
        with pytest.raises(AssertionError):
            _row_stats_check(bad)


# ---------------------------------------------------------------- ddp_step
CFG = dict(vocab=17, ctx=8, dim=16, heads=2, layers=2, dtype="float64")


def _setup(W, seed=3):
    c = model.GPTConfig(**CFG)
    P = model.dtrain_init(c, seed=seed)
    xs, ys = model.synthetic_tokens(c, batch=2, seed=seed + 1, replicas=W)
    return c, P, [(xs[r], ys[r]) for r in range(W)]


def _copy(P):
    return {k: v.copy() for k, v in P.items()}


def test_ddp_step_world_1_equals_single_step_bits():
    c, P, batches = _setup(1)
    Pa, Pb = _copy(P), _copy(P)
    la, na, ga = step.ddp_step(Pa, c, batches, optim.AdamW(list(Pa.values()), lr=1e-2), clip=0.5)
    lb, nb, gb = step.single_step(Pb, c, batches, optim.AdamW(list(Pb.values()), lr=1e-2), clip=0.5)
    assert la == lb and na == nb
    for k in P:
        assert Pa[k].tobytes() == Pb[k].tobytes(), k
    for a, b in zip(ga, gb):
        assert a.tobytes() == b.tobytes()


def _emulate_world_check(ddp_fn, W=4, steps=3):
    """dtrain tests/test_training.py:57-62: DDP over W ranks and one process
    emulating W ranks reach the same parameters to 1e-10."""
    c, P, batches = _setup(W)
    Pa, Pb = _copy(P), _copy(P)
    oa = optim.AdamW(list(Pa.values()), lr=3e-3)
    ob = optim.AdamW(list(Pb.values()), lr=3e-3)
    for _ in range(steps):
        la, _, _ = ddp_fn(Pa, c, batches, oa, clip=1.0)
        lb, _, _ = step.single_step(Pb, c, batches, ob, clip=1.0, emulate_world=W)
        assert abs(la - lb) <= 1e-12 * abs(lb)
    for k in P:
        assert np.max(np.abs(Pa[k] - Pb[k])) <= 1e-10, k


def test_ddp_step_equals_emulated_world():
    _emulate_world_check(step.ddp_step)


def test_ddp_step_bucket_size_changes_no_bit():
    c, P, batches = _setup(4, seed=7)
    finals = []
    for mb in (1e-4, 1.0, 100.0):
        Pk = _copy(P)
        opt = optim.AdamW(list(Pk.values()), lr=1e-2)
        for _ in range(2):
            step.ddp_step(Pk, c, batches, opt, clip=0.5, bucket_mb=mb)
        finals.append(np.concatenate([v.reshape(-1) for v in Pk.values()]))
    assert finals[0].tobytes() == finals[1].tobytes() == finals[2].tobytes()


def test_planted_mistake_in_ddp_step_is_caught():
    """A sum without the 1/W of ddp.py:104-106, or the clip applied per
    replica, fails the emulated-world equivalence."""
    def no_average(P, c, batches, opt, clip=1.0, bucket_mb=1.0):
        names = list(P)
        W = len(batches)
        reps, losses = [], []
        for x, y in batches:
            loss, g = model.loss_and_grads(P, c, x, y)
            reps.append([g[k] for k in names])
            losses.append(float(loss))
        avg = ddp_average(reps, 8, bucket_mb)
        avg = [a * W for a in avg]  # the average left as a sum
        sq = optim.global_sq_norm(avg)
        opt.step([a * optim.clip_scale(sq, clip) for a in avg])
        return sum(losses) / W, float(np.sqrt(sq)), avg

    def loss_unscaled(P, c, batches, opt, clip=1.0, bucket_mb=1.0):
        # each replica's gradient of the summed (not mean) batch loss
        names = list(P)
        W = len(batches)
        reps, losses = [], []
        for x, y in batches:
            loss, g = model.loss_and_grads(P, c, x, y, loss_scale=float(x.size))
            reps.append([g[k] for k in names])
            losses.append(float(loss))
        avg = ddp_average(reps, 8, bucket_mb)
        sq = optim.global_sq_norm(avg)
        opt.step([a * optim.clip_scale(sq, clip) for a in avg])
        return sum(losses) / W, float(np.sqrt(sq)), avg
    for bad in (no_average, loss_unscaled):
        with pytest.raises(AssertionError):
            _emulate_world_check(bad, steps=1)
