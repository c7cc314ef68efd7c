"""Parity at the GPT-2-small shape (12 layers, d_model 768, 12 heads, T 1024,
vocab 50304, float32), the configuration the headline throughput is measured
on, and the kernels at the shapes only that configuration reaches:

- the whole training step (dtrain/train.py:128-159 with --mode ddp): 4
  simulated replicas of one 1024-token sequence each through forward and
  backward, every replica's 149 gradient tensors and loss against the oracle
  (dtrain/nn.py:131-139, autograd.py), the bucketed average bit-exact on the
  device's own replica gradients in both of dtrain's all-reduce orders (ring
  and direct; ddp.py:84-110, comm.py:292-303, 342-391), the global norm and
  clip (train.py:155-158), and AdamW bit-exact on the averaged gradients
  (optim.py:21-33);
- one replica at the benchmark's 8 x 1024 tokens, forward and backward
  against the oracle;
- causal attention at (B, H, T, D) = (2, 12, 1024, 64) (autograd.py:226-247);
- cross entropy over 8192 x 50304 logits (autograd.py:250-266);
- the vocabulary head's forward, dX and dW at M = 8192, K/N = 50304
  (autograd.py:102-109).

Bar: float32 normwise relative error <= 1e-5 (float64 <= 1e-12); the average
and AdamW bit-exact.
"""
import numpy as np
import pytest

from helpers import bits_equal, rel_err
from oracle import model as OM, ops, optim as OO
from oracle.ddp import ddp_average, fixed_order_sum

pytestmark = pytest.mark.gpu

GPT2 = dict(vocab=50304, ctx=1024, dim=768, heads=12, layers=12)
TOL = {np.float32: 1e-5, np.float64: 1e-12}


def _api():
    from dtmi import ddp as P, device as D, kernels as K, nn as N, optim as O, replicas as R, train as S
    return D, K, N, O, P, R, S


def _split_rows(rows, names, shapes, offs):
    """A [W, n] gradient buffer back into per-replica lists of parameter arrays."""
    return [[rows[r, offs[i]:offs[i + 1]].reshape(shapes[k]) for i, k in enumerate(names)]
            for r in range(rows.shape[0])]


@pytest.mark.parametrize("algo", ["direct", "ring"])
def test_gpt2_small_ddp_step_matches_oracle(dev, algo):
    """One step of the headline workload at 1 sequence per replica, with each
    of dtrain's all-reduce orders (`--algo ring` is what the benchmark runs):
    loss and gradients of every replica within 1e-5 of the oracle; the
    51-bucket average (merged launches of adjacent buckets, up to 16 rank-order
    segments each) bit-exact to dtrain's DDP.finish restated over the device's
    own replica rows (ddp.py:84-110 with comm.py:292-303, 342-372 for ring,
    374-391 for direct); norm and clip factor within 1e-5; AdamW bit-exact on
    the averaged gradients."""
    D, K, N, O, P, R, S = _api()
    W = 4
    oc = OM.GPTConfig(dtype="float32", **GPT2)
    weights = OM.synthetic_init(oc, seed=5)
    xs, ys = OM.synthetic_tokens(oc, batch=1, seed=5, replicas=W)
    m = N.GPT(N.GPTConfig(dtype="float32", **GPT2), seed=5)
    m.load_numpy(weights)
    names = [n for n, _ in m.named_parameters()]
    assert len(names) == 149
    pg = R.SimGroup(W)
    ddp = P.DDP(m, pg, bucket_mb=1.0, overlap=True, algo=algo)
    assert len(ddp.buckets) == 51
    launches = []
    average = pg.average
    pg.average = lambda out, rows, **kw: (launches.append(kw.get("segments")), average(out, rows, **kw))
    lr = 3e-4
    opt = O.AdamW([p.data for p in m.parameters()], lr=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    res = S.step_ddp(m, ddp, opt, [[(xs[r], ys[r])] for r in range(W)], clip=1.0)
    rows = ddp.grads.rows.numpy()  # [W, n]: every replica's gradients, forward order
    avg_dev = ddp.avg.numpy()[:ddp.grads.n]
    p_dev = m.flat.numpy()
    # adjacent buckets share launches; the ring order gives several segments per launch
    assert 1 < len(launches) < 51
    if algo == "ring":
        assert max(len(s) for s in launches) > 4

    shapes = {k: weights[k].shape for k in names}
    offs = np.cumsum([0] + [weights[k].size for k in names])
    # the average of the device's own replica gradients: bit-exact to dtrain's
    # bucketed all-reduce in the chosen order, times 1/W
    dev_avg_ref = ddp_average(_split_rows(rows, names, shapes, offs), 4, 1.0, algo=algo)
    assert bits_equal(avg_dev, np.concatenate([a.reshape(-1) for a in dev_avg_ref]))
    del dev_avg_ref
    if algo == "ring":  # the ring order is not the rank order: some bits must differ
        assert not bits_equal(avg_dev, fixed_order_sum(list(rows)) * np.float32(0.25))

    losses, replica_grads = [], []
    for r in range(W):
        loss, G = OM.loss_and_grads(weights, oc, xs[r], ys[r])
        losses.append(float(loss))
        for i, k in enumerate(names):
            got = rows[r, offs[i]:offs[i + 1]]
            assert rel_err(got, G[k].reshape(-1)) <= 1e-5, (r, k)
        replica_grads.append([G[k] for k in names])
        del G
    ref_loss = sum(losses) / W
    assert abs(res.loss - ref_loss) <= 1e-5 * abs(ref_loss)

    # within tolerance of the oracle's average of its own gradients
    ref_avg = ddp_average(replica_grads, 4, 1.0, algo=algo)
    del replica_grads
    for i, k in enumerate(names):
        assert rel_err(avg_dev[offs[i]:offs[i + 1]], ref_avg[i].reshape(-1)) <= 1e-5, k
    sq_ref = OO.global_sq_norm(ref_avg)
    assert abs(res.grad_norm - np.sqrt(sq_ref)) <= 1e-5 * np.sqrt(sq_ref)
    # clip factor from the device's norm, dtrain's formula (optim.py:49-52)
    s = res.clip_scale
    assert s == OO.clip_scale(res.grad_norm ** 2, 1.0) or abs(s - OO.clip_scale(res.grad_norm ** 2, 1.0)) <= 1e-15
    assert abs(s - OO.clip_scale(sq_ref, 1.0)) <= 1e-5 * s
    # AdamW on the device's averaged gradients times its clip factor
    p_ref = np.concatenate([weights[k].reshape(-1) for k in names])
    opt_ref = OO.AdamW([p_ref], lr=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    opt_ref.step([avg_dev * s])
    assert bits_equal(p_dev, p_ref)


def test_gpt2_small_replica_at_8_sequences_matches_oracle(dev):
    """One replica at the benchmark's batch (8 x 1024 tokens, so every Linear
    runs at M = 8192 with the tile and split-K choices of the benchmark):
    forward and backward through the model, loss and all 149 gradients within
    1e-5 of the oracle."""
    D, K, N, O, P, R, S = _api()
    oc = OM.GPTConfig(dtype="float32", **GPT2)
    weights = OM.synthetic_init(oc, seed=5)
    xs, ys = OM.synthetic_tokens(oc, batch=8, seed=5, replicas=1)
    m = N.GPT(N.GPTConfig(dtype="float32", **GPT2), seed=5)
    m.load_numpy(weights)
    m.zero_grad()
    _, loss = m(xs[0], ys[0])
    loss.backward()
    got_loss = float(loss.numpy())
    got = {k: p.grad.numpy() for k, p in m.named_parameters()}
    del m, loss
    ref_loss, G = OM.loss_and_grads(weights, oc, xs[0], ys[0])
    assert abs(got_loss - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    assert len(got) == 149
    for k, g in got.items():
        assert rel_err(g, G[k]) <= 1e-5, k


@pytest.mark.parametrize("dt,B", [(np.float32, 2), (np.float64, 1)])
def test_attention_at_gpt2_small_shape(dev, dt, B):
    """(B, 12, 1024, 64): the aligned path with the longest-first block order,
    forward and backward against the oracle."""
    D, K = _api()[:2]
    shape = (B, 12, 1024, 64)
    rng = np.random.default_rng(1024 + B)
    q, k, v, g = (rng.standard_normal(shape).astype(dt) for _ in range(4))
    o_ref, p, scale = ops.attention_fwd(q, k, v)
    gq, gk, gv = ops.attention_bwd(g, q, k, v, p, scale)
    del p
    dq_, dk_, dv_ = D.from_numpy(q), D.from_numpy(k), D.from_numpy(v)
    o, rmax, rsum = K.attn_fwd(dq_, dk_, dv_)
    assert rel_err(o.numpy(), o_ref) <= TOL[dt]
    got = K.attn_bwd(dq_, dk_, dv_, o, D.from_numpy(g), rmax, rsum)
    for a, ref, name in zip(got, (gq, gk, gv), "qkv"):
        assert rel_err(a.numpy(), ref) <= TOL[dt], name


def test_cross_entropy_at_gpt2_small_shape(dev):
    """8192 rows of 50304 float32 logits: the single-pass training kernel
    (loss and the gradient for an upstream gradient of 1, then rescaled by a
    loss scale) and the forward-only kernel, against the oracle."""
    D, K = _api()[:2]
    rng = np.random.default_rng(50304)
    rows, V = 8192, 50304
    z = (rng.standard_normal((rows, V), dtype=np.float32) * np.float32(2.0))
    t = rng.integers(0, V, rows)
    ref_loss, cache = ops.cross_entropy_fwd(z, t)
    ref_g = ops.cross_entropy_bwd(np.float32(0.25), z, t, cache)
    del cache
    dz = D.from_numpy(z)
    dt_ = D.from_numpy(t.astype(np.int64))
    loss, rmax, rsum, grad = K.xent_fused(dz, dt_)
    assert rel_err(loss.numpy(), ref_loss) <= 1e-5
    K.xent_grad_scale(grad, D.from_numpy(np.array([0.25], np.float32)))
    assert rel_err(grad.numpy(), ref_g) <= 1e-5
    del grad
    loss2, rmax2, rsum2 = K.xent_fwd(dz, dt_)
    assert rel_err(loss2.numpy(), ref_loss) <= 1e-5
    # the forward-only kernel's row statistics drive the unfused backward
    g2 = K.xent_bwd(dz, dt_, rmax2, rsum2, g_host=0.25)
    assert rel_err(g2.numpy(), ref_g) <= 1e-5


def test_vocabulary_head_gemms_at_gpt2_small_shape(dev):
    """logits = h @ W (K = 768), dX = dY @ W^T (K = 50304), dW = h^T @ dY
    (K = 8192) with h [8192, 768], W [768, 50304]: the 256 x 128 tile path
    with long k ranges, against the oracle's float32 products."""
    D, K = _api()[:2]
    rng = np.random.default_rng(8192)
    M, C, V = 8192, 768, 50304
    h = rng.standard_normal((M, C), dtype=np.float32)
    w = rng.standard_normal((C, V), dtype=np.float32) * np.float32(0.02)
    dy = rng.standard_normal((M, V), dtype=np.float32) * np.float32(1e-4)
    dh, dw_, ddy = D.from_numpy(h), D.from_numpy(w), D.from_numpy(dy)
    y = K.linear_fwd(dh, dw_, None)
    assert rel_err(y.numpy(), h @ w) <= 1e-5
    del y
    dx, dw, db = K.linear_bwd(dh, dw_, ddy, need_db=False)
    gx, gw = ops.matmul_bwd(dy, h, w)
    assert rel_err(dx.numpy(), gx) <= 1e-5
    assert rel_err(dw.numpy(), gw) <= 1e-5


def test_layernorm_backward_taking_split_k_partials_changes_no_bit(dev):
    """8 x 1024 tokens at GPT-2 width (2 layers, vocabulary 65): the qkv and fc
    input gradients split in two and handed to the LayerNorm backwards as
    partials give every parameter gradient and the loss bit for bit as
    summing the partials first."""
    D, K, N, O, P, R, S = _api()
    cfg = dict(vocab=65, ctx=1024, dim=768, heads=12, layers=2)
    oc = OM.GPTConfig(dtype="float32", **cfg)
    weights = OM.synthetic_init(oc, seed=7)
    xs, ys = OM.synthetic_tokens(oc, batch=8, seed=7, replicas=1)
    out = {}
    for split in (True, False):
        N.LN_SPLIT_SUM = split
        try:
            m = N.GPT(N.GPTConfig(dtype="float32", **cfg), seed=7)
            m.load_numpy(weights)
            m.zero_grad()
            _, loss = m(xs[0], ys[0])
            loss.backward()
            out[split] = (loss.numpy(), [p.grad.numpy() for p in m.parameters()])
        finally:
            N.LN_SPLIT_SUM = True
    assert bits_equal(out[True][0], out[False][0])
    for a, b in zip(out[True][1], out[False][1]):
        assert bits_equal(a, b)


def test_split_k_partials_reaching_a_layernorm_output_read_twice(dev, monkeypatch):
    """A LayerNorm output read by two Linears at GPT-2 width (8192 x 768 rows;
    the qkv- and fc-shaped products split their input gradients in two): each
    product hands its dX over as split-K partials, the backward engine forms
    their values to add the two gradients in its own order, and the LayerNorm
    backward then takes a plain dy. Every gradient, the leaf input's
    included, is bit for bit the path that sums the partials inside the
    products."""
    D, K, N, O, P, R, S = _api()
    from dtmi.autograd import Tensor
    rng = np.random.default_rng(11)
    M, C = 8192, 768
    hx = rng.standard_normal((M, C)).astype(np.float32)
    c1 = rng.standard_normal((M, 3 * C)).astype(np.float32)
    c2 = rng.standard_normal((M, 4 * C)).astype(np.float32)
    formed = []
    value = K.SplitSum.value
    monkeypatch.setattr(K.SplitSum, "value", lambda self: formed.append(self.n) or value(self))
    out = {}
    for split in (True, False):
        N.LN_SPLIT_SUM = split
        try:
            wr = np.random.default_rng(12)
            ln, l1, l2 = N.LayerNorm(C), N.Linear(C, 3 * C, wr), N.Linear(C, 4 * C, wr)
            x = Tensor(D.from_numpy(hx), requires_grad=True)
            h = ln(x)
            loss = (l1(h) * Tensor(D.from_numpy(c1))).sum() + (l2(h) * Tensor(D.from_numpy(c2))).sum()
            loss.backward()
            out[split] = [t.grad.numpy() for t in (x, ln.w, ln.b, l1.w, l1.b, l2.w, l2.b)]
        finally:
            N.LN_SPLIT_SUM = True
        if split:
            assert formed == [2, 2]  # both products split, both partial sets formed once
            formed.clear()
    assert not formed
    for a, b in zip(out[True], out[False]):
        assert bits_equal(a, b)
