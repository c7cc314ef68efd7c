"""The float32 GEMM in its split-bf16 arithmetic ("bf16x6": each operand split
exactly into three bf16 parts, the six largest partial products on the bf16
MFMA, float32 accumulation) against the oracle, at the float32 bar (normwise
relative error <= 1e-5), plus a tighter bound that only holds when all six
partial products are present (dropping the three second-order ones leaves an
error near 2^-16, about 4e-6 on these inputs; the full six give ~2e-7)."""
import numpy as np
import pytest

from helpers import bits_equal, rel_err
from oracle import ops

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _dev():
    from dtmi import device as D, kernels as K
    return D, K


@pytest.fixture
def x6(dev):
    from dtmi import _lib
    with _lib.use_gemm_math("bf16x6"):
        yield


def _ref(a, b, akc, bkc):
    A = a if akc else np.swapaxes(a, -1, -2)
    B = b if not bkc else np.swapaxes(b, -1, -2)
    return A.astype(np.float64) @ B.astype(np.float64)


def test_mode_switch_round_trips(dev):
    import os
    from dtmi import _lib
    start = _lib.gemm_math()
    assert start == os.environ.get("DTMI_GEMM_MATH", "f32")
    for mode in ("bf16x6", "f32"):
        with _lib.use_gemm_math(mode):
            assert _lib.gemm_math() == mode
        assert _lib.gemm_math() == start
    with pytest.raises(ValueError):
        _lib.set_gemm_math("tf32")


@pytest.mark.parametrize("akc,bkc", [(True, False), (True, True), (False, False), (False, True)])
@pytest.mark.parametrize("M,N,K", [(256, 192, 64), (300, 68, 64), (132, 68, 36), (260, 132, 1000), (4, 4, 4),
                                   (512, 2304, 768), (2000, 2040, 2052), (128, 128, 16), (8, 12, 20)])
def test_layouts_ragged_edges_and_k_tails(x6, akc, bkc, M, N, K):
    D, K_ = _dev()
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    a = rng.standard_normal((M, K) if akc else (K, M)).astype(np.float32)
    b = rng.standard_normal((N, K) if bkc else (K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    ref = _ref(a, b, akc, bkc) + bias
    got = K_.gemm(D.from_numpy(a), D.from_numpy(b), a_kcontig=akc, b_kcontig=bkc, bias=D.from_numpy(bias)).numpy()
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("akc,bkc", [(True, False), (True, True), (False, False)])
def test_all_six_partial_products_are_present(x6, akc, bkc):
    D, K_ = _dev()
    rng = np.random.default_rng(5)
    M, N, K = 512, 384, 768
    a = rng.standard_normal((M, K) if akc else (K, M)).astype(np.float32)
    b = rng.standard_normal((N, K) if bkc else (K, N)).astype(np.float32)
    got = K_.gemm(D.from_numpy(a), D.from_numpy(b), a_kcontig=akc, b_kcontig=bkc).numpy()
    assert rel_err(got, _ref(a, b, akc, bkc)) <= 1e-6


def test_exact_on_integer_operands(x6):
    """Small integers split into one bf16 part and products/sums stay exact."""
    D, K_ = _dev()
    rng = np.random.default_rng(6)
    a = rng.integers(-8, 9, size=(256, 512)).astype(np.float32)
    b = rng.integers(-8, 9, size=(512, 192)).astype(np.float32)
    got = K_.gemm(D.from_numpy(a), D.from_numpy(b)).numpy()
    assert np.array_equal(got, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


def test_wide_dynamic_range(x6):
    """Operands spanning 1e-20 .. 1e20 (rows scaled): the split is exact at any
    exponent, so the relative error stays at the float32 bar."""
    D, K_ = _dev()
    rng = np.random.default_rng(7)
    a = rng.standard_normal((256, 768)) * (10.0 ** rng.uniform(-20, 20, size=(256, 1)))
    b = rng.standard_normal((768, 256))
    a, b = a.astype(np.float32), b.astype(np.float32)
    got = K_.gemm(D.from_numpy(a), D.from_numpy(b)).numpy()
    ref = _ref(a, b, True, False)
    row_err = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert row_err.max() <= TOL


@pytest.mark.parametrize("akc,bkc", [(True, False), (False, False), (True, True)])
def test_split_k_deterministic_with_partial_last_tile(x6, akc, bkc):
    D, K_ = _dev()
    rng = np.random.default_rng(13)
    M, N, K = 200, 132, 1000
    a = rng.standard_normal((M, K) if akc else (K, M)).astype(np.float32)
    b = rng.standard_normal((N, K) if bkc else (K, N)).astype(np.float32)
    ref = _ref(a, b, akc, bkc)
    outs = [K_.gemm(D.from_numpy(a), D.from_numpy(b), a_kcontig=akc, b_kcontig=bkc, splits=s).numpy()
            for s in (1, 3, 3, 0)]
    for o in outs:
        assert rel_err(o, ref) <= TOL
    assert bits_equal(outs[1], outs[2])


def test_batched(x6):
    D, K_ = _dev()
    rng = np.random.default_rng(12)
    a = rng.standard_normal((3, 200, 96)).astype(np.float32)
    b = rng.standard_normal((3, 96, 136)).astype(np.float32)
    got = K_.gemm(D.from_numpy(a), D.from_numpy(b)).numpy()
    assert rel_err(got, a.astype(np.float64) @ b.astype(np.float64)) <= TOL


def test_linear_backward_with_bias_gradient(x6):
    """dX, dW and db (the column sums taken inside the dW GEMM) of the
    LayerNorm + Linear workload shape x [16384, 768] -> [16384, 3072]."""
    D, K = _dev()
    rng = np.random.default_rng(2)
    M, Cin, N = 16384, 768, 3072
    h = rng.standard_normal((M, Cin)).astype(np.float32)
    W = (rng.standard_normal((Cin, N)) * 0.02).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    gh, gW = ops.matmul_bwd(dY, h, W)
    gb = ops.unbroadcast(dY, (N,))
    hd, Wd = D.from_numpy(h), D.from_numpy(W)
    y = K.linear_fwd(hd, Wd, D.from_numpy(b))
    assert rel_err(y.numpy(), h.astype(np.float64) @ W + b) <= TOL
    dh, dW, db = K.linear_bwd(hd, Wd, D.from_numpy(dY))
    assert rel_err(dh.numpy(), gh) <= TOL
    assert rel_err(dW.numpy(), gW) <= TOL
    assert rel_err(db.numpy(), gb) <= TOL


@pytest.mark.parametrize("M,K,N", [(1024, 256, 512), (300, 68, 132), (4096, 1024, 2048)])
def test_fused_epilogues_equal_the_unfused_ops(x6, M, K, N):
    D, K_ = _dev()
    rng = np.random.default_rng(M + K + N)
    x = D.from_numpy(rng.standard_normal((M, K)).astype(np.float32))
    w = D.from_numpy((rng.standard_normal((K, N)) * 0.05).astype(np.float32))
    b = D.from_numpy(rng.standard_normal(N).astype(np.float32))
    r = D.from_numpy(rng.standard_normal((M, N)).astype(np.float32))
    y0 = K_.linear_fwd(x, w, b)
    y_res, _ = K_.linear_fwd_fused(x, w, b, residual=r)
    assert bits_equal(y_res.numpy(), K_.binary("add", r, y0).numpy())
    h, act = K_.linear_fwd_fused(x, w, b, gelu=True)
    assert bits_equal(h.numpy(), y0.numpy())
    assert bits_equal(act.numpy(), K_.gelu_fwd(y0).numpy())
    pre = D.from_numpy(rng.standard_normal((M, K)).astype(np.float32))
    g = D.from_numpy(rng.standard_normal((M, N)).astype(np.float32))
    dx_plain, _, _ = K_.linear_bwd(x, w, g, need_db=False)
    dx_fused, _, _ = K_.linear_bwd(x, w, g, need_db=False, gelu_pre=pre)
    assert bits_equal(dx_fused.numpy(), K_.gelu_bwd(pre, dx_plain).numpy())
    ref = (x.numpy().astype(np.float64) @ w.numpy().astype(np.float64)) + b.numpy() + r.numpy()
    assert rel_err(y_res.numpy(), ref) <= TOL


@pytest.mark.parametrize("dt", [np.float32])
def test_full_model_gradients_under_bf16x6(x6, dt):
    import test_gpu_api as T
    T.test_full_model_gradients_match_oracle(None, dt)


def test_two_training_steps_match_dtrain_golden_under_bf16x6(x6, golden):
    import test_gpu_api as T
    T.test_two_training_steps_match_dtrain_golden(None, golden, "float32")
