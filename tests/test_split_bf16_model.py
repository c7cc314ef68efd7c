"""CPU model of the split-bf16 float32 GEMM arithmetic (the GPU kernel's
DTMI_GEMM_MATH_BF16X6): each float32 operand split exactly into three bf16
parts (round-to-nearest-even at each step), the partial products a_i*b_j
exact, summed in float32. Pins the claims the kernel relies on: the split is
exact, six products (i + j <= 2) are as accurate as a float32 product, and
three are not."""
import numpy as np


def _bf16_rne(x):
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def _split(x):
    x0 = _bf16_rne(x)
    r1 = (x - x0).astype(np.float32)
    x1 = _bf16_rne(r1)
    x2 = _bf16_rne((r1 - x1).astype(np.float32))
    return x0, x1, x2


def _gemm(a, b, terms):
    pa, pb = _split(a), _split(b)
    acc = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for i, j in sorted(terms, key=lambda t: -(t[0] + t[1])):  # smallest first
        acc = (acc + (pa[i].astype(np.float64) @ pb[j].astype(np.float64)).astype(np.float32)).astype(np.float32)
    return acc.astype(np.float64)


def _rel(x, ref):
    return np.linalg.norm(x - ref) / np.linalg.norm(ref)


def test_split_is_exact_and_parts_are_bf16():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(100000) * 10.0 ** rng.uniform(-30, 30, 100000)).astype(np.float32)
    p = _split(x)
    assert np.array_equal((p[0].astype(np.float64) + p[1] + p[2]), x.astype(np.float64))
    for part in p:  # representable in bf16: low 16 bits zero
        assert not np.any(part.view(np.uint32) & 0xFFFF)
    # |x1| <= 2^-8 |x|, |x2| <= 2^-16 |x|
    ax = np.abs(x.astype(np.float64))
    assert np.all(np.abs(p[1]) <= ax * 2.0 ** -8) and np.all(np.abs(p[2]) <= ax * 2.0 ** -16)


def test_six_products_match_float32_accuracy_three_do_not():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((96, 768)).astype(np.float32)
    b = rng.standard_normal((768, 80)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    e32 = _rel((a @ b).astype(np.float64), ref)
    six = [(0, 0), (0, 1), (1, 0), (0, 2), (1, 1), (2, 0)]
    e6 = _rel(_gemm(a, b, six), ref)
    e9 = _rel(_gemm(a, b, [(i, j) for i in range(3) for j in range(3)]), ref)
    e3 = _rel(_gemm(a, b, [(0, 0), (0, 1), (1, 0)]), ref)
    assert e6 <= 2 * e32 and e6 <= 1.5 * e9
    assert e6 <= 1e-6 < e3  # the bound the GPU test uses to detect a missing product
