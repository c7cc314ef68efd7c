"""Host-side logic of the dtmi package that needs no GPU: DDP bucket layout,
ZeRO partition, the learning-rate schedule and the parameter order/init of
the model definition (checked without touching the device)."""
import numpy as np

from dtmi.ddp import bucket_layout
from dtmi.replicas import partition
from dtmi.train import lr_at
from oracle import model as OM


def test_bucket_layout_matches_dtrain(golden):
    G = golden("dtrain_layout.npz")
    for tag, cfg in (("charGPT", OM.GPTConfig(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64")),
                     ("gpt2small", OM.GPTConfig(vocab=50304, ctx=1024, dim=768, heads=12, layers=12,
                                                dtype="float32"))):
        sizes = [int(np.prod(s)) for _, s in OM.param_spec(cfg)]
        rows = []
        for bi, idx in enumerate(bucket_layout(sizes, np.dtype(cfg.dtype).itemsize, 1.0)):
            off = 0
            for i in idx:
                rows.append((bi, i, off, sizes[i]))
                off += sizes[i]
        assert np.array_equal(np.array(rows, dtype=np.int64), G[f"{tag}/layout"])


def test_partition_matches_dtrain(golden):
    for row in golden("dtrain_layout.npz")["partition"]:
        n, w = int(row[0]), int(row[1])
        assert partition(n, w) == [int(x) for x in row[2:3 + w]]


def test_lr_schedule_closed_form():
    lr = 1e-3
    assert lr_at(0, lr, 0, 100) == lr
    assert lr_at(0, lr, 4, 100) == lr * 1 / 4
    assert lr_at(3, lr, 4, 100) == lr
    assert abs(lr_at(4, lr, 4, 100) - lr) < 1e-18          # cosine starts at lr
    assert abs(lr_at(100, lr, 4, 100) - 0.1 * lr) < 1e-18  # and ends at lr / 10
    mid = lr_at(52, lr, 4, 100)
    assert abs(mid - lr * (0.1 + 0.9 * 0.5)) < 1e-15


def test_model_parameter_order_matches_dtrain_names():
    """dtmi.nn builds its modules in dtrain's attribute order; the names it
    reports follow from the class structure alone."""
    import dtmi.nn as N
    assert [f.name for f in N.GPTConfig.__dataclass_fields__.values()] == \
        ["vocab", "ctx", "dim", "heads", "layers", "dtype"]
    assert list(N.Block.__init__.__code__.co_names).index("ln1") < list(N.Block.__init__.__code__.co_names).index("qkv")


def _segmented_average(rows, segs, W):
    """What dtmi_bucket_average_ring computes, element by element on the host:
    element i summed starting at the first rank of its segment."""
    n = rows.shape[1]
    starts = [s for s, _ in segs] + [n]
    out = np.empty(n, rows.dtype)
    for j, (s, f) in enumerate(segs):
        for i in range(s, starts[j + 1]):
            acc = rows[f, i]
            for r in range(1, W):
                acc = acc + rows[(f + r) % W, i]
            out[i] = acc
    return out * rows.dtype.type(1.0 / W)


def test_ring_segments_reproduce_dtrains_ring_buckets(golden):
    """The segments of every bucket, applied to the forward-order layout, give
    dtrain's DDP ring average bit for bit (its own fixture: 3 and 4 ranks,
    256-byte buckets)."""
    from dtmi.replicas import ring_segments
    G = golden("dtrain_ddp_reduce.npz")
    shapes = [(7, 5), (3,), (13, 4), (1,), (33,), (6, 6), (2,), (41,)]
    sizes = [int(np.prod(s)) for s in shapes]
    offs = np.cumsum([0] + sizes)
    for W in (3, 4):
        for dt in ("float64", "float32"):
            reps = np.stack([np.concatenate([G[f"w{W}/{dt}/g{r}/{i}"].reshape(-1) for i in range(len(shapes))])
                             for r in range(W)])
            for idx in bucket_layout(sizes, np.dtype(dt).itemsize, 256 / (1 << 20)):
                fwd = sorted(idx)
                lo, hi = offs[fwd[0]], offs[fwd[-1] + 1]
                segs = ring_segments([sizes[i] for i in fwd], W)
                assert [s for s, _ in segs] == sorted(s for s, _ in segs) and segs[0][0] == 0
                got = _segmented_average(reps[:, lo:hi], segs, W)
                for i in fwd:
                    ref = G[f"w{W}/{dt}/ddp_ring/{i}"].reshape(-1)
                    assert got[offs[i] - lo:offs[i + 1] - lo].tobytes() == ref.tobytes(), (W, dt, i)


def test_ring_segments_cover_gpt2_small_buckets():
    """At the GPT-2-small layout (51 buckets, 4 ranks) every bucket needs at
    most a few segments, all within one launch (16 per launch)."""
    from dtmi.replicas import ring_segments
    cfg = OM.GPTConfig(vocab=50304, ctx=1024, dim=768, heads=12, layers=12, dtype="float32")
    sizes = [int(np.prod(s)) for _, s in OM.param_spec(cfg)]
    for idx in bucket_layout(sizes, 4, 1.0):
        segs = ring_segments([sizes[i] for i in sorted(idx)], 4)
        assert 1 <= len(segs) <= 16
        assert {f for _, f in segs} <= {0, 1, 2, 3}


def test_benchmark_inputs_equal_the_oracles():
    """bench.py draws its weights and tokens with dtmi.workload; they are the
    oracle's synthetic inputs bit for bit (one source of truth for both)."""
    from dtmi import workload as Wk
    from dtmi.nn import GPTConfig
    for cfg in (dict(vocab=65, ctx=32, dim=64, heads=4, layers=2, dtype="float64"),
                dict(vocab=50304, ctx=16, dim=48, heads=4, layers=2, dtype="float32")):
        c, oc = GPTConfig(**cfg), OM.GPTConfig(**cfg)
        assert Wk.param_spec(c) == OM.param_spec(oc)
        a, b = Wk.synthetic_weights(c, 5), OM.synthetic_init(oc, seed=5)
        assert list(a) == list(b)
        for k in a:
            assert a[k].dtype == b[k].dtype and a[k].tobytes() == b[k].tobytes(), k
        xa, ya = Wk.synthetic_tokens(c, 3, 7, 4)
        xb, yb = OM.synthetic_tokens(oc, batch=3, seed=7, replicas=4)
        for u, v in zip(xa + ya, xb + yb):
            assert np.array_equal(u, v)
    gpt2 = GPTConfig(vocab=50304, ctx=1024, dim=768, heads=12, layers=12)
    assert sum(int(np.prod(s)) for _, s in Wk.param_spec(gpt2)) == 163_109_376


def test_split_k_partials_offered_to_the_layernorm_backward():
    """The product reading a LayerNorm output leaves at most as many split-K
    partials of dx as the LayerNorm backward adds in its row loads (four
    for rows of up to 4 16-byte vectors per lane, two up to 8, else none)."""
    from dtmi.kernels import ln_fusable_parts
    assert ln_fusable_parts(np.float32, 768) == 4  # GPT-2: 3 vectors per lane
    assert ln_fusable_parts(np.float32, 1024) == 4
    assert ln_fusable_parts(np.float32, 1028) == 2
    assert ln_fusable_parts(np.float32, 2048) == 2
    assert ln_fusable_parts(np.float32, 2052) == 0
    assert ln_fusable_parts(np.float32, 770) == 0  # rows not in 16-byte vectors
    assert ln_fusable_parts(np.float64, 768) == 2  # 6 vectors per lane
    assert ln_fusable_parts(np.float64, 512) == 4
    assert ln_fusable_parts(np.float64, 1025) == 0
