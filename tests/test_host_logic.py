"""Host-side logic of the dtmi package that needs no GPU: DDP bucket layout,
ZeRO partition, the learning-rate schedule, embedding segment construction and
the parameter order/init of the model definition (checked without touching
the device)."""
import numpy as np

from dtmi.ddp import bucket_layout
from dtmi.kernels import embedding_segments
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


def test_embedding_segments_reproduce_add_at_order():
    rng = np.random.default_rng(0)
    idx = rng.integers(0, 7, (5, 9))
    perm, start, row = embedding_segments(idx)
    flat = idx.reshape(-1)
    assert start[0] == 0 and start[-1] == flat.size
    seen = []
    for s in range(row.size):
        pos = perm[start[s]:start[s + 1]]
        assert np.all(flat[pos] == row[s])
        assert np.all(np.diff(pos) > 0)  # increasing position order == np.add.at order
        seen.extend(pos.tolist())
    assert sorted(seen) == list(range(flat.size))
    assert list(row) == sorted(set(flat.tolist()))


def test_model_parameter_order_matches_dtrain_names():
    """dtmi.nn builds its modules in dtrain's attribute order; the names it
    reports follow from the class structure alone."""
    import dtmi.nn as N
    assert [f.name for f in N.GPTConfig.__dataclass_fields__.values()] == \
        ["vocab", "ctx", "dim", "heads", "layers", "dtype"]
    assert list(N.Block.__init__.__code__.co_names).index("ln1") < list(N.Block.__init__.__code__.co_names).index("qkv")
