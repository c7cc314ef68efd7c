"""Host-only parts of the training driver: character data and per-rank
batches against dtrain's own outputs, the checkpoint format (written and read
by dtrain and by dtmi), and the command line."""
import json
import os
from pathlib import Path

import numpy as np
import pytest

from dtmi import checkpoint, data
from dtmi import train as T
from oracle import model as OM, optim as OO, step as OS

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_chardata_and_rank_batches_match_dtrain():
    g = np.load(GOLDEN / "dtrain_data.npz")
    text = g["text"].tobytes().decode()
    d = data.CharData(text)
    assert d.vocab == int(g["vocab"])
    assert d.train.dtype == np.int32
    np.testing.assert_array_equal(d.train, g["train"])
    np.testing.assert_array_equal(d.val, g["val"])
    i = 0
    while f"case{i}" in g.files:
        step, micro, bs, ctx, seed, rank, world = (int(v) for v in g[f"case{i}"])
        x, y = data.rank_batch(d.train, step, micro, bs, ctx, seed, rank, world)
        np.testing.assert_array_equal(x, g[f"x{i}"])
        np.testing.assert_array_equal(y, g[f"y{i}"])
        i += 1
    assert i >= 4


def test_rank_batches_tile_the_global_batch():
    ids = np.arange(1000, dtype=np.int32) % 37
    gx, gy = data.global_batch(ids, 5, 1, 12, 20, 3)
    np.testing.assert_array_equal(gx[:, 1:], gy[:, :-1])  # y is x shifted by one token
    parts = [data.rank_batch(ids, 5, 1, 4, 20, 3, r, 3) for r in range(3)]
    np.testing.assert_array_equal(np.concatenate([p[0] for p in parts]), gx)
    np.testing.assert_array_equal(np.concatenate([p[1] for p in parts]), gy)


def test_load_text_requires_a_file(tmp_path):
    with pytest.raises(ValueError):
        data.load_text(None)
    p = tmp_path / "t.txt"
    p.write_text("hello")
    assert data.load_text(str(p)) == "hello"


def test_reads_a_checkpoint_written_by_dtrain():
    ck = GOLDEN / "dtrain_ckpt"
    d = checkpoint.latest(str(ck))
    assert d is not None and d.endswith("step_000002")
    for r in range(2):
        step, st = checkpoint.load(d, r, 2)
        assert step == 2
        want = np.load(GOLDEN / f"dtrain_ckpt_state_rank{r}.npz")
        assert sorted(st) == sorted(want.files)
        for k in want.files:
            np.testing.assert_array_equal(st[k], want[k])
    with pytest.raises(ValueError, match="ranks"):
        checkpoint.load(d, 0, 3)


def test_checkpoint_round_trip_latest_and_corruption(tmp_path):
    rng = np.random.default_rng(0)
    states = [{"params": rng.standard_normal(10), "t": 4, "m": rng.standard_normal(5)} for _ in range(2)]
    root = str(tmp_path / "ck")
    checkpoint.save_group(root, 2, states)
    calls = []
    for r in (1, 0):  # per-rank API, rank 0 last as after a barrier
        checkpoint.save(root, 4, r, 2, states[r], lambda: calls.append(r))
    assert calls == [1, 1, 0, 0]  # every rank meets both barriers (before and after the manifest)
    d = checkpoint.latest(root)
    assert d.endswith("step_000004")
    man = json.loads(Path(d, "manifest.json").read_text())
    assert man["step"] == 4 and man["world"] == 2 and set(man["shards"]) == {"rank0.npz", "rank1.npz"}
    for r in range(2):
        step, st = checkpoint.load(d, r, 2)
        assert step == 4 and int(st["t"]) == 4
        np.testing.assert_array_equal(st["params"], states[r]["params"])
    assert not any(name.endswith(".tmp") for name in os.listdir(d))
    shard = Path(d, "rank1.npz")
    b = bytearray(shard.read_bytes())
    b[len(b) // 2] ^= 0xFF
    shard.write_bytes(bytes(b))
    with pytest.raises(ValueError, match="checksum mismatch"):
        checkpoint.load(d, 1, 2)
    checkpoint.load(d, 0, 2)  # the other shard is intact


def test_driver_flags_match_dtrain():
    a = T.parse(["--mode", "zero", "--world", "4", "--steps", "8", "--accum", "2", "--ckpt-dir", "x",
                 "--ckpt-every", "2", "--resume", "--stop-after", "4", "--emulate-world", "2", "--algo", "direct"])
    assert (a.mode, a.world, a.steps, a.accum, a.ckpt_every, a.resume, a.stop_after) == ("zero", 4, 8, 2, 2, True, 4)
    d = T.parse([])
    assert (d.batch, d.ctx, d.dim, d.heads, d.layers, d.lr, d.wd, d.clip, d.bucket_mb, d.algo) == \
        (8, 64, 128, 4, 4, 1e-3, 0.1, 1.0, 1.0, "ring")


# dtrain's training driver run (tests/golden/make_golden_driver.py): --mode single
# --emulate-world 2 --accum 2 --steps 6 with the tiny float64 flags of dtrain's
# tests/test_training.py:15-16
DRIVER = dict(steps=6, world=2, accum=2, batch=2, ctx=16, dim=16, heads=2, layers=2, lr=3e-3, warmup=2, wd=0.1,
              clip=1.0, seed=0)


def test_schedule_and_batches_reproduce_dtrain_driver_run():
    """dtmi.train.lr_at and dtmi.data.rank_batch, driven as dtrain's main loop
    drives them (train.py:118-159: lr_at(step), rank_batch(step, micro, ...,
    vr, W), micro-steps outer), with the oracle's arithmetic for the steps:
    every logged lr is identical, and loss, grad_norm and the final
    parameters are dtrain's bit for bit."""
    g = np.load(GOLDEN / "dtrain_driver_run.npz")
    a = DRIVER
    d = data.CharData(g["corpus"].tobytes().decode())
    c = OM.GPTConfig(vocab=d.vocab, ctx=a["ctx"], dim=a["dim"], heads=a["heads"], layers=a["layers"],
                     dtype="float64")
    P = OM.dtrain_init(c, seed=a["seed"])
    opt = OO.AdamW(list(P.values()), lr=a["lr"], weight_decay=a["wd"])
    for step in range(a["steps"]):
        lr = T.lr_at(step, a["lr"], a["warmup"], a["steps"])
        assert lr == g["log/lr"][step]
        opt.lr = lr
        batches = [[data.rank_batch(d.train, step, micro, a["batch"], a["ctx"], a["seed"], vr, a["world"])
                    for micro in range(a["accum"])] for vr in range(a["world"])]
        loss, gnorm, _ = OS.single_step(P, c, batches, opt, clip=a["clip"], emulate_world=a["world"],
                                        accum=a["accum"])
        assert loss == g["log/loss"][step]
        assert gnorm == g["log/grad_norm"][step]
    for k, v in P.items():
        np.testing.assert_array_equal(v, g[f"param/{k}"])


def test_reads_the_checkpoint_of_a_dtrain_driver_run():
    """dtrain's driver stopped after step 3 (--stop-after 3 --ckpt-every 3):
    its checkpoint holds the parameters it saved at that point, AdamW's step
    count 3 and one m and v per parameter (train.py:170-180)."""
    g = np.load(GOLDEN / "dtrain_driver_run.npz")
    d = checkpoint.latest(str(GOLDEN / "dtrain_driver_ckpt"))
    assert d.endswith("step_000003")
    step, st = checkpoint.load(d, 0, 1)
    names = [k[len("part_param/"):] for k in g.files if k.startswith("part_param/")]
    assert step == 3 and int(st["t"]) == 3
    np.testing.assert_array_equal(st["params"], np.concatenate([g[f"part_param/{k}"].reshape(-1) for k in names]))
    assert sorted(k for k in st if k[0] in "mv") == sorted([f"m{i}" for i in range(len(names))] +
                                                          [f"v{i}" for i in range(len(names))])
