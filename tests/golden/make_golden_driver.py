"""Write golden fixtures for the training driver's data and checkpoint formats
from dtrain itself (run where the dtrain source tree exists; the fixtures are
committed, so the GPU tests never need dtrain).

    python tests/golden/make_golden_driver.py [/path/to/DISTRIBUTED-TRAINING]

  - dtrain_data.npz: CharData of a fixed synthetic text (vocabulary, train /
    validation ids) and rank_batch windows for several (step, micro, seed,
    rank, world) (dtrain/data.py:35-56);
  - dtrain_ckpt/: a 2-rank checkpoint written by dtrain/checkpoint.py:save
    (step directory, per-rank npz shards, manifest with SHA-256, LATEST);
  - dtrain_driver_run.npz and dtrain_driver_ckpt/: dtrain's training driver
    (dtrain/train.py:72-190) run in-process on the corpus of dtrain's own
    training tests (tests/test_training.py:19-26) with the tiny float64 flags
    (:15-16) and `--mode single --emulate-world 2 --accum 2 --steps 6`: the
    per-step lr, loss and grad_norm of its JSON log, its final parameters
    (--save-params), and the checkpoint a run stopped after step 3 wrote
    (--stop-after 3 --ckpt-dir --ckpt-every 3), from which a resumed run
    continues.
"""
from __future__ import annotations

import shutil
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
sys.path.insert(0, str(REF))

import json  # noqa: E402
import tempfile  # noqa: E402

from dtrain import checkpoint  # noqa: E402
from dtrain import train as dtrain_train  # noqa: E402
from dtrain.data import CharData, rank_batch  # noqa: E402

TINY = ["--dim", "16", "--heads", "2", "--layers", "2", "--ctx", "16", "--batch", "2", "--dtype", "float64",
        "--lr", "3e-3", "--warmup", "2"]
DRIVER = ["--mode", "single", "--emulate-world", "2", "--accum", "2", "--steps", "6"]


def synthetic_text(n=5000, seed=7):
    rng = np.random.default_rng(seed)
    alphabet = np.array(list("abcdefghij klmnop,.\nQRS"))
    return "".join(alphabet[rng.integers(0, len(alphabet), n)])


def test_corpus():
    """The corpus of dtrain's training tests (tests/test_training.py:19-26)."""
    rng = np.random.default_rng(0)
    words = ["the", "king", "and", "queen", "of", "rome", "said", "to", "thee", "now"]
    return " ".join(rng.choice(words, 4000)) + "\n"


def driver_runs():
    """dtrain.train.main in-process: a 6-step run, and a run stopped after
    step 3 that leaves its checkpoint."""
    text = test_corpus()
    with tempfile.TemporaryDirectory() as tmp:
        tmp = Path(tmp)
        corpus = tmp / "corpus.txt"
        corpus.write_text(text)
        out = {"corpus": np.frombuffer(text.encode(), dtype=np.uint8)}
        full, log = tmp / "full.npz", tmp / "full.jsonl"
        dtrain_train.main([*DRIVER, *TINY, "--data", str(corpus), "--save-params", str(full), "--log", str(log)])
        lines = [json.loads(line) for line in open(log)]
        assert [d["step"] for d in lines] == list(range(1, 7))
        for key in ("lr", "loss", "grad_norm"):
            out[f"log/{key}"] = np.array([d[key] for d in lines], np.float64)
        with np.load(full) as z:
            for k in z.files:
                out[f"param/{k}"] = z[k]
        ck = HERE / "dtrain_driver_ckpt"
        if ck.exists():
            shutil.rmtree(ck)
        part, plog = tmp / "part.npz", tmp / "part.jsonl"
        dtrain_train.main([*DRIVER, *TINY, "--data", str(corpus), "--stop-after", "3", "--ckpt-dir", str(ck),
                           "--ckpt-every", "3", "--save-params", str(part), "--log", str(plog)])
        assert (ck / "LATEST").read_text() == "step_000003"
        plines = [json.loads(line) for line in open(plog)]
        assert [d["loss"] for d in plines] == [d["loss"] for d in lines[:3]]
        with np.load(part) as z:
            for k in z.files:
                out[f"part_param/{k}"] = z[k]
    np.savez(HERE / "dtrain_driver_run.npz", **out)
    print("wrote", HERE / "dtrain_driver_run.npz", ck)


def main():
    driver_runs()
    text = synthetic_text()
    data = CharData(text)
    out = {"text": np.frombuffer(text.encode(), dtype=np.uint8), "vocab": np.int64(data.vocab),
           "train": data.train, "val": data.val}
    cases = [(0, 0, 4, 16, 0, 0, 1), (3, 1, 4, 16, 0, 1, 2), (7, 0, 2, 32, 5, 2, 4), (11, 2, 8, 8, 1, 0, 3)]
    for i, (step, micro, bs, ctx, seed, rank, world) in enumerate(cases):
        x, y = rank_batch(data.train, step, micro, bs, ctx, seed, rank, world)
        out[f"case{i}"] = np.array([step, micro, bs, ctx, seed, rank, world])
        out[f"x{i}"], out[f"y{i}"] = x, y
    np.savez(HERE / "dtrain_data.npz", **out)

    ck = HERE / "dtrain_ckpt"
    if ck.exists():
        shutil.rmtree(ck)
    rng = np.random.default_rng(9)
    params = rng.standard_normal(37)
    for rank in (1, 0):  # rank 0 last: its manifest covers both shards
        st = {"params": params, "t": 3, "m": rng.standard_normal(19 - rank), "v": np.abs(rng.standard_normal(19 - rank))}
        np.savez(HERE / f"dtrain_ckpt_state_rank{rank}.npz", **st)
        checkpoint.save(str(ck), 2, rank, 2, st, lambda: None)
    print("wrote", HERE / "dtrain_data.npz", ck)


if __name__ == "__main__":
    main()
