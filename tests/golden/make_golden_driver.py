"""Write golden fixtures for the training driver's data and checkpoint formats
from dtrain itself (run where the dtrain source tree exists; the fixtures are
committed, so the GPU tests never need dtrain).

    python tests/golden/make_golden_driver.py [/path/to/DISTRIBUTED-TRAINING]

  - dtrain_data.npz: CharData of a fixed synthetic text (vocabulary, train /
    validation ids) and rank_batch windows for several (step, micro, seed,
    rank, world) (dtrain/data.py:35-56);
  - dtrain_ckpt/: a 2-rank checkpoint written by dtrain/checkpoint.py:save
    (step directory, per-rank npz shards, manifest with SHA-256, LATEST).
"""
from __future__ import annotations

import shutil
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
sys.path.insert(0, str(REF))

from dtrain import checkpoint  # noqa: E402
from dtrain.data import CharData, rank_batch  # noqa: E402


def synthetic_text(n=5000, seed=7):
    rng = np.random.default_rng(seed)
    alphabet = np.array(list("abcdefghij klmnop,.\nQRS"))
    return "".join(alphabet[rng.integers(0, len(alphabet), n)])


def main():
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
