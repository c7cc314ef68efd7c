"""Character-level text data and deterministic per-rank batches (dtrain/data.py).

The batch of (step, micro-step) is a pure function of the seed: the global
batch of `bs_per_rank * world` windows is drawn from
`default_rng([seed, step, micro])` (dtrain/data.py:38-43) and rank r takes rows
[r * bs, (r + 1) * bs) (data.py:46-49). A run resumed from a checkpoint sees
the batches it would have seen, and W simulated replicas in one process see
exactly the batches of a W-process dtrain job.

There is no network here: `load_text` needs a local file (dtrain downloads
tiny-shakespeare when no path is given, data.py:16-32).
"""
from __future__ import annotations

import numpy as np


def load_text(path: str | None) -> str:
    if not path:
        raise ValueError("load_text: a local text file is required (no download)")
    with open(path, encoding="utf-8") as f:
        return f.read()


class CharData:
    """Vocabulary = the sorted distinct characters; ids as int32; the last
    `val_fraction` of the text is the validation split (data.py:35-42)."""

    def __init__(self, text: str, val_fraction: float = 0.1):
        chars = sorted(set(text))
        self.vocab = len(chars)
        self.stoi = {ch: i for i, ch in enumerate(chars)}
        ids = np.fromiter((self.stoi[ch] for ch in text), dtype=np.int32, count=len(text))
        cut = int(len(ids) * (1 - val_fraction))
        self.train, self.val = ids[:cut], ids[cut:]


def global_batch(ids: np.ndarray, step: int, micro: int, global_bs: int, ctx: int, seed: int):
    """x, y [global_bs, ctx]: windows at starts drawn from default_rng([seed, step, micro])."""
    rng = np.random.default_rng([seed, step, micro])
    starts = rng.integers(0, len(ids) - ctx - 1, size=global_bs)
    win = starts[:, None] + np.arange(ctx + 1)[None, :]
    tok = ids[win]
    return tok[:, :-1], tok[:, 1:]


def rank_batch(ids, step, micro, bs_per_rank, ctx, seed, rank, world):
    """Rank `rank`'s rows of the global batch of `bs_per_rank * world` windows."""
    x, y = global_batch(ids, step, micro, bs_per_rank * world, ctx, seed)
    lo = rank * bs_per_rank
    return x[lo:lo + bs_per_rank], y[lo:lo + bs_per_rank]
