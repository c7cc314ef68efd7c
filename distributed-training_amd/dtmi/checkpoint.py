"""Sharded, atomic, checksummed checkpoints in dtrain's on-disk format
(dtrain/checkpoint.py), so either side can resume from the other's files.

    root/step_000100/rank0.npz ... rank{W-1}.npz   one state dict per rank
    root/step_000100/manifest.json                {"step", "world", "shards": {name: sha256}}
    root/LATEST                                   name of the newest complete step directory

Each shard is written to a temporary name, flushed and renamed; the manifest
and then LATEST are replaced only after every shard is complete, so a crash
leaves LATEST at the previous complete checkpoint (checkpoint.py:40-75). On
load the shard's SHA-256 must match the manifest (checkpoint.py:85-92).

Values may be device arrays (copied to the host) or NumPy arrays / scalars.
With W simulated replicas in one process, `save_group` writes every rank's
shard and then the manifest.
"""
from __future__ import annotations

import hashlib
import io
import json
import os

import numpy as np


def _sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            block = f.read(1 << 20)
            if not block:
                break
            h.update(block)
    return h.hexdigest()


def _sync_dir(path: str):
    fd = os.open(path, os.O_RDONLY)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def _write_atomic(path: str, data: bytes):
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(data)
        f.flush()
        os.fsync(f.fileno())
    os.replace(tmp, path)


def _step_dir(root: str, step: int) -> tuple[str, str]:
    name = f"step_{step:06d}"
    return name, os.path.join(root, name)


def _write_shard(d: str, rank: int, state: dict):
    buf = io.BytesIO()
    np.savez(buf, **{k: np.asarray(v) for k, v in state.items()})
    _write_atomic(os.path.join(d, f"rank{rank}.npz"), buf.getvalue())


def _commit(root: str, name: str, d: str, step: int, world: int):
    shards = {f"rank{r}.npz": _sha256(os.path.join(d, f"rank{r}.npz")) for r in range(world)}
    _write_atomic(os.path.join(d, "manifest.json"), json.dumps({"step": step, "world": world, "shards": shards}).encode())
    _sync_dir(d)
    _write_atomic(os.path.join(root, "LATEST"), name.encode())
    _sync_dir(root)


def save(root: str, step: int, rank: int, world: int, state: dict, barrier) -> str:
    """dtrain/checkpoint.py:40-75: every rank calls this with its own state."""
    name, d = _step_dir(root, step)
    os.makedirs(d, exist_ok=True)
    _write_shard(d, rank, state)
    barrier()
    if rank == 0:
        _commit(root, name, d, step, world)
    barrier()
    return d


def save_group(root: str, step: int, states: list) -> str:
    """All W ranks' shards from one process (states[r] = rank r's state dict)."""
    name, d = _step_dir(root, step)
    os.makedirs(d, exist_ok=True)
    for r, st in enumerate(states):
        _write_shard(d, r, st)
    _commit(root, name, d, step, len(states))
    return d


def latest(root: str) -> str | None:
    p = os.path.join(root, "LATEST")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return os.path.join(root, f.read().strip())


def load(d: str, rank: int, world: int) -> tuple[int, dict]:
    """(step, state) of `rank`, after checking the world size and the shard's checksum."""
    with open(os.path.join(d, "manifest.json")) as f:
        man = json.load(f)
    if man["world"] != world:
        raise ValueError(f"checkpoint was written by {man['world']} ranks, this job has {world}")
    shard = os.path.join(d, f"rank{rank}.npz")
    if _sha256(shard) != man["shards"][f"rank{rank}.npz"]:
        raise ValueError(f"checksum mismatch in {shard}")
    with np.load(shard, allow_pickle=False) as z:
        return man["step"], {k: z[k] for k in z.files}
