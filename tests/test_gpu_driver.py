"""End-to-end training through the driver on the GPU: dtrain's own training
tests (tests/test_training.py:57-130) with the ranks as simulated replicas in
one process. float64 and a tiny model, so equivalences are checked tightly;
the corpus is generated (no network)."""
import json
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = ["--dim", "16", "--heads", "2", "--layers", "2", "--ctx", "16", "--batch", "2", "--dtype", "float64",
        "--lr", "3e-3", "--warmup", "2"]
STEPS = ["--steps", "6"]


@pytest.fixture(scope="module")
def corpus(tmp_path_factory):
    rng = np.random.default_rng(0)
    words = ["the", "king", "and", "queen", "of", "rome", "said", "to", "thee", "now"]
    text = " ".join(rng.choice(words, 4000)) + "\n"
    p = tmp_path_factory.mktemp("data") / "corpus.txt"
    p.write_text(text)
    return str(p)


def train(tmp: Path, name, corpus, mode, world=1, extra=()):
    from dtmi import train as T
    out, log = tmp / f"{name}.npz", tmp / f"{name}.jsonl"
    args = ["--mode", mode, "--world", str(world), "--data", corpus, "--save-params", str(out), "--log", str(log),
            *TINY, *extra]
    assert T.main(args) == 0
    params = dict(np.load(out)) if out.exists() else None
    logs = [json.loads(line) for line in open(log)] if log.exists() else []
    return params, logs


def assert_close(a, b, tol):
    assert a.keys() == b.keys()
    worst = max(float(np.max(np.abs(a[k] - b[k]))) for k in a)
    assert worst <= tol, f"max abs param difference {worst:g} > {tol:g}"


def test_ddp_matches_single_process(dev, tmp_path, corpus):
    ref, ref_log = train(tmp_path, "single", corpus, "single", extra=[*STEPS, "--emulate-world", "4"])
    ddp, ddp_log = train(tmp_path, "ddp", corpus, "ddp", 4, extra=STEPS)
    assert_close(ddp, ref, 1e-10)
    assert len(ref_log) == len(ddp_log) == 6
    for a, b in zip(ref_log, ddp_log):
        assert abs(a["loss"] - b["loss"]) < 1e-10
        assert set(a) == {"step", "lr", "loss", "grad_norm", "step_s", "tokens_per_s", "comm_wait_s"}


def test_zero_matches_ddp_and_shards_state(dev, tmp_path, corpus):
    ddp, _ = train(tmp_path, "ddp", corpus, "ddp", 4, extra=STEPS)
    zero, zlog = train(tmp_path, "zero", corpus, "zero", 4, extra=STEPS)
    assert_close(zero, ddp, 1e-10)
    nparams = sum(v.size for v in ddp.values())
    state = [line for line in zlog if "optimizer_state_bytes_per_rank" in line][0]["optimizer_state_bytes_per_rank"]
    assert state == 2 * 8 * -(-nparams // 4)  # rank 0's float64 m and v for ceil(n / 4) elements


def test_overlap_bucket_size_and_algorithm_do_not_change_results(dev, tmp_path, corpus):
    a, _ = train(tmp_path, "a", corpus, "ddp", 3, extra=[*STEPS, "--bucket-mb", "0.001"])
    b, _ = train(tmp_path, "b", corpus, "ddp", 3, extra=[*STEPS, "--no-overlap", "--bucket-mb", "100"])
    c, _ = train(tmp_path, "c", corpus, "ddp", 3, extra=[*STEPS, "--algo", "direct"])
    # dtrain's tolerance: the ring's chunk edges move with the bucket size
    assert_close(a, b, 1e-12)
    assert_close(a, c, 1e-12)


def test_gradient_accumulation_matches_larger_batch(dev, tmp_path, corpus):
    ref, _ = train(tmp_path, "ref", corpus, "single", extra=[*STEPS, "--emulate-world", "2", "--accum", "2"])
    acc, _ = train(tmp_path, "acc", corpus, "ddp", 2, extra=[*STEPS, "--accum", "2"])
    assert_close(acc, ref, 1e-10)


@pytest.mark.parametrize("mode", ["ddp", "zero"])
def test_checkpoint_resume_is_exact(dev, tmp_path, corpus, mode, capsys):
    full, _ = train(tmp_path, f"{mode}-full", corpus, mode, 2, extra=["--steps", "8"])
    ck = tmp_path / f"ck-{mode}"
    train(tmp_path, f"{mode}-part", corpus, mode, 2,
          extra=["--steps", "8", "--stop-after", "4", "--ckpt-dir", str(ck), "--ckpt-every", "2"])
    assert (ck / "LATEST").read_text() == "step_000004"
    resumed, _ = train(tmp_path, f"{mode}-res", corpus, mode, 2,
                       extra=["--steps", "8", "--ckpt-dir", str(ck), "--ckpt-every", "2", "--resume"])
    assert "resumed from step 4" in capsys.readouterr().err
    assert_close(resumed, full, 0.0)  # bit-identical


def test_corrupt_checkpoint_is_rejected(dev, tmp_path, corpus):
    ck = tmp_path / "ck-bad"
    train(tmp_path, "w", corpus, "ddp", 2, extra=["--steps", "2", "--ckpt-dir", str(ck), "--ckpt-every", "2"])
    shard = ck / "step_000002" / "rank1.npz"
    b = bytearray(shard.read_bytes())
    b[len(b) // 2] ^= 0xFF
    shard.write_bytes(bytes(b))
    with pytest.raises(ValueError, match="checksum mismatch"):
        train(tmp_path, "r", corpus, "ddp", 2, extra=["--steps", "4", "--ckpt-dir", str(ck), "--resume"])
