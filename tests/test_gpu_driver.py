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


# ---------------------------------------------- against a run of dtrain's driver
DRIVER = ["--mode", "single", "--emulate-world", "2", "--accum", "2", "--steps", "6"]


@pytest.fixture(scope="module")
def dtrain_run(golden, tmp_path_factory):
    """dtrain's own driver (dtrain/train.py:72-190) on the corpus of its tests,
    with DRIVER and the tiny float64 flags (tests/golden/make_golden_driver.py):
    per-step log, final parameters, and the checkpoint its run stopped after
    step 3 wrote."""
    g = golden("dtrain_driver_run.npz")
    p = tmp_path_factory.mktemp("dtrain") / "corpus.txt"
    p.write_bytes(g["corpus"].tobytes())
    params = {k[len("param/"):]: g[k] for k in g.files if k.startswith("param/")}
    log = {k: g[f"log/{k}"] for k in ("lr", "loss", "grad_norm")}
    return str(p), params, log


def _check_log(lines, ref, steps):
    """lr identical; loss and gradient norm within 1e-12 (relative) of dtrain's
    log lines for the given 1-based steps."""
    assert [d["step"] for d in lines] == list(steps)
    for d in lines:
        i = d["step"] - 1
        assert d["lr"] == ref["lr"][i], d["step"]
        assert abs(d["loss"] - ref["loss"][i]) <= 1e-12 * abs(ref["loss"][i]), d["step"]
        assert abs(d["grad_norm"] - ref["grad_norm"][i]) <= 1e-12 * ref["grad_norm"][i], d["step"]


def test_driver_matches_a_dtrain_driver_run(dev, tmp_path, dtrain_run):
    """dtmi.train.main with dtrain's flags against dtrain's main on the same
    corpus: every step's lr (warm-up then cosine) identical, loss and gradient
    norm within 1e-12, final parameters within 1e-10 (dtrain's own bar for
    runs that sum in different orders, tests/test_training.py:48-51)."""
    corpus, ref_params, ref_log = dtrain_run
    params, log = train(tmp_path, "single", corpus, "single", extra=DRIVER)
    _check_log(log, ref_log, range(1, 7))
    assert_close(params, ref_params, 1e-10)


def test_ddp_driver_matches_a_dtrain_driver_run(dev, tmp_path, dtrain_run):
    """2 simulated ranks x 2 micro-steps against dtrain's single process
    emulating 2 ranks with 2 micro-steps (dtrain's
    test_gradient_accumulation_matches_larger_batch, with dtrain's run as the
    reference): the losses within 1e-12, parameters within 1e-10."""
    corpus, ref_params, ref_log = dtrain_run
    params, log = train(tmp_path, "ddp", corpus, "ddp", 2, extra=["--accum", "2", "--steps", "6"])
    for d in log:
        i = d["step"] - 1
        assert d["lr"] == ref_log["lr"][i]
        assert abs(d["loss"] - ref_log["loss"][i]) <= 1e-12 * abs(ref_log["loss"][i])
    assert_close(params, ref_params, 1e-10)


def test_resume_from_a_checkpoint_dtrain_wrote_during_training(dev, tmp_path, dtrain_run, capsys):
    """dtmi.train.main --resume from the checkpoint dtrain's driver wrote at
    step 3 (dtrain/checkpoint.py:40-88, train.py:98-112): steps 4-6 log
    dtrain's lr, loss and gradient norm, and the final parameters are within
    1e-10 of dtrain's uninterrupted run."""
    import shutil
    corpus, ref_params, ref_log = dtrain_run
    ck = tmp_path / "ck"
    shutil.copytree(Path(__file__).resolve().parent / "golden" / "dtrain_driver_ckpt", ck)
    params, log = train(tmp_path, "resumed", corpus, "single",
                        extra=[*DRIVER, "--ckpt-dir", str(ck), "--ckpt-every", "3", "--resume"])
    assert "resumed from step 3" in capsys.readouterr().err
    _check_log(log, ref_log, range(4, 7))
    assert_close(params, ref_params, 1e-10)
    # and it wrote its own step-6 checkpoint in the same format
    assert (ck / "LATEST").read_text() == "step_000006"
