"""The triton-mla-bench CSV keeps the reference's column types
(src/triton_mla/bench.py:17, 93-104): batch, seqlen, heads, num_splits and
bytes parse as integers and the time columns as floats (empty when a leg did
not run), for the balanced default and an explicit split count."""

import csv
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("splits", ["balanced", "4"])
def test_csv_columns_parse(gpu, tmp_path, splits):
    path = tmp_path / "bench.csv"
    env = dict(os.environ, PYTHONPATH=os.path.join(ROOT, "triton-mla_amd"))
    print(f"triton-mla-bench --batch 1 --seqlen 1024 --splits {splits}", flush=True)
    subprocess.run([sys.executable, "-m", "triton_mla.bench", "--batch", "1", "--seqlen", "1024", "--no-compile",
                    "--reps", "5", "--splits", splits, "--csv", str(path)], check=True, env=env, timeout=300)
    rows = list(csv.DictReader(open(path)))
    assert len(rows) == 1
    r = rows[0]
    for k in ("batch", "seqlen", "heads", "num_splits", "bytes"):
        assert str(int(r[k])) == r[k], (k, r[k])
    for k in ("triton_us", "eager_us", "compile_us"):
        if r[k]:
            float(r[k])
    assert r["compile_us"] == ""  # --no-compile
    assert float(r["triton_us"]) > 0
    # B=1, 1K over the device's compute units: 16 tiles, one per worker
    assert int(r["num_splits"]) == (16 if splits == "balanced" else 4)


@pytest.mark.parametrize("dims,dtype", [(("128", "32"), "fp32"), (("256", "32"), "bf16")])
def test_other_dims_through_the_cli(gpu, tmp_path, dims, dtype):
    """--head-dim-v / --rope-dim (the reference make_inputs' d_latent / d_rope)
    and --dtype fp32 run the generic decode; the run checks it against the
    eager torch path (the reference's 2e-2 gate) and writes the same columns."""
    path = tmp_path / "bench.csv"
    env = dict(os.environ, PYTHONPATH=os.path.join(ROOT, "triton-mla_amd"))
    args = ["--batch", "2", "--seqlen", "1000", "--heads", "16", "--no-compile", "--reps", "5",
            "--head-dim-v", dims[0], "--rope-dim", dims[1], "--dtype", dtype, "--csv", str(path)]
    print("triton-mla-bench " + " ".join(args), flush=True)
    subprocess.run([sys.executable, "-m", "triton_mla.bench"] + args, check=True, env=env, timeout=300)
    rows = list(csv.DictReader(open(path)))
    assert len(rows) == 1
    r = rows[0]
    for k in ("batch", "seqlen", "heads", "num_splits", "bytes"):
        assert str(int(r[k])) == r[k], (k, r[k])
    assert f"generic-{dims[0]}+{dims[1]}" in r["config"]
    assert float(r["triton_us"]) > 0 and float(r["eager_us"]) > 0
