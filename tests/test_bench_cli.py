"""CPU tests of bench.py's contract (no GPU needed):

* ``--gpus N`` with N > 1 exits with status 2 and says that one GPU is what
  this build measures; with no GPU visible the bench exits 1 (it never falls
  back to a CPU path);
* the algorithmic work it reports: valid slots exclude ``-1`` and count
  duplicates, F_alg = 4 h d N_valid, gathered bytes = 2 d N_valid, and the
  compulsory bytes count each (batch, row) once;
* every configuration has a measured traffic figure, and the track-02
  scenarios are the reference's (track-02/workloads.py:19-24).
"""
import os
import subprocess
import sys

import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

import bench  # noqa: E402
import sa_workloads as wl  # noqa: E402


def run_bench(*args):
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="")
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args],
                          capture_output=True, text=True, env=env, timeout=300)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_no_gpu_exits_loudly():
    if torch.cuda.is_available():
        return  # only meaningful on a host without a GPU
    r = run_bench("--steps", "1", "--warmup", "0")
    assert r.returncode == 1
    assert "no GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_algorithmic_work():
    idx = torch.tensor([[[3, 3, -1, 7], [-1, -1, -1, -1], [0, 7, 7, 7]]], dtype=torch.int32)
    b, m = 1, 3
    n_valid, flops, gathered, uniq, compulsory = bench.algorithmic(idx, b, m)
    assert n_valid == 7                      # duplicates count, -1 does not
    assert flops == 4.0 * 16 * 512 * 7
    assert gathered == 7 * 512 * 2
    assert uniq == 3                         # rows 0, 3, 7 of batch 0
    io = b * m * 16 * 512 * 2 * 2 + idx.numel() * 4 + 16 * 4
    assert compulsory == 3 * 512 * 2 + io


def test_tables():
    # traffic of every BASELINE config and every track-03 workload comes from
    # a committed profile summary that names the commit it measured
    for name in list(wl.CONFIGS) + [f"moe{i}" for i in range(len(bench.MOE_WORKLOADS))]:
        tr = bench.traffic_of(name)
        assert tr is not None and tr[0] > 0, name
        assert tr[1] and os.path.exists(os.path.join(bench.REPO, tr[2])), name
    assert len(bench.MOE_WORKLOADS) == 8
    shapes = {(d, p) for _, d, _, p, _ in bench.HC_WORKLOADS}
    assert shapes == {((1, 1), (1, 16384)), ((16, 1), (16, 4096)), ((64, 1), (64, 1024))}
    assert [n for n, *_ in bench.HC_WORKLOADS] == ["16k-1k-1", "4k-1k-16", "1k-1k-64", "1k-1-64"]
