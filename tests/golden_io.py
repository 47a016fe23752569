"""Loader for the golden fixtures in ``tests/golden`` (plain ``numpy.load``)."""
import glob
import os

import numpy as np
import torch

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture_names():
    return sorted(os.path.splitext(os.path.basename(p))[0]
                  for p in glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))


def _bf16(a):
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)


def load_fixture(name):
    z = np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"))
    return dict(
        q=_bf16(z["q"]), kv=_bf16(z["kv"]), sink=torch.from_numpy(z["sink"].copy()),
        idx=torch.from_numpy(z["idx"].copy()), scale=float(z["scale"]),
        expected_f64=z["expected_f64"].astype(np.float64),
        expected_ref_bf16=_bf16(z["expected_ref_bf16"]))
