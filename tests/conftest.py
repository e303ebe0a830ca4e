import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "g1.cu_amd", "scripts"), os.path.join(ROOT, "g1.cu_amd"),
          ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the HIP library)")


def relerr_rows(a, b, eps=1e-12):
    """Per-state ||a-b||_2 / ||b||_2 (the reference's gate metric, src/test_envqacc.cu:74-86)."""
    a = np.asarray(a, np.float64).reshape(len(a), -1)
    b = np.asarray(b, np.float64).reshape(len(b), -1)
    return np.linalg.norm(a - b, axis=1) / (np.linalg.norm(b, axis=1) + eps)


def load_contact_validate():
    raw = open(os.path.join(GOLDEN, "contact_validate.bin"), "rb").read()
    n = int(np.frombuffer(raw[:4], np.int32)[0])
    o = 4
    out = {}
    for key, w in (("qpos", 36), ("qvel", 35), ("qacc", 35)):
        out[key] = np.frombuffer(raw[o:o + n * w * 4], np.float32).reshape(n, w).copy()
        o += n * w * 4
    out["label"] = np.frombuffer(raw[o:o + 4 * n], np.int32).copy()
    return out


def envqacc_states(n, seed=999):
    """The reference gate's state family (src/test_envqacc.cu:29-39): stand pose + U(-0.2,0.2) on
    every qpos entry, base dropped up to 0.15 m, renormalised quaternion, qvel U(-1,1)."""
    import g1_model as gm
    rng = np.random.default_rng(seed)
    qp = (gm.qpos_stand.astype(np.float32)[None] + 0.2 * (rng.random((n, 36), np.float32) * 2 - 1)).astype(np.float32)
    qp[:, 2] -= 0.15 * rng.random(n, np.float32)
    qp[:, 3:7] /= np.linalg.norm(qp[:, 3:7], axis=1, keepdims=True)
    qv = (rng.random((n, 35), np.float32) * 2 - 1).astype(np.float32)
    return qp, qv


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def ref_traj():
    return np.load(os.path.join(GOLDEN, "ref_traj_subset.npz"), allow_pickle=False)
