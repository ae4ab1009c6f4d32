"""Shared test fixtures.

Markers: ``gpu`` tests need a real MI355X and call the HIP library through its C ABI;
everything else runs on the CPU (the oracle against golden vectors and closed forms, the
host logic, and that the C-ABI library loads and exports its declared symbols).
"""
import os
import sys

import numpy as np
import pytest

REPO = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
for sub in ("scunet-rs_amd", "oracle", os.path.join("tests", "golden")):
    p = os.path.join(REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def weights_path():
    from scunet_hip import synth
    return synth.weights_file(seed=0)


@pytest.fixture(scope="session")
def weights_path_affine():
    """A checkpoint whose LayerNorm gamma/beta are random, so affine indexing is exercised."""
    from scunet_hip import synth
    return synth.weights_file(seed=3, ln_affine="random")


@pytest.fixture(scope="session")
def owt(weights_path):
    import oracle
    return oracle.Weights.load(weights_path)


@pytest.fixture(scope="session")
def golden():
    return np.load(os.path.join(REPO, "tests", "golden", "golden.npz"))


def close(what, want, got, tol):
    """The reference tests' structural bound (tests/cuda_ops.rs:49-73): the worst absolute
    difference must be within ``tol`` times the data's own magnitude."""
    want = np.asarray(want, np.float32).ravel()
    got = np.asarray(got, np.float32).ravel()
    assert want.shape == got.shape, f"{what}: length {want.shape} vs {got.shape}"
    scale = max(1e-6, float(np.abs(want).max()))
    d = np.abs(want - got)
    i = int(d.argmax())
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert d[i] <= tol * scale, (f"{what}: worst |diff| {d[i]:.3e} at {i} against a scale of "
                                 f"{scale:.3e} (tolerance {tol:.1e} of scale)")
    return float(d[i])


def max_abs(want, got):
    want = np.asarray(want, np.float32).ravel()
    got = np.asarray(got, np.float32).ravel()
    assert want.shape == got.shape
    assert np.isfinite(got).all()
    return float(np.abs(want - got).max())


@pytest.fixture(scope="session")
def weights_path_gray():
    """The grayscale variant (in_nc = 1), benchmark config 4's network."""
    from scunet_hip import synth
    return synth.weights_file(seed=5, in_nc=1)
