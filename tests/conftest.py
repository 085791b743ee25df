"""Shared pytest setup: the `gpu` marker, repo-root imports, comparison helpers."""

import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (runs on the MI355X box)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda", 0)


def lim_ratio(got, ref, rtol, atol):
    """max |got - ref| / (atol + rtol |ref|) -- <= 1 means within tolerance."""
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return ((got - ref).abs() / (atol + rtol * ref.abs())).max().item() if ref.numel() else 0.0


def assert_parity(name, gpu, cpu32, ref64, rtol=1e-4, atol=1e-5):
    """Elementwise parity with the fp32 CPU restatement of the reference.

    Where the fp32 CPU value itself is off from the fp64 evaluation of the same
    formula, an element is also accepted when the GPU value is at least as close
    to fp64 as the CPU is (|gpu - ref64| <= |cpu32 - ref64| + tol).
    """
    g = gpu.detach().double().cpu()
    c = cpu32.detach().double().cpu()
    r = ref64.detach().double().cpu()
    assert g.shape == c.shape == r.shape, (name, g.shape, c.shape, r.shape)
    tol_c = atol + rtol * c.abs()
    ok = (g - c).abs() <= tol_c
    if not bool(ok.all()):
        tie = (g - r).abs() <= (c - r).abs() + atol + rtol * r.abs()
        bad = ~(ok | tie)
        n = int(bad.sum())
        assert n == 0, (
            f"{name}: {n} of {g.numel()} elements outside rtol={rtol} atol={atol} "
            f"(vs cpu32 {lim_ratio(g, c, rtol, atol):.3g}x, vs fp64 {lim_ratio(g, r, rtol, atol):.3g}x)")


def assert_close64(name, gpu, ref64, rtol=1e-4, atol=1e-5):
    """Parity against the fp64 evaluation of the reference formula."""
    ratio = lim_ratio(gpu, ref64, rtol, atol)
    assert ratio <= 1.0, f"{name}: {ratio:.3g}x the tolerance (rtol={rtol}, atol={atol}) vs fp64"
