"""Shared pytest setup: import paths, the `gpu` marker, seeded inputs."""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "ma-transformer_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libma_attn.so")


def randn(shape, seed, scale=1.0):
    """i.i.d. N(0,1)*scale float32 from numpy's PCG64 (identical on every host)."""
    return (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * scale).astype(np.float32)


def qkv(shape, seed, scale=1.0):
    return randn(shape, seed, scale), randn(shape, seed + 1, scale), randn(shape, seed + 2, scale)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    return O


@pytest.fixture
def kernel_env(monkeypatch):
    """Set MA_ATTN_* kernel-selection switches for one test: the library reads
    them when it loads, so they are re-read after setting and after the test."""
    import ma_attn

    def set_env(name, value):
        monkeypatch.setenv(name, value)
        ma_attn.reload_options()

    yield set_env
    monkeypatch.undo()
    ma_attn.reload_options()


# Gradient tolerances: float32 max-abs <= 1e-4; bfloat16 / float16 per element
# |got - ref| <= GRAD16_ATOL + GRAD16_RTOL * |ref| (the kernels compute in fp32
# on the 16-bit inputs, with 16-bit P and dS operands on the MFMA path, and
# round each gradient once to the input dtype).
GRAD32_ATOL = 1e-4
GRAD16_ATOL = 1e-2
GRAD16_RTOL = 1e-2


def check_grad(name, got, ref, is_f32):
    """Assert one gradient tensor (numpy float32) against the oracle's; prints
    the max error and, for 16-bit, the worst ratio to the per-element bound."""
    assert np.isfinite(got).all(), f"{name}: non-finite"
    if got.size == 0:
        return
    err = np.abs(got - ref)
    if is_f32:
        print(f"  {name}: max|err| = {err.max():.3e} (tol {GRAD32_ATOL:.0e})", flush=True)
        assert err.max() <= GRAD32_ATOL, (name, float(err.max()))
        return
    ratio = err / (GRAD16_ATOL + GRAD16_RTOL * np.abs(ref))
    print(f"  {name}: max|err| = {err.max():.3e}, worst err/(atol + rtol|ref|) = {ratio.max():.3f}", flush=True)
    assert ratio.max() <= 1.0, (name, float(err.max()), float(ratio.max()))
