"""Seeded random band geometries, forward and backward, against the oracle.

Each case draws left/right (including windows wider than a block, one-sided
and empty-side ones), dilation, sequence length (ragged, shorter and longer
than the band), heads and dtype from a fixed seed, so a failure names a
reproducible case.  Head_dim is 64 (the MFMA paths: stream kernels, shifted
block grids, fixed-window tiles, per-tile backward with dead sub-tiles).
Tolerances as the other parity suites: forward 1e-5 (fp32) / 2e-2 (16-bit)
max-abs; backward 1e-4 (fp32) max-abs / per element 1e-2 + 1e-2 * |ref| (16-bit).
"""
import numpy as np
import pytest
import torch

from conftest import check_grad, qkv, randn

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _case(i):
    rng = np.random.default_rng(20260 + i)
    left = int(rng.choice([0, 1, 15, 16, 17, 31, 32, 33, 47, 63, 64, 65, 100, 127, 150]))
    right = int(rng.choice([0, 0, 1, 16, 31, 32, 47, 63, 64, 90]))
    dil = int(rng.choice([1, 1, 1, 2, 3, 4]))
    N = int(rng.integers(1, 700))
    H = int(rng.choice([1, 2, 3]))
    dtype = DTYPES[int(rng.integers(0, 3))]
    return left, right, dil, N, H, dtype


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import sparse_attention_cuda
    return sparse_attention_cuda


def _dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).to("cuda")


@pytest.mark.parametrize("i", range(100))
def test_random_band_forward_backward(ext, oracle, i):
    left, right, dil, N, H, dtype = _case(i)
    print(f"  case {i}: left={left} right={right} dil={dil} N={N} H={H} {dtype}", flush=True)
    shape = (1, N, H, 64)
    q, k, v = qkv(shape, 500 + i)
    g = randn(shape, 900 + i)
    dev = [_dev(a, dtype) for a in (q, k, v, g)]
    up = [t.float().cpu().numpy() for t in dev]
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right, dilation=dil)

    o = ext.sliding_forward(dev[0], dev[1], dev[2], left, right, dil).float().cpu().numpy()
    ref = oracle.forward(spec, *up[:3])
    assert np.isfinite(o).all()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert float(np.abs(o - ref).max()) <= tol, ("forward", float(np.abs(o - ref).max()))

    got = ext.sliding_backward(*dev, left, right, dil)
    for name, a, b in zip("qkv", got, oracle.backward(spec, *up)):
        check_grad("d" + name, a.float().cpu().numpy(), b, dtype == torch.float32)
