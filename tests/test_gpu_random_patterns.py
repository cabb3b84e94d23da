"""Seeded random block-sparse tables and Longformer geometries, forward,
against the oracle.

Block-sparse: random tables (ascending, -1 padded, 1..width valid entries;
widths 1-4 take the short-row kernel, wider ones the streaming walk), ragged
sequence lengths, batches and heads.  Longformer: the global count G (1-16,
the tiled kernel; above 16 the row kernel), left/right windows around and
beyond one block, lengths shorter and longer than the band.  Each case is
drawn from a fixed seed, so a failure names a reproducible case.
Tolerances as the other parity suites: max-abs 1e-5 (fp32) / 2e-2 (16-bit).
"""
import numpy as np
import pytest
import torch

from conftest import qkv

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import sparse_attention_cuda
    return sparse_attention_cuda


def _dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).to("cuda")


def _table(rng, nb, width):
    tab = np.full((nb, width), -1, dtype=np.int32)
    for r in range(nb):
        n = min(int(rng.integers(1, width + 1)), nb)
        tab[r, :n] = np.sort(rng.choice(nb, size=n, replace=False))
    return tab


def _check(o, ref, dtype):
    o = o.float().cpu().numpy()
    assert np.isfinite(o).all()
    err = float(np.abs(o - ref).max())
    assert err <= (1e-5 if dtype == torch.float32 else 2e-2), err


@pytest.mark.parametrize("i", range(40))
def test_random_block_sparse(ext, oracle, i):
    rng = np.random.default_rng(31000 + i)
    N = int(rng.integers(1, 1500))
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
    width = int(rng.choice([1, 2, 3, 4, 4, 4, 6, 9]))
    dtype = DTYPES[int(rng.integers(0, 3))]
    nb = (N + 63) // 64
    tab = _table(rng, nb, width)
    print(f"  case {i}: B={B} N={N} H={H} width={width} {dtype}", flush=True)
    shape = (B, N, H, 64)
    q, k, v = qkv(shape, 600 + i, 0.5)
    dev = [_dev(a, dtype) for a in (q, k, v)]
    up = [t.float().cpu().numpy() for t in dev]
    table = torch.from_numpy(tab)
    arg = ext.BlockTable(table, N, 64) if i % 2 else table
    o = ext.block_sparse_forward(*dev, arg, 64)
    spec = oracle.Spec(*shape, pattern="block_sparse", block_size=64, table=tab)
    _check(o, oracle.forward(spec, *up), dtype)


@pytest.mark.parametrize("i", range(40))
def test_random_longformer(ext, oracle, i):
    rng = np.random.default_rng(32000 + i)
    G = int(rng.choice([1, 2, 7, 15, 16, 16, 20]))
    left = int(rng.choice([0, 3, 31, 63, 64, 127, 128, 200]))
    right = int(rng.choice([0, 0, 0, 5, 63, 64]))
    N = int(rng.integers(1, 1200))
    H = int(rng.integers(1, 4))
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    print(f"  case {i}: N={N} H={H} G={G} left={left} right={right} {dtype}", flush=True)
    shape = (1, N, H, 64)
    q, k, v = qkv(shape, 700 + i)
    dev = [_dev(a, dtype) for a in (q, k, v)]
    up = [t.float().cpu().numpy() for t in dev]
    o = ext.longformer_forward(*dev, left, right, G)
    spec = oracle.Spec(*shape, pattern="longformer", left=left, right=right, num_global=G)
    _check(o, oracle.forward(spec, *up), dtype)
