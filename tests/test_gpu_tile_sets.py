"""Explicit key sets on the tiled MFMA kernels (an IndexSet with a tile plan,
head_dim 64): forward and backward against the oracle, with tile rows and
key-block columns split over several work items (small tile_seg) and not.

Sets: random (sparse, dense, with empty rows), skewed (sparse rows plus full
rows and full columns, the Longformer global shape), windows, the
block-sparse and Longformer patterns' own key sets.  Tolerances: forward
max-abs 1e-5 (fp32) / 2e-2 (16-bit); gradients as the backward suites
(conftest.check_grad).
"""
import numpy as np
import pytest
import torch

from conftest import check_grad, qkv, randn

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import sparse_attention_cuda
    return sparse_attention_cuda


def _csr_of(m):
    off = np.zeros(m.shape[0] + 1, np.int64)
    off[1:] = np.cumsum(m.sum(1))
    return off, np.nonzero(m)[1].astype(np.int32)


def _set(kind, N, rng):
    i = np.arange(N)[:, None]
    j = np.arange(N)[None, :]
    if kind == "random":
        m = rng.random((N, N)) < 0.15
    elif kind == "dense":
        m = rng.random((N, N)) < 0.9
    elif kind == "skewed":
        m = rng.random((N, N)) < 0.03
        m[rng.choice(N, 4, replace=False)] = True
        m[:, rng.choice(N, 4, replace=False)] = True
        m[rng.choice(N, 5, replace=False)] = False  # empty rows
    elif kind == "window":
        m = (j <= i) & (j >= i - 63)
    elif kind == "window2":
        m = (j >= i - 40) & (j <= i + 17)
    elif kind == "global":
        m = (j <= i) & (j >= i - 100)
        m[:16] = True
        m[:, :16] = True
    else:
        raise ValueError(kind)
    return _csr_of(m)


def _inputs(shape, seed, dtype):
    arrs = list(qkv(shape, seed)) + [randn(shape, seed + 7)]
    dev = [torch.from_numpy(a).to(dtype).to("cuda") for a in arrs]
    return dev, [t.float().cpu().numpy() for t in dev]


@pytest.mark.parametrize("kind,N", [("random", 300), ("dense", 130), ("skewed", 700), ("window", 1000),
                                    ("window2", 513), ("global", 1200)])
@pytest.mark.parametrize("seg", [0, 2])
@pytest.mark.parametrize("dtype", DTYPES)
def test_tiled_set_forward_backward(ext, oracle, kind, N, seg, dtype):
    rng = np.random.default_rng(N + len(kind))
    off, keys = _set(kind, N, rng)
    shape = (2, N, 2, 64)
    dev, up = _inputs(shape, 9100 + N, dtype)
    iset = ext.IndexSet(torch.from_numpy(off), torch.from_numpy(keys), N, tiles=True, tile_seg=seg)
    h = iset.tile_header
    print(f"  {kind} N={N} seg={h.seg}: {h.num_entries} entries, {h.num_q_split} split tiles, "
          f"{h.num_k_split} split key blocks", flush=True)
    spec = oracle.Spec(*shape, pattern="index_set", offsets=off, keys=keys)
    o = ext.index_set_forward(*dev[:3], iset)
    err = float(np.abs(o.float().cpu().numpy() - oracle.forward(spec, *up[:3])).max())
    print(f"  forward max|err| = {err:.3e}", flush=True)
    assert np.isfinite(o.float().cpu().numpy()).all() and err <= TOL[dtype]
    got = ext.index_set_backward(*dev, iset)
    for name, a, b in zip("qkv", got, oracle.backward(spec, *up)):
        check_grad("d" + name, a.float().cpu().numpy(), b, dtype == torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_tiled_matches_gather(ext, dtype):
    """The same set with and without its tile plan: the tiled and gather
    kernels agree to the tolerance."""
    rng = np.random.default_rng(3)
    off, keys = _set("skewed", 900, rng)
    shape = (1, 900, 3, 64)
    dev, _ = _inputs(shape, 9300, dtype)
    a = ext.IndexSet(torch.from_numpy(off), torch.from_numpy(keys), 900, tiles=True)
    b = ext.IndexSet(torch.from_numpy(off), torch.from_numpy(keys), 900, tiles=False)
    assert b.tile_plan is None
    oa, ob = ext.index_set_forward(*dev[:3], a), ext.index_set_forward(*dev[:3], b)
    assert float((oa.float() - ob.float()).abs().max()) <= TOL[dtype]


@pytest.mark.parametrize("pattern,N", [("block_sparse", 1500), ("block_sparse", 1536), ("longformer", 1500)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pattern_sets_on_tiles(ext, oracle, pattern, N, dtype):
    """The key sets block-sparse and Longformer train on (pattern_index_set)
    get a tile plan; their tiled forward and backward match the oracle's.  A
    block table over whole blocks (N a multiple of 64) gives a plan with no
    masked entry, which runs the kernels' mask-free variant."""
    shape = (2, N, 2, 64)
    if pattern == "block_sparse":
        nb = (N + 63) // 64
        tab = ext.make_block_table(11, nb, 2)
        iset = ext.pattern_index_set("block_sparse", N, "cuda", block_table=ext.BlockTable(tab, N, 64), block_size=64)
        spec = oracle.Spec(*shape, pattern="block_sparse", block_size=64, table=tab.numpy())
    else:
        iset = ext.pattern_index_set("longformer", N, "cuda", left=127, right=0, num_global=16)
        spec = oracle.Spec(*shape, pattern="longformer", left=127, right=0, num_global=16)
    assert iset.tile_plan is not None
    assert (iset.tile_header.num_masked == 0) == (pattern == "block_sparse" and N % 64 == 0)
    dev, up = _inputs(shape, 9400, dtype)
    out = ext.index_set_forward(*dev[:3], iset)
    err = float(np.abs(out.float().cpu().numpy() - oracle.forward(spec, *up[:3])).max())
    assert err <= TOL[dtype], err
    got = ext.index_set_backward(*dev, iset)
    for name, a, b in zip("qkv", got, oracle.backward(spec, *up)):
        check_grad("d" + name, a.float().cpu().numpy(), b, dtype == torch.float32)


def test_tiled_plan_for_another_length_rejected(ext):
    off = torch.tensor([0, 1, 2], dtype=torch.int64)
    keys = torch.tensor([0, 1], dtype=torch.int32)
    s = ext.IndexSet(off, keys, 2, tiles=True)
    q = torch.randn(1, 3, 1, 64, device="cuda")
    with pytest.raises(RuntimeError, match="S=2"):
        ext.index_set_forward(q, q, q, s)
