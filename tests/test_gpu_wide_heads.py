"""head_dim above 512 on the GPU: the row kernels read the row from memory
and produce the output columns in passes of 512, recomputing the scores per
pass.  Forward and backward against the oracle (which, like the reference's
ma_core.cpp:202-239 and .cu:228-258, loops over any head_dim), for head_dims
with a whole pass, a ragged last pass and a short last pass.

Tolerances: forward max-abs 1e-5 (fp32) / 2e-2 (16-bit); gradients per
check_grad (fp32 1e-4)."""
import numpy as np
import pytest
import torch

from conftest import check_grad, qkv, randn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import sparse_attention_cuda
    return sparse_attention_cuda


def _inputs(shape, seed, dtype):
    arrs = qkv(shape, seed, 0.25)
    dev = [torch.from_numpy(a).to(dtype).cuda() for a in arrs]
    return dev, [t.float().cpu().numpy() for t in dev]


@pytest.mark.parametrize("D", [520, 1024, 1100])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_wide_forward_sliding_and_dense(ext, oracle, D, dtype):
    shape = (1, 70, 2, D)
    (q, k, v), up = _inputs(shape, 7000 + D, dtype)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, out, spec in (
            ("sliding w=5", ext.forward(q, k, v, 5), oracle.Spec(*shape, pattern="sliding", left=5, right=5)),
            ("causal 9", ext.sliding_forward(q, k, v, 9, 0),
             oracle.Spec(*shape, pattern="sliding", left=9, right=0)),
            ("dense causal", ext.dense_forward(q, k, v, True), oracle.Spec(*shape, pattern="dense", causal=True))):
        err = float(np.abs(out.float().cpu().numpy() - oracle.forward(spec, *up)).max())
        print(f"D={D} {dtype} {name}: max|err| = {err:.3e}", flush=True)
        assert out.shape == q.shape and err <= tol


@pytest.mark.parametrize("D", [520, 1100])
def test_wide_backward(ext, oracle, D):
    shape = (1, 50, 2, D)
    (q, k, v), up = _inputs(shape, 7100 + D, torch.float32)
    g = torch.from_numpy(randn(shape, 7200 + D, 0.5)).cuda()
    got = ext.sliding_backward(q, k, v, g, 4, 3)
    ref = oracle.backward(oracle.Spec(*shape, pattern="sliding", left=4, right=3), *up, g.cpu().numpy())
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        check_grad(name, a.cpu().numpy(), b, True)


def test_wide_index_set_and_ma_core(ext, oracle):
    """An explicit key set at head_dim 600, and ma_core with a value head_dim of
    700 against a query head_dim of 600 (zero-padded to 700)."""
    import ma_core
    N, D = 40, 600
    shape = (1, N, 1, D)
    (q, k, v), up = _inputs(shape, 7300, torch.float32)
    rng = np.random.default_rng(5)
    rows = [np.flatnonzero(rng.random(N) < 0.2) for _ in range(N)]
    off = np.zeros(N + 1, dtype=np.int64)
    off[1:] = np.cumsum([len(r) for r in rows])
    keys = np.concatenate(rows).astype(np.int32)
    out = ext.index_set_forward(q, k, v, (torch.from_numpy(off), torch.from_numpy(keys)))
    ref = oracle.forward(oracle.Spec(*shape, pattern="index_set", offsets=off, keys=keys), *up)
    assert float(np.abs(out.cpu().numpy() - ref).max()) <= 1e-5
    vv = randn((1, N, 1, 700), 7301, 0.25)
    tq, tk, tv = (ma_core.create_tensor(list(a.shape)) for a in (up[0], up[1], vv))
    for t, a in ((tq, up[0]), (tk, up[1]), (tv, vv)):
        t.copy_from_numpy(a)
    o = ma_core.compute_sparse_attention(tq, tk, tv, 3).to_numpy()
    ref = oracle.forward_value_dim(oracle.Spec(*shape, pattern="sliding", left=3, right=3), up[0], up[1], vv)
    assert o.shape == (1, N, 1, 700) and float(np.abs(o - ref).max()) <= 1e-5
