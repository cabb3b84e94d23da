"""``ma_core`` attention on the GPU: the reference's own outputs (golden
vectors from ma_core.cpp compiled unchanged, tests/golden) reproduced through
the module's host Tensors, staged to the MI355X kernels and back.

Tolerance: max-abs <= 1e-5 (float32, the north_star bound), plus the
reference's own CPU test tolerance (rtol 1e-5, atol 1e-6,
tests/python/test_cpu_attention_cpp.py:24-56) through the bridge converters.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def mc():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ma_core
    return ma_core


def _t(mc, x):
    t = mc.create_tensor(list(x.shape))
    t.copy_from_numpy(x)
    return t


@pytest.mark.parametrize("name", ["ref_sparse_s10_w2", "ref_sparse_s256_w64", "ref_sparse_s33_w0"])
def test_sparse_matches_reference_bits(mc, name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    out = mc.compute_sparse_attention(_t(mc, z["q"]), _t(mc, z["k"]), _t(mc, z["v"]), int(z["w"]))
    got = out.to_numpy()
    assert got.shape == z["o"].shape
    err = float(np.abs(got - z["o"]).max())
    print(f"{name}: max|err| vs the reference's ma_core = {err:.3e}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_dense_matches_reference_bits(mc, causal):
    z = np.load(os.path.join(GOLDEN, "ref_dense_s32.npz"))
    out = mc.compute_dense_attention(_t(mc, z["q"]), _t(mc, z["k"]), _t(mc, z["v"]), use_causal_mask=causal)
    ref = z["o_causal" if causal else "o_full"]
    err = float(np.abs(out.to_numpy() - ref).max())
    print(f"dense causal={causal}: max|err| vs the reference's ma_core = {err:.3e}", flush=True)
    assert err <= 1e-5


def test_reference_cpu_tests_through_converters(mc):
    """tests/python/test_cpu_attention_cpp.py:24-56 as written: torch tensors
    through pytorch_to_ma_core / ma_core_to_pytorch, against the PyTorch
    implementations, at the reference's tolerance."""
    from layers.ma_core_bridge import (ma_core_to_pytorch, pytorch_dense_attention,
                                       pytorch_sparse_attention, pytorch_to_ma_core)
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 6, 2, 4) for _ in range(3))
    out = mc.compute_dense_attention(pytorch_to_ma_core(q), pytorch_to_ma_core(k), pytorch_to_ma_core(v), False)
    y = ma_core_to_pytorch(out, torch.device("cpu"), torch.float32)
    torch.testing.assert_close(y, pytorch_dense_attention(q, k, v, use_causal_mask=False), rtol=1e-5, atol=1e-6)
    torch.manual_seed(1)
    q, k, v = (torch.randn(1, 10, 2, 4) for _ in range(3))
    out = mc.compute_sparse_attention(pytorch_to_ma_core(q), pytorch_to_ma_core(k), pytorch_to_ma_core(v), 2)
    y = ma_core_to_pytorch(out, torch.device("cpu"), torch.float32)
    torch.testing.assert_close(y, pytorch_sparse_attention(q, k, v, window_size=2), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("shape,w", [((2, 300, 4, 64), 64), ((1, 1000, 2, 16), 5), ((3, 17, 3, 40), 8),
                                     ((1, 129, 1, 64), 200), ((2, 50, 2, 32), -1)])
def test_sparse_matches_oracle(mc, oracle, shape, w):
    from conftest import qkv
    q, k, v = qkv(shape, 4400 + shape[1], 1.0)
    out = mc.compute_sparse_attention(_t(mc, q), _t(mc, k), _t(mc, v), window_size=w)
    ref = oracle.forward(oracle.Spec(*shape, pattern="sliding", left=w, right=w), q, k, v)
    err = float(np.abs(out.to_numpy() - ref).max())
    print(f"{shape} w={w}: max|err| vs oracle = {err:.3e}", flush=True)
    assert err <= 1e-5


def test_uniform_inputs(mc):
    """test_attention_computation.py:85-108: Q = K = 1, V = 2 gives O = 2 for
    dense and every window."""
    q, k, v = (mc.create_tensor([1, 3, 1, 4]) for _ in range(3))
    q.fill(1.0)
    k.fill(1.0)
    v.fill(2.0)
    for out in (mc.compute_dense_attention(q, k, v), mc.compute_sparse_attention(q, k, v, window_size=1),
                mc.compute_sparse_attention(q, k, v, window_size=2)):
        assert np.allclose(out.to_numpy(), 2.0, rtol=0, atol=1e-6)


def test_random_tensors_through_engine(mc):
    """test_attention_computation.py:55-70: random inputs, several windows: finite,
    shaped like the query, inputs left unchanged."""
    q, k, v = (mc.create_random_tensor([2, 64, 4, 32], mean=0.0, std=0.1) for _ in range(3))
    before = q.to_numpy()
    for w in (1, 4, 16, 64):
        out = mc.compute_sparse_attention(q, k, v, window_size=w)
        s = out.shape()
        assert (s.batch_size, s.sequence_length, s.num_heads, s.head_dim) == (2, 64, 4, 32)
        assert np.isfinite(out.to_numpy()).all()
    assert np.array_equal(before, q.to_numpy())


@pytest.mark.parametrize("dv", [8, 24, 40])
def test_value_head_dim_matches_reference_bits(mc, dv):
    """V with a head_dim of its own (ma_core.cpp:84-90, :178-183): O takes the
    value's head_dim; sparse (w=5), dense and causal against the reference's
    own outputs (tests/golden/ref_value_dim.npz)."""
    z = np.load(os.path.join(GOLDEN, "ref_value_dim.npz"))
    q, k, v = _t(mc, z["q"]), _t(mc, z["k"]), _t(mc, z[f"v_{dv}"])
    for name, out in (("sparse", mc.compute_sparse_attention(q, k, v, int(z["w"]))),
                      ("dense", mc.compute_dense_attention(q, k, v, False)),
                      ("causal", mc.compute_dense_attention(q, k, v, use_causal_mask=True))):
        got = out.to_numpy()
        ref = z[f"o_{name}_{dv}"]
        assert got.shape == ref.shape
        err = float(np.abs(got - ref).max())
        print(f"Dv={dv} {name}: max|err| vs the reference's ma_core = {err:.3e}", flush=True)
        assert err <= 1e-5


@pytest.mark.parametrize("shape,dv,w", [((2, 300, 3, 16), 40, 16), ((1, 257, 2, 64), 24, 64),
                                        ((1, 130, 2, 32), 96, 7)])
def test_value_head_dim_matches_oracle(mc, oracle, shape, dv, w):
    """Larger shapes against the oracle's column blocks (oracle.forward_value_dim)."""
    from conftest import qkv, randn
    q, k, _ = qkv(shape, 5100 + dv, 1.0)
    v = randn(shape[:3] + (dv,), 5200 + dv)
    out = mc.compute_sparse_attention(_t(mc, q), _t(mc, k), _t(mc, v), window_size=w).to_numpy()
    ref = oracle.forward_value_dim(oracle.Spec(*shape, pattern="sliding", left=w, right=w), q, k, v)
    err = float(np.abs(out - ref).max())
    print(f"{shape} Dv={dv} w={w}: max|err| vs oracle = {err:.3e}", flush=True)
    assert out.shape == ref.shape and err <= 1e-5


def test_wider_key_value_tensors(mc, oracle):
    """K and V with more batches and heads than Q: the reference reads Q's
    (batch, head) range of them with their own strides (tensor.cpp:104-114);
    fewer raise RuntimeError."""
    from conftest import randn
    q = randn((1, 50, 2, 16), 61)
    k, v = randn((2, 50, 3, 16), 62), randn((2, 50, 3, 16), 63)
    out = mc.compute_sparse_attention(_t(mc, q), _t(mc, k), _t(mc, v), window_size=4).to_numpy()
    ks, vs = np.ascontiguousarray(k[:1, :, :2]), np.ascontiguousarray(v[:1, :, :2])
    ref = oracle.forward(oracle.Spec(1, 50, 2, 16, pattern="sliding", left=4, right=4), q, ks, vs)
    assert out.shape == q.shape and float(np.abs(out - ref).max()) <= 1e-5
    with pytest.raises(RuntimeError):
        mc.compute_sparse_attention(_t(mc, k), _t(mc, q), _t(mc, k), window_size=4)
