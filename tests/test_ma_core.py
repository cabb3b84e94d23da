"""The ``ma_core`` module (the reference's src/csrc pybind surface,
src/csrc/main.cpp:10-98) on the host: tensors, patterns, statistics, errors.

Patterns and statistics are held against the reference's own outputs frozen
in tests/golden (ref_patterns.npz, ref_pattern_stats.json, written by
tests/golden/make_golden.py from ma_core.cpp compiled unchanged).  The
attention entry points run on the GPU (tests/test_gpu_ma_core.py); here they
must refuse to run without one.
"""
import json
import os

import numpy as np
import pytest
import torch

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def mc():
    import ma_core
    return ma_core


def test_module_surface(mc):
    for name in ("add", "create_tensor", "create_random_tensor", "create_sliding_window_pattern",
                 "get_pattern_statistics", "compute_dense_attention", "compute_sparse_attention",
                 "SparseTensor", "TensorShape", "Tensor", "Device"):
        assert hasattr(mc, name), name
    assert "MA Transformer Core" in mc.__doc__
    assert "add" in mc.add.__doc__.lower()


def test_add_int64(mc):
    """test_ma_core_extension.py:38-146 cases."""
    assert mc.add(1, 2) == 3 and mc.add(-1, 1) == 0 and mc.add(10, -15) == -5
    assert mc.add(2 ** 31, 2 ** 31) == 2 ** 32
    assert mc.add(2 ** 60, 0) == 2 ** 60
    assert mc.add(-2 ** 63, 0) == -2 ** 63 and mc.add(2 ** 63 - 1, -1) == 2 ** 63 - 2
    for bad in (("1", 2), (1, "2"), (1.5, 2), (1, 2.5)):
        with pytest.raises(TypeError):
            mc.add(*bad)
    with pytest.raises(TypeError):
        mc.add(1)
    with pytest.raises(TypeError):
        mc.add(1, 2, 3)


@pytest.mark.parametrize("shape", [[1, 1, 1, 1], [2, 8, 4, 64], [1, 512, 8, 64], [4, 128, 12, 64], [0, 4, 2, 8]])
def test_create_tensor(mc, shape):
    t = mc.create_tensor(shape)
    n = int(np.prod(shape))
    assert t.size() == n and t.nbytes() == 4 * n and t.empty() == (n == 0)
    s = t.shape()
    assert (s.batch_size, s.sequence_length, s.num_heads, s.head_dim) == tuple(shape)
    assert s.total_elements() == n
    assert not t.to_numpy().any()


def test_create_tensor_errors(mc):
    """test_tensor_functionality.py:86-99 and :275-283."""
    for shape in ([], [1], [1, 2], [1, 2, 3], [1, 2, 3, 4, 5]):
        with pytest.raises(RuntimeError) as e:
            mc.create_tensor(shape)
        assert "4 dimensions" in str(e.value) and "batch, seq, heads, dim" in str(e.value)
    assert mc.create_tensor([1, 4, 2, 8], "CPU").size() == 64


def test_tensor_fill_copy_roundtrip(mc):
    t = mc.create_tensor([2, 3, 2, 4])
    t.fill(3.25)
    assert (t.to_numpy() == np.float32(3.25)).all()
    t.zero()
    assert not t.to_numpy().any()
    src = np.arange(48, dtype=np.float64).reshape(2, 3, 2, 4) / 7.0
    t.copy_from_numpy(src)
    out = t.to_numpy()
    assert out.dtype == np.float32 and out.shape == (2, 3, 2, 4)
    assert np.array_equal(out, src.astype(np.float32))
    out[0, 0, 0, 0] = 99.0  # to_numpy gives a copy
    assert t.to_numpy()[0, 0, 0, 0] == 0.0
    with pytest.raises(RuntimeError):
        t.copy_from_numpy(np.zeros(47, np.float32))


def test_random_tensor(mc):
    t = mc.create_random_tensor([1, 64, 8, 64], mean=1.5, std=0.5)
    x = t.to_numpy()
    assert x.dtype == np.float32 and x.shape == (1, 64, 8, 64)
    assert abs(x.mean() - 1.5) < 0.02 and abs(x.std() - 0.5) < 0.02


def test_device_enum(mc):
    assert mc.Device.CPU == mc.Device.CPU and mc.Device.CPU != mc.Device.MPS
    assert {mc.Device.CPU, mc.Device.MPS, mc.Device.CUDA, mc.Device.ROCm} == set(mc.Device)


def test_pattern_nnz_matches_reference(mc):
    """nnz of create_sliding_window_pattern against the reference's own
    (ref_patterns.npz), including (4,4) and (4,10) => 16 of
    test_tensor_functionality.py:174-179."""
    z = np.load(os.path.join(GOLDEN, "ref_patterns.npz"))
    for (n, w), nnz in zip(z["cases"], z["nnz"]):
        p = mc.create_sliding_window_pattern(int(n), int(w))
        assert p.nnz() == int(nnz), (n, w)
        assert p.shape.sequence_length == n and p.shape.batch_size == 1
        assert p.empty() == (nnz == 0)
    assert mc.create_sliding_window_pattern(4, 4).nnz() == 16
    assert mc.create_sliding_window_pattern(4, 10).nnz() == 16


def test_pattern_entries_match_reference(mc):
    """The (row, col) entries themselves, in the reference's order."""
    z = np.load(os.path.join(GOLDEN, "ref_patterns.npz"))
    for n, w in z["small"]:
        p = mc.create_sliding_window_pattern(int(n), int(w))
        assert np.array_equal(p.row_indices, z[f"rows_{n}_{w}"]), (n, w)
        assert np.array_equal(p.col_indices, z[f"cols_{n}_{w}"]), (n, w)


def test_pattern_entries_match_oracle_large(mc, oracle):
    """A long pattern row by row against the oracle's key lists."""
    n, w = 3000, 37
    p = mc.create_sliding_window_pattern(n, w)
    rows, cols = p.row_indices, p.col_indices
    offs = np.searchsorted(rows, np.arange(n + 1))
    spec = oracle.Spec(1, n, 1, 16, pattern="sliding", left=w, right=w)
    for i in (0, 1, 36, 37, 38, 1500, 2962, 2963, 2999):
        assert cols[offs[i]:offs[i + 1]].tolist() == oracle.row_keys(spec, i).tolist()


def test_pattern_edge_cases(mc):
    assert mc.create_sliding_window_pattern(0, 1).nnz() == 0
    assert mc.create_sliding_window_pattern(2, 1).nnz() == 4
    assert mc.create_sliding_window_pattern(5, -1).empty()
    with pytest.raises(TypeError):
        mc.create_sliding_window_pattern(8, 1.5)


def test_pattern_statistics_match_reference(mc):
    """get_pattern_statistics strings against the reference's own, character for character."""
    with open(os.path.join(GOLDEN, "ref_pattern_stats.json")) as f:
        golden = json.load(f)
    for key, text in golden.items():
        n, w = (int(x) for x in key.split(","))
        assert mc.get_pattern_statistics(mc.create_sliding_window_pattern(n, w)) == text, key


def test_pattern_statistics_parse(mc):
    """test_tensor_functionality.py:181-202."""
    stats = mc.get_pattern_statistics(mc.create_sliding_window_pattern(16, 3))
    lines = stats.split("\n")
    total = int([l for l in lines if "Total elements" in l][0].split(": ")[1])
    nonzero = int([l for l in lines if "Non-zero elements" in l][0].split(": ")[1])
    assert total == 256 and 0 < nonzero < total


def test_attention_shape_errors(mc):
    """The reference's messages for mismatched sequence length / head_dim
    (ma_core.cpp:72-80; test_attention_computation.py:123-145), raised before
    any device work."""
    q = mc.create_random_tensor([1, 4, 2, 8])
    with pytest.raises(RuntimeError, match="sequence length"):
        mc.compute_dense_attention(q, mc.create_random_tensor([1, 6, 2, 8]), q)
    with pytest.raises(RuntimeError, match="head dimension"):
        mc.compute_dense_attention(q, mc.create_random_tensor([1, 4, 2, 16]), q)
    # a value head_dim of its own is accepted (ma_core.cpp:84-90); fewer value
    # heads than the query's would be read out of range and raise
    with pytest.raises(RuntimeError, match="number of heads"):
        mc.compute_sparse_attention(q, q, mc.create_random_tensor([1, 4, 1, 16]), 2)
    with pytest.raises(TypeError):
        mc.compute_sparse_attention(q, q, np.zeros((1, 4, 2, 8), np.float32), 2)


def test_empty_tensors_need_no_device(mc):
    z = mc.create_tensor([0, 4, 2, 8])
    assert mc.compute_sparse_attention(z, z, z, 3).size() == 0
    # O takes the value's head_dim, also when empty
    q, v = mc.create_tensor([1, 4, 2, 8]), mc.create_tensor([1, 4, 2, 0])
    s = mc.compute_dense_attention(q, q, v).shape()
    assert (s.batch_size, s.sequence_length, s.num_heads, s.head_dim) == (1, 4, 2, 0)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the refusal on a host without a GPU")
def test_attention_refuses_without_gpu(mc):
    """No CPU arithmetic path: without a GPU the attention entry points raise."""
    q = mc.create_random_tensor([1, 8, 2, 16])
    with pytest.raises(RuntimeError, match="no GPU"):
        mc.compute_sparse_attention(q, q, q, 2)
    with pytest.raises(RuntimeError, match="no GPU"):
        mc.compute_dense_attention(q, q, q)
