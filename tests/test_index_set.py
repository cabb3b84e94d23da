"""INDEX_SET (explicit key set per query row, CSR), on the CPU: the oracle's
index-set path pinned against its already-pinned closed-form patterns and
against float64 textbook attention, malformed sets rejected, and the
module's CSR construction from the reference's COO entry lists."""
import numpy as np
import pytest
import torch

from conftest import qkv


def _csr_of(oracle, spec):
    """The CSR rows of any pattern, from the oracle's closed-form key lists."""
    rows = [oracle.row_keys(spec, i) for i in range(spec.N)]
    offsets = np.zeros(spec.N + 1, dtype=np.int64)
    offsets[1:] = np.cumsum([len(r) for r in rows])
    keys = np.concatenate(rows).astype(np.int32) if offsets[-1] else np.zeros(0, np.int32)
    return offsets, keys


def _random_csr(rng, N, density):
    rows = [np.flatnonzero(rng.random(N) < density) for _ in range(N)]
    offsets = np.zeros(N + 1, dtype=np.int64)
    offsets[1:] = np.cumsum([len(r) for r in rows])
    keys = np.concatenate(rows).astype(np.int32) if offsets[-1] else np.zeros(0, np.int32)
    return offsets, keys


@pytest.mark.parametrize("pattern,kw", [
    ("sliding", dict(left=3, right=2)), ("sliding", dict(left=5, right=0, dilation=3)),
    ("dense", dict(causal=True)), ("longformer", dict(left=4, right=1, num_global=3)),
])
def test_index_set_equals_closed_form_patterns(oracle, pattern, kw):
    """The same key lists as an explicit set give the same bits."""
    shape = (2, 37, 3, 16)
    q, k, v = qkv(shape, 41)
    spec = oracle.Spec(*shape, pattern=pattern, **kw)
    off, keys = _csr_of(oracle, spec)
    iset = oracle.Spec(*shape, pattern="index_set", offsets=off, keys=keys)
    assert np.array_equal(oracle.forward(iset, q, k, v), oracle.forward(spec, q, k, v))
    for a, b in zip(oracle.backward(iset, q, k, v, v), oracle.backward(spec, q, k, v, v)):
        assert np.array_equal(a, b)


def test_index_set_block_sparse_equal(oracle):
    shape = (1, 200, 2, 16)
    q, k, v = qkv(shape, 42)
    tab = oracle.block_table(5, 4, 1)
    spec = oracle.Spec(*shape, pattern="block_sparse", block_size=64, table=tab)
    off, keys = _csr_of(oracle, spec)
    iset = oracle.Spec(*shape, pattern="index_set", offsets=off, keys=keys)
    assert np.array_equal(oracle.forward(iset, q, k, v), oracle.forward(spec, q, k, v))


@pytest.mark.parametrize("density", [0.0, 0.05, 0.3, 1.0])
def test_index_set_vs_float64(oracle, density):
    """Random sets (empty rows included) against float64 masked attention."""
    rng = np.random.default_rng(int(density * 100) + 7)
    shape = (2, 29, 2, 16)
    q, k, v = qkv(shape, 43)
    off, keys = _random_csr(rng, 29, density)
    spec = oracle.Spec(*shape, pattern="index_set", offsets=off, keys=keys)
    mask = oracle.mask_dense(spec)
    assert mask.sum() == keys.size
    assert np.abs(oracle.forward(spec, q, k, v) - oracle.forward_f64(q, k, v, mask)).max() <= 1e-5
    empty = np.diff(off) == 0
    assert np.all(oracle.forward(spec, q, k, v)[:, empty] == 0.0)


@pytest.mark.parametrize("bad", ["unsorted", "repeat", "range", "offsets"])
def test_oracle_rejects_malformed_sets(oracle, bad):
    N = 6
    off = np.array([0, 2, 3, 3, 5, 6, 7], dtype=np.int64)
    keys = np.array([0, 1, 2, 1, 4, 5, 3], dtype=np.int32)
    if bad == "unsorted":
        keys[0], keys[1] = 1, 0
    elif bad == "repeat":
        keys[4] = 1
    elif bad == "range":
        keys[6] = N
    else:
        off[2] = 1
    spec = oracle.Spec(1, N, 1, 4, pattern="index_set", offsets=off, keys=keys)
    q, k, v = qkv((1, N, 1, 4), 44)
    with pytest.raises(ValueError):
        oracle.forward(spec, q, k, v)


def test_module_validation_and_coo():
    """The module's host checks and the COO -> CSR conversion (repeats dropped)."""
    import sparse_attention_cuda as ext
    N = 5
    ok_off, ok_keys = torch.tensor([0, 2, 2, 3, 5, 6]), torch.tensor([0, 4, 2, 1, 3, 0])
    ext._validated_index_set(ok_off, ok_keys, N)
    for off, keys, msg in [
        (torch.tensor([0, 2, 2, 3, 5]), ok_keys, "offsets"),
        (torch.tensor([1, 2, 2, 3, 5, 6]), ok_keys, "offsets"),
        (torch.tensor([0, 2, 1, 3, 5, 6]), ok_keys, "offsets"),
        (ok_off, torch.tensor([0, 5, 2, 1, 3, 0]), "lie in"),
        (ok_off, torch.tensor([4, 0, 2, 1, 3, 0]), "ascending"),
        (ok_off, torch.tensor([0, 4, 2, 3, 3, 0]), "ascending"),
    ]:
        with pytest.raises(RuntimeError, match=msg):
            ext._validated_index_set(off, keys, N)
    # the reference's Longformer COO lists window and global entries twice
    # (sparse_attention.cpp:234-259); the set keeps each once, sorted per row
    rows = [0, 0, 1, 1, 1, 3, 3, 3, 3, 2]
    cols = [0, 1, 0, 1, 0, 4, 0, 2, 4, 2]
    s = ext.IndexSet.from_coo(rows, cols, N, device="cpu")
    assert s.offsets.tolist() == [0, 2, 4, 5, 8, 8]
    assert s.keys.tolist() == [0, 1, 0, 1, 2, 0, 2, 4]
    assert s.num_indices == 8
    empty = ext.IndexSet.from_coo([], [], N, device="cpu")
    assert empty.offsets.tolist() == [0] * (N + 1) and empty.num_indices == 0


def test_abi_index_set_rules():
    import ma_attn
    d = ma_attn.make_desc(1, 8, 1, 16, ma_attn.F32, ma_attn.INDEX_SET, num_indices=4)
    with pytest.raises(RuntimeError, match="index_offsets"):
        ma_attn.validate(d)
    d = ma_attn.make_desc(1, 8, 1, 16, ma_attn.F32, ma_attn.INDEX_SET, index_offsets_ptr=64, num_indices=4)
    with pytest.raises(RuntimeError, match="index_keys"):
        ma_attn.validate(d)
    d = ma_attn.make_desc(1, 8, 1, 16, ma_attn.F32, ma_attn.INDEX_SET, index_offsets_ptr=64,
                          index_keys_ptr=64, num_indices=-1)
    with pytest.raises(RuntimeError, match="num_indices"):
        ma_attn.validate(d)
    d = ma_attn.make_desc(1, 8, 1, 16, ma_attn.F32, ma_attn.INDEX_SET, index_offsets_ptr=64,
                          index_keys_ptr=64, num_indices=4)
    ma_attn.validate(d)
    with pytest.raises(ValueError, match="own input"):
        ma_attn.row_keys(d, 0)


def test_bench_window_csr_matches_oracle(oracle):
    """bench.py's index_set workload builds the target's window as a set: the
    same rows as the oracle's closed form, and the key count it reports."""
    import bench
    N = 300
    off, keys = bench.window_csr(N, 63, 0)
    spec = oracle.Spec(1, N, 1, 16, pattern="sliding", left=63, right=0)
    for i in range(N):
        assert keys[off[i]:off[i + 1]].tolist() == oracle.row_keys(spec, i).tolist()
    assert int(off[-1]) == bench.key_count(N, dict(pattern="index_set", left=63, right=0))
    off, keys = bench.window_csr(50, 3, 5)
    spec = oracle.Spec(1, 50, 1, 16, pattern="sliding", left=3, right=5)
    assert all(keys[off[i]:off[i + 1]].tolist() == oracle.row_keys(spec, i).tolist() for i in range(50))


def test_index_set_transpose():
    """IndexSet's transposed set (queries per key, ascending) against brute force."""
    import sparse_attention_cuda as ext
    rng = np.random.default_rng(9)
    N = 40
    rows, cols = np.nonzero(rng.random((N, N)) < 0.15)
    s = ext.IndexSet.from_coo(rows, cols, N, device="cpu")
    t_off, t_q = s.t_offsets.tolist(), s.t_queries.tolist()
    for j in range(N):
        assert t_q[t_off[j]:t_off[j + 1]] == sorted(int(i) for i in rows[cols == j])


@pytest.mark.parametrize("pattern,kw,okw", [
    ("longformer", dict(left=7, right=2, num_global=3), dict(left=7, right=2, num_global=3)),
    ("block_sparse", dict(block_size=16), dict(block_size=16)),
])
def test_pattern_index_set_matches_oracle(oracle, pattern, kw, okw):
    """The explicit set the layer trains block-sparse / Longformer on holds
    exactly the oracle's key lists."""
    import sparse_attention_cuda as ext
    N = 90
    if pattern == "block_sparse":
        tab = oracle.block_table(4, 6, 2)
        kw = dict(kw, block_table=torch.from_numpy(tab))
        okw = dict(okw, table=tab)
    s = ext.pattern_index_set(pattern, N, "cpu", **kw)
    spec = oracle.Spec(1, N, 1, 16, pattern=pattern, **okw)
    off, keys = s.offsets.tolist(), s.keys.tolist()
    for i in range(N):
        assert keys[off[i]:off[i + 1]] == oracle.row_keys(spec, i).tolist()
