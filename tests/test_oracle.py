"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own formulas:
* bit-exact equality with the reference's own compiled engine (oracle/_ref)
  and with committed golden vectors produced by it;
* a float64 dense-masked softmax(QK^T)V (textbook attention) for every pattern;
* index sets against a brute-force membership predicate and closed-form counts;
* special cases fixed by the mathematics (w=0 => O=V, constant V => O=V,
  identical keys => mean of V, window >= N => dense).
"""
import os

import numpy as np
import pytest

from conftest import qkv, randn

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _spec(O, shape, **kw):
    B, N, H, D = shape
    return O.Spec(B, N, H, D, **kw)


# ----------------------------------------------------------------- golden vectors

@pytest.mark.parametrize("name", ["ref_sparse_s10_w2", "ref_sparse_s256_w64", "ref_sparse_s33_w0"])
def test_oracle_matches_reference_golden_sparse(oracle, name):
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    B, N, H, D = g["q"].shape
    w = int(g["w"])
    o = oracle.forward(_spec(oracle, (B, N, H, D), pattern="sliding", left=w, right=w),
                       g["q"], g["k"], g["v"])
    assert np.array_equal(o, g["o"]), np.abs(o - g["o"]).max()


def test_oracle_matches_reference_golden_dense(oracle):
    g = np.load(os.path.join(GOLDEN, "ref_dense_s32.npz"))
    shape = g["q"].shape
    for causal, key in ((False, "o_full"), (True, "o_causal")):
        o = oracle.forward(_spec(oracle, shape, pattern="dense", causal=causal), g["q"], g["k"], g["v"])
        assert np.array_equal(o, g[key])


@pytest.mark.parametrize("dv", [8, 24, 40])
def test_oracle_matches_reference_golden_value_dim(oracle, dv):
    """A value head_dim of its own (ma_core.cpp:84-90): the oracle's column
    blocks against the reference's bits, sparse (w=5), dense and causal."""
    g = np.load(os.path.join(GOLDEN, "ref_value_dim.npz"))
    q, k, v = g["q"], g["k"], g[f"v_{dv}"]
    w = int(g["w"])
    for kw, key in ((dict(pattern="sliding", left=w, right=w), "o_sparse"), (dict(pattern="dense"), "o_dense"),
                    (dict(pattern="dense", causal=True), "o_causal")):
        o = oracle.forward_value_dim(_spec(oracle, q.shape, **kw), q, k, v)
        assert o.shape == v.shape
        assert np.array_equal(o, g[f"{key}_{dv}"]), (key, np.abs(o - g[f"{key}_{dv}"]).max())


def test_golden_w0_is_value(oracle):
    g = np.load(os.path.join(GOLDEN, "ref_sparse_s33_w0.npz"))
    assert np.array_equal(g["o"], g["v"])


def test_sliding_nnz_matches_reference_pattern(oracle):
    g = np.load(os.path.join(GOLDEN, "ref_patterns.npz"))
    for (n, w), nnz in zip(g["cases"], g["nnz"]):
        s = _spec(oracle, (1, int(n), 1, 1), pattern="sliding", left=int(w), right=int(w))
        total = sum(len(oracle.row_keys(s, i)) for i in range(int(n)))
        assert total == nnz
    # test_tensor_functionality.py:173-179: window >= N is fully dense
    assert dict(zip(map(tuple, g["cases"].tolist()), g["nnz"].tolist()))[(4, 4)] == 16


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "_ref",
                                                    "libma_core_ref.so")),
                    reason="reference engine not built here (oracle/_ref)")
@pytest.mark.parametrize("shape,w", [((1, 10, 2, 4), 2), ((2, 64, 3, 8), 4), ((1, 100, 2, 16), 64),
                                     ((2, 17, 2, 16), 0), ((1, 5, 1, 4), 9)])
def test_oracle_bitexact_vs_reference_engine(oracle, shape, w):
    q, k, v = qkv(shape, 100 + w)
    o = oracle.forward(_spec(oracle, shape, pattern="sliding", left=w, right=w), q, k, v)
    assert np.array_equal(o, oracle.ref_sparse_forward(q, k, v, w))


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "_ref",
                                                    "libma_core_ref.so")),
                    reason="reference engine not built here (oracle/_ref)")
@pytest.mark.parametrize("causal", [False, True])
def test_oracle_bitexact_vs_reference_dense(oracle, causal):
    shape = (2, 48, 2, 8)
    q, k, v = qkv(shape, 5)
    o = oracle.forward(_spec(oracle, shape, pattern="dense", causal=causal), q, k, v)
    assert np.array_equal(o, oracle.ref_dense_forward(q, k, v, causal))


# ----------------------------------------------------------------- float64 textbook attention

def _table(oracle, N, bs, extra, seed):
    nb = (N + bs - 1) // bs
    return oracle.block_table(seed, nb, extra)


PATTERN_CASES = [
    ("sliding", dict(left=63, right=0)),              # cfg 1 / target (causal 64)
    ("sliding", dict(left=32, right=31)),             # cfg 2
    ("sliding", dict(left=63, right=0, dilation=4)),  # cfg 5
    ("sliding", dict(left=2, right=5, dilation=3)),
    ("sliding", dict(left=-1, right=-1)),             # empty window
    ("dense", dict(causal=True)),
    ("dense", dict(causal=False)),
    ("longformer", dict(left=7, right=0, num_global=3)),
    ("longformer", dict(left=4, right=4, num_global=0)),
]


@pytest.mark.parametrize("pattern,kw", PATTERN_CASES)
def test_oracle_vs_float64(oracle, pattern, kw):
    shape = (2, 40, 2, 16)
    q, k, v = qkv(shape, 11)
    s = _spec(oracle, shape, pattern=pattern, **kw)
    o = oracle.forward(s, q, k, v)
    ref = oracle.forward_f64(q, k, v, oracle.mask_dense(s))
    assert np.abs(o - ref).max() <= 1e-5


def test_oracle_block_sparse_vs_float64(oracle):
    shape = (1, 70, 2, 8)
    q, k, v = qkv(shape, 12)
    s = _spec(oracle, shape, pattern="block_sparse", block_size=8, table=_table(oracle, 70, 8, 2, 3))
    assert np.abs(oracle.forward(s, q, k, v) - oracle.forward_f64(q, k, v, oracle.mask_dense(s))).max() <= 1e-5


# ----------------------------------------------------------------- index sets

INDEX_CASES = PATTERN_CASES + [
    ("sliding", dict(left=3, right=3)), ("sliding", dict(left=0, right=0)),
    ("sliding", dict(left=100, right=100)), ("sliding", dict(left=-2, right=5)),
    ("sliding", dict(left=9, right=2, dilation=7)), ("longformer", dict(left=127, right=0, num_global=16)),
    ("longformer", dict(left=2, right=1, num_global=50)),
]


@pytest.mark.parametrize("pattern,kw", INDEX_CASES)
@pytest.mark.parametrize("N", [1, 5, 37])
def test_row_keys_vs_bruteforce(oracle, pattern, kw, N):
    s = _spec(oracle, (1, N, 1, 1), pattern=pattern, **kw)
    for i in range(N):
        brute = [j for j in range(N) if oracle.member(s, i, j)]
        assert oracle.row_keys(s, i).tolist() == brute


def test_block_sparse_row_keys_vs_bruteforce(oracle):
    for N, bs in ((70, 8), (64, 64), (130, 64), (5, 2)):
        s = _spec(oracle, (1, N, 1, 1), pattern="block_sparse", block_size=bs,
                  table=_table(oracle, N, bs, 2, 9))
        for i in range(N):
            assert oracle.row_keys(s, i).tolist() == [j for j in range(N) if oracle.member(s, i, j)]


def _count(oracle, s):
    return sum(len(oracle.row_keys(s, i)) for i in range(s.N))


def test_key_counts_closed_form(oracle):
    # causal window 64 at N=1024: 1024*64 - 63*64/2
    assert _count(oracle, _spec(oracle, (1, 1024, 1, 1), pattern="sliding", left=63, right=0)) == 63520
    # cfg 2 per (b,h): 64 per row minus the clipped edges (32*33/2 + 31*32/2)
    assert _count(oracle, _spec(oracle, (1, 8192, 1, 1), pattern="sliding", left=32, right=31)) == \
        8192 * 64 - 32 * 33 // 2 - 31 * 32 // 2
    # target per (b,h): 65536*64 - 63*64/2
    assert _count(oracle, _spec(oracle, (1, 65536, 1, 1), pattern="sliding", left=63, right=0)) == \
        65536 * 64 - 63 * 64 // 2
    # cfg 5 per (b,h): 4 residue classes of 16384, each a causal-64 window
    assert _count(oracle, _spec(oracle, (1, 65536, 1, 1), pattern="sliding", left=63, right=0,
                                dilation=4)) == 4 * (16384 * 64 - 63 * 64 // 2)
    # cfg 4 per (b,h): 16 dense rows + rows 16..142 see i+1 keys + 144 keys after
    assert _count(oracle, _spec(oracle, (1, 32768, 1, 1), pattern="longformer", left=127, right=0,
                                num_global=16)) == 16 * 32768 + sum(i + 1 for i in range(16, 143)) + 144 * (32768 - 143)


# ----------------------------------------------------------------- block table

def test_block_table_fixture_and_invariants(oracle):
    t = oracle.block_table(1234, 256, 2)
    fix = np.fromfile(os.path.join(GOLDEN, "block_table_seed1234_nb256_r2.bin"), dtype="<i4").reshape(256, 4)
    assert np.array_equal(t, fix)
    assert t[0, 3] == -1 and t[0, 0] == 0          # row 0: {0} + 2 picks
    for r in range(256):
        row = [c for c in t[r] if c >= 0]
        assert row == sorted(set(row))                 # ascending, distinct
        assert r in row and (r == 0 or r - 1 in row)   # diagonal + previous block
        assert len(row) == (3 if r == 0 else 4)
        assert all(0 <= c < 256 for c in row)


def test_block_table_small_and_seeds(oracle):
    t = oracle.block_table(5, 3, 2)                    # only one block left to pick
    assert t[0].tolist() == [0, 1, 2, -1] and t[1].tolist() == [0, 1, 2, -1]
    assert not np.array_equal(oracle.block_table(1, 64, 2), oracle.block_table(2, 64, 2))
    # picks are spread over the whole range (uniform draw, not neighbours)
    t = oracle.block_table(99, 1024, 2)
    picks = np.concatenate([[c for c in row if c not in (r, r - 1) and c >= 0] for r, row in enumerate(t)])
    assert picks.min() < 100 and picks.max() > 900


# ----------------------------------------------------------------- special cases

def test_special_cases(oracle):
    shape = (1, 50, 2, 8)
    q, k, v = qkv(shape, 21)
    # w = 0 => O = V exactly
    assert np.array_equal(oracle.forward(_spec(oracle, shape, pattern="sliding", left=0, right=0), q, k, v), v)
    # constant V (per head) => O = V
    vc = np.broadcast_to(randn((1, 1, 2, 8), 3), shape).copy()
    o = oracle.forward(_spec(oracle, shape, pattern="sliding", left=5, right=2), q, k, vc)
    assert np.abs(o - vc).max() <= 1e-6
    # identical keys => uniform weights => mean of V over the window
    kc = np.broadcast_to(randn((1, 1, 2, 8), 4), shape).copy()
    s = _spec(oracle, shape, pattern="sliding", left=3, right=0)
    o = oracle.forward(s, q, kc, v)
    for i in (0, 1, 10, 49):
        lo = max(0, i - 3)
        assert np.abs(o[0, i] - v[0, lo:i + 1].mean(axis=0)).max() <= 1e-6
    # window covering the whole sequence == dense
    a = oracle.forward(_spec(oracle, shape, pattern="sliding", left=60, right=60), q, k, v)
    b = oracle.forward(_spec(oracle, shape, pattern="dense"), q, k, v)
    assert np.array_equal(a, b)
    # empty window => zero rows
    assert not oracle.forward(_spec(oracle, shape, pattern="sliding", left=-1, right=-1), q, k, v).any()


# ----------------------------------------------------------------- backward

def _autograd_f64(q, k, v, dout, mask):
    """torch float64 autograd of dense-masked softmax(QK^T * scale)V (CPU)."""
    import torch
    t = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v)]
    B, N, H, D = q.shape
    scale = 1.0 / float(np.sqrt(np.float32(D)))
    qh, kh, vh = (x.permute(0, 2, 1, 3) for x in t)
    s = torch.matmul(qh, kh.transpose(-1, -2).contiguous()) * scale
    m = torch.tensor(mask)
    s = s.masked_fill(~m, float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    o = torch.matmul(p, vh).permute(0, 2, 1, 3)
    o.backward(torch.tensor(dout, dtype=torch.float64))
    return [x.grad.numpy() for x in t]


@pytest.mark.parametrize("pattern,kw", PATTERN_CASES)
def test_oracle_backward_vs_autograd(oracle, pattern, kw):
    """Restated .cu:265-346 against float64 autograd of textbook attention."""
    shape = (2, 40, 2, 16)
    q, k, v = qkv(shape, 31)
    dout = randn(shape, 32)
    s = _spec(oracle, shape, pattern=pattern, **kw)
    got = oracle.backward(s, q, k, v, dout)
    ref = _autograd_f64(q, k, v, dout, oracle.mask_dense(s))
    for g, r in zip(got, ref):
        assert np.abs(g - r).max() <= 2e-5


def test_oracle_backward_block_sparse_vs_autograd(oracle):
    shape = (1, 70, 2, 8)
    q, k, v = qkv(shape, 33)
    dout = randn(shape, 34)
    s = _spec(oracle, shape, pattern="block_sparse", block_size=8, table=_table(oracle, 70, 8, 2, 3))
    for g, r in zip(oracle.backward(s, q, k, v, dout), _autograd_f64(q, k, v, dout, oracle.mask_dense(s))):
        assert np.abs(g - r).max() <= 2e-5


@pytest.mark.parametrize("pattern,kw", [("sliding", dict(left=2, right=1)), ("sliding", dict(left=3, right=0, dilation=2)),
                                        ("dense", dict(causal=True)), ("longformer", dict(left=2, right=0, num_global=2))])
def test_oracle_backward_finite_differences(oracle, pattern, kw):
    """Central differences of the float64 forward, L = sum(O * dout): no gradient formula involved."""
    shape = (1, 7, 1, 3)
    q, k, v = qkv(shape, 35)
    dout = randn(shape, 36)
    s = _spec(oracle, shape, pattern=pattern, **kw)
    mask = oracle.mask_dense(s)
    got = oracle.backward(s, q, k, v, dout)
    x = [a.astype(np.float64) for a in (q, k, v)]
    eps = 1e-6
    for which in range(3):
        fd = np.zeros_like(x[which])
        for idx in np.ndindex(*shape):
            for sgn in (1, -1):
                y = [a.copy() for a in x]
                y[which][idx] += sgn * eps
                fd[idx] += sgn * float((oracle.forward_f64(*y, mask) * dout).sum()) / (2 * eps)
        assert np.abs(got[which] - fd).max() <= 2e-5, which


def test_oracle_backward_special_cases(oracle):
    shape = (2, 30, 2, 8)
    q, k, v = qkv(shape, 37)
    dout = randn(shape, 38)
    # w = 0: O = V, so dV = dout and dQ = dK = 0 exactly
    dq, dk, dv = oracle.backward(_spec(oracle, shape, pattern="sliding", left=0, right=0), q, k, v, dout)
    assert np.array_equal(dv, dout) and not dq.any() and not dk.any()
    # empty window: all zero
    assert not any(g.any() for g in oracle.backward(_spec(oracle, shape, pattern="sliding", left=-1, right=-1),
                                                    q, k, v, dout))
    # rows of P sum to 1 => sum_j dV_j = sum_i dout_i; rows of dS sum to 0 => sum_j dK_j = 0
    dq, dk, dv = oracle.backward(_spec(oracle, shape, pattern="sliding", left=4, right=2, dilation=2), q, k, v, dout)
    assert np.abs(dv.sum(axis=1) - dout.sum(axis=1)).max() <= 1e-4
    assert np.abs(dk.sum(axis=1)).max() <= 1e-4
