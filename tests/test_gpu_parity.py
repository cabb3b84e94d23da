"""GPU parity: the HIP kernels (through the C-ABI, via sparse_attention_cuda)
against the CPU oracle on identical seeded inputs.

Tolerances (north_star): max-abs <= 1e-5 for float32; <= 2e-2 for bfloat16 /
float16, measured against the float32 oracle run on the upcast 16-bit inputs.
Full-size benchmark configs compare the oracle on sampled row ranges (first,
middle and last rows of some heads) -- the oracle computes exactly those rows.
"""
import os

import numpy as np
import pytest
import torch

from conftest import qkv

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import sparse_attention_cuda
    return sparse_attention_cuda


def _dev(x, dtype):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dtype)
    return t.to("cuda")


def _inputs(shape, seed, dtype, scale=1.0):
    """Device tensors in dtype plus the float32 values the oracle must see."""
    q, k, v = qkv(shape, seed, scale)
    tq, tk, tv = (_dev(a, dtype) for a in (q, k, v))
    up = [t.float().cpu().numpy() for t in (tq, tk, tv)] if dtype != torch.float32 else [q, k, v]
    return (tq, tk, tv), up


def _max_err(out, ref, heads=None, rows=None):
    o = out.float().cpu().numpy()
    h0, h1 = heads if heads else (0, o.shape[2])
    i0, i1 = rows if rows else (0, o.shape[1])
    a = o[:, i0:i1, h0:h1]
    b = ref[:, i0:i1, h0:h1]
    assert np.isfinite(a).all(), "non-finite output"
    return float(np.abs(a - b).max()) if a.size else 0.0


def _check_sampled(oracle, spec, up, out, dtype, heads, row_ranges):
    for rows in row_ranges:
        ref = oracle.forward(spec, *up, heads=heads, rows=rows)
        err = _max_err(out, ref, heads, rows)
        print(f"  rows {rows} heads {heads}: max|err| = {err:.3e}", flush=True)
        assert err <= TOL[dtype], (rows, err)


# ------------------------------------------------------- reference test cases

@pytest.mark.parametrize("S", [1, 17, 33, 64, 127])
@pytest.mark.parametrize("W", [0, 1, 4, 8])
def test_forward_launch_edgecases(ext, oracle, S, W):
    """test_cuda_sparse_kernel_launch.py:15-30 shapes, against the oracle at 1e-5."""
    from layers.ma_core_bridge import pytorch_sparse_attention
    (q, k, v), up = _inputs((2, S, 2, 16), 123 + S + W, torch.float32)
    y = ext.forward(q, k, v, W)
    spec = oracle.Spec(2, S, 2, 16, pattern="sliding", left=W, right=W)
    assert _max_err(y, oracle.forward(spec, *up)) <= 1e-5
    torch.testing.assert_close(y, pytorch_sparse_attention(q, k, v, window_size=W), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("name", ["ref_sparse_s10_w2", "ref_sparse_s256_w64", "ref_sparse_s33_w0"])
def test_forward_matches_reference_golden(ext, name):
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    q, k, v = (_dev(g[x], torch.float32) for x in "qkv")
    y = ext.forward(q, k, v, int(g["w"])).cpu().numpy()
    assert np.abs(y - g["o"]).max() <= 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_dense_forward_golden_and_oracle(ext, oracle, causal):
    g = np.load(os.path.join(GOLDEN, "ref_dense_s32.npz"))
    q, k, v = (_dev(g[x], torch.float32) for x in "qkv")
    y = ext.dense_forward(q, k, v, causal).cpu().numpy()
    assert np.abs(y - g["o_causal" if causal else "o_full"]).max() <= 1e-5
    (q, k, v), up = _inputs((2, 300, 3, 40), 77, torch.float32)
    y = ext.dense_forward(q, k, v, causal)
    spec = oracle.Spec(2, 300, 3, 40, pattern="dense", causal=causal)
    assert _max_err(y, oracle.forward(spec, *up)) <= 1e-5


@pytest.mark.parametrize("shape,W", [((1, 32, 2, 16), 1), ((2, 64, 4, 32), 8), ((1, 50, 3, 5), 3),
                                     ((1, 40, 2, 130), 6), ((2, 65, 2, 64), 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_forward_shapes_dtypes(ext, oracle, shape, W, dtype):
    (q, k, v), up = _inputs(shape, 31, dtype)
    y = ext.forward(q, k, v, W)
    assert y.dtype == dtype and y.shape == q.shape
    spec = oracle.Spec(*shape, pattern="sliding", left=W, right=W)
    assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]


# ------------------------------------------------------- streaming kernels, window / length / dilation geometry

@pytest.mark.parametrize("N,left,right,dil", [
    (1, 63, 0, 1), (63, 63, 0, 1), (64, 63, 0, 1), (65, 63, 0, 1), (300, 63, 0, 1),
    (257, 32, 31, 1), (200, 64, 64, 1), (130, 0, 0, 1), (190, 5, 200, 1), (77, 300, 0, 1),
    (1000, 63, 0, 4), (999, 10, 3, 3), (500, 150, 150, 2), (129, 1, 1, 7),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_band_kernel_geometry(ext, oracle, N, left, right, dil, dtype):
    shape = (2, N, 3, 64)
    (q, k, v), up = _inputs(shape, N + left + dil, dtype)
    y = ext.sliding_forward(q, k, v, left, right, dil)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right, dilation=dil)
    assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]


@pytest.mark.parametrize("N,D,left,right", [(1000, 24, 40, 20), (777, 8, 100, 50), (300, 16, 63, 0),
                                             (129, 32, 0, 5), (64, 13, 3, 3)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_narrow_head_geometry(ext, oracle, N, D, left, right, dtype):
    """head_dim <= 32 sliding windows (one query per lane, window split over 4 waves)."""
    shape = (2, N, 3, D)
    (q, k, v), up = _inputs(shape, 1500 + N + D, dtype)
    y = ext.sliding_forward(q, k, v, left, right)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right)
    assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]


@pytest.mark.parametrize("shape,left,right,dtype", [((2, 16384, 8, 16), 63, 0, torch.float32),
                                                    ((1, 9000, 64, 24), 40, 20, torch.bfloat16)])
def test_narrow_head_large_grid(ext, oracle, shape, left, right, dtype):
    """head_dim <= 32 on large grids (thousands of workgroups), against the oracle."""
    (q, k, v), up = _inputs(shape, 1700 + shape[1], dtype)
    y = ext.sliding_forward(q, k, v, left, right)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right)
    assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]


# ------------------------------------------------------- block-sparse and Longformer kernels

def _random_table(nb, width, seed, rng_extra_pad=True):
    """Ascending, -1 padded block table with 1..width valid entries per row."""
    rng = np.random.default_rng(seed)
    tab = np.full((nb, width), -1, dtype=np.int32)
    for r in range(nb):
        n = int(rng.integers(1, width + 1)) if rng_extra_pad else width
        n = min(n, nb)
        tab[r, :n] = np.sort(rng.choice(nb, size=n, replace=False))
    return tab


@pytest.mark.parametrize("N", [64, 65, 200, 1000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_block_sparse_geometry(ext, oracle, N, dtype):
    shape = (2, N, 3, 64)
    (q, k, v), up = _inputs(shape, 500 + N, dtype, scale=0.5)
    nb = (N + 63) // 64
    for tab in (ext.make_block_table(77 + N, nb, 2).numpy(), _random_table(nb, 5, N)):
        y = ext.block_sparse_forward(q, k, v, torch.from_numpy(tab), 64)
        spec = oracle.Spec(*shape, pattern="block_sparse", block_size=64, table=tab)
        assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]


@pytest.mark.parametrize("N,G,left,right", [
    (16, 16, 127, 0), (17, 16, 127, 0), (100, 5, 127, 0), (300, 16, 127, 0), (1000, 16, 127, 0),
    (257, 1, 3, 0), (300, 7, 20, 9), (130, 16, 200, 0), (500, 3, 64, 64), (10, 4, 2, 1),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_longformer_geometry(ext, oracle, N, G, left, right, dtype):
    shape = (2, N, 3, 64)
    (q, k, v), up = _inputs(shape, 900 + N + G, dtype)
    y = ext.longformer_forward(q, k, v, left, right, G)
    spec = oracle.Spec(*shape, pattern="longformer", left=left, right=right, num_global=G)
    assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]


@pytest.mark.parametrize("shape,G,left,dtype", [
    ((1, 8192, 1, 64), 16, 127, torch.bfloat16),  # one stream: 128 chunks of one tile
    ((1, 3000, 2, 64), 5, 40, torch.float16),     # 47 chunks: a second batch of 15
    ((1, 8192, 2, 64), 16, 127, torch.float32),   # fp32 (one workgroup per CU): 128 chunks of one tile
])
def test_longformer_many_chunks(ext, oracle, shape, G, left, dtype):
    """Few (batch, head) streams over a long sequence: the grid splits each
    stream into more than 32 chunks, so longformer_combine merges each global
    row's partials in several batches of 32 (the last one ragged).  Whole
    output against the oracle, global rows included."""
    (q, k, v), up = _inputs(shape, 950 + shape[1] + G, dtype)
    y = ext.longformer_forward(q, k, v, left, 0, G)
    spec = oracle.Spec(*shape, pattern="longformer", left=left, right=0, num_global=G)
    ref = oracle.forward(spec, *up)
    assert _max_err(y, ref, rows=(0, G)) <= TOL[dtype]
    assert _max_err(y, ref) <= TOL[dtype]


@pytest.mark.parametrize("N", [1, 63, 64, 65, 200, 1000])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dense_mfma_geometry(ext, oracle, N, causal, dtype):
    """dense_forward at head_dim 64 (the block kernel with every block; fp32
    on 16x16x4 MFMA with two-slot blocks)."""
    shape = (2, N, 3, 64)
    (q, k, v), up = _inputs(shape, 1300 + N + causal, dtype)
    y = ext.dense_forward(q, k, v, causal)
    spec = oracle.Spec(*shape, pattern="dense", causal=causal)
    assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dense_mfma_long(ext, oracle, causal, dtype):
    """B=2 H=4 N=8000: many key blocks per row, causal rows in reverse order."""
    (q, k, v), up = _inputs((2, 8000, 4, 64), 1400 + causal, dtype)
    y = ext.dense_forward(q, k, v, causal)
    spec = oracle.Spec(2, 8000, 4, 64, pattern="dense", causal=causal)
    _check_sampled(oracle, spec, up, y, dtype, (0, 4), [(0, 70), (3990, 4100), (7900, 8000)])


@pytest.mark.parametrize("width,padded", [(2, False), (2, True), (4, False), (4, True), (3, True)])
def test_block_sparse_many_rows(ext, oracle, width, padded):
    """4032 (batch, head, block) rows, renumbered over the XCDs, N not a
    multiple of 64; full and -1 padded tables of several widths."""
    shape = (4, 4000, 16, 64)
    (q, k, v), up = _inputs(shape, 4321 + width, torch.bfloat16, scale=0.5)
    nb = (4000 + 63) // 64
    tab = _random_table(nb, width, 99 + width, rng_extra_pad=padded)
    # a checked device-resident table for the padded cases, a plain tensor otherwise
    arg = ext.BlockTable(torch.from_numpy(tab), 4000, 64) if padded else torch.from_numpy(tab)
    y = ext.block_sparse_forward(q, k, v, arg, 64)
    spec = oracle.Spec(*shape, pattern="block_sparse", block_size=64, table=tab)
    _check_sampled(oracle, spec, up, y, torch.bfloat16, (0, 2), [(0, 4000)])
    _check_sampled(oracle, spec, up, y, torch.bfloat16, (15, 16), [(0, 4000)])


@pytest.mark.parametrize("shape", [
    (1, 64, 1, 64),     # one row
    (1, 448, 1, 64),    # 7 rows: fewer than the 8 XCDs
    (3, 190, 3, 64),    # 27 rows, not a multiple of 8
    (1, 6400, 11, 64),  # 1100 rows
])
def test_block_sparse_every_row(ext, oracle, shape):
    """Row counts around the XCD renumbering (tables of <= 4 entries): every
    (batch, head, block) row is computed once.  All rows are checked."""
    B, N, H, D = shape
    (q, k, v), up = _inputs(shape, 7000 + N + H, torch.bfloat16, scale=0.5)
    nb = (N + 63) // 64
    for tab in (ext.make_block_table(31 + N, nb, min(2, max(nb - 2, 0))).numpy(), _random_table(nb, 4, N)):
        y = ext.block_sparse_forward(q, k, v, torch.from_numpy(tab), 64)
        spec = oracle.Spec(*shape, pattern="block_sparse", block_size=64, table=tab)
        assert _max_err(y, oracle.forward(spec, *up)) <= TOL[torch.bfloat16]


def test_block_table_validation(ext):
    q = torch.randn(1, 128, 1, 64, device="cuda", dtype=torch.bfloat16)
    ok = torch.tensor([[0, -1, -1], [0, 1, -1]], dtype=torch.int32)
    ext.block_sparse_forward(q, q, q, ok, 64)  # multiple -1 pads are fine
    for bad in ([[1, 0, -1], [0, 1, -1]], [[-1, 0, -1], [0, 1, -1]], [[0, 2, -1], [0, 1, -1]],
                [[0, 0, -1], [0, 1, -1]]):
        with pytest.raises(RuntimeError):
            ext.block_sparse_forward(q, q, q, torch.tensor(bad, dtype=torch.int32), 64)
        with pytest.raises(RuntimeError):
            ext.BlockTable(torch.tensor(bad, dtype=torch.int32), 128, 64)
    bt = ext.BlockTable(ok, 128, 64)
    torch.testing.assert_close(ext.block_sparse_forward(q, q, q, bt, 64), ext.block_sparse_forward(q, q, q, ok, 64))
    with pytest.raises(RuntimeError):  # made for another sequence length
        ext.block_sparse_forward(q[:, :64].contiguous(), q[:, :64].contiguous(), q[:, :64].contiguous(), bt, 64)


# ------------------------------------------------------- benchmark configs

def test_cfg1_causal_fp32(ext, oracle):
    """B=1 H=4 N=1024 D=16, causal window 64, float32 -- whole output."""
    (q, k, v), up = _inputs((1, 1024, 4, 16), 1235, torch.float32)
    y = ext.sliding_forward(q, k, v, 63, 0)
    spec = oracle.Spec(1, 1024, 4, 16, pattern="sliding", left=63, right=0)
    err = _max_err(y, oracle.forward(spec, *up))
    print(f"  cfg1 fp32 whole output: max|err| = {err:.3e}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cfg2_symmetric(ext, oracle, dtype):
    """B=4 H=8 N=8192 D=64, keys [i-32, i+31]."""
    (q, k, v), up = _inputs((4, 8192, 8, 64), 1236, dtype)
    y = ext.sliding_forward(q, k, v, 32, 31)
    spec = oracle.Spec(4, 8192, 8, 64, pattern="sliding", left=32, right=31)
    _check_sampled(oracle, spec, up, y, dtype, (0, 2), [(0, 300), (4000, 4200), (7900, 8192)])
    _check_sampled(oracle, spec, up, y, dtype, (7, 8), [(0, 8192)])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cfg5_dilated(ext, oracle, dtype):
    """B=1 H=8 N=65536 D=64, keys i-4k for k=0..63."""
    (q, k, v), up = _inputs((1, 65536, 8, 64), 1239, dtype)
    y = ext.sliding_forward(q, k, v, 63, 0, 4)
    spec = oracle.Spec(1, 65536, 8, 64, pattern="sliding", left=63, right=0, dilation=4)
    _check_sampled(oracle, spec, up, y, dtype, (0, 8), [(0, 600), (30000, 30300), (65000, 65536)])
    _check_sampled(oracle, spec, up, y, dtype, (5, 6), [(0, 65536)])  # one whole head


def test_target_causal_bf16(ext, oracle):
    """The headline workload: B=1 H=8 N=65536 D=64, causal w=64, bf16."""
    (q, k, v), up = _inputs((1, 65536, 8, 64), 1240, torch.bfloat16)
    y = ext.sliding_forward(q, k, v, 63, 0)
    spec = oracle.Spec(1, 65536, 8, 64, pattern="sliding", left=63, right=0)
    _check_sampled(oracle, spec, up, y, torch.bfloat16, (0, 8), [(0, 400), (32700, 33000), (65300, 65536)])
    _check_sampled(oracle, spec, up, y, torch.bfloat16, (3, 4), [(0, 65536)])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_cfg3_block_sparse(ext, oracle, dtype):
    """B=2 H=8 N=16384 D=64, block 64, diag + previous + 2 seeded blocks; inputs N(0,1)*0.5
    (BASELINE's bf16, and fp16 on the same kernel)."""
    (q, k, v), up = _inputs((2, 16384, 8, 64), 1237, dtype, scale=0.5)
    table = ext.make_block_table(1234, 256, 2)
    y = ext.block_sparse_forward(q, k, v, table, 64)
    spec = oracle.Spec(2, 16384, 8, 64, pattern="block_sparse", block_size=64, table=table.numpy())
    _check_sampled(oracle, spec, up, y, dtype, (0, 2), [(0, 256), (8000, 8256), (16128, 16384)])
    _check_sampled(oracle, spec, up, y, dtype, (6, 7), [(0, 16384)])  # one whole head


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_cfg4_longformer(ext, oracle, dtype):
    """B=2 H=12 N=32768 D=64, causal w=128 plus 16 global tokens (BASELINE's bf16, fp16 on
    the same kernel, and fp32 on its fp32 instantiation at 1e-5)."""
    (q, k, v), up = _inputs((2, 32768, 12, 64), 1238, dtype)
    y = ext.longformer_forward(q, k, v, 127, 0, 16)
    spec = oracle.Spec(2, 32768, 12, 64, pattern="longformer", left=127, right=0, num_global=16)
    _check_sampled(oracle, spec, up, y, dtype, (0, 2), [(0, 300), (16000, 16100), (32700, 32768)])
    _check_sampled(oracle, spec, up, y, dtype, (9, 10), [(0, 32768)])  # one whole head, globals included


# ------------------------------------------------------- properties at full size

def test_target_properties(ext):
    """Constant V => O = V; determinism; independence from other heads' data."""
    torch.manual_seed(0)
    q = torch.randn(1, 65536, 8, 64, device="cuda", dtype=torch.bfloat16)
    k = torch.randn_like(q)
    vc = torch.randn(1, 1, 8, 64, device="cuda", dtype=torch.bfloat16).expand(1, 65536, 8, 64).contiguous()
    y = ext.sliding_forward(q, k, vc, 63, 0)
    assert (y.float() - vc.float()).abs().max().item() <= 2e-2
    v = torch.randn_like(q)
    y1 = ext.sliding_forward(q, k, v, 63, 0)
    y2 = ext.sliding_forward(q, k, v, 63, 0)
    assert torch.equal(y1, y2)
    v2 = v.clone()
    v2[:, :, 5] = 7.0  # perturb head 5 only
    y3 = ext.sliding_forward(q, k, v2, 63, 0)
    assert torch.equal(y3[:, :, :5], y1[:, :, :5]) and torch.equal(y3[:, :, 6:], y1[:, :, 6:])


def test_side_stream(ext, oracle):
    (q, k, v), up = _inputs((1, 512, 2, 64), 5, torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        y = ext.sliding_forward(q, k, v, 63, 0)
    torch.cuda.current_stream().wait_stream(s)
    spec = oracle.Spec(1, 512, 2, 64, pattern="sliding", left=63, right=0)
    assert _max_err(y, oracle.forward(spec, *up)) <= 2e-2


# ------------------------------------------------------- errors (reference TORCH_CHECK contract)

def test_errors(ext):
    q = torch.randn(1, 16, 2, 8, device="cuda")
    with pytest.raises(RuntimeError):
        ext.forward(q.transpose(1, 2), q.transpose(1, 2), q.transpose(1, 2), 2)  # non-contiguous
    with pytest.raises(RuntimeError):
        ext.forward(q.cpu(), q.cpu(), q.cpu(), 2)
    with pytest.raises(RuntimeError):
        ext.forward(q, q.half(), q, 2)
    with pytest.raises(RuntimeError):
        ext.forward(q, q[:, :8].contiguous(), q, 2)
    with pytest.raises(RuntimeError):
        ext.forward(q[0], q[0], q[0], 2)
    with pytest.raises(RuntimeError):
        ext.forward(q.double(), q.double(), q.double(), 2)
    with pytest.raises(RuntimeError):
        ext.sliding_forward(q, q, q, 3, 3, 0)
    with pytest.raises(RuntimeError):
        ext.block_sparse_forward(q, q, q, torch.zeros(3, 2, dtype=torch.int32), 8)  # wrong rows
    y = ext.forward(q, q, q, 2)  # still usable after errors
    assert torch.isfinite(y).all()


# ------------------------------------------------------- bridge on the device

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bridge_eval_uses_native(ext, oracle, dtype):
    from layers.ma_core_bridge import MACoreAttention
    (q, k, v), up = _inputs((2, 200, 4, 64), 9, dtype)
    attn = MACoreAttention(sparse=True, window_size=8, fallback_training=False).eval()
    y = attn(q, k, v)
    spec = oracle.Spec(2, 200, 4, 64, pattern="sliding", left=8, right=8)
    assert y.dtype == dtype
    assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]
    causal = MACoreAttention(sparse=True, window_size=64, causal=True).eval()
    y = causal(q, k, v)
    spec = oracle.Spec(2, 200, 4, 64, pattern="sliding", left=63, right=0)
    assert _max_err(y, oracle.forward(spec, *up)) <= TOL[dtype]
    dense = MACoreAttention(sparse=False, use_causal_mask=True).eval()
    spec = oracle.Spec(2, 200, 4, 64, pattern="dense", causal=True)
    assert _max_err(dense(q, k, v), oracle.forward(spec, *up)) <= TOL[dtype]


def test_bridge_backward_on_device(ext):
    from layers.ma_core_bridge import MACoreAttention, pytorch_sparse_attention
    torch.manual_seed(3)
    q, k, v = (torch.randn(1, 40, 2, 16, device="cuda", requires_grad=True) for _ in range(3))
    attn = MACoreAttention(sparse=True, window_size=4, fallback_training=False)
    attn(q, k, v).sum().backward()
    g = [t.grad.clone() for t in (q, k, v)]
    q2, k2, v2 = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    pytorch_sparse_attention(q2, k2, v2, 4).sum().backward()
    for a, b in zip(g, (q2.grad, k2.grad, v2.grad)):
        assert (a - b).abs().max().item() <= 1e-4


def test_timed_entry_points(ext):
    """ma_attn_forward_timed / ma_attn_backward_timed: same results as the
    untimed calls, and the event pair brackets the kernels (positive,
    shorter than the host-side wall time of the synchronised call)."""
    import time
    q, k, v, g = (torch.randn(1, 4096, 4, 64, device="cuda", dtype=torch.bfloat16) for _ in range(4))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    torch.cuda.synchronize()
    ref = ext.sliding_forward(q, k, v, 63, 0)
    t = time.perf_counter()
    with ext.kernel_events(e0, e1):
        out = ext.sliding_forward(q, k, v, 63, 0)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t) * 1e3
    assert torch.equal(out, ref)
    assert 0.0 < e0.elapsed_time(e1) <= wall_ms
    ref_g = ext.sliding_backward(q, k, v, g, 63, 0)
    with ext.kernel_events(e0, e1):
        got_g = ext.sliding_backward(q, k, v, g, 63, 0)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(got_g, ref_g))
    assert e0.elapsed_time(e1) > 0.0


@pytest.mark.parametrize("shape", [(1, 0, 2, 64), (0, 37, 2, 64), (2, 0, 3, 16)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_empty_inputs(ext, shape, dtype):
    """Empty batches or sequences launch nothing and return empty outputs of
    the inputs' shape, forward and backward, on every entry point."""
    q = torch.randn(shape, device="cuda").to(dtype)
    for y in (ext.forward(q, q, q, 8), ext.dense_forward(q, q, q, True), ext.sliding_forward(q, q, q, 63, 0),
              ext.longformer_forward(q, q, q, 127, 0, 16)):
        assert y.shape == q.shape and y.dtype == dtype
    for grads in (ext.backward(q, q, q, q, 8), ext.dense_backward(q, q, q, q, True),
                  ext.sliding_backward(q, q, q, q, 32, 31)):
        assert [tuple(g.shape) for g in grads] == [tuple(shape)] * 3
    torch.cuda.synchronize()
    y = ext.forward(*[torch.randn(1, 16, 1, 16, device="cuda")] * 3, 2)  # still usable afterwards
    assert torch.isfinite(y).all()
