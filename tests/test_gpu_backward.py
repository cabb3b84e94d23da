"""GPU parity of the HIP backward (ma_attn_backward through sparse_attention_cuda)
against the CPU oracle's restatement of the reference backward kernel
(src/cuda/sparse_attention_kernel.cu:265-346; dense :104-175).

Tolerances: float32 max-abs <= 1e-4 (sums of up to a few hundred products per
gradient element, in another order than the oracle's); bfloat16 / float16
per element |err| <= 1e-2 + 1e-2 * |ref| -- the kernels compute in fp32 on the
16-bit inputs (16-bit P and dS operands on the MFMA path) and round each
gradient once to the input dtype (2^-8 relative for bf16).  The reference's own tests compare against torch autograd at
1e-3 / 2e-3 (test_cuda_backward.py:75-101, test_cuda_extensive.py:168-193);
those checks are repeated here as written.
"""
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


def _dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).to("cuda")


def _case(shape, seed, dtype):
    q, k, v = qkv(shape, seed)
    g = randn(shape, seed + 1)
    dev = [_dev(a, dtype) for a in (q, k, v, g)]
    up = [t.float().cpu().numpy() for t in dev]
    return dev, up


def _check(got, ref, dtype):
    for name, a, b in zip("qkv", got, ref):
        check_grad("d" + name, a.float().cpu().numpy(), b, dtype == torch.float32)


# ------------------------------------------------------- the reference's own tests

def _torch_dense(q, k, v, causal=False):
    B, S, H, D = q.shape
    scale = 1.0 / (D ** 0.5)
    qh, kh, vh = ((t * scale if i == 0 else t).transpose(1, 2).contiguous() for i, t in enumerate((q, k, v)))
    s = torch.matmul(qh, kh.transpose(-2, -1).contiguous())
    if causal:
        s = s.masked_fill(~torch.tril(torch.ones(S, S, dtype=torch.bool, device=s.device)), -1e9)
    return torch.matmul(torch.softmax(s, dim=-1), vh).transpose(1, 2).contiguous()


def _torch_sparse(q, k, v, window):
    B, S, H, D = q.shape
    scale = 1.0 / (D ** 0.5)
    i = torch.arange(S, device=q.device)
    mask = (i.view(1, -1) >= i.view(-1, 1) - window) & (i.view(1, -1) <= i.view(-1, 1) + window)
    qh, kh, vh = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    s = torch.matmul(qh * scale, kh.transpose(-2, -1).contiguous()).masked_fill(~mask, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vh).transpose(1, 2).contiguous()


def _ref_grads(fn, q, k, v, loss):
    q2, k2, v2 = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    loss(fn(q2, k2, v2)).backward()
    return q2.grad, k2.grad, v2.grad


def test_reference_dense_backward(ext):
    """test_cuda_backward.py:48-73: B=1 S=8 H=2 D=4, atol = rtol = 1e-3."""
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 8, 2, 4, device="cuda") for _ in range(3))
    dO = torch.ones_like(q)  # d(out.sum())/d(out)
    got = ext.dense_backward(q, k, v, dO, False)
    for a, b in zip(got, _ref_grads(_torch_dense, q, k, v, lambda o: o.sum())):
        assert torch.allclose(a, b, atol=1e-3, rtol=1e-3)


def test_reference_sparse_backward(ext):
    """test_cuda_backward.py:75-101: B=1 S=10 H=2 D=4, window 2, atol = rtol = 1e-3."""
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 10, 2, 4, device="cuda") for _ in range(3))
    got = ext.backward(q, k, v, torch.ones_like(q), 2)
    for a, b in zip(got, _ref_grads(lambda a, b, c: _torch_sparse(a, b, c, 2), q, k, v, lambda o: o.sum())):
        assert torch.allclose(a, b, atol=1e-3, rtol=1e-3)


def test_reference_bridge_training_grads(ext):
    """test_cuda_extensive.py:168-193: MACoreAttention(sparse, W=3, fallback_training=False)."""
    from layers.ma_core_bridge import MACoreAttention
    torch.manual_seed(10)
    q, k, v = (torch.randn(2, 17, 2, 8, device="cuda", requires_grad=True) for _ in range(3))
    attn = MACoreAttention(sparse=True, window_size=3, fallback_training=False)
    attn(q, k, v).sin().pow(2).mean().backward()
    ref = _ref_grads(lambda a, b, c: _torch_sparse(a, b, c, 3), q, k, v, lambda o: o.sin().pow(2).mean())
    for a, b in zip((q.grad, k.grad, v.grad), ref):
        assert (a - b).abs().max().item() < 2e-3


# ------------------------------------------------------- against the oracle

@pytest.mark.parametrize("N,left,right,dil", [
    (1, 3, 3, 1), (10, 2, 2, 1), (65, 63, 0, 1), (300, 63, 0, 1), (257, 32, 31, 1),
    (200, 0, 0, 1), (190, 5, 40, 1), (333, 63, 0, 4), (129, 2, 7, 3), (50, -1, -1, 1),
    # one-sided bands (left or right negative): the gather kernels over the
    # transposed band, on non-empty key sets
    (97, -2, 9, 1), (120, 7, -3, 2),
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_sliding_backward_geometry(ext, oracle, N, left, right, dil, dtype):
    shape = (2, N, 3, 64)
    (q, k, v, g), up = _case(shape, 700 + N + left + dil, dtype)
    got = ext.sliding_backward(q, k, v, g, left, right, dil)
    assert all(t.dtype == dtype and t.shape == q.shape for t in got)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right, dilation=dil)
    _check(got, oracle.backward(spec, *up), dtype)


@pytest.mark.parametrize("shape", [(1, 7, 2, 16), (2, 33, 2, 40), (1, 20, 1, 130)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_backward_geometry(ext, oracle, shape, causal, dtype):
    (q, k, v, g), up = _case(shape, 800 + shape[1] + causal, dtype)
    got = ext.dense_backward(q, k, v, g, causal)
    spec = oracle.Spec(*shape, pattern="dense", causal=causal)
    _check(got, oracle.backward(spec, *up), dtype)


@pytest.mark.parametrize("N", [1, 64, 65, 300])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dense_backward_mfma(ext, oracle, N, causal, dtype):
    """head_dim 64: the MFMA backward with the band [i-(N-1), i(+N-1)]."""
    shape = (2, N, 3, 64)
    (q, k, v, g), up = _case(shape, 850 + N + causal, dtype)
    got = ext.dense_backward(q, k, v, g, causal)
    _check(got, oracle.backward(oracle.Spec(*shape, pattern="dense", causal=causal), *up), dtype)


@pytest.mark.parametrize("N,left,right,dil", [(300, 63, 0, 1), (257, 32, 31, 4), (129, 2, 7, 3)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sliding_backward_row_kernels(ext, oracle, kernel_env, N, left, right, dil, dtype):
    """The VALU row kernels for head_dim 64 (the MFMA path's cases), forced
    with MA_ATTN_KERNEL=rows, stay correct."""
    kernel_env("MA_ATTN_KERNEL", "rows")
    shape = (2, N, 3, 64)
    (q, k, v, g), up = _case(shape, 860 + N, dtype)
    got = ext.sliding_backward(q, k, v, g, left, right, dil)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right, dilation=dil)
    _check(got, oracle.backward(spec, *up), dtype)


@pytest.mark.parametrize("N,H,left,right,dil", [(5000, 16, 63, 0, 1), (4099, 8, 63, 0, 4), (3000, 8, 0, 0, 1),
                                                 (2500, 8, 10, 0, 3), (3333, 8, 0, 64, 1), (4000, 8, 32, 31, 1),
                                                 (3001, 8, 32, 31, 4), (2000, 8, 5, 40, 1), (2222, 8, 47, 16, 2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_chunked(ext, oracle, N, H, left, right, dil, dtype):
    """Bands of at most two blocks stream several tiles per workgroup (the
    last chunk of each residue class ragged): whole gradients vs the oracle.
    fp32 runs the same kernels on 16x16x4 MFMA with two-slot blocks."""
    shape = (2, N, H, 64)
    (q, k, v, g), up = _case(shape, 880 + N + dil, dtype)
    got = ext.sliding_backward(q, k, v, g, left, right, dil)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right, dilation=dil)
    _check(got, oracle.backward(spec, *up), dtype)


@pytest.mark.parametrize("N,H,left,right,dil", [(5000, 16, 63, 0, 1), (4099, 8, 63, 0, 4), (4000, 8, 32, 31, 1),
                                                 (3001, 8, 32, 31, 4)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_chunked_generic(ext, oracle, kernel_env, N, H, left, right, dil, dtype):
    """The bands with fixed-window tiles (causal 64, [i-32, i+31]) on the
    generic stream tiles (MA_ATTN_BWD_NO_FIXED) stay correct."""
    kernel_env("MA_ATTN_BWD_NO_FIXED", "1")
    shape = (2, N, H, 64)
    (q, k, v, g), up = _case(shape, 890 + N + dil, dtype)
    got = ext.sliding_backward(q, k, v, g, left, right, dil)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right, dilation=dil)
    _check(got, oracle.backward(spec, *up), dtype)


@pytest.mark.parametrize("N,H,left,right,dil", [(5000, 16, 63, 0, 1), (4099, 8, 63, 0, 4), (300, 2, 63, 0, 1),
                                                 (4000, 8, 32, 31, 1), (3001, 8, 32, 31, 4), (257, 2, 32, 31, 1)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_backward_unfused_fixed_windows(ext, oracle, kernel_env, N, H, left, right, dil, dtype):
    """The fixed windows in 16 bits on the two-launch kernels (dQ, then
    dK/dV; MA_ATTN_BWD_UNFUSED) instead of the fused one: whole gradients
    vs the oracle."""
    kernel_env("MA_ATTN_BWD_UNFUSED", "1")
    shape = (2, N, H, 64)
    (q, k, v, g), up = _case(shape, 870 + N + dil, dtype)
    got = ext.sliding_backward(q, k, v, g, left, right, dil)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right, dilation=dil)
    _check(got, oracle.backward(spec, *up), dtype)


@pytest.mark.parametrize("shape,left,right,dil", [((1, 65536, 8, 64), 63, 0, 1), ((1, 65536, 8, 64), 63, 0, 4),
                                                  ((4, 8192, 8, 64), 32, 31, 1)])
def test_backward_fused_matches_unfused_full_size(ext, kernel_env, shape, left, right, dil):
    """bf16 at the target shape (causal 64; dilation 4 is cfg 5) and at cfg
    2's ([i-32, i+31], B=4 H=8 N=8192): the fused kernel's gradients against
    the two-launch kernels'.  Both run the same fixed-window score arithmetic
    on interior tiles; P and dS enter dK, dV through the fused kernel's
    exchange (P as e/l instead of exp2(s - lse)), so elements differ by
    roundings."""
    gen = torch.Generator(device="cuda").manual_seed(41 + dil + left)
    q, k, v, g = (torch.randn(shape, device="cuda", generator=gen).bfloat16() for _ in range(4))
    fused = ext.sliding_backward(q, k, v, g, left, right, dil)
    kernel_env("MA_ATTN_BWD_UNFUSED", "1")
    split = ext.sliding_backward(q, k, v, g, left, right, dil)
    for name, a, b in zip("qkv", fused, split):
        a, b = a.float(), b.float()
        diff = (a - b).abs()
        print(f"  d{name}: max|fused - unfused| = {diff.max().item():.3e}, "
              f"differing elements {int((diff > 0).sum().item())}", flush=True)
        assert torch.isfinite(a).all()
        assert (diff <= 1e-2 + 1e-2 * b.abs()).all()


@pytest.mark.parametrize("N", [64, 127, 128, 129, 191, 192, 255, 256, 257, 1000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("left,right", [(63, 0), (32, 31)])
def test_backward_fixed_window_edges(ext, oracle, N, dtype, left, right):
    """The fixed-window bands (fixed-window tiles inside, generic tiles at
    the sequence ends): lengths around the interior-tile bounds."""
    shape = (1, N, 4, 64)
    (q, k, v, g), up = _case(shape, 910 + N, dtype)
    got = ext.sliding_backward(q, k, v, g, left, right, 1)
    spec = oracle.Spec(*shape, pattern="sliding", left=left, right=right)
    _check(got, oracle.backward(spec, *up), dtype)


def test_backward_target_shape(ext, oracle):
    """The headline shape in bf16 (B=1 H=8 N=65536 D=64, causal w=64): whole
    gradients against the oracle."""
    shape = (1, 65536, 8, 64)
    (q, k, v, g), up = _case(shape, 900, torch.bfloat16)
    got = ext.sliding_backward(q, k, v, g, 63, 0, 1)
    spec = oracle.Spec(*shape, pattern="sliding", left=63, right=0)
    _check(got, oracle.backward(spec, *up), torch.bfloat16)


@pytest.mark.parametrize("shape,left,right,dil", [((4, 8192, 8, 64), 32, 31, 1), ((1, 65536, 8, 64), 63, 0, 4)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_full_config_shapes_one_head(ext, oracle, shape, left, right, dil, dtype):
    """cfg 2 (B=4 H=8 N=8192, [i-32, i+31]) and cfg 5 (B=1 H=8 N=65536,
    dilation 4) at their full shapes, both dtypes: every gradient element of
    heads 0 and H-1 against the oracle's backward of those heads (heads are
    independent, so the oracle runs on them alone)."""
    (q, k, v, g), up = _case(shape, 950 + left + dil, dtype)
    got = ext.sliding_backward(q, k, v, g, left, right, dil)
    H = shape[2]
    for h in (0, H - 1):
        one = [np.ascontiguousarray(a[:, :, h:h + 1]) for a in up]
        spec = oracle.Spec(shape[0], shape[1], 1, shape[3], pattern="sliding", left=left, right=right, dilation=dil)
        print(f"head {h}:", flush=True)
        _check([t[:, :, h:h + 1] for t in got], oracle.backward(spec, *one), dtype)


@pytest.mark.parametrize("left,right,dil", [(63, 0, 1), (32, 31, 1), (63, 0, 4)])
def test_backward_sum_identities_full_size(ext, left, right, dil):
    """fp32 at B=1 H=8 N=65536 D=64: rows of P sum to 1 and rows of dS to 0,
    so per head sum_j dV_j = sum_i dout_i and sum_j dK_j = 0."""
    shape = (1, 65536, 8, 64)
    gen = torch.Generator(device="cuda").manual_seed(5 + left + dil)
    q, k, v, g = (torch.randn(shape, device="cuda", generator=gen) for _ in range(4))
    dq, dk, dv = ext.sliding_backward(q, k, v, g, left, right, dil)
    gs = g.double().sum(dim=1)
    assert (dv.double().sum(dim=1) - gs).abs().max().item() <= 1e-2
    assert dk.double().sum(dim=1).abs().max().item() <= 1e-2


def test_backward_rejects_unsupported(ext):
    q = torch.randn(1, 64, 1, 64, device="cuda", dtype=torch.bfloat16)
    from ma_attn import BLOCK_SPARSE, LONGFORMER
    with pytest.raises(RuntimeError):
        ext._backward(q, q, q, q, BLOCK_SPARSE)
    # LONGFORMER only in the one-pass kernel's domain (16-bit, left < 128, right = 0)
    for t, kw in ((q.float(), dict(num_global=4)), (q, dict(left=200, num_global=4)),
                  (q, dict(left=3, right=2, num_global=4))):
        with pytest.raises(RuntimeError, match="LONGFORMER"):
            ext._backward(t, t, t, t, LONGFORMER, **kw)
    with pytest.raises(RuntimeError):
        ext.backward(q, q, q, q.float())  # mixed dtypes


def test_longformer_backward_workspace_through_the_c_abi(ext):
    """ma_attn_backward on a LONGFORMER descriptor through the C-ABI: the
    workspace ma_attn_backward_workspace_size names (statistics, delta and
    both passes' partials) is taken, one byte less or none is refused with a
    message naming the size, and nothing is written then."""
    import ma_attn as _ma
    B, N, H, D = 1, 1000, 2, 64
    q, k, v, g = (torch.randn(B, N, H, D, device="cuda", dtype=torch.bfloat16) for _ in range(4))
    desc = _ma.make_desc(B, N, H, D, _ma.BF16, _ma.LONGFORMER, left=127, right=0, num_global=16)
    need = _ma.backward_workspace_size(desc)
    saved_need = 2 * 4 * B * N * H  # at least the statistics and delta, 4 B each per row
    assert need > saved_need
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    ptrs = [t.data_ptr() for t in (q, k, v, g)]
    for nbytes, wsp in ((need - 1, ws.data_ptr()), (need, 0)):
        outs = [torch.full_like(q, 7.0) for _ in range(3)]
        with pytest.raises(RuntimeError, match=f"workspace of {need} bytes"):
            _ma.backward_raw(desc, *ptrs, *(t.data_ptr() for t in outs), wsp, nbytes)
        torch.cuda.synchronize()
        assert all(bool((t == 7.0).all()) for t in outs)
    outs = [torch.empty_like(q) for _ in range(3)]
    _ma.backward_raw(desc, *ptrs, *(t.data_ptr() for t in outs), ws.data_ptr(), need)
    ref = ext.longformer_backward(q, k, v, g, 127, 0, 16)
    torch.cuda.synchronize()
    for a, b in zip(outs, ref):
        assert torch.equal(a, b)
