"""The one-pass Longformer backward from saved statistics (bwd_lf_kernel +
bwd_lf_combine, ma_attn_backward_saved on a LONGFORMER descriptor) against
the oracle's backward (oracle.c, the restatement of the reference's backward
kernel, /root/reference src/cuda/sparse_attention_kernel.cu:265-346, over the
Longformer key sets).

Cases: windows [i-L, i] with L in {0, 40, 100, 127}, 1 to 16 global tokens,
sequence lengths around the 128-row tile (ragged last tiles, a single tile,
fewer rows than global tokens), one and several tiles per workgroup,
workgroup runs of tiles that cross a head's end, 12 seeded random geometries,
and the full cfg4 shape (B=2 H=12 N=32768) on three heads against the oracle
and on all heads against the tiled backward (fp16 without saved statistics:
two heads against the oracle).  The oracle cases and the random geometries
run both routes: from saved statistics and without them.  Tolerance: check_grad's 16-bit
bound, per element |got - ref| <= 1e-2 + 1e-2 |ref|; against float64 from the
same saved statistics, twice the worst case of the 16-bit roundings.
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


def _case(ext, shape, seed, dtype, L, G):
    """Device inputs, the forward's output and statistics, and the float32
    values the oracle sees."""
    q, k, v = qkv(shape, seed)
    g = randn(shape, seed + 7)
    dev = [torch.from_numpy(a).to(dtype).cuda() for a in (q, k, v, g)]
    out, lse = ext.longformer_forward(dev[0], dev[1], dev[2], L, 0, G, return_lse=True)
    up = [t.float().cpu().numpy() for t in dev]
    return dev, out, lse, up


def _check_heads(oracle, got, up, shape, L, G, heads):
    B, N, H, D = shape
    spec = oracle.Spec(B, N, 1, D, pattern="longformer", left=L, right=0, num_global=G)
    for h in heads:
        one = [np.ascontiguousarray(a[:, :, h:h + 1]) for a in up]
        ref = oracle.backward(spec, *one)
        print(f"head {h}:", flush=True)
        for name, a, r in zip(("dq", "dk", "dv"), got, ref):
            check_grad(name, a[:, :, h:h + 1].float().cpu().numpy(), r, False)


@pytest.mark.parametrize("shape,L,G", [
    ((1, 300, 2, 64), 127, 16),    # ragged last tile
    ((2, 128, 2, 64), 127, 16),    # one tile
    ((1, 1000, 3, 64), 100, 5),
    ((1, 129, 1, 64), 40, 1),      # a tile of one row
    ((1, 700, 2, 64), 0, 16),      # window of the key itself
    ((1, 10, 2, 64), 127, 16),     # fewer rows than global tokens
    ((2, 2000, 2, 64), 127, 16),
    ((1, 8192, 1, 64), 127, 16),   # one stream: 64 chunks, each global sum merged over all of them
    ((1, 12928, 3, 64), 127, 16),  # 3 x 101 tiles in runs of 2: runs cross the heads' ends
    ((1, 12928, 3, 64), 40, 5),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("saved", [True, False], ids=["saved", "nostats"])
def test_longformer_backward_vs_oracle(ext, oracle, shape, L, G, dtype, saved):
    """saved: from the forward's O and statistics (ma_attn_backward_saved);
    nostats: ma_attn_backward (the forward in delta mode, then the same pass)."""
    dev, out, lse, up = _case(ext, shape, 6100 + shape[1] + L, dtype, L, G)
    assert ext.longformer_fused_applies(dev[0], L, 0, G)
    got = ext.longformer_backward(*dev, L, 0, G, **(dict(out=out, lse=lse) if saved else {}))
    _check_heads(oracle, got, up, shape, L, G, range(shape[2]))


@pytest.mark.parametrize("saved", [True, False], ids=["saved", "nostats"])
@pytest.mark.parametrize("i", range(12))
def test_random_longformer_backward(ext, oracle, i, saved):
    """Seeded random geometries in the one-pass kernel's domain (16-bit,
    L <= 127, 1 to 16 globals): sequence lengths from one row to 15 000, 1 to
    12 (batch, head) streams.  The odd cases have more than 256 tiles and an
    odd tile count per stream, so the workgroups' equal runs (2 to 5 tiles)
    start and end at varied places and cross the streams' ends.  Every head
    against the oracle.  In bf16, windows narrower than 63 keys are drawn
    only up to N = 2000: over longer sequences the global keys' dK gather a
    systematic term from delta = dO . O with the forward's bf16 O.  When the
    global keys carry much of every row's softmax, every row's O is nearly the
    same vector, so its roundings add up over the rows instead of averaging
    out; against the float32 oracle that exceeded check_grad's bound at
    N = 12316, G = 11 (2.3x at L = 0, 1.2x at L = 17), while bf16 at L >= 63
    and fp16 at any L stayed within it.  test_longformer_backward_long_key_only_window
    holds the kernel to float64 from the same statistics in that regime.
    Without saved statistics (nostats: delta = sum_j P_ij dP_ij from the
    forward in fp32) every window is drawn at every length."""
    rng = np.random.default_rng(41000 + i)
    if i % 2:  # more than 256 tiles, an odd count per stream: runs of 2+ tiles cross the heads' ends
        B, H = 1 + (i % 4 == 1), int(rng.integers(3, 7))
        nt = int(rng.integers(256 // (B * H) + 2, 121)) | 1
        N = 128 * (nt - 1) + int(rng.integers(1, 129))
    else:
        N = int(rng.choice([int(rng.integers(1, 700)), int(rng.integers(2000, 9000))]))
        B, H = int(rng.integers(1, 3)), int(rng.integers(1, 7))
    G = int(rng.integers(1, 17))
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(0, 2))]
    narrow = N <= 2000 or dtype == torch.float16 or not saved
    L = int(rng.choice([0, 17, 63, 64, 100, 127] if narrow else [63, 64, 100, 127]))
    tiles = B * H * ((N + 127) // 128)
    print(f"  case {i}: B={B} N={N} H={H} L={L} G={G} {dtype}, {tiles} tiles in runs of "
          f"{max(1, (tiles + 255) // 256)}", flush=True)
    shape = (B, N, H, 64)
    dev, out, lse, up = _case(ext, shape, 42000 + i, dtype, L, G)
    assert ext.longformer_fused_applies(dev[0], L, 0, G)
    got = ext.longformer_backward(*dev, L, 0, G, **(dict(out=out, lse=lse) if saved else {}))
    _check_heads(oracle, got, up, shape, L, G, range(H))


def _same_statistics_grads(dev, out, lse, L, G):
    """float64 dQ, dK, dV of every (batch, head) from the forward's saved
    statistics (lse2, and delta = dO . O with the forward's 16-bit O): the
    quantities the saved-statistics backward computes, without its 16-bit
    operand and output roundings; and, for each element, the sum of its
    terms' magnitudes (scale |dS| |K|, scale |dS|^T |Q|, |P|^T |dO|)."""
    Q, K, V, dO = (t.double().cpu().numpy() for t in dev)
    Ob, l2 = out.double().cpu().numpy(), lse.double().cpu().numpy()
    B, N, H, D = Q.shape
    scale = 1.0 / np.sqrt(np.float32(D)).astype(np.float64)
    i = np.arange(N)[:, None]
    j = np.arange(N)[None, :]
    member = (i < G) | (j < G) | ((j <= i) & (j >= i - L))
    grads = [np.zeros_like(Q) for _ in range(3)]
    mags = [np.zeros_like(Q) for _ in range(3)]
    for b in range(B):
        for h in range(H):
            q, k, v, go = Q[b, :, h], K[b, :, h], V[b, :, h], dO[b, :, h]
            p = np.where(member, 2.0 ** ((q @ k.T) * scale * np.log2(np.e) - l2[b, :, h, None]), 0.0)
            delta = (go * Ob[b, :, h]).sum(-1, keepdims=True)
            ds = p * (go @ v.T - delta)
            grads[0][b, :, h] = scale * ds @ k
            grads[1][b, :, h] = scale * ds.T @ q
            grads[2][b, :, h] = p.T @ go
            mags[0][b, :, h] = scale * np.abs(ds) @ np.abs(k)
            mags[1][b, :, h] = scale * np.abs(ds).T @ np.abs(q)
            mags[2][b, :, h] = p.T @ np.abs(go)
    return grads, mags


@pytest.mark.parametrize("shape,L,G", [((1, 600, 2, 64), 0, 3), ((2, 300, 1, 64), 127, 16), ((1, 520, 2, 64), 64, 1)])
def test_longformer_backward_vs_same_statistics(ext, shape, L, G):
    """The kernel's arithmetic against float64 from the same saved statistics,
    element by element: within twice the worst case of its 16-bit roundings,
    one bf16 rounding (2^-9 relative) of each term's P or dS operand and one
    of the output: 2^-8 (sum of the terms' magnitudes + |result|) + 2e-3.
    The comparison with the oracle above also carries the statistics' own
    rounding (delta from the 16-bit forward output), which dominates where
    few keys share each row (L = 0, G = 3: four keys, three of them global)."""
    dev, out, lse, _ = _case(ext, shape, 6600 + shape[1] + L, torch.bfloat16, L, G)
    got = ext.longformer_backward(*dev, L, 0, G, out=out, lse=lse)
    refs, mags = _same_statistics_grads(dev, out, lse, L, G)
    for name, a, r, m in zip(("dq", "dk", "dv"), got, refs, mags):
        a = a.double().cpu().numpy()
        err = np.abs(a - r)
        bound = 2e-3 + 2.0 ** -8 * (m + np.abs(r))
        print(f"  {name}: max|err| = {err.max():.3e}, worst err/bound = {(err / bound).max():.3f}", flush=True)
        assert (err <= bound).all(), name


def test_longformer_backward_long_key_only_window(ext):
    """L = 0 over a long sequence in bf16 (B=1 N=12316 H=1, G=11, runs of
    tiles crossing nothing but the chunking of one stream): every element of
    dQ, dK, dV against float64 from the same saved statistics (lse2, and delta
    from the forward's bf16 O), within twice the worst case of the kernel's
    16-bit roundings, as test_longformer_backward_vs_same_statistics.  Against
    the float32 oracle this geometry exceeds check_grad's bound on the global
    keys (delta's rounding, see test_random_longformer_backward); here the
    kernel's own arithmetic is held to its bound."""
    shape, L, G = (1, 12316, 1, 64), 0, 11
    dev, out, lse, _ = _case(ext, shape, 42001, torch.bfloat16, L, G)
    got = ext.longformer_backward(*dev, L, 0, G, out=out, lse=lse)
    Q, K, V, dO = (t.double().cpu().numpy()[0, :, 0] for t in dev)
    Ob, l2 = out.double().cpu().numpy()[0, :, 0], lse.double().cpu().numpy()[0, :, 0]
    N = shape[1]
    scale = 1.0 / np.sqrt(np.float32(64)).astype(np.float64)
    refs = [np.zeros((N, 64)) for _ in range(3)]
    mags = [np.zeros((N, 64)) for _ in range(3)]
    j = np.arange(N)[None, :]
    for lo in range(0, N, 2048):  # row blocks: the float64 matrices stay at 2048 x N
        hi = min(N, lo + 2048)
        i = np.arange(lo, hi)[:, None]
        member = (i < G) | (j < G) | ((j <= i) & (j >= i - L))
        p = np.where(member, 2.0 ** ((Q[lo:hi] @ K.T) * scale * np.log2(np.e) - l2[lo:hi, None]), 0.0)
        delta = (dO[lo:hi] * Ob[lo:hi]).sum(-1, keepdims=True)
        ds = p * (dO[lo:hi] @ V.T - delta)
        refs[0][lo:hi] = scale * ds @ K
        refs[1] += scale * ds.T @ Q[lo:hi]
        refs[2] += p.T @ dO[lo:hi]
        mags[0][lo:hi] = scale * np.abs(ds) @ np.abs(K)
        mags[1] += scale * np.abs(ds).T @ np.abs(Q[lo:hi])
        mags[2] += p.T @ np.abs(dO[lo:hi])
    for name, a, r, m in zip(("dq", "dk", "dv"), got, refs, mags):
        a = a.double().cpu().numpy()[0, :, 0]
        err = np.abs(a - r)
        bound = 2e-3 + 2.0 ** -8 * (m + np.abs(r))
        print(f"  {name}: max|err| = {err.max():.3e}, worst err/bound = {(err / bound).max():.3f}", flush=True)
        assert (err <= bound).all(), name


@pytest.mark.parametrize("L,G", [(0, 11), (17, 11)])
def test_longformer_backward_long_narrow_window_without_statistics(ext, oracle, L, G):
    """The regime where delta from the forward's bf16 O exceeds the bound
    (B=2 N=12316 H=2, bf16): without saved statistics the forward sums
    delta = sum_j P_ij dP_ij in fp32, and every gradient element of both
    heads is within check_grad's bound of the oracle's."""
    shape = (2, 12316, 2, 64)
    dev, _, _, up = _case(ext, shape, 42001, torch.bfloat16, L, G)
    got = ext.longformer_backward(*dev, L, 0, G)
    _check_heads(oracle, got, up, shape, L, G, range(shape[2]))


def test_longformer_backward_several_tiles_per_chunk(ext, oracle):
    """64 (batch, head) streams: 4 chunks of 8 tiles each (the chunk's carried
    key block and its extra key pass for the next chunk's first tile)."""
    shape = (4, 4096, 16, 64)
    dev, out, lse, up = _case(ext, shape, 6200, torch.bfloat16, 127, 16)
    got = ext.longformer_backward(*dev, 127, 0, 16, out=out, lse=lse)
    _check_heads(oracle, got, up, shape, 127, 16, (0, 15))
    again = ext.longformer_backward(*dev, 127, 0, 16, out=out, lse=lse)
    for a, b in zip(got, again):  # one writer per row, partials summed in a fixed order
        assert torch.equal(a, b)


def test_longformer_backward_cfg4_shape(ext, oracle):
    """cfg4 (B=2 H=12 N=32768, w=128, 16 globals): heads 0, 5 and 11 against
    the oracle; every row from 16 on, in every head, against the tiled
    backward from the same statistics (both within the 16-bit bound of each
    other's values there; on the 16 global keys the tiled backward's long
    16-bit sums are the less accurate of the two)."""
    shape = (2, 32768, 12, 64)
    dev, out, lse, up = _case(ext, shape, 6300, torch.bfloat16, 127, 16)
    got = ext.longformer_backward(*dev, 127, 0, 16, out=out, lse=lse)
    _check_heads(oracle, got, up, shape, 127, 16, (0, 5, 11))
    iset = ext.pattern_index_set("longformer", shape[1], dev[0].device, left=127, right=0, num_global=16)
    tiled = ext.index_set_backward(*dev, iset, out=out, lse=lse)
    for name, a, b in zip(("dq", "dk", "dv"), got, tiled):
        a, b = a[:, 16:].float(), b[:, 16:].float()
        diff = (a - b).abs()
        print(f"  {name}: max|fused - tiled| = {diff.max().item():.3e}", flush=True)
        assert torch.isfinite(a).all()
        assert bool((diff <= 1e-2 + 1e-2 * b.abs()).all())


def test_longformer_backward_falls_back(ext, oracle):
    """Shapes the one-pass kernel does not take (a right window, more than 16
    global tokens, float32, no statistics) run the tiled backward."""
    shape = (1, 300, 2, 64)
    for dtype, L, R, G in ((torch.bfloat16, 20, 3, 5), (torch.bfloat16, 127, 0, 20), (torch.float32, 127, 0, 16)):
        q, k, v = qkv(shape, 6400 + G + R)
        g = randn(shape, 6401)
        dev = [torch.from_numpy(a).to(dtype).cuda() for a in (q, k, v, g)]
        assert not ext.longformer_fused_applies(dev[0], L, R, G)
        got = ext.longformer_backward(*dev, L, R, G)
        up = [t.float().cpu().numpy() for t in dev]
        ref = oracle.backward(oracle.Spec(*shape, pattern="longformer", left=L, right=R, num_global=G), *up)
        for name, a, r in zip(("dq", "dk", "dv"), got, ref):
            check_grad(name, a.float().cpu().numpy(), r, dtype == torch.float32)


def test_layer_longformer_training_uses_the_one_pass_kernel(ext, oracle, monkeypatch):
    """MACoreAttention(pattern="longformer", fallback_training=False) in bf16:
    the forward keeps its statistics and the backward runs longformer_backward
    from them (no tiled backward), with the oracle's gradients."""
    from layers.ma_core_bridge import MACoreAttention
    calls = []
    f = ext.longformer_backward
    monkeypatch.setattr(ext, "longformer_backward", lambda *a, **k_: calls.append(k_) or f(*a, **k_))
    monkeypatch.setattr(ext, "index_set_backward", lambda *a, **k_: pytest.fail("tiled backward used"))
    shape = (1, 500, 2, 64)
    q, k, v = qkv(shape, 6500)
    g = randn(shape, 6501)
    dev = [torch.from_numpy(a).bfloat16().cuda().requires_grad_(True) for a in (q, k, v)]
    gd = torch.from_numpy(g).bfloat16().cuda()
    att = MACoreAttention(sparse=True, window_size=64, pattern="longformer", window_left=127, window_right=0,
                          num_global_tokens=16, fallback_training=False).train()
    att(*dev).backward(gd)
    assert len(calls) == 1 and calls[0].get("lse") is not None
    up = [t.detach().float().cpu().numpy() for t in dev] + [gd.float().cpu().numpy()]
    ref = oracle.backward(oracle.Spec(*shape, pattern="longformer", left=127, right=0, num_global=16), *up)
    for name, t, r in zip(("dq", "dk", "dv"), dev, ref):
        check_grad(name, t.grad.float().cpu().numpy(), r, False)


@pytest.mark.parametrize("shape,L,G", [((1, 700, 2, 64), 127, 16), ((2, 300, 1, 64), 40, 5)])
def test_longformer_backward_without_statistics(ext, oracle, shape, L, G):
    """longformer_backward without out / lse (ma_attn_backward on the
    LONGFORMER descriptor: the forward writing each row's statistic and
    delta = sum_j P_ij dP_ij, then the one-pass kernel): the oracle's
    gradients, the saved-statistics call's within the 16-bit bound (the two
    differ only in delta's rounding), bit-identical repeats; under
    kernel_events both launches' kernels are stamped as one span."""
    dev, out, lse, up = _case(ext, shape, 6700 + shape[1] + L, torch.bfloat16, L, G)
    got = ext.longformer_backward(*dev, L, 0, G)
    saved = ext.longformer_backward(*dev, L, 0, G, out=out, lse=lse)
    for name, a, b in zip(("dq", "dk", "dv"), got, saved):
        check_grad(name, a.float().cpu().numpy(), b.float().cpu().numpy(), False)
    for a, b in zip(got, ext.longformer_backward(*dev, L, 0, G)):
        assert torch.equal(a, b)
    _check_heads(oracle, got, up, shape, L, G, range(shape[2]))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    torch.cuda.synchronize()
    with ext.kernel_events(e0, e1):
        ext.longformer_backward(*dev, L, 0, G)
    torch.cuda.synchronize()
    assert e0.elapsed_time(e1) > 0.0


def test_longformer_backward_cfg4_shape_fp16_without_statistics(ext, oracle):
    """cfg4's shape (B=2 H=12 N=32768, w=128, 16 globals) in fp16 without
    saved statistics (the delta-mode forward, then the one-pass kernel):
    heads 0 and 11 against the oracle, every element within check_grad's
    16-bit bound."""
    shape = (2, 32768, 12, 64)
    dev, _, _, up = _case(ext, shape, 6350, torch.float16, 127, 16)
    got = ext.longformer_backward(*dev, 127, 0, 16)
    _check_heads(oracle, got, up, shape, 127, 16, (0, 11))
