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


# ---------------------------------------------------------------- saved statistics (ma_attn_forward_lse / _backward_saved)

def _lse_ref(up, off, keys):
    """float64 log2 of each row's softmax denominator over its key set (in
    units of the scaled scores), [B, N, H]; 0 for a row with no key."""
    q, k = (x.astype(np.float64) for x in up[:2])
    B, N, H, D = q.shape
    sl2 = np.log2(np.e) / np.sqrt(D)
    out = np.zeros((B, N, H))
    for i in range(N):
        kk = keys[off[i]:off[i + 1]]
        if kk.size == 0:
            continue
        s = np.einsum("bhd,bkhd->bhk", q[:, i], k[:, kk]) * sl2  # [B, H, keys]
        m = s.max(-1, keepdims=True)
        out[:, i] = (m[..., 0] + np.log2(np.exp2(s - m).sum(-1)))
    return out


@pytest.mark.parametrize("kind,N,seg", [("random", 300, 0), ("skewed", 700, 2), ("window", 1000, 0),
                                        ("global", 1200, 0), ("global", 1200, 3)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_saved_statistics_index_set(ext, oracle, kind, N, seg, dtype):
    """index_set_forward(return_lse=True) writes each row's log-sum-exp; the
    backward from the saved O and statistics matches the oracle's gradients
    and the backward that recomputes them."""
    rng = np.random.default_rng(N + 7 * len(kind))
    off, keys = _set(kind, N, rng)
    shape = (2, N, 2, 64)
    dev, up = _inputs(shape, 9500 + N, dtype)
    iset = ext.IndexSet(torch.from_numpy(off), torch.from_numpy(keys), N, tiles=True, tile_seg=seg)
    out, lse = ext.index_set_forward(*dev[:3], iset, return_lse=True)
    assert float((out.float() - ext.index_set_forward(*dev[:3], iset).float()).abs().max()) == 0.0
    err = float(np.abs(lse.cpu().numpy() - _lse_ref(up, off, keys)).max())
    print(f"  {kind} N={N} {dtype}: max|lse err| = {err:.2e}", flush=True)
    assert err <= 1e-3, err
    saved = ext.index_set_backward(*dev, iset, out=out, lse=lse)
    spec = oracle.Spec(*shape, pattern="index_set", offsets=off, keys=keys)
    for name, a, b in zip("qkv", saved, oracle.backward(spec, *up)):
        check_grad("d" + name, a.float().cpu().numpy(), b, dtype == torch.float32)
    again = ext.index_set_backward(*dev, iset)
    for a, b in zip(saved, again):
        assert float((a.float() - b.float()).abs().max()) <= (2e-5 if dtype == torch.float32 else 3e-2)


@pytest.mark.parametrize("pattern,N", [("block_sparse", 1536), ("block_sparse", 1500), ("longformer", 1500),
                                       ("longformer", 700)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_saved_statistics_patterns(ext, oracle, pattern, N, dtype):
    """block_sparse_forward / longformer_forward with return_lse=True give the
    statistics of their key sets (block-row and Longformer stream kernels), and
    the tiled backward of those sets from them matches the oracle."""
    import ma_attn
    shape = (2, N, 2, 64)
    dev, up = _inputs(shape, 9600 + N, dtype)
    if pattern == "block_sparse":
        nb = (N + 63) // 64
        tab = ext.make_block_table(5, nb, 2)
        bt = ext.BlockTable(tab, N, 64)
        out, lse = ext.block_sparse_forward(*dev[:3], bt, 64, return_lse=True)
        ref_out = ext.block_sparse_forward(*dev[:3], bt, 64)
        iset = ext.pattern_index_set("block_sparse", N, "cuda", block_table=bt, block_size=64)
        spec = oracle.Spec(*shape, pattern="block_sparse", block_size=64, table=tab.numpy())
        pd = ma_attn.make_desc(1, N, 1, 64, ma_attn.F32, ma_attn.BLOCK_SPARSE, block_table_ptr=tab.data_ptr(),
                               blocks_per_row=int(tab.shape[1]), block_size=64)
        off, keys = ma_attn.pattern_csr(pd, tab)
    else:
        out, lse = ext.longformer_forward(*dev[:3], 127, 0, 16, return_lse=True)
        ref_out = ext.longformer_forward(*dev[:3], 127, 0, 16)
        iset = ext.pattern_index_set("longformer", N, "cuda", left=127, right=0, num_global=16)
        spec = oracle.Spec(*shape, pattern="longformer", left=127, right=0, num_global=16)
        pd = ma_attn.make_desc(1, N, 1, 64, ma_attn.F32, ma_attn.LONGFORMER, left=127, right=0, num_global=16)
        off, keys = ma_attn.pattern_csr(pd)
    assert float((out.float() - ref_out.float()).abs().max()) == 0.0
    off, keys = np.asarray(off, np.int64), np.asarray(keys, np.int64)
    err = float(np.abs(lse.cpu().numpy() - _lse_ref(up, off, keys)).max())
    print(f"  {pattern} N={N} {dtype}: max|lse err| = {err:.2e}", flush=True)
    assert err <= 1e-3, err
    saved = ext.index_set_backward(*dev, iset, out=out, lse=lse)
    for name, a, b in zip("qkv", saved, oracle.backward(spec, *up)):
        check_grad("d" + name, a.float().cpu().numpy(), b, dtype == torch.float32)


def test_saved_statistics_rejected(ext):
    """Kernels that write no statistics refuse return_lse; a malformed lse is
    rejected before any launch."""
    q = torch.randn(1, 256, 2, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="statistics"):
        ext._launch(q, q, q, __import__("ma_attn").SLIDING, True, left=63, right=0, dilation=1)
    off = torch.arange(0, 257, dtype=torch.int64)
    iset = ext.IndexSet(off, torch.arange(256, dtype=torch.int32), 256, tiles=True)
    out, lse = ext.index_set_forward(q, q, q, iset, return_lse=True)
    with pytest.raises(RuntimeError, match="lse"):
        ext.index_set_backward(q, q, q, q, iset, out=out, lse=lse[:, :128])


@pytest.mark.parametrize("pattern", ["block_sparse", "longformer", "dense"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_layer_trains_from_saved_statistics(ext, oracle, pattern, dtype, monkeypatch):
    """MACoreAttention training on the device (fallback_training=False) keeps
    the forward's statistics and runs the backward from them (16-bit
    Longformer on the one-pass longformer_backward, fp32 Longformer on the
    tiled index-set kernels); gradients match the oracle's."""
    from layers.ma_core_bridge import MACoreAttention
    N = 1536
    shape = (2, N, 2, 64)
    dev, up = _inputs(shape, 9700, dtype)
    if pattern == "block_sparse":
        tab = ext.make_block_table(3, N // 64, 2)
        layer = MACoreAttention(pattern="block_sparse", block_table=tab, block_size=64, fallback_training=False)
        spec = oracle.Spec(*shape, pattern="block_sparse", block_size=64, table=tab.numpy())
    elif pattern == "longformer":
        layer = MACoreAttention(pattern="longformer", window_size=128, causal=True, num_global_tokens=16,
                                fallback_training=False)
        spec = oracle.Spec(*shape, pattern="longformer", left=127, right=0, num_global=16)
    else:  # the reference's own dense layer (no pattern keywords)
        layer = MACoreAttention(sparse=False, use_causal_mask=True, fallback_training=False)
        spec = oracle.Spec(*shape, pattern="dense", causal=True)
    layer.train()
    calls = []
    if pattern == "dense":
        fn = "dense_backward"
    elif pattern == "longformer" and dtype != torch.float32:
        fn = "longformer_backward"
    else:
        fn = "index_set_backward"
    real = getattr(ext, fn)

    def spy(*a, **kw):
        calls.append(kw.get("lse") is not None)
        return real(*a, **kw)

    monkeypatch.setattr(ext, fn, spy)
    q, k, v = (t.clone().requires_grad_(True) for t in dev[:3])
    layer(q, k, v).backward(dev[3])
    assert calls == [True]
    for name, t, ref in zip("qkv", (q, k, v), oracle.backward(spec, *up)):
        check_grad("d" + name, t.grad.float().cpu().numpy(), ref, dtype == torch.float32)


@pytest.mark.parametrize("N,causal", [(700, True), (1000, False), (64, True), (4096, True)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_saved_statistics_dense(ext, oracle, N, causal, dtype):
    """dense_forward(return_lse=True) (block-row kernel) writes each row's
    log-sum-exp; dense_backward from the saved O and statistics matches the
    oracle and the recomputing backward."""
    shape = (2, N, 2, 64)
    dev, up = _inputs(shape, 9800 + N, dtype)
    out, lse = ext.dense_forward(*dev[:3], causal, return_lse=True)
    assert float((out.float() - ext.dense_forward(*dev[:3], causal).float()).abs().max()) == 0.0
    off = np.concatenate([[0], np.cumsum(np.arange(1, N + 1) if causal else np.full(N, N))]).astype(np.int64)
    keys = np.concatenate([np.arange(i + 1 if causal else N) for i in range(N)]).astype(np.int64)
    err = float(np.abs(lse.cpu().numpy() - _lse_ref(up, off, keys)).max())
    print(f"  dense N={N} causal={causal} {dtype}: max|lse err| = {err:.2e}", flush=True)
    assert err <= 1e-3, err
    saved = ext.dense_backward(*dev, causal, out=out, lse=lse)
    spec = oracle.Spec(*shape, pattern="dense", causal=causal)
    for name, a, b in zip("qkv", saved, oracle.backward(spec, *up)):
        check_grad("d" + name, a.float().cpu().numpy(), b, dtype == torch.float32)
    again = ext.dense_backward(*dev, causal)
    for a, b in zip(saved, again):
        assert float((a.float() - b.float()).abs().max()) <= (2e-5 if dtype == torch.float32 else 3e-2)


@pytest.mark.parametrize("workload", ["cfg3", "cfg4"])
def test_saved_statistics_full_size(ext, workload):
    """At the BASELINE shapes (cfg3: B2 H8 N16384 block-sparse; cfg4: B2 H12
    N32768 Longformer; bf16), the backward from saved statistics agrees with
    the backward that recomputes them on every element, and the statistics
    satisfy sum_j exp2(s_ij*sl2 - lse_i) = 1 on sampled rows."""
    torch.manual_seed(11)
    if workload == "cfg3":
        B, H, N = 2, 8, 16384
    else:
        B, H, N = 2, 12, 32768
    q, k, v, g = (torch.randn(B, N, H, 64, device="cuda").to(torch.bfloat16) for _ in range(4))
    if workload == "cfg3":
        tab = ext.BlockTable(ext.make_block_table(1234, N // 64, 2), N, 64)
        out, lse = ext.block_sparse_forward(q, k, v, tab, 64, return_lse=True)
        iset = ext.pattern_index_set("block_sparse", N, "cuda", block_table=tab, block_size=64)
    else:
        out, lse = ext.longformer_forward(q, k, v, 127, 0, 16, return_lse=True)
        iset = ext.pattern_index_set("longformer", N, "cuda", left=127, right=0, num_global=16)
    saved = ext.index_set_backward(q, k, v, g, iset, out=out, lse=lse)
    again = ext.index_set_backward(q, k, v, g, iset)
    for name, a, b in zip(("dq", "dk", "dv"), saved, again):
        a, b = a.float(), b.float()
        bound = 1e-2 + 1e-2 * b.abs()
        worst = float(((a - b).abs() / bound).max())
        print(f"  {workload} {name}: max |saved - recomputed| / (1e-2 + 1e-2|x|) = {worst:.3f}", flush=True)
        assert worst <= 1.0
    # the statistics normalise their rows: a sample of query rows of head 0, batch 0
    off = iset.offsets.cpu().numpy()
    keys = iset.keys.cpu().numpy()
    sl2 = 1.4426950408889634 / 8.0
    qs, ks = q[0, :, 0].float(), k[0, :, 0].float()
    for i in list(range(0, 20)) + [N // 2, N - 1]:
        kk = torch.from_numpy(keys[off[i]:off[i + 1]].astype(np.int64)).cuda()
        s = (ks[kk] @ qs[i]) * sl2
        total = float(torch.exp2(s - lse[0, i, 0]).sum())
        assert abs(total - 1.0) <= 1e-4, (i, total)


def test_block_sparse_backward_cfg3_shape_vs_oracle(ext, oracle):
    """cfg3 at full size (B=2 H=8 N=16384, block 64, diagonal + previous + 2
    seeded blocks, bf16): the tiled backward over the table's key sets,
    recomputing and from the forward's saved statistics, on heads 0 and 7
    against the oracle's backward of those heads (heads are independent),
    every element within check_grad's 16-bit bound."""
    B, N, H, D = 2, 16384, 8, 64
    q, k, v = qkv((B, N, H, D), 7100)
    g = randn((B, N, H, D), 7101)
    dev = [torch.from_numpy(a).bfloat16().cuda() for a in (q, k, v, g)]
    up = [t.float().cpu().numpy() for t in dev]
    host = ext.make_block_table(1234, N // 64, 2)
    tab = ext.BlockTable(host, N, 64)
    out, lse = ext.block_sparse_forward(dev[0], dev[1], dev[2], tab, 64, return_lse=True)
    iset = ext.pattern_index_set("block_sparse", N, "cuda", block_table=tab, block_size=64)
    routes = {"recomputed": ext.index_set_backward(*dev, iset),
              "saved": ext.index_set_backward(*dev, iset, out=out, lse=lse)}
    spec = oracle.Spec(B, N, 1, D, pattern="block_sparse", block_size=64, table=host.numpy())
    for h in (0, H - 1):
        ref = oracle.backward(spec, *(np.ascontiguousarray(a[:, :, h:h + 1]) for a in up))
        for route, got in routes.items():
            print(f"head {h}, {route}:", flush=True)
            for name, a, r in zip(("dq", "dk", "dv"), got, ref):
                check_grad(name, a[:, :, h:h + 1].float().cpu().numpy(), r, False)
