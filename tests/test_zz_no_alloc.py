"""ma_attn_forward_noalloc: the allocation-free forward entry point, through
the C-ABI, against ma_attn_forward on the same inputs.

Two forward kernels use scratch: the Longformer stream kernel (its per-chunk
partials of the global rows) and the tiled index-set kernel (the partial
results of a tile plan's split rows).  The no-alloc entry point takes it from
the library's static device array instead of a caller workspace.  Both entry
points launch the same kernels, so the outputs must agree bit for bit.  For
each scratch user: two calls in a row, the second smaller (the array keeps the
first call's contents); then a pattern with no scratch, then a call whose
scratch need is above the array's size, which must be rejected with nothing
launched.
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ma():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ma_attn
    return ma_attn


def _inputs(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g).to(dtype).cuda() for _ in range(3)]


def _both(ma, desc, q, k, v):
    """(ma_attn_forward with a workspace, ma_attn_forward_noalloc) outputs."""
    stream = torch.cuda.current_stream().cuda_stream
    o_ws, o_na = torch.empty_like(q), torch.empty_like(q)
    nbytes = ma.workspace_size(desc)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    ma.forward_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), o_ws.data_ptr(), ws.data_ptr(), nbytes, stream)
    ma.forward_noalloc_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), o_na.data_ptr(), stream)
    torch.cuda.synchronize()
    return o_ws, o_na, nbytes


def _longformer_desc(ma, shape, dtype, left, G):
    B, N, H, D = shape
    return ma.make_desc(B, N, H, D, ma.DTYPES[dtype], ma.LONGFORMER, left=left, right=0, num_global=G)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_workspace_entry_point(ma, oracle, dtype):
    # first call: the Longformer benchmark geometry at a quarter of its length
    shape1 = (2, 8192, 12, 64)
    q, k, v = _inputs(shape1, 11, dtype)
    desc = _longformer_desc(ma, shape1, dtype, 127, 16)
    o_ws, o_na, nbytes = _both(ma, desc, q, k, v)
    print(f"call 1 {shape1} {dtype}: scratch {nbytes} B", flush=True)
    assert 0 < nbytes <= ma.NOALLOC_SCRATCH_BYTES
    assert torch.equal(o_ws, o_na)
    # the global rows and a few local rows against the oracle as well
    up = [t.float().cpu().numpy() for t in (q, k, v)]
    spec = oracle.Spec(*shape1, pattern="longformer", left=127, right=0, num_global=16)
    ref = oracle.forward(spec, *up, heads=(0, 2), rows=(0, 40))
    err = float(np.abs(o_na.float().cpu().numpy()[:, :40, :2] - ref[:, :40, :2]).max())
    print(f"  rows 0-40 heads 0-1 vs oracle: {err:.3e}", flush=True)
    assert err <= 2e-2
    # second call, smaller: fewer chunks and globals; stale partials of call 1 stay in the array
    shape2 = (1, 3000, 4, 64)
    q, k, v = _inputs(shape2, 12, dtype)
    desc = _longformer_desc(ma, shape2, dtype, 100, 5)
    o_ws, o_na, nbytes = _both(ma, desc, q, k, v)
    print(f"call 2 {shape2} {dtype}: scratch {nbytes} B", flush=True)
    assert 0 < nbytes
    assert torch.equal(o_ws, o_na)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_tiled_index_set(ma, oracle, dtype):
    """A tiled index set whose plan splits rows (the Longformer key sets: the
    global rows' tiles hold every key block): its partials in the static array."""
    import sparse_attention_cuda as ext
    calls = [((1, 8192, 4, 64), 127, 16, 21), ((1, 3000, 2, 64), 60, 5, 22)]  # the second smaller
    for n, (shape, left, G, seed) in enumerate(calls):
        B, N, H, D = shape
        iset = ext.pattern_index_set("longformer", N, "cuda:0", left=left, right=0, num_global=G)
        assert iset.tile_plan is not None and int(iset.tile_header.num_q_split) > 0
        q, k, v = _inputs(shape, seed, dtype)
        desc = ma.make_desc(B, N, H, D, ma.DTYPES[dtype], ma.INDEX_SET, index_offsets_ptr=iset.offsets.data_ptr(),
                            index_keys_ptr=iset.keys.data_ptr(), num_indices=iset.num_indices, **iset._tile_kw())
        o_ws, o_na, nbytes = _both(ma, desc, q, k, v)
        print(f"call {n + 1} {shape} {dtype}: tiled set, {int(iset.tile_header.num_q_split)} split rows, "
              f"scratch {nbytes} B", flush=True)
        assert 0 < nbytes <= ma.NOALLOC_SCRATCH_BYTES
        assert torch.equal(o_ws, o_na)
        # the split (global) rows against the oracle
        up = [t.float().cpu().numpy() for t in (q, k, v)]
        spec = oracle.Spec(*shape, pattern="longformer", left=left, right=0, num_global=G)
        ref = oracle.forward(spec, *up, heads=(0, 1), rows=(0, G + 8))
        err = float(np.abs(o_na.float().cpu().numpy()[:, :G + 8, :1] - ref[:, :G + 8, :1]).max())
        print(f"  rows 0-{G + 8} head 0 vs oracle: {err:.3e}", flush=True)
        assert err <= 2e-2


def test_noalloc_without_scratch(ma):
    """A pattern whose kernels use no scratch: the same output as ma_attn_forward."""
    shape = (1, 4096, 8, 64)
    q, k, v = _inputs(shape, 13, torch.bfloat16)
    desc = ma.make_desc(*shape, ma.BF16, ma.SLIDING, left=63, right=0, dilation=1)
    o_ws, o_na, nbytes = _both(ma, desc, q, k, v)
    assert nbytes == 0 and torch.equal(o_ws, o_na)


def test_noalloc_rejects_oversized_scratch(ma):
    """2048 (batch, head) streams of Longformer partials need more than the
    static array holds: rejected with a message, the output left untouched."""
    shape = (16, 64, 128, 64)
    desc = _longformer_desc(ma, shape, torch.bfloat16, 7, 4)
    assert ma.workspace_size(desc) > ma.NOALLOC_SCRATCH_BYTES
    q = torch.zeros(shape, dtype=torch.bfloat16, device="cuda")
    o = torch.full(shape, 7.0, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="static scratch"):
        ma.forward_noalloc_raw(desc, q.data_ptr(), q.data_ptr(), q.data_ptr(), o.data_ptr(),
                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert bool((o == 7.0).all())
