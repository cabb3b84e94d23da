"""The entry points under HIP graph capture (serving loops replay captured
launches).  The library allocates, clears and synchronises nothing on its
launch path (outputs and workspaces come from the caller / torch's allocator,
every workspace word is written before it is read), so a captured sequence
replays to the eager results.  Replays are interleaved with eager work on the
same inputs and each replay is checked, bit-exactly (the kernels are
deterministic), against the eager outputs."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import sparse_attention_cuda
    return sparse_attention_cuda


def test_graph_capture_replays(ext):
    gen = torch.Generator(device="cuda").manual_seed(11)
    shape = (1, 4096, 4, 64)
    q, k, v, g = (torch.randn(shape, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(4))
    qf, kf, vf, gf = (t.float() for t in (q, k, v, g))
    table = ext.BlockTable(ext.make_block_table(7, 64, 2), 4096, 64)
    rows = torch.arange(4096).repeat_interleave(3)
    iset = ext.IndexSet.from_coo(rows, (rows * 7 + torch.arange(3).repeat(4096) * 13) % 4096, 4096)

    def work():
        lo, llse = ext.longformer_forward(q, k, v, 127, 0, 16, return_lse=True)
        return [ext.sliding_forward(q, k, v, 63, 0),
                ext.sliding_forward(q, k, v, 32, 31, 2),
                ext.block_sparse_forward(q, k, v, table, 64),
                ext.longformer_forward(q, k, v, 127, 0, 16),  # workspace of partials + combine launch
                ext.dense_forward(qf, kf, vf, True),
                ext.index_set_forward(q, k, v, iset),  # gather kernel over a device-resident set
                *ext.sliding_backward(q, k, v, g, 63, 0, 1),  # statistics workspace, two launches
                *ext.sliding_backward(qf, kf, vf, gf, 63, 0, 1),
                # one-pass Longformer backward: from the saved statistics, and without them (the
                # delta-mode forward, then the same pass); per-segment partials + combines
                lo, llse, *ext.longformer_backward(q, k, v, g, 127, 0, 16, out=lo, lse=llse),
                *ext.longformer_backward(q, k, v, g, 127, 0, 16)]

    eager = work()  # the first calls also reserve the kernels' dynamic LDS
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = work()
    for rep in range(3):
        other = ext.sliding_forward(k, q, v, 63, 0)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), (rep, i)
        assert torch.isfinite(other.float()).all()


def test_graph_capture_tiled_and_saved_backward(ext):
    """The tiled backward of a block-sparse table's key sets (tile plan,
    split-tile partials and their sums), recomputing and from the forward's
    saved statistics, and the dense causal backward from saved statistics,
    under capture: every replay bit-identical to the eager results."""
    gen = torch.Generator(device="cuda").manual_seed(12)
    shape = (1, 4096, 4, 64)
    q, k, v, g = (torch.randn(shape, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(4))
    table = ext.BlockTable(ext.make_block_table(9, 64, 2), 4096, 64)
    bset = ext.pattern_index_set("block_sparse", 4096, q.device, block_table=table, block_size=64)

    def work():
        bo, blse = ext.index_set_forward(q, k, v, bset, return_lse=True)
        do, dlse = ext.dense_forward(q, k, v, True, return_lse=True)
        return [bo, blse, *ext.index_set_backward(q, k, v, g, bset),
                *ext.index_set_backward(q, k, v, g, bset, out=bo, lse=blse),
                do, dlse, *ext.dense_backward(q, k, v, g, True, out=do, lse=dlse)]

    eager = work()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = work()
    for rep in range(3):
        other = ext.index_set_backward(k, q, v, g, bset)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), (rep, i)
        assert all(torch.isfinite(t.float()).all() for t in other)
