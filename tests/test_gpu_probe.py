"""ma_attn_copy_probe (a forward kernel's access pattern without its
arithmetic, a measurement entry point).  SLIDING: every O element is Q xor K
xor V of its own position, for the window shapes bench.py measures it on.
BLOCK_SPARSE: O row i is Q row i xor the K and V rows at the same offset in
every block its table row lists.  ma_attn_backward_copy_probe (the fused
backward's pattern): dQ = Q xor dO, dK = K, dV = V at every position."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape,left,right,dil,dtype", [
    ((1, 5000, 8, 64), 63, 0, 1, torch.bfloat16),
    ((2, 3000, 4, 64), 32, 31, 1, torch.bfloat16),
    ((1, 4099, 8, 64), 63, 0, 4, torch.bfloat16),
    ((2, 2000, 4, 64), 32, 31, 1, torch.float32),
])
def test_copy_probe_covers_every_element(shape, left, right, dil, dtype):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ma_attn
    g = torch.Generator(device="cuda").manual_seed(1)
    q, k, v = (torch.randn(shape, device="cuda", generator=g).to(dtype) for _ in range(3))
    o = torch.full_like(q, 3.0)
    desc = ma_attn.make_desc(*shape, ma_attn.DTYPES[dtype], ma_attn.SLIDING, left=left, right=right, dilation=dil)
    ma_attn.copy_probe_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    it = torch.int16 if dtype != torch.float32 else torch.int32
    want = q.view(it) ^ k.view(it) ^ v.view(it)
    # the halo blocks' K/V words are folded into the first two words of each
    # 16-byte chunk; compare the untouched words exactly, the rest must be written
    w = want.view(torch.int32).reshape(-1, 4)
    got = o.view(torch.int32).reshape(-1, 4)
    assert torch.equal(got[:, 2:], w[:, 2:])
    assert not torch.equal(o.view(it), torch.full_like(o, 3.0).view(it))


@pytest.mark.parametrize("shape,dtype,width", [
    ((2, 1000, 4, 64), torch.bfloat16, 4),
    ((1, 4096, 8, 64), torch.float16, 4),
    ((2, 1500, 2, 64), torch.float32, 4),
    ((1, 777, 3, 64), torch.bfloat16, 3),
])
def test_block_probe_reads_every_listed_block(shape, dtype, width):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ma_attn
    import sparse_attention_cuda as sac
    B, N, H, D = shape
    nb = (N + 63) // 64
    table = sac.make_block_table(7, nb, 2)
    if width < 4:  # rows of 3 entries, every third row padded after its first two
        table = table[:, :width].clone()
        table[::3, 2] = -1
    tab = sac._validated_table(table, nb)
    g = torch.Generator(device="cuda").manual_seed(2)
    q, k, v = (torch.randn(shape, device="cuda", generator=g).to(dtype) for _ in range(3))
    o = torch.full_like(q, 3.0)
    dtab = tab.to("cuda")
    desc = ma_attn.make_desc(*shape, ma_attn.DTYPES[dtype], ma_attn.BLOCK_SPARSE, block_size=64,
                             block_table_ptr=dtab.data_ptr(), blocks_per_row=tab.shape[1])
    ma_attn.copy_probe_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    it = torch.int16 if dtype != torch.float32 else torch.int32
    pad = nb * 64 - N
    kp = torch.nn.functional.pad(k.view(it), (0, 0, 0, 0, 0, pad))  # rows past N read as zero
    vp = torch.nn.functional.pad(v.view(it), (0, 0, 0, 0, 0, pad))
    want = q.view(it).clone()
    i = torch.arange(N, device="cuda")
    for e in range(tab.shape[1]):
        c = dtab[i // 64, e].long()
        src = torch.where(c >= 0, 64 * c + i % 64, 0)
        x = kp[:, src] ^ vp[:, src]
        want ^= torch.where((c >= 0).view(1, N, 1, 1), x, torch.zeros_like(x))
    assert torch.equal(o.view(it), want)


def test_copy_probe_rejects_other_patterns():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ma_attn
    q = torch.zeros(1, 64, 1, 64, device="cuda", dtype=torch.bfloat16)
    desc = ma_attn.make_desc(1, 64, 1, 64, ma_attn.BF16, ma_attn.DENSE)
    with pytest.raises(RuntimeError, match="SLIDING"):
        ma_attn.copy_probe_raw(desc, q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr())


@pytest.mark.parametrize("shape,left,right,dil,dtype", [
    ((1, 5000, 8, 64), 63, 0, 1, torch.bfloat16),
    ((2, 3000, 4, 64), 32, 31, 1, torch.bfloat16),
    ((1, 4099, 8, 64), 63, 0, 4, torch.bfloat16),
    ((2, 1000, 3, 64), 32, 31, 2, torch.float16),
    ((1, 100, 2, 64), 63, 0, 1, torch.float16),
])
def test_backward_copy_probe_writes_every_row_once(shape, left, right, dil, dtype):
    """ma_attn_backward_copy_probe: every dQ row is Q xor dO of its position,
    every dK / dV row a copy of K / V, so the fused kernel's chunks and steps
    reach each query tile and key block with one writer."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ma_attn
    g = torch.Generator(device="cuda").manual_seed(3)
    q, k, v, dout = (torch.randn(shape, device="cuda", generator=g).to(dtype) for _ in range(4))
    dq, dk, dv = (torch.full_like(q, 3.0) for _ in range(3))
    desc = ma_attn.make_desc(*shape, ma_attn.DTYPES[dtype], ma_attn.SLIDING, left=left, right=right, dilation=dil)
    ma_attn.backward_copy_probe_raw(desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), dout.data_ptr(), dq.data_ptr(),
                                    dk.data_ptr(), dv.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(dq.view(torch.int16), q.view(torch.int16) ^ dout.view(torch.int16))
    assert torch.equal(dk.view(torch.int16), k.view(torch.int16))
    assert torch.equal(dv.view(torch.int16), v.view(torch.int16))


@pytest.mark.parametrize("dtype,left,right", [(torch.float32, 63, 0), (torch.bfloat16, 40, 0)])
def test_backward_copy_probe_rejects_unfused_windows(dtype, left, right):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ma_attn
    q = torch.zeros(1, 128, 1, 64, device="cuda", dtype=dtype)
    desc = ma_attn.make_desc(1, 128, 1, 64, ma_attn.DTYPES[dtype], ma_attn.SLIDING, left=left, right=right)
    p = q.data_ptr()
    with pytest.raises(RuntimeError, match="fused backward does not take"):
        ma_attn.backward_copy_probe_raw(desc, p, p, p, p, p, p, p)
