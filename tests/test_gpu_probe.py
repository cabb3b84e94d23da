"""ma_attn_copy_probe (the stream kernel's access pattern without its
arithmetic, a measurement entry point): every O element is Q xor K xor V of
its own position, for the window shapes bench.py measures it on."""
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


def test_copy_probe_rejects_other_patterns():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import ma_attn
    q = torch.zeros(1, 64, 1, 64, device="cuda", dtype=torch.bfloat16)
    desc = ma_attn.make_desc(1, 64, 1, 64, ma_attn.BF16, ma_attn.DENSE)
    with pytest.raises(RuntimeError, match="SLIDING"):
        ma_attn.copy_probe_raw(desc, q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr())
