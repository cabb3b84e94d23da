"""The toy TransformerModel end to end on the GPU: inference through the HIP
forward kernels and a training step through the HIP forward + backward
kernels, against the same weights on the PyTorch path (float32)."""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import sparse_attention_cuda
    return sparse_attention_cuda


def _count_calls(monkeypatch, ext, names):
    calls = {n: 0 for n in names}
    for n in names:
        f = getattr(ext, n)

        def wrap(*a, _f=f, _n=n, **kw):
            calls[_n] += 1
            return _f(*a, **kw)
        monkeypatch.setattr(ext, n, wrap)
    return calls


@pytest.mark.parametrize("model_dim,num_layers", [(32, 2), (64, 4)])
def test_model_inference_native(ext, monkeypatch, model_dim, num_layers):
    from model import TransformerModel
    torch.manual_seed(1)
    m = TransformerModel(input_dim=5, model_dim=model_dim, num_heads=2, num_layers=num_layers).eval()
    src = torch.randn(64, 10, 5)
    with torch.no_grad():
        ref = m(src)  # host tensors: the PyTorch path
        calls = _count_calls(monkeypatch, ext, ["forward"])
        out = m.cuda()(src.cuda())
    assert calls["forward"] == num_layers
    torch.testing.assert_close(out.cpu(), ref, rtol=1e-4, atol=1e-4)


def test_model_training_step_native(ext, monkeypatch):
    """fallback_training=False: loss, every parameter gradient and the
    updated weights match the PyTorch path (dropout 0)."""
    from model import TransformerModel
    torch.manual_seed(2)
    native = TransformerModel(input_dim=5, model_dim=64, num_heads=2, num_layers=2, dropout=0.0,
                              fallback_training=False).cuda().train()
    torch_path = copy.deepcopy(native)
    for layer in torch_path.encoder_layers:
        layer.self_attn.use_ma_core = False  # SparseAttention._pytorch_forward (window w-1)
        layer.self_attn.window_size += 1     # same key set |i-j| <= 3 as the engine's window 3
    src = torch.randn(64, 10, 5, device="cuda")
    tgt = torch.randn(64, 1, device="cuda")
    calls = _count_calls(monkeypatch, ext, ["forward", "backward"])
    losses = []
    for m in (native, torch_path):
        opt = torch.optim.Adam(m.parameters(), lr=1e-3)
        opt.zero_grad()
        loss = torch.nn.functional.mse_loss(m(src), tgt)
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert calls == {"forward": 2, "backward": 2}
    assert abs(losses[0] - losses[1]) <= 1e-5
    for (n, a), (_, b) in zip(native.named_parameters(), torch_path.named_parameters()):
        torch.testing.assert_close(a.grad, b.grad, rtol=1e-4, atol=1e-5, msg=n)
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5, msg=n)
