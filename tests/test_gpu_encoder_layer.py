"""The fused encoder layer (ma_encoder_layer_forward): one HIP kernel for the
reference's CustomTransformerEncoderLayer in eval mode (src/model.py:42-53).

Checked in float32 against
* a float64 CPU evaluation of the layer (textbook masked attention over keys
  [i-w, i+w], LayerNorm, Linear, ReLU): max-abs <= 1e-5, and
* the layer's own PyTorch operations on the GPU (the unfused forward, whose
  attention is the engine's sliding-window kernel): max-abs <= 1e-5.
"""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module")
def model_mod():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import model
    return model


def _layer(model_mod, d, window, seed):
    torch.manual_seed(seed)
    layer = model_mod.CustomTransformerEncoderLayer(d_model=d, num_heads=1, window_size=window, fused=True)
    with torch.no_grad():  # non-trivial LayerNorm affine parameters
        for n in (layer.norm1, layer.norm2):
            n.weight.uniform_(0.5, 1.5)
            n.bias.uniform_(-0.2, 0.2)
    return layer.cuda().eval()


def _ref64(layer, src, window):
    """The layer in float64 on the CPU."""
    x = src.detach().double().cpu()
    B, S, D = x.shape
    g = {n: p.detach().double().cpu() for n, p in layer.named_parameters()}
    i = torch.arange(S).unsqueeze(1)
    j = torch.arange(S).unsqueeze(0)
    band = (j >= i - window) & (j <= i + window)
    s = (x @ x.transpose(1, 2)) / (D ** 0.5)
    s = s.masked_fill(~band, float("-inf"))
    attn = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0) @ x
    ln = torch.nn.functional.layer_norm
    h = ln(x + attn, (D,), g["norm1.weight"], g["norm1.bias"], layer.norm1.eps)
    z = torch.relu(h @ g["linear1.weight"].T + g["linear1.bias"])
    y = z @ g["linear2.weight"].T + g["linear2.bias"]
    return ln(h + y, (D,), g["norm2.weight"], g["norm2.bias"], layer.norm2.eps)


def _unfused(layer, src):
    layer.fused = False
    try:
        return layer(src)
    finally:
        layer.fused = True


@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("B,S,window", [(64, 10, 3), (3, 37, 3), (2, 100, 7), (5, 1, 3), (4, 20, 25)])
def test_fused_layer_matches_layer(model_mod, d, B, S, window):
    layer = _layer(model_mod, d, window, 100 + d + S)
    src = torch.randn(B, S, d, device="cuda")
    with torch.no_grad():
        out = layer(src)
        unfused = _unfused(layer, src)
    ref = _ref64(layer, src, window)
    err64 = (out.double().cpu() - ref).abs().max().item()
    err_ops = (out - unfused).abs().max().item()
    print(f"d={d} B={B} S={S} w={window}: max|err| vs float64 {err64:.2e}, vs the layer's ops {err_ops:.2e}",
          flush=True)
    assert err64 <= TOL and err_ops <= TOL


@pytest.mark.parametrize("d", [32, 64])
def test_fused_block_with_given_attention(model_mod, d):
    """attn given: only the post-attention block runs in the kernel."""
    layer = _layer(model_mod, d, 3, 7 + d)
    src = torch.randn(64, 10, d, device="cuda")
    with torch.no_grad():
        attn = layer.self_attn(src, src, src)
        out = model_mod.encoder_layer_forward(layer, src, attn)
        unfused = _unfused(layer, src)
    assert (out - unfused).abs().max().item() <= TOL
    assert (out.double().cpu() - _ref64(layer, src, 3)).abs().max().item() <= TOL


def test_fused_layer_window_edges(model_mod):
    """Window 0 (attention output = src) and a window wider than the sequence
    (dense attention), through the C-ABI's window field."""
    layer = _layer(model_mod, 64, 3, 5)
    src = torch.randn(8, 12, 64, device="cuda")
    with torch.no_grad():
        for w in (0, 11, 40):
            layer.self_attn.window_size = w
            out = model_mod.encoder_layer_forward(layer, src)
            err = (out.double().cpu() - _ref64(layer, src, w)).abs().max().item()
            assert err <= TOL, (w, err)


def test_fused_model_matches_unfused(model_mod):
    """TransformerModel(fused_layers=True) at the reference's configuration
    (batch 64, sequence 10, input 5, model_dim 64, 4 layers): the same
    prediction as the unfused model, with no separate attention launch."""
    import sparse_attention_cuda as ext
    torch.manual_seed(3)
    fused = model_mod.TransformerModel(input_dim=5, model_dim=64, num_heads=2, num_layers=4,
                                       fused_layers=True).cuda().eval()
    plain = copy.deepcopy(fused)
    for layer in plain.encoder_layers:
        layer.fused = False
    src = torch.randn(64, 10, 5, device="cuda")
    calls = {"n": 0}
    orig = ext.forward

    def counting(*a, **kw):
        calls["n"] += 1
        return orig(*a, **kw)
    ext.forward = counting
    try:
        with torch.no_grad():
            y_fused = fused(src)
            n_fused = calls["n"]
            y_plain = plain(src)
    finally:
        ext.forward = orig
    assert n_fused == 0 and calls["n"] == 4
    err = (y_fused - y_plain).abs().max().item()
    print(f"model: max|err| fused vs unfused {err:.2e}", flush=True)
    assert err <= TOL


def test_fused_layer_not_taken_when_recording_gradients(model_mod):
    """With gradients recorded (or in training mode) the layer runs its
    operations, so backward works; the result equals the fused inference."""
    layer = _layer(model_mod, 32, 3, 9)
    src = torch.randn(4, 10, 32, device="cuda", requires_grad=True)
    out = layer(src)
    assert out.grad_fn is not None
    out.sum().backward()
    assert src.grad is not None and layer.linear1.weight.grad is not None
    with torch.no_grad():
        assert (layer(src) - out.detach()).abs().max().item() <= TOL


def test_fused_layer_rejects(model_mod):
    import ma_attn
    layer = _layer(model_mod, 48, 3, 1)  # d_model 48: no kernel instantiation
    src = torch.randn(2, 10, 48, device="cuda")
    with torch.no_grad(), pytest.raises(RuntimeError, match="d_model"):
        model_mod.encoder_layer_forward(layer, src)  # the kernel itself; the layer runs its operations
    layer = _layer(model_mod, 64, 3, 1)
    src = torch.randn(2, 10, 64, device="cuda")
    L = ma_attn.EncoderLayer()
    L.batch, L.seq_len, L.d_model, L.d_ff, L.window, L.ln_eps = 2, 10, 64, 256, 3, 1e-5
    params = [layer.norm1.weight, layer.norm1.bias, layer.linear1.weight, layer.linear1.bias,
              layer.linear2.weight, layer.linear2.bias, layer.norm2.weight, layer.norm2.bias]
    (L.norm1_weight, L.norm1_bias, L.linear1_weight, L.linear1_bias, L.linear2_weight, L.linear2_bias,
     L.norm2_weight, L.norm2_bias) = (p.data_ptr() for p in params)
    with pytest.raises(RuntimeError, match="overlaps"):
        ma_attn.encoder_layer_forward_raw(L, src.data_ptr(), 0, src.data_ptr())
    L.d_ff = 128
    out = torch.empty_like(src)
    with pytest.raises(RuntimeError, match="d_ff"):
        ma_attn.encoder_layer_forward_raw(L, src.data_ptr(), 0, out.data_ptr())


def test_fused_model_other_width_runs_its_operations(model_mod):
    """fused_layers=True with a model width the fused kernel has no
    instantiation for (48): the layers run their separate operations, with the
    unfused model's result."""
    import sparse_attention_cuda as ext
    torch.manual_seed(4)
    fused = model_mod.TransformerModel(input_dim=5, model_dim=48, num_heads=2, num_layers=2,
                                       fused_layers=True).cuda().eval()
    plain = copy.deepcopy(fused)
    for layer in plain.encoder_layers:
        layer.fused = False
    src = torch.randn(8, 10, 5, device="cuda")
    calls = {"n": 0}
    orig = ext.forward

    def counting(*a, **kw):
        calls["n"] += 1
        return orig(*a, **kw)
    ext.forward = counting
    try:
        with torch.no_grad():
            y_fused = fused(src)
            y_plain = plain(src)
    finally:
        ext.forward = orig
    assert calls["n"] == 4  # two layers, each through the attention entry point, twice
    assert torch.equal(y_fused, y_plain)
