"""The toy TransformerModel (reference src/model.py) on the engine's attention:
structure and CPU semantics (no GPU needed)."""
import math

import pytest
import torch
import torch.nn.functional as F


def _window_attention(x, w):
    """Single-head attention over keys |i - j| <= w, written with torch SDPA."""
    S, D = x.shape[1], x.shape[2]
    i = torch.arange(S)
    mask = (i.view(-1, 1) - i.view(1, -1)).abs() <= w
    return F.scaled_dot_product_attention(x.unsqueeze(1), x.unsqueeze(1), x.unsqueeze(1), attn_mask=mask,
                                          scale=1.0 / math.sqrt(D)).squeeze(1)


def _manual_forward(m, src):
    """The reference forward (model.py:80-91, :42-52) restated with SDPA."""
    x = m.encoder(src) * math.sqrt(m.model_dim)
    x = x + m.pos_encoder.pe[:x.size(0), :]
    for layer in m.encoder_layers:
        x = layer.norm1(x + _window_attention(x, layer.self_attn.window_size))
        x = layer.norm2(x + layer.linear2(F.relu(layer.linear1(x))))
    return m.decoder(x[:, -1, :])


def test_state_dict_names_match_reference():
    from model import TransformerModel
    m = TransformerModel(input_dim=5, model_dim=32, num_heads=2, num_layers=2)
    want = {"encoder.weight", "encoder.bias", "pos_encoder.pe", "decoder.weight", "decoder.bias"}
    for l in range(2):
        for n in ("linear1", "linear2", "norm1", "norm2"):
            want |= {f"encoder_layers.{l}.{n}.weight", f"encoder_layers.{l}.{n}.bias"}
    assert set(m.state_dict()) == want
    assert m.pos_encoder.pe.shape == (5000, 1, 32)


@pytest.mark.parametrize("model_dim,num_layers", [(32, 2), (64, 4)])
def test_cpu_forward_matches_restatement(model_dim, num_layers):
    from model import TransformerModel
    torch.manual_seed(0)
    m = TransformerModel(input_dim=5, model_dim=model_dim, num_heads=2, num_layers=num_layers).eval()
    src = torch.randn(64, 10, 5)
    with torch.no_grad():
        out = m(src)
        ref = _manual_forward(m, src)
    assert out.shape == (64, 1)
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
