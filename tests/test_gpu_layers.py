"""The reference's layer-level tests on device tensors, through the HIP kernels.

The reference runs these module calls on its CPU engine and checks shapes,
dtypes and finiteness (tests/integration/test_ma_core_bridge.py,
test_error_handling.py, test_pytorch_compatibility.py).  Here the same calls
take device tensors, with the native path forced (eval mode, or
``fallback_training=False``), and the values are also checked against the
oracle: fp32 forward <= 1e-5, fp32 backward <= 1e-4.
"""
import numpy as np
import pytest
import torch
import torch.nn as nn

from conftest import qkv
from layers.ma_core_bridge import MACoreAttention
from layers.sparse_attention import SparseAttention

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def ext():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import sparse_attention_cuda
    return sparse_attention_cuda


@pytest.fixture
def calls(ext, monkeypatch):
    """Counts the engine's forward/backward entry points, so a test can show
    that the native path ran."""
    n = {}
    for name in ("forward", "dense_forward", "backward", "dense_backward"):
        f = getattr(ext, name)

        def wrap(*a, _f=f, _n=name, **kw):
            n[_n] = n.get(_n, 0) + 1
            return _f(*a, **kw)
        monkeypatch.setattr(ext, name, wrap)
    return n


def _spec(O, shape, sparse, w, causal=False):
    B, N, H, D = shape
    if sparse:
        return O.Spec(B, N, H, D, "sliding", left=w, right=w)
    return O.Spec(B, N, H, D, "dense", causal=causal)


def _oracle_fwd(O, q, k, v, sparse, w=0, causal=False):
    spec = _spec(O, q.shape, sparse, w, causal)
    return torch.from_numpy(O.forward(spec, q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()))


def _dev(*arrays):
    return [torch.from_numpy(a).to(DEV) for a in arrays]


# -- test_ma_core_bridge.py: forward --------------------------------------------------------

def test_dense_attention_forward(ext, oracle, calls):
    """:23-37 (small tensors 1x4x2x8)."""
    q, k, v = _dev(*qkv((1, 4, 2, 8), 11))
    att = MACoreAttention(sparse=False).eval()
    out = att(q, k, v)
    assert out.shape == q.shape and out.dtype == q.dtype and out.is_cuda
    assert calls.get("dense_forward") == 1
    torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, False), rtol=0, atol=1e-5)


@pytest.mark.parametrize("w", [2, 4, 8, 16])
def test_sparse_attention_forward(ext, oracle, calls, w):
    """:39-53 with the window_sizes fixture (2, 4, 8, 16)."""
    q, k, v = _dev(*qkv((1, 4, 2, 8), 12 + w))
    out = MACoreAttention(sparse=True, window_size=w).eval()(q, k, v)
    assert calls.get("forward") == 1
    torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, True, w), rtol=0, atol=1e-5)


def test_causal_mask_attention(ext, oracle):
    """:55-66."""
    q, k, v = _dev(*qkv((1, 4, 2, 8), 13))
    out = MACoreAttention(sparse=False, use_causal_mask=True).eval()(q, k, v)
    torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, False, causal=True), rtol=0, atol=1e-5)


def test_attention_module_modes(ext, calls):
    """:68-88: training mode (PyTorch path, fallback_training=True) and eval
    mode (engine) agree on the same inputs."""
    q, k, v = _dev(*qkv((1, 4, 2, 8), 14))
    att = MACoreAttention(sparse=True, window_size=4, fallback_training=True)
    train_out = att.train()(q, k, v)
    assert not calls
    with torch.no_grad():
        eval_out = att.eval()(q, k, v)
    assert calls.get("forward") == 1
    torch.testing.assert_close(eval_out, train_out, rtol=0, atol=1e-5)


# -- test_ma_core_bridge.py: gradients -----------------------------------------------------

@pytest.mark.parametrize("sparse", [False, True])
def test_attention_gradients(ext, oracle, calls, sparse):
    """:95-140 with fallback_training=False, so the HIP backward produces the
    gradients; checked against the oracle's backward."""
    qn, kn, vn = qkv((1, 4, 2, 8), 15)
    q, k, v = (t.requires_grad_(True) for t in _dev(qn, kn, vn))
    att = MACoreAttention(sparse=sparse, window_size=2, fallback_training=False).train()
    out = att(q, k, v)
    out.sum().backward()
    assert calls.get("backward" if sparse else "dense_backward") == 1
    spec = _spec(oracle, qn.shape, sparse, 2)
    dq, dk, dv = oracle.backward(spec, qn, kn, vn, np.ones_like(qn))
    for g, r in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        assert g.shape == q.shape
        torch.testing.assert_close(g.cpu(), torch.from_numpy(r), rtol=0, atol=1e-4)


def test_gradient_accumulation(ext):
    """:143-170: a second backward adds to the first (here: exactly twice it)."""
    q, k, v = (t.requires_grad_(True) for t in _dev(*qkv((1, 4, 2, 8), 16)))
    att = MACoreAttention(sparse=True, window_size=2, fallback_training=False).train()
    att(q, k, v).sum().backward()
    first = [t.grad.clone() for t in (q, k, v)]
    att(q, k, v).sum().backward()
    for t, g1 in zip((q, k, v), first):
        assert not torch.equal(t.grad, g1)
        torch.testing.assert_close(t.grad, 2 * g1, rtol=0, atol=0)


# -- test_ma_core_bridge.py: numerics -------------------------------------------------------

def test_attention_self_consistency(ext):
    """:176-189: identical calls give identical bits (Q = K, V = 2)."""
    torch.manual_seed(42)
    q = torch.randn(1, 8, 2, 16, device=DEV)
    v = torch.full((1, 8, 2, 16), 2.0, device=DEV)
    att = MACoreAttention(sparse=False).eval()
    with torch.no_grad():
        o1, o2 = att(q, q.clone(), v), att(q, q.clone(), v)
    assert torch.equal(o1, o2)
    torch.testing.assert_close(o1, v, rtol=0, atol=1e-6)  # constant V: O = V


def test_attention_symmetry(ext):
    """:191-208: Q = K = ones gives equal scores, so every row is the mean of V."""
    v = torch.randn(1, 4, 1, 8, device=DEV)
    q = torch.ones(1, 4, 1, 8, device=DEV)
    with torch.no_grad():
        out = MACoreAttention(sparse=False).eval()(q, q.clone(), v)
    torch.testing.assert_close(out, v.mean(dim=1, keepdim=True).expand_as(v), rtol=0, atol=1e-6)


def test_attention_scale_invariance(ext, oracle):
    """:211-232: inputs scaled by 2 (a different softmax, still exact against the oracle)."""
    q, k, v = _dev(*qkv((1, 4, 2, 8), 17))
    att = MACoreAttention(sparse=False).eval()
    with torch.no_grad():
        for s in (1.0, 2.0):
            out = att(q * s, k * s, v)
            torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q * s, k * s, v, False), rtol=0, atol=1e-5)


def test_extreme_window_sizes(ext, oracle):
    """:281-296: window 1 and a window longer than the sequence (= dense)."""
    q, k, v = _dev(*qkv((1, 4, 2, 8), 18))
    for w in (1, 100):
        out = MACoreAttention(sparse=True, window_size=w).eval()(q, k, v)
        torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, True, w), rtol=0, atol=1e-5)
    dense = MACoreAttention(sparse=False).eval()(q, k, v)
    torch.testing.assert_close(MACoreAttention(sparse=True, window_size=100).eval()(q, k, v), dense,
                               rtol=0, atol=1e-6)


@pytest.mark.parametrize("shape", [(1, 4, 2, 8), (2, 8, 4, 16), (1, 16, 8, 32)])
@pytest.mark.parametrize("sparse,w,causal", [(True, 2, False), (True, 8, False), (True, 16, False),
                                             (False, 0, True), (False, 0, False)])
def test_attention_configurations(ext, oracle, shape, sparse, w, causal):
    """:329-357 (tensor_shapes fixture x sparse x window x causal)."""
    q, k, v = _dev(*qkv(shape, 19))
    att = (MACoreAttention(sparse=True, window_size=w) if sparse
           else MACoreAttention(sparse=False, use_causal_mask=causal)).eval()
    out = att(q, k, v)
    torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, sparse, w, causal), rtol=0, atol=1e-5)


@pytest.mark.parametrize("shape", [(1, 8, 1, 16), (1, 8, 4, 16), (2, 16, 2, 32), (1, 32, 8, 64)])
def test_various_tensor_sizes(ext, oracle, shape):
    """:360-377 (window 4)."""
    q, k, v = _dev(*qkv(shape, 20))
    out = MACoreAttention(sparse=True, window_size=4).eval()(q, k, v)
    torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, True, 4), rtol=0, atol=1e-5)


# -- test_error_handling.py on device tensors ------------------------------------------------

@pytest.mark.parametrize("training", [True, False])
def test_mismatched_shapes_on_device(ext, calls, training):
    """:17-61: mismatches raise before the engine is called."""
    att = MACoreAttention(sparse=True, window_size=4, fallback_training=False).train(training)
    good = torch.randn(1, 8, 2, 16, device=DEV)
    for bad in ((1, 6, 2, 16), (1, 8, 2, 32), (2, 8, 2, 16)):
        with pytest.raises(ValueError):
            att(good, torch.randn(*bad, device=DEV), good)
    with pytest.raises(ValueError):
        z = torch.randn(0, 8, 2, 16, device=DEV)
        att(z, z, z)
    assert not calls


def test_engine_rejects_what_the_module_would(ext):
    """The module-level checks have engine twins (RuntimeError, .cu:427-432)."""
    q = torch.randn(1, 8, 2, 16, device=DEV)
    with pytest.raises(RuntimeError):
        ext.forward(q, torch.randn(1, 6, 2, 16, device=DEV), q, 4)
    with pytest.raises(RuntimeError):
        ext.forward(q, q, q.cpu(), 4)
    with pytest.raises(RuntimeError):
        ext.dense_forward(q, q.half(), q, False)


def test_extreme_values(ext, oracle):
    """:99-122: inputs x100 and x1e-6 stay finite; the small ones match the oracle."""
    att = MACoreAttention(sparse=True, window_size=4).eval()
    qn, kn, vn = qkv((1, 8, 2, 16), 21)
    q, k, v = _dev(qn * 100, kn * 100, vn * 100)
    assert torch.isfinite(att(q, k, v)).all()
    q, k, v = _dev(qn * 1e-6, kn * 1e-6, vn * 1e-6)
    out = att(q, k, v)
    torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, True, 4), rtol=1e-5, atol=1e-12)


def test_nan_input_handling(ext, oracle):
    """:124-144: a NaN in query row 0 may only reach output row 0 (dense)."""
    qn, kn, vn = qkv((1, 4, 1, 8), 22)
    qn[0, 0, 0, 0] = np.nan
    q, k, v = _dev(qn, kn, vn)
    out = MACoreAttention(sparse=False).eval()(q, k, v).cpu()
    ref = _oracle_fwd(oracle, q, k, v, False)
    assert torch.isfinite(out[:, 1:]).all()
    torch.testing.assert_close(out[:, 1:], ref[:, 1:], rtol=0, atol=1e-5)


def test_inf_input_handling(ext, oracle):
    """:146-165: an inf in key 0 may only reach rows whose window holds key 0."""
    qn, kn, vn = qkv((1, 4, 1, 8), 23)
    kn[0, 0, 0, 0] = np.inf
    q, k, v = _dev(qn, kn, vn)
    out = MACoreAttention(sparse=True, window_size=2).eval()(q, k, v).cpu()
    ref = _oracle_fwd(oracle, q, k, v, True, 2)
    torch.testing.assert_close(out[:, 3:], ref[:, 3:], rtol=0, atol=1e-5)


def test_gradient_numerical_stability(ext):
    """:167-187 with the HIP backward: Q, K x10 and V x0.1 give finite gradients."""
    base = _dev(*qkv((1, 6, 1, 8), 24))
    q = (base[0] * 10).requires_grad_(True)
    k = (base[1] * 10).requires_grad_(True)
    v = (base[2] * 0.1).requires_grad_(True)
    att = MACoreAttention(sparse=True, window_size=3, fallback_training=False).train()
    att(q, k, v).sum().backward()
    for t in (q, k, v):
        assert torch.isfinite(t.grad).all()


def test_single_element_tensors(ext):
    """:193-205: one key, so O = V."""
    q, k, v = (torch.randn(1, 1, 1, 1, device=DEV) for _ in range(3))
    out = MACoreAttention(sparse=True, window_size=1).eval()(q, k, v)
    assert out.shape == (1, 1, 1, 1)
    torch.testing.assert_close(out, v, rtol=0, atol=0)


def test_very_long_sequences(ext, oracle):
    """:207-222 (1x1024x2x16, window 8)."""
    q, k, v = _dev(*qkv((1, 1024, 2, 16), 25))
    out = MACoreAttention(sparse=True, window_size=8).eval()(q, k, v)
    torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, True, 8), rtol=0, atol=1e-5)


def test_identical_and_orthogonal_qk(ext, oracle):
    """:240-273."""
    t = torch.from_numpy(qkv((1, 4, 2, 8), 26)[0]).to(DEV)
    att = MACoreAttention(sparse=False).eval()
    torch.testing.assert_close(att(t, t, t).cpu(), _oracle_fwd(oracle, t, t, t, False), rtol=0, atol=1e-5)
    q = torch.eye(4, device=DEV).view(1, 4, 1, 4)
    k = q[:, [1, 0, 3, 2]].contiguous()
    v = torch.randn(1, 4, 1, 4, device=DEV)
    torch.testing.assert_close(att(q, k, v).cpu(), _oracle_fwd(oracle, q, k, v, False), rtol=0, atol=1e-5)


def test_error_recovery(ext, oracle):
    """:338-359: a rejected call leaves the module working."""
    att = MACoreAttention(sparse=True, window_size=4).eval()
    with pytest.raises(ValueError):
        att(torch.randn(1, 4, 2, 8, device=DEV), torch.randn(1, 6, 2, 8, device=DEV),
            torch.randn(1, 4, 2, 8, device=DEV))
    q, k, v = _dev(*qkv((1, 4, 2, 8), 27))
    torch.testing.assert_close(att(q, k, v).cpu(), _oracle_fwd(oracle, q, k, v, True, 4), rtol=0, atol=1e-5)


# -- test_pytorch_compatibility.py -----------------------------------------------------------

class SimpleTransformerBlock(nn.Module):
    """The reference test's block (:15-63): LayerNorm, Q/K/V projections to
    [B, S, heads, head_dim], MACoreAttention or SparseAttention, output
    projection, residual."""

    def __init__(self, model_dim=64, num_heads=4, use_ma_core=True, window_size=8, fallback_training=True):
        super().__init__()
        self.model_dim, self.num_heads, self.head_dim = model_dim, num_heads, model_dim // num_heads
        self.q_proj = nn.Linear(model_dim, model_dim)
        self.k_proj = nn.Linear(model_dim, model_dim)
        self.v_proj = nn.Linear(model_dim, model_dim)
        self.out_proj = nn.Linear(model_dim, model_dim)
        if use_ma_core:
            self.attention = MACoreAttention(sparse=True, window_size=window_size,
                                             fallback_training=fallback_training)
        else:
            self.attention = SparseAttention(window_size=window_size, use_ma_core=False)
        self.norm = nn.LayerNorm(model_dim)

    def forward(self, x):
        residual = x
        x = self.norm(x)
        b, s, m = x.shape
        if getattr(self.attention, "sparse", False):
            shape = (b, s, self.num_heads, self.head_dim)
            a = self.attention(self.q_proj(x).view(shape), self.k_proj(x).view(shape),
                               self.v_proj(x).view(shape)).reshape(b, s, m)
        else:
            a = self.attention(self.q_proj(x), self.k_proj(x), self.v_proj(x))
        return residual + self.out_proj(a)


def test_sparse_attention_basic(ext, oracle, calls):
    """:74-88: SparseAttention [B, S, Dm] (one head) on the engine."""
    q, k, v = _dev(*(x[:, :, 0] for x in qkv((2, 16, 1, 32), 28)))
    with torch.no_grad():
        out = SparseAttention(window_size=3).eval()(q, k, v)
    assert out.shape == (2, 16, 32) and calls.get("forward") == 1
    ref = _oracle_fwd(oracle, q.unsqueeze(2), k.unsqueeze(2), v.unsqueeze(2), True, 3).squeeze(2)
    torch.testing.assert_close(out.cpu(), ref, rtol=0, atol=1e-5)


@pytest.mark.parametrize("model_dim,heads,w,seq", [(32, 4, 4, 8), (32, 4, 6, 12), (24, 3, 4, 6)])
def test_transformer_block_inference(ext, calls, model_dim, heads, w, seq):
    """:146-156, :179-192, :194-213: the block on the engine against the same
    weights on the host (PyTorch path)."""
    torch.manual_seed(model_dim + w)
    cpu = SimpleTransformerBlock(model_dim, heads, True, w).eval()
    x = torch.randn(2, seq, model_dim)
    with torch.no_grad():
        ref = cpu(x)
        out = SimpleTransformerBlock(model_dim, heads, True, w).to(DEV).eval()
        out.load_state_dict(cpu.state_dict())
        y = out(x.to(DEV))
    assert calls.get("forward") == 1
    torch.testing.assert_close(y.cpu(), ref, rtol=1e-4, atol=1e-4)


def test_transformer_block_training(ext, calls):
    """:158-177 with fallback_training=False: three Adam steps on the engine's
    forward and backward track the same steps on the host."""
    torch.manual_seed(3)
    host = SimpleTransformerBlock(16, 2, True, 2, fallback_training=False)
    dev = SimpleTransformerBlock(16, 2, True, 2, fallback_training=False).to(DEV)
    dev.load_state_dict(host.state_dict())
    opt_h = torch.optim.Adam(host.parameters(), lr=1e-3)
    opt_d = torch.optim.Adam(dev.parameters(), lr=1e-3)
    for step in range(3):
        x, tgt = torch.randn(1, 4, 16), torch.randn(1, 4, 16)
        losses = []
        for m, opt, xx, tt in ((host, opt_h, x, tgt), (dev, opt_d, x.to(DEV), tgt.to(DEV))):
            opt.zero_grad()
            loss = nn.functional.mse_loss(m(xx), tt)
            loss.backward()
            opt.step()
            losses.append(loss.item())
        assert np.isfinite(losses[1])
        assert abs(losses[0] - losses[1]) <= 1e-5 * max(1.0, abs(losses[0]))
    assert calls.get("forward") == 3 and calls.get("backward") == 3
    # A bias added to every key shifts all of a query's scores equally, so the
    # softmax ignores it: k_proj.bias has a zero gradient in exact arithmetic,
    # and Adam scales the rounding noise left in it to full-size steps.  It
    # is checked for that zero instead (the column sums of dK vanish).
    assert dev.k_proj.bias.grad.abs().max().item() <= 1e-5
    for (n, p), q in zip(host.named_parameters(), dev.parameters()):
        if n != "k_proj.bias":
            torch.testing.assert_close(q.detach().cpu(), p.detach(), rtol=1e-4, atol=1e-4, msg=n)


@pytest.mark.parametrize("batch_size", [1, 2, 4])
def test_different_batch_sizes(ext, oracle, batch_size):
    """:215-229."""
    q, k, v = _dev(*qkv((batch_size, 8, 2, 16), 29))
    out = MACoreAttention(sparse=True, window_size=4).eval()(q, k, v)
    torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, True, 4), rtol=0, atol=1e-5)


def test_large_sequence_sparse_attention(ext, oracle):
    """:231-245 (1x64x4x32, window 8) and :247-281 (1x128x4x64, window 16)."""
    for shape, w in (((1, 64, 4, 32), 8), ((1, 128, 4, 64), 16)):
        q, k, v = _dev(*qkv(shape, 30))
        with torch.no_grad():
            out = MACoreAttention(sparse=True, window_size=w).eval()(q, k, v)
        torch.testing.assert_close(out.cpu(), _oracle_fwd(oracle, q, k, v, True, w), rtol=0, atol=1e-5)


def test_model_state_dict(ext):
    """:283-306: a reloaded block gives the same bits on the engine."""
    torch.manual_seed(4)
    a = SimpleTransformerBlock(32, 4, True, 8).to(DEV).eval()
    b = SimpleTransformerBlock(32, 4, True, 8).to(DEV).eval()
    b.load_state_dict(a.state_dict())
    x = torch.randn(1, 8, 32, device=DEV)
    with torch.no_grad():
        assert torch.equal(a(x), b(x))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mixed_precision_compatibility(ext, calls, dtype):
    """:344-358: the half-precision block runs on the engine (the reference
    skips when it cannot) and stays within 16-bit rounding of fp32."""
    torch.manual_seed(5)
    ref_block = SimpleTransformerBlock(32, 4, True, 8).to(DEV).eval()
    x = torch.randn(1, 8, 32, device=DEV)
    with torch.no_grad():
        ref = ref_block(x)
        half = SimpleTransformerBlock(32, 4, True, 8).to(DEV).eval()
        half.load_state_dict(ref_block.state_dict())
        out = half.to(dtype)(x.to(dtype))
    assert out.dtype == dtype and calls.get("forward") == 2
    torch.testing.assert_close(out.float(), ref, rtol=0, atol=2e-2 if dtype == torch.float16 else 1e-1)


def test_device_consistency(ext):
    """:360-371: outputs stay on the input's device, host or GPU."""
    torch.manual_seed(6)
    m = SimpleTransformerBlock(16, 2, True, 8).eval()
    x = torch.randn(1, 4, 16)
    with torch.no_grad():
        assert m(x).device.type == "cpu"
        assert m.to(DEV)(x.to(DEV)).device.type == "cuda"

