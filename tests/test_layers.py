"""The layer surface's construction and validation rules, on the CPU.

These are the reference's own layer tests that need no device
(tests/integration/test_error_handling.py, test_ma_core_bridge.py:299-326,
test_pytorch_compatibility.py:283-342): constructor and factory errors,
input validation before any engine call, and module state after an error.
The same calls on device tensors, routed to the HIP kernels, are in
test_gpu_layers.py.
"""
import pytest
import torch
import torch.nn as nn

from layers.ma_core_bridge import MACoreAttention, create_attention_layer
from layers.sparse_attention import SparseAttention


def _t(*shape):
    return torch.randn(*shape)


def test_invalid_window_sizes():
    """test_error_handling.py:85-93: window 0 and -1 are refused at construction."""
    for w in (0, -1):
        with pytest.raises(ValueError):
            MACoreAttention(sparse=True, window_size=w, fallback_training=True)
    with pytest.raises(TypeError):
        MACoreAttention(sparse=True, window_size=2.5)
    # the window is not checked for dense modules (reference :272-280)
    assert MACoreAttention(sparse=False, window_size=0).window_size == 0


def test_sparse_attention_invalid_construction():
    """test_error_handling.py:279-287."""
    for w in (-1, 0):
        with pytest.raises(ValueError):
            SparseAttention(window_size=w)
    with pytest.raises(TypeError):
        SparseAttention(window_size=3.0)


def test_create_attention_layer():
    """test_ma_core_bridge.py:302-319."""
    dense = create_attention_layer("dense", use_causal_mask=True)
    assert isinstance(dense, MACoreAttention) and not dense.sparse and dense.use_causal_mask
    sparse = create_attention_layer("sparse", window_size=16)
    assert sparse.sparse and sparse.window_size == 16
    auto = create_attention_layer("auto", window_size=32)
    assert auto.sparse and auto.window_size == 32


@pytest.mark.parametrize("name", ["invalid_type", "nonexistent_type"])
def test_invalid_attention_type(name):
    """test_ma_core_bridge.py:321-326, test_error_handling.py:317-322."""
    with pytest.raises(ValueError) as e:
        create_attention_layer(name)
    assert "unknown attention type" in str(e.value).lower()


def test_invalid_factory_parameters():
    """test_error_handling.py:324-332."""
    assert create_attention_layer("sparse", window_size=8).window_size == 8
    with pytest.raises(ValueError):
        create_attention_layer("sparse", window_size=-1)


@pytest.mark.parametrize("training", [True, False])
def test_mismatched_shapes(training):
    """test_error_handling.py:17-61 and test_ma_core_bridge.py:238-266: sequence,
    head-dim and batch mismatches raise with a message naming the problem, in
    both modes (checked before any engine call)."""
    att = MACoreAttention(sparse=False, fallback_training=True).train(training)
    cases = [
        (_t(1, 8, 2, 16), _t(1, 6, 2, 16), _t(1, 8, 2, 16)),
        (_t(1, 8, 2, 16), _t(1, 8, 2, 16), _t(1, 8, 2, 32)),
        (_t(1, 8, 2, 16), _t(2, 8, 2, 16), _t(1, 8, 2, 16)),
    ]
    for q, k, v in cases:
        with pytest.raises(ValueError) as e:
            att(q, k, v)
        msg = str(e.value).lower()
        assert any(w in msg for w in ("sequence", "length", "mismatch", "size", "dimension", "head"))


@pytest.mark.parametrize("shape", [(0, 8, 2, 16), (1, 0, 2, 16)])
def test_zero_dimensions(shape):
    """test_error_handling.py:63-82 and test_ma_core_bridge.py:269-279."""
    att = MACoreAttention(sparse=False, fallback_training=True)
    with pytest.raises(ValueError):
        att(_t(*shape), _t(*shape), _t(*shape))


def test_rank_other_than_four():
    att = MACoreAttention(sparse=True, window_size=2)
    with pytest.raises(ValueError):
        att(_t(8, 16), _t(8, 16), _t(8, 16))


def test_sparse_attention_wrong_inputs():
    """test_error_handling.py:289-310: mismatched and 2-D inputs raise."""
    sa = SparseAttention(window_size=2, use_ma_core=True).train()
    with pytest.raises(Exception):
        sa(_t(1, 8, 16), _t(1, 6, 16), _t(1, 8, 16))
    with pytest.raises(Exception):
        SparseAttention(window_size=3)(_t(8, 16), _t(1, 8, 16), _t(1, 8, 16))


def test_module_state_after_error():
    """test_error_handling.py:338-384: an error leaves the module usable and unchanged."""
    att = MACoreAttention(sparse=True, window_size=4, fallback_training=True)
    state = (att.sparse, att.window_size, att.use_causal_mask, att.spec)
    for q, k, v in [(_t(1, 4, 2, 8), _t(1, 6, 2, 8), _t(1, 4, 2, 8)),
                    (_t(0, 4, 2, 8),) * 3]:
        with pytest.raises(ValueError):
            att(q, k, v)
    assert (att.sparse, att.window_size, att.use_causal_mask, att.spec) == state
    x = _t(1, 4, 2, 8)
    out = att(x, x, x)
    assert out.shape == (1, 4, 2, 8) and torch.isfinite(out).all()


def test_training_state_propagates():
    """test_pytorch_compatibility.py:308-322."""
    block = nn.Sequential(nn.Linear(16, 16), MACoreAttention(sparse=True, window_size=4))
    block.train()
    assert all(m.training for m in block.modules())
    block.eval()
    assert not any(m.training for m in block.modules())


def test_pattern_arguments_rejected():
    """The keyword-only pattern arguments keep the reference's error types."""
    with pytest.raises(ValueError):
        MACoreAttention(sparse=True, window_size=4, pattern="ring")
    with pytest.raises(ValueError):
        MACoreAttention(sparse=True, window_size=4, pattern="sliding", dilation=0)
    with pytest.raises(ValueError):
        MACoreAttention(sparse=True, window_size=4, pattern="block_sparse")  # no table


def test_pattern_defaults_follow_window():
    """causal=True gives keys [i-(w-1), i]; the plain module keeps the reference's [i-w, i+w]."""
    assert MACoreAttention(sparse=True, window_size=4).spec is None
    s = MACoreAttention(sparse=True, window_size=4, causal=True).spec
    assert (s.pattern, s.left, s.right, s.dilation) == ("sliding", 3, 0, 1)
    s = MACoreAttention(sparse=True, window_size=4, dilation=4).spec
    assert (s.left, s.right, s.dilation) == (4, 4, 4)
    s = MACoreAttention(sparse=False, use_causal_mask=True, pattern="dense").spec
    assert s.causal


def test_saved_statistics_choice():
    """When the native backward starts from the forward's saved statistics:
    tiled sets whose query tiles average more than two entries, and dense rows
    longer than two 64-key blocks at head_dim 64; never for sliding windows
    (their kernels keep a tile's scores in registers)."""
    import types
    from layers import ma_core_bridge as br

    def iset(entries, items):
        return types.SimpleNamespace(tile_header=types.SimpleNamespace(num_entries=entries, num_q_items=items))

    assert br._saved_statistics_pay(iset(1024, 256))      # block-sparse: 4 entries per tile
    assert not br._saved_statistics_pay(iset(2048, 1024))  # a causal 64 window: 2 per tile
    assert not br._saved_statistics_pay(types.SimpleNamespace(tile_header=None))  # no tile plan
    q = torch.empty(1, 1024, 2, 64)
    assert br._saved_statistics_plan(None, False, q) == ("dense", None)       # the reference's dense layer
    assert br._saved_statistics_plan(None, True, q) is None                   # its sliding layer
    assert br._saved_statistics_plan(None, False, torch.empty(1, 128, 2, 64)) is None  # two blocks
    assert br._saved_statistics_plan(None, False, torch.empty(1, 1024, 2, 32)) is None  # head_dim 32
    assert br._saved_statistics_plan(br.PatternSpec(pattern="sliding", left=63, right=0), True, q) is None
    assert br._saved_statistics_plan(br.PatternSpec(pattern="dense", causal=True), False, q) == ("dense", None)
    assert br._saved_statistics_plan(br.PatternSpec(pattern="index_set", index_set=iset(900, 300)), False,
                                     q)[0] == "set"
    assert br._saved_statistics_plan(br.PatternSpec(pattern="index_set", index_set=iset(600, 300)), False,
                                     q) is None


def test_bench_saved_stats_needs_a_tiled_or_dense_backward():
    """bench.py refuses --saved-stats outside the backward of dense, block-sparse,
    Longformer and index-set workloads (before touching any device)."""
    import subprocess
    import sys
    import os
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for argv in (["--saved-stats"], ["--saved-stats", "--pass", "backward"],
                 ["--workload", "cfg3", "--saved-stats"]):
        r = subprocess.run([sys.executable, os.path.join(repo, "bench.py"), *argv], capture_output=True, text=True,
                           timeout=300, env={**os.environ, "HIP_VISIBLE_DEVICES": ""})
        assert r.returncode == 2 and "--saved-stats applies" in r.stderr, (argv, r.returncode, r.stderr[-300:])
