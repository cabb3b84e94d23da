"""GPU tick-feature pass (ma_tick_features) against the oracle restatement of
the reference's TickDataset preprocessing (src/data_loader.py:15-28).

Tolerances: means and stds relative 1e-12 (float64, another summation
order).  The float32 rows are compared bit-exactly with the oracle's float64
per-tick features normalised by the statistics the GPU returned: every
per-tick operation is one correctly rounded IEEE float64 operation on both
sides, so only the statistics may differ, and they are checked separately.
(Comparing against the oracle's own statistics instead would let a row near
zero differ by many float32 ulps: (f - mean) cancels.)
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

COLS = ["timestamp", "price", "bid_price", "ask_price", "bid_volume", "ask_volume"]


@pytest.fixture(scope="module")
def tf():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import tick_features
    return tick_features


def _dev_cols(cols):
    return {c: torch.from_numpy(cols[c]).cuda() for c in COLS}


@pytest.mark.parametrize("n", [2, 3, 17, 1000, 4097, 100_003, 3_000_001])
def test_tick_features_vs_oracle(tf, n):
    from oracle import features as F
    cols = F.synthetic_ticks(n, 100 + n % 97)
    f_ref = F.raw_features(*(cols[c] for c in COLS))
    _, m_ref, s_ref = F.tick_features(*(cols[c] for c in COLS))
    z, m, s = tf.compute_tick_features(_dev_cols(cols))
    z, m, s = z.cpu().numpy(), m.cpu().numpy(), s.cpu().numpy()
    np.testing.assert_allclose(m, m_ref, rtol=1e-12, atol=0)
    np.testing.assert_allclose(s, s_ref, rtol=1e-12, atol=0)
    z_ref = F.normalize(f_ref, m, s)
    bad = np.argwhere(z.view(np.uint32) != z_ref.view(np.uint32))
    assert bad.size == 0, (bad[:4].tolist(), z[tuple(bad[0])], z_ref[tuple(bad[0])])


def test_tick_features_single_tick_and_errors(tf):
    from oracle import features as F
    cols = F.synthetic_ticks(1, 5)
    z, m, s = tf.compute_tick_features(_dev_cols(cols))
    assert torch.isnan(s).all() and torch.isnan(z).all()  # sample std of one value, as pandas
    with pytest.raises(RuntimeError):
        bad = _dev_cols(F.synthetic_ticks(10, 5))
        bad["price"] = bad["price"][:5]
        tf.compute_tick_features(bad)
    with pytest.raises(RuntimeError):
        tf.compute_tick_features({c: torch.zeros(4) for c in COLS})  # host tensors


def test_tick_dataset_csv_matches_reference_items(tf, tmp_path):
    """TickDataset from a CSV: items (window, next WAP) and statistics as the
    reference dataset produces them (pandas preprocessing, float32 items)."""
    import pandas as pd
    from oracle import features as F
    cols = F.synthetic_ticks(5000, 11)
    path = tmp_path / "ticks.csv"
    pd.DataFrame(cols).to_csv(path, index=False)
    ds = tf.TickDataset(str(path), sequence_length=10)
    df = pd.read_csv(path)
    z_ref, m_ref, s_ref = F.tick_features(*(df[c].to_numpy() for c in COLS))
    assert len(ds) == 5000 - 10
    np.testing.assert_allclose(ds.feature_means.to_numpy(), m_ref, rtol=1e-12)
    assert list(ds.feature_stds.index) == F.FEATURES
    for idx in (0, 1234, len(ds) - 1):
        x, y = ds[idx]
        assert x.shape == (10, 5) and x.dtype == torch.float32
        np.testing.assert_allclose(x.cpu().numpy(), z_ref[idx:idx + 10], rtol=0, atol=1e-6)
        assert abs(float(y) - float(z_ref[idx + 10, 2])) <= 1e-6
    # the GPU dataset feeds the model directly
    from model import TransformerModel
    m = TransformerModel(input_dim=5, model_dim=32, num_heads=2, num_layers=2).cuda().eval()
    xb = torch.stack([ds[i][0] for i in range(64)])
    with torch.no_grad():
        assert m(xb).shape == (64, 1)


def test_tick_features_timed_matches(tf):
    """ma_tick_features_timed: the same rows and statistics, and a positive
    stamped duration for the pass."""
    from oracle import features as F
    dc = _dev_cols(F.synthetic_ticks(50_000, 3))
    z0, m0, s0 = tf.compute_tick_features(dc)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    b.record()
    torch.cuda.synchronize()
    z1, m1, s1 = tf.compute_tick_features(dc, events=(a, b))
    torch.cuda.synchronize()
    assert torch.equal(z0, z1) and torch.equal(m0, m1) and torch.equal(s0, s1)
    assert a.elapsed_time(b) > 0
