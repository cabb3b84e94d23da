"""Pins the tick-feature oracle (oracle/features.py) before it checks the GPU
pass: against pandas running the reference's own DataFrame operations
(src/data_loader.py:15-28), and against what the definitions fix."""
import numpy as np
import pandas as pd
import pytest


def _reference_pandas(cols):
    """The reference's preprocessing, operation for operation, in pandas."""
    df = pd.DataFrame(cols)
    df["bid_ask_spread"] = df["ask_price"] - df["bid_price"]
    df["wap"] = (df["bid_price"] * df["ask_volume"] + df["ask_price"] * df["bid_volume"]) / \
        (df["bid_volume"] + df["ask_volume"])
    df["order_book_imbalance"] = df["bid_volume"] / (df["bid_volume"] + df["ask_volume"])
    df["time_diff"] = df["timestamp"].diff().fillna(0)
    feats = ["price", "bid_ask_spread", "wap", "order_book_imbalance", "time_diff"]
    means, stds = df[feats].mean(), df[feats].std()
    return df[feats].to_numpy(), ((df[feats] - means) / stds).to_numpy().astype(np.float32), means, stds


@pytest.mark.parametrize("n,seed", [(2, 1), (17, 2), (1000, 3), (100_003, 4)])
def test_oracle_matches_reference_pandas(n, seed):
    from oracle import features as F
    cols = F.synthetic_ticks(n, seed)
    raw, z_ref, means, stds = _reference_pandas(cols)
    z, m, s = F.tick_features(*(cols[c] for c in ["timestamp", "price", "bid_price", "ask_price",
                                                   "bid_volume", "ask_volume"]))
    np.testing.assert_allclose(m, means.to_numpy(), rtol=1e-13, atol=0)
    np.testing.assert_allclose(s, stds.to_numpy(), rtol=1e-12, atol=0)  # ddof 1, as pandas
    # per-tick features bit-exact with pandas' (the same IEEE float64 operations)
    f = F.raw_features(*(cols[c] for c in ["timestamp", "price", "bid_price", "ask_price",
                                           "bid_volume", "ask_volume"]))
    assert np.array_equal(f, raw)
    # float32 rows bit-exact given pandas' statistics (only the statistics' summation order differs)
    assert np.array_equal(F.normalize(f, means.to_numpy(), stds.to_numpy()).view(np.uint32), z_ref.view(np.uint32))


def test_oracle_definitions():
    from oracle import features as F
    cols = F.synthetic_ticks(5000, 9)
    z, m, s = F.tick_features(*(cols[c] for c in ["timestamp", "price", "bid_price", "ask_price",
                                                   "bid_volume", "ask_volume"]))
    # z-scored columns: mean 0, sample std 1
    assert np.abs(z.astype(np.float64).mean(axis=0)).max() < 1e-6
    assert np.abs(z.astype(np.float64).std(axis=0, ddof=1) - 1.0).max() < 1e-6
    # un-normalised features from the statistics: wap between bid and ask, imbalance in (0, 1),
    # first time difference zero, then the timestamp gaps
    raw = z.astype(np.float64) * s + m
    assert np.all(raw[:, 2] >= cols["bid_price"] - 1e-9) and np.all(raw[:, 2] <= cols["ask_price"] + 1e-9)
    assert np.all((raw[:, 3] > 0) & (raw[:, 3] < 1))
    assert abs(raw[0, 4]) < 1e-9
    np.testing.assert_allclose(raw[1:, 4], np.diff(cols["timestamp"]), atol=1e-9)
    # one tick: the sample std is undefined (NaN), as in pandas
    with np.errstate(invalid="ignore", divide="ignore"), pytest.warns(RuntimeWarning):
        _, _, s1 = F.tick_features(*(cols[c][:1] for c in ["timestamp", "price", "bid_price", "ask_price",
                                                           "bid_volume", "ask_volume"]))
    assert np.isnan(s1).all()
