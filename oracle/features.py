"""CPU oracle for the tick-feature pass -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s cpu_baseline leg import this module, as
the checker / the timed CPU baseline; the product never does.

Restates the reference's TickDataset preprocessing
(/root/reference src/data_loader.py:15-28) in numpy float64:
  spread = ask - bid                                   (:16)
  wap    = (bid * askv + ask * bidv) / (bidv + askv)   (:17)
  obi    = bidv / (bidv + askv)                        (:18)
  dt     = ts.diff().fillna(0)                         (:19)
  columns [price, spread, wap, obi, dt] z-scored with the column mean and
  the sample std (pandas' default ddof = 1)            (:22-26)
and the float32 rows the dataset hands to the model (:38).
"""
from __future__ import annotations

import numpy as np

FEATURES = ["price", "bid_ask_spread", "wap", "order_book_imbalance", "time_diff"]


def raw_features(ts, price, bid, ask, bidv, askv):
    """-> float64 [n, 5] un-normalised rows [price, spread, wap, obi, dt]
    (src/data_loader.py:16-19), each an IEEE float64 expression evaluated in
    the reference's operation order."""
    ts, price, bid, ask, bidv, askv = (np.asarray(x, dtype=np.float64) for x in (ts, price, bid, ask, bidv, askv))
    spread = ask - bid
    wap = (bid * askv + ask * bidv) / (bidv + askv)
    obi = bidv / (bidv + askv)
    dt = np.empty_like(ts)
    dt[:1] = 0.0
    dt[1:] = ts[1:] - ts[:-1]
    return np.stack([price, spread, wap, obi, dt], axis=1)


def normalize(f, mean, std):
    """float32 rows (f - mean) / std (src/data_loader.py:26, :38), the
    float64 quotient rounded once to float32."""
    return ((np.asarray(f, np.float64) - mean) / std).astype(np.float32)


def tick_features(ts, price, bid, ask, bidv, askv):
    """-> (float32 [n, 5] z-scored rows, float64 means [5], float64 stds [5])."""
    f = raw_features(ts, price, bid, ask, bidv, askv)
    mean = f.mean(axis=0)
    std = f.std(axis=0, ddof=1)
    return normalize(f, mean, std), mean, std


def synthetic_ticks(n: int, seed: int):
    """Seeded tick columns with the shape of the reference's GBM generator
    (data/generate_synthetic_ticks.py): sorted timestamps, a positive mid
    price path, a small spread, integer volumes >= 1."""
    rng = np.random.default_rng(seed)
    ts = np.sort(rng.uniform(0.0, 1.0, n))
    mid = 100.0 * np.exp(np.cumsum(rng.standard_normal(n)) * 0.001)
    spread = mid * 0.2 * rng.uniform(0.0005, 0.0015, n)
    bid, ask = mid - spread / 2, mid + spread / 2
    price = mid + (spread / 2) * rng.choice([-1.0, 0.0, 1.0], n, p=[0.4, 0.2, 0.4])
    bidv = np.maximum(rng.poisson(100 * np.abs(1 + 0.5 * rng.standard_normal(n))), 1).astype(np.float64)
    askv = np.maximum(rng.poisson(100 * np.abs(1 + 0.5 * rng.standard_normal(n))), 1).astype(np.float64)
    return {"timestamp": ts, "price": price, "bid_price": bid, "ask_price": ask,
            "bid_volume": bidv, "ask_volume": askv}
