"""GPU-resident tick preprocessing: the reference's TickDataset on MI355X.

Reference: /root/reference src/data_loader.py.  ``TickDataset`` and
``create_data_loaders`` keep the reference's names, arguments and item
format ((features[idx:idx+L], next WAP), float32); the microstructure features
and their z-scoring run on the GPU (``ma_tick_features`` in libma_attn.so,
include/ma_features.h) instead of in pandas, and the feature matrix stays in
device memory.  ``feature_means`` / ``feature_stds`` are pandas Series, as the
reference's.
"""
from __future__ import annotations

import ctypes

import torch

import ma_attn as _ma

FEATURES = ["price", "bid_ask_spread", "wap", "order_book_imbalance", "time_diff"]
COLUMNS = ["timestamp", "price", "bid_price", "ask_price", "bid_volume", "ask_volume"]

_lib = _ma.LIB
_lib.ma_tick_features_workspace_size.restype = ctypes.c_size_t
_lib.ma_tick_features_workspace_size.argtypes = [ctypes.c_int64]
_lib.ma_tick_features.restype = ctypes.c_int
_lib.ma_tick_features.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                                          ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
_lib.ma_tick_features_timed.restype = ctypes.c_int
_lib.ma_tick_features_timed.argtypes = _lib.ma_tick_features.argtypes + [ctypes.c_void_p] * 2


def compute_tick_features(columns: dict, events=None):
    """columns: the six raw tick columns (COLUMNS) as 1-D device tensors of one
    length.  Returns (float32 [n, 5] z-scored features, float64 [5] means,
    float64 [5] sample stds), all on the device.  events: optional
    (start, stop) torch.cuda.Event pair (recorded once already) stamped on the
    pass's first kernel start and last kernel end."""
    cols = []
    for name in COLUMNS:
        t = columns[name]
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise RuntimeError(f"column {name} must be a device tensor")
        cols.append(t.to(torch.float64).contiguous())
    n = cols[0].numel()
    if any(c.dim() != 1 or c.numel() != n for c in cols) or any(c.device != cols[0].device for c in cols):
        raise RuntimeError("tick columns must be 1-D, of one length, on one device")
    dev = cols[0].device
    out = torch.empty((n, 5), dtype=torch.float32, device=dev)
    stats = torch.empty(10, dtype=torch.float64, device=dev)
    nbytes = int(_lib.ma_tick_features_workspace_size(n))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        args = [*(c.data_ptr() for c in cols), n, out.data_ptr(), stats.data_ptr(), ws.data_ptr(), nbytes,
                stream or None]
        if events is not None:
            rc = _lib.ma_tick_features_timed(*args, events[0].cuda_event or None, events[1].cuda_event or None)
        else:
            rc = _lib.ma_tick_features(*args)
    if rc != 0:
        raise RuntimeError(_ma.last_error())
    return out, stats[:5], stats[5:]


class TickDataset(torch.utils.data.Dataset):
    """Reference TickDataset (data_loader.py:8-38) with GPU preprocessing.

    file_path: CSV with the COLUMNS (read on the host); or pass ``columns``
    (a dict of arrays / tensors) instead.  Items are (features[idx:idx+L],
    z-scored WAP of tick idx+L), float32, on ``device``.
    """

    def __init__(self, file_path=None, sequence_length=10, *, columns=None, device=None):
        import pandas as pd
        self.sequence_length = sequence_length
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if columns is None:
            df = pd.read_csv(file_path)
            columns = {c: df[c].to_numpy() for c in COLUMNS}
        cols = {c: torch.as_tensor(columns[c], dtype=torch.float64).to(dev) for c in COLUMNS}
        self.features, means, stds = compute_tick_features(cols)
        self.feature_means = pd.Series(means.cpu().numpy(), index=FEATURES)
        self.feature_stds = pd.Series(stds.cpu().numpy(), index=FEATURES)

    def __len__(self):
        return len(self.features) - self.sequence_length

    def __getitem__(self, idx):
        x = self.features[idx:idx + self.sequence_length]
        y = self.features[idx + self.sequence_length, 2]  # WAP
        return x, y


def create_data_loaders(file_path, sequence_length, batch_size, train_split=0.8):
    """Reference create_data_loaders (data_loader.py:40-52) over the GPU dataset."""
    dataset = TickDataset(file_path, sequence_length)
    train_size = int(train_split * len(dataset))
    val_size = len(dataset) - train_size
    train_dataset, val_dataset = torch.utils.data.random_split(dataset, [train_size, val_size])
    train_loader = torch.utils.data.DataLoader(train_dataset, batch_size=batch_size, shuffle=True)
    val_loader = torch.utils.data.DataLoader(val_dataset, batch_size=batch_size, shuffle=False)
    return train_loader, val_loader, dataset
