"""Single-head sparse-attention layer over [batch, seq_len, model_dim].

Reference: /root/reference src/layers/sparse_attention.py:26-110.  Same
constructor (``window_size=3, use_ma_core=True``), the same TypeError /
ValueError rules, the same reshape to one head ([B,S,Dm] -> [B,S,1,Dm]) and
the same ``_pytorch_forward`` fallback.  "ma_core" in the argument name keeps
the reference API; the engine behind it is the MI355X one (``MACoreAttention``).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .ma_core_bridge import MACoreAttention, pytorch_sparse_attention  # noqa: F401

MA_CORE_AVAILABLE = True  # the engine module imported (reference :9-16)
CUDA_AVAILABLE = False     # the reference's legacy ma_transformer_cuda path (:18-23)


class SparseAttention(nn.Module):
    """Sliding-window attention; priority engine > PyTorch fallback."""

    def __init__(self, window_size=3, use_ma_core=True, *, fallback_training=True):
        """fallback_training (keyword-only, not in the reference): False runs
        the native forward and backward kernels in training mode too."""
        super().__init__()
        if not isinstance(window_size, int):
            raise TypeError("window_size must be an integer for SparseAttention")
        if window_size <= 0:
            raise ValueError("window_size must be > 0 for SparseAttention")
        self.window_size = window_size
        self.use_ma_core = use_ma_core
        if MA_CORE_AVAILABLE and use_ma_core:
            self.ma_core_attention = MACoreAttention(sparse=True, window_size=window_size,
                                                     fallback_training=fallback_training)

    def forward(self, q, k, v):
        """q, k, v: [batch, seq_len, model_dim] -> [batch, seq_len, model_dim]."""
        if MA_CORE_AVAILABLE and self.use_ma_core and hasattr(self, "ma_core_attention"):
            out = self.ma_core_attention(q.unsqueeze(2), k.unsqueeze(2), v.unsqueeze(2))
            return out.squeeze(2)
        return self._pytorch_forward(q, k, v)

    def _pytorch_forward(self, q, k, v):
        """Reference fallback (:88-110): mask |i-j| <= window_size-1, fill -1e9."""
        batch_size, seq_len, model_dim = q.size()
        q = q / math.sqrt(model_dim)
        mask = torch.ones(seq_len, seq_len, device=q.device).tril(self.window_size - 1) \
            .triu(-self.window_size + 1).bool()
        attn_scores = torch.matmul(q, k.transpose(-2, -1))
        attn_scores = attn_scores.masked_fill(mask == 0, -1e9)
        attn_weights = F.softmax(attn_scores, dim=-1)
        return torch.matmul(attn_weights, v)
