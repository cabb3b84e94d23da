"""The reference's toy forecasting model on this engine's attention.

Reference: /root/reference src/model.py:1-92 -- PositionalEncoding,
CustomTransformerEncoderLayer (single-head SparseAttention, window 3, then a
ReLU feed-forward block, post-norm residuals) and TransformerModel
(Linear encoder * sqrt(model_dim), positional encoding, the layer stack, a
Linear decoder on the last time step).  Same class names, constructor
arguments, parameter names (so the reference's state_dicts load unchanged)
and forward semantics, including PositionalEncoding indexing its table by
``x.size(0)`` as the reference does (:19-20).  The attention inside each
layer is ``layers.SparseAttention``: the HIP kernels in eval mode, the
PyTorch path in training mode unless ``fallback_training=False``.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from layers.sparse_attention import SparseAttention


class PositionalEncoding(nn.Module):
    """Sinusoidal table pe[pos, 2i] = sin(pos w_i), pe[pos, 2i+1] = cos(pos w_i),
    w_i = 10000^(-2i/d_model) (reference model.py:7-20)."""

    def __init__(self, d_model, max_len=5000):
        super().__init__()
        position = torch.arange(0, max_len, dtype=torch.float).unsqueeze(1)
        freq = torch.exp(torch.arange(0, d_model, 2).float() * (-math.log(10000.0) / d_model))
        table = torch.zeros(max_len, d_model)
        table[:, 0::2] = torch.sin(position * freq)
        table[:, 1::2] = torch.cos(position * freq)
        self.register_buffer("pe", table.unsqueeze(0).transpose(0, 1))  # [max_len, 1, d_model]

    def forward(self, x):
        return x + self.pe[:x.size(0), :]


class CustomTransformerEncoderLayer(nn.Module):
    """Self-attention (SparseAttention) + feed-forward, each with residual,
    dropout and post-LayerNorm (reference model.py:28-52)."""

    def __init__(self, d_model, num_heads, dropout=0.1, window_size=3, *, fallback_training=True):
        super().__init__()
        self.self_attn = SparseAttention(window_size=window_size, fallback_training=fallback_training)
        self.linear1 = nn.Linear(d_model, d_model * 4)
        self.dropout = nn.Dropout(dropout)
        self.linear2 = nn.Linear(d_model * 4, d_model)
        self.norm1 = nn.LayerNorm(d_model)
        self.norm2 = nn.LayerNorm(d_model)
        self.dropout1 = nn.Dropout(dropout)
        self.dropout2 = nn.Dropout(dropout)

    def forward(self, src):
        attn = self.self_attn(src, src, src)
        src = self.norm1(src + self.dropout1(attn))
        ff = self.linear2(self.dropout(F.relu(self.linear1(src))))
        return self.norm2(src + self.dropout2(ff))


class TransformerModel(nn.Module):
    """[batch, seq_len, input_dim] -> [batch, 1] (reference model.py:54-92).

    num_heads is accepted and unused, as in the reference (its layers are
    single-head)."""

    def __init__(self, input_dim, model_dim, num_heads, num_layers, dropout=0.1, *,
                 fallback_training=True):
        super().__init__()
        self.model_dim = model_dim
        self.encoder = nn.Linear(input_dim, model_dim)
        self.pos_encoder = PositionalEncoding(model_dim)
        self.encoder_layers = nn.ModuleList([
            CustomTransformerEncoderLayer(d_model=model_dim, num_heads=num_heads, dropout=dropout,
                                          fallback_training=fallback_training)
            for _ in range(num_layers)
        ])
        self.decoder = nn.Linear(model_dim, 1)
        self.init_weights()

    def init_weights(self):
        r = 0.1
        self.encoder.weight.data.uniform_(-r, r)
        self.decoder.bias.data.zero_()
        self.decoder.weight.data.uniform_(-r, r)

    def forward(self, src):
        x = self.pos_encoder(self.encoder(src) * math.sqrt(self.model_dim))
        for layer in self.encoder_layers:
            x = layer(x)
        return self.decoder(x[:, -1, :])
