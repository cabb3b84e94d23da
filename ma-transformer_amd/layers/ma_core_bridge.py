"""PyTorch bridge to the MI355X sparse-attention engine.

Keeps the public surface of the reference bridge
(/root/reference src/layers/ma_core_bridge.py):

* ``MACoreAttentionFunction``  autograd.Function (:44-154)
* ``MACoreAttention``          nn.Module with the same constructor defaults and
                               ValueError / TypeError rules (:250-330)
* ``create_attention_layer``   factory (:333-352)
* ``pytorch_dense_attention``, ``pytorch_sparse_attention`` the PyTorch
                               reference implementations (:184-247)
* ``pytorch_to_ma_core``, ``ma_core_to_pytorch`` converters (:157-181) to and
                               from this package's ``ma_core`` module (host
                               Tensors whose attention runs on the GPU kernels).

Routing differs from the reference in one deliberate way: device tensors of
every supported dtype (float32, bfloat16, float16) go to the native HIP
kernels; the reference sent non-float32 device tensors to a Python loop
(:77-80).  If device tensors arrive and the native library is missing, the
call raises -- there is no silent fallback on a GPU.  CPU tensors use the
PyTorch reference implementations, as the reference's CPU branch computes on
the host; ``ma_core`` (whose attention stages host buffers to the GPU) is
reached through the converters, as the reference's bridge reaches it.

New, keyword-only constructor arguments select the benchmark patterns and
default to the reference behaviour: ``pattern`` ("sliding", "dense",
"block_sparse", "longformer", "index_set"), ``causal``, ``window_left``,
``window_right``, ``dilation``, ``block_size``, ``block_table``,
``num_global_tokens``, ``index_set`` (an explicit key set per query row: a
``sparse_attention_cuda.IndexSet`` or an (offsets, keys) CSR pair).
"""
from __future__ import annotations

import os
import sys
from dataclasses import dataclass, field
from typing import Optional, Tuple

import torch
import torch.nn as nn

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _PKG_DIR not in sys.path:
    sys.path.insert(0, _PKG_DIR)


def _try_import_sparse_ext():
    """Import the native extension.  On a machine with a GPU a failure is fatal."""
    try:
        import sparse_attention_cuda  # noqa: F401
        return sparse_attention_cuda
    except ImportError:
        if torch.cuda.is_available():
            raise
        return None


sparse_attention_cuda = _try_import_sparse_ext()
_HAS_SPARSE_CUDA = sparse_attention_cuda is not None

try:  # this package's ma_core module (the reference's src/csrc surface), for the two converters
    import ma_core  # type: ignore  # noqa: F401
except ImportError:  # pragma: no cover - without libma_attn.so
    ma_core = None


@dataclass(frozen=True)
class PatternSpec:
    """A resolved index-set choice (see include/ma_attn.h for the sets)."""

    pattern: str = "sliding"       # sliding | dense | block_sparse | longformer | index_set
    left: int = 64
    right: int = 64
    dilation: int = 1
    causal: bool = False
    block_size: int = 64
    block_table: Optional[torch.Tensor] = None
    num_global: int = 0
    index_set: Optional[object] = None  # IndexSet or (offsets, keys)
    # device-side forms built on first use and kept: (device, seq_len) ->
    # BlockTable (block_sparse) or IndexSet (index_set given as a CSR pair)
    device_forms: dict = field(default_factory=dict, compare=False, hash=False, repr=False)

    def native_table(self, seq_len: int, device):
        """The block table as a BlockTable for (seq_len, device): checked and
        uploaded once; its key sets (pattern_index_set) are then built once too."""
        key = ("table", int(seq_len), str(device))
        hit = self.device_forms.get(key)
        if hit is None:
            hit = self.device_forms[key] = sparse_attention_cuda.BlockTable(
                self.block_table, seq_len, self.block_size, device)
        return hit

    def native_index_set(self, seq_len: int, device):
        """The index set as an IndexSet on device (a CSR pair is converted once)."""
        s = self.index_set
        if not isinstance(s, (tuple, list)):  # an IndexSet already
            return s
        key = ("set", int(seq_len), str(device))
        hit = self.device_forms.get(key)
        if hit is None:
            offsets, keys = s
            hit = self.device_forms[key] = sparse_attention_cuda.IndexSet(
                torch.as_tensor(offsets), torch.as_tensor(keys), seq_len, device)
        return hit

    def _csr(self, device):
        s = self.index_set
        off, keys = (s.offsets, s.keys[:s.num_indices]) if hasattr(s, "offsets") else s
        return (torch.as_tensor(off, device=device).long(), torch.as_tensor(keys, device=device).long())

    def mask(self, N: int, device) -> torch.Tensor:
        """[N, N] boolean membership mask (for the PyTorch paths)."""
        i = torch.arange(N, device=device).unsqueeze(1)
        j = torch.arange(N, device=device).unsqueeze(0)
        if self.pattern == "sliding":
            d = j - i
            t = torch.div(d, self.dilation, rounding_mode="floor")
            return (d % self.dilation == 0) & (t >= -self.left) & (t <= self.right)
        if self.pattern == "dense":
            return j <= i if self.causal else torch.ones(N, N, dtype=torch.bool, device=device)
        if self.pattern == "block_sparse":
            bs = self.block_size
            tab = self.block_table.to(device=device, dtype=torch.long)
            rb = (torch.arange(N, device=device) // bs)
            kb = (torch.arange(N, device=device) // bs)
            hit = (tab[rb].unsqueeze(-1) == kb.view(1, 1, N)).any(dim=1)
            return hit
        if self.pattern == "longformer":
            G = self.num_global
            local = (j >= i - self.left) & (j <= i + self.right)
            return (i < G) | (j < G) | local
        if self.pattern == "index_set":
            off, keys = self._csr(device)
            rows = torch.repeat_interleave(torch.arange(N, device=device), off[1:] - off[:-1])
            m = torch.zeros(N, N, dtype=torch.bool, device=device)
            m[rows, keys] = True
            return m
        raise ValueError(f"unknown pattern {self.pattern}")


def _pattern_set(spec: PatternSpec, seq_len: int, device):
    """The explicit key sets the native backward of a block-sparse, Longformer
    or index-set pattern runs on, built on the first step and kept: on the
    spec's BlockTable (block-sparse), in pattern_index_set's geometry cache
    (Longformer), or on the spec (an index set given as a CSR pair)."""
    ext = sparse_attention_cuda
    if spec.pattern == "index_set":
        return spec.native_index_set(seq_len, device)
    if spec.pattern == "block_sparse":
        return ext.pattern_index_set("block_sparse", seq_len, device,
                                     block_table=spec.native_table(seq_len, device), block_size=spec.block_size)
    return ext.pattern_index_set(spec.pattern, seq_len, device, left=spec.left, right=spec.right,
                                 num_global=spec.num_global)


def _saved_statistics_pay(iset) -> bool:
    """Whether the backward should run from the forward's saved statistics:
    a tile plan whose query tiles average more than two entries.  There the
    dQ pass would stream the tile's key blocks twice; on two-entry tiles both
    blocks stay resident and reading O costs more than the statistics pass it
    replaces (bench.py --saved-stats: cfg3 backward 152 -> 131 us, cfg4
    548 -> 434 us, the target's sets 188 -> 194 us)."""
    h = getattr(iset, "tile_header", None)
    return h is not None and int(h.num_entries) > 2 * int(h.num_q_items)


def _saved_statistics_plan(spec: Optional[PatternSpec], sparse: bool, q: torch.Tensor):
    """("set", IndexSet), ("longformer", None) or ("dense", None) when the
    native backward should start from the forward's saved statistics, else
    None.  Longformer windows of at most 128 keys with 1 to 16 global tokens
    (16-bit, head_dim 64) take the one-pass kernel.  Dense rows longer
    than two 64-key blocks take the one-tile dQ kernel, whose statistics pass
    streams every key block once more (bench.py --saved-stats on
    dense_causal_*); shorter rows keep their scores in registers."""
    if spec is None or spec.pattern == "dense":
        if (spec is None and sparse) or q.shape[1] <= 128 or q.shape[3] != 64:
            return None
        return ("dense", None)
    if spec.pattern == "longformer" and sparse_attention_cuda.longformer_fused_applies(
            q, spec.left, spec.right, spec.num_global):
        return ("longformer", None)  # one pass from the statistics (bwd_lf_kernel)
    if spec.pattern in ("block_sparse", "longformer", "index_set"):
        iset = _pattern_set(spec, q.shape[1], q.device)
        return ("set", iset) if _saved_statistics_pay(iset) else None
    return None


def _native_forward(q, k, v, sparse, window_size, use_causal_mask, spec: Optional[PatternSpec],
                    return_lse: bool = False):
    ext = sparse_attention_cuda
    cq, ck, cv = q.contiguous(), k.contiguous(), v.contiguous()
    if return_lse:  # dense, block-sparse, Longformer and index sets only
        if spec is None or spec.pattern == "dense":
            causal = bool(use_causal_mask) if spec is None else spec.causal
            return ext.dense_forward(cq, ck, cv, causal, return_lse=True)
        if spec.pattern == "block_sparse":
            return ext.block_sparse_forward(cq, ck, cv, spec.native_table(cq.shape[1], cq.device), spec.block_size,
                                            return_lse=True)
        if spec.pattern == "longformer":
            return ext.longformer_forward(cq, ck, cv, spec.left, spec.right, spec.num_global, return_lse=True)
        return ext.index_set_forward(cq, ck, cv, spec.native_index_set(cq.shape[1], cq.device), return_lse=True)
    if spec is None:
        if sparse:
            return ext.forward(cq, ck, cv, int(window_size))
        return ext.dense_forward(cq, ck, cv, bool(use_causal_mask))
    if spec.pattern == "sliding":
        return ext.sliding_forward(cq, ck, cv, spec.left, spec.right, spec.dilation)
    if spec.pattern == "dense":
        return ext.dense_forward(cq, ck, cv, spec.causal)
    if spec.pattern == "block_sparse":
        return ext.block_sparse_forward(cq, ck, cv, spec.native_table(cq.shape[1], cq.device), spec.block_size)
    if spec.pattern == "longformer":
        return ext.longformer_forward(cq, ck, cv, spec.left, spec.right, spec.num_global)
    if spec.pattern == "index_set":
        return ext.index_set_forward(cq, ck, cv, spec.native_index_set(cq.shape[1], cq.device))
    raise ValueError(f"unknown pattern {spec.pattern}")


def pytorch_pattern_attention(query, key, value, spec: PatternSpec) -> torch.Tensor:
    """Differentiable masked attention for any PatternSpec (float32 math)."""
    B, S, H, D = query.shape
    scale = 1.0 / (D ** 0.5)
    mask = spec.mask(S, query.device)
    qh, kh, vh = (t.transpose(1, 2).float() for t in (query, key, value))
    s = torch.matmul(qh * scale, kh.transpose(-2, -1))
    s = s.masked_fill(~mask, float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    return torch.matmul(p, vh).transpose(1, 2).to(query.dtype).contiguous()


class MACoreAttentionFunction(torch.autograd.Function):
    """Autograd function: native forward; native backward for every pattern:
    sliding and dense on their own kernels (which recompute the softmax),
    index sets, block-sparse and Longformer on the tiled index-set kernels
    (the latter two as their explicit key sets).  When those sets' tiles
    average more than two entries, the forward also keeps each row's softmax
    statistic and the backward starts from it and the saved output; the
    16-bit Longformer with a causal window of at most 128 keys and 1 to 16
    global tokens then runs the one-pass kernel (longformer_backward).

    Reference: src/layers/ma_core_bridge.py:44-154.  The extra trailing
    argument ``spec`` (a PatternSpec or None) selects a non-reference pattern.
    Device-side pattern data (a block-sparse pattern's BlockTable and the key
    sets of its backward, an index set given as a CSR pair) is built on the
    first call and kept on the PatternSpec, so later steps only launch.
    """

    @staticmethod
    def forward(ctx, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                sparse: bool = False, window_size: int = 64,
                use_causal_mask: bool = False, spec: Optional[PatternSpec] = None) -> torch.Tensor:
        ctx.sparse = sparse
        ctx.window_size = window_size
        ctx.use_causal_mask = use_causal_mask
        ctx.spec = spec
        ctx.saved_plan = None
        on_device = query.is_cuda or key.is_cuda or value.is_cuda
        if on_device:
            if not _HAS_SPARSE_CUDA:
                raise RuntimeError("device tensors given but the native sparse-attention "
                                   "library (libma_attn.so) is not loaded")
            plan = _saved_statistics_plan(spec, sparse, query) if any(ctx.needs_input_grad[:3]) else None
            if plan is not None:
                try:
                    out, lse = _native_forward(query, key, value, sparse, window_size, use_causal_mask, spec,
                                               return_lse=True)
                except RuntimeError:  # a kernel that writes no statistics takes this shape
                    pass
                else:
                    ctx.saved_plan = plan
                    ctx.save_for_backward(query, key, value, out, lse)
                    return out
            ctx.save_for_backward(query, key, value)
            return _native_forward(query, key, value, sparse, window_size, use_causal_mask, spec)
        ctx.save_for_backward(query, key, value)
        if spec is not None:
            return pytorch_pattern_attention(query, key, value, spec)
        if sparse:
            return pytorch_sparse_attention(query, key, value, window_size)
        return pytorch_dense_attention(query, key, value, use_causal_mask)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor) -> Tuple[Optional[torch.Tensor], ...]:
        query, key, value = ctx.saved_tensors[:3]
        spec = ctx.spec
        native = spec is None or spec.pattern in ("sliding", "dense", "index_set", "block_sparse", "longformer")
        if _HAS_SPARSE_CUDA and query.is_cuda and native:
            ext = sparse_attention_cuda
            cq, ck, cv, cgo = (t.contiguous() for t in (query, key, value, grad_output))
            cgo = cgo.to(cq.dtype)
            if ctx.saved_plan is not None:  # from the forward's output and statistics
                out, lse = ctx.saved_tensors[3:]
                kind, iset = ctx.saved_plan
                if kind == "longformer":
                    dQ, dK, dV = ext.longformer_backward(cq, ck, cv, cgo, spec.left, spec.right, spec.num_global,
                                                         out=out, lse=lse)
                elif kind == "set":
                    dQ, dK, dV = ext.index_set_backward(cq, ck, cv, cgo, iset, out=out, lse=lse)
                else:
                    causal = bool(ctx.use_causal_mask) if spec is None else spec.causal
                    dQ, dK, dV = ext.dense_backward(cq, ck, cv, cgo, causal, out=out, lse=lse)
            elif spec is not None and spec.pattern == "sliding":
                dQ, dK, dV = ext.sliding_backward(cq, ck, cv, cgo, spec.left, spec.right, spec.dilation)
            elif spec is not None and spec.pattern in ("index_set", "block_sparse", "longformer"):
                # the pattern's key sets as an explicit set (built on the first step, kept)
                dQ, dK, dV = ext.index_set_backward(cq, ck, cv, cgo, _pattern_set(spec, cq.shape[1], cq.device))
            elif spec is not None:
                dQ, dK, dV = ext.dense_backward(cq, ck, cv, cgo, spec.causal)
            elif ctx.sparse:
                dQ, dK, dV = ext.backward(cq, ck, cv, cgo, int(ctx.window_size))
            else:
                dQ, dK, dV = ext.dense_backward(cq, ck, cv, cgo, bool(ctx.use_causal_mask))
            return (dQ if ctx.needs_input_grad[0] else None,
                    dK if ctx.needs_input_grad[1] else None,
                    dV if ctx.needs_input_grad[2] else None, None, None, None, None)
        # Host tensors: recompute with the PyTorch implementation and
        # differentiate, as the reference does (:140-154)
        with torch.enable_grad():
            q, k, v = (t.detach().requires_grad_(True) for t in (query, key, value))
            if spec is not None:
                out = pytorch_pattern_attention(q, k, v, spec)
            elif ctx.sparse:
                out = pytorch_sparse_attention(q, k, v, ctx.window_size)
            else:
                out = pytorch_dense_attention(q, k, v, ctx.use_causal_mask)
            dq, dk, dv = torch.autograd.grad(out, (q, k, v), grad_output)
        return (dq if ctx.needs_input_grad[0] else None,
                dk if ctx.needs_input_grad[1] else None,
                dv if ctx.needs_input_grad[2] else None, None, None, None, None)


def pytorch_to_ma_core(tensor: torch.Tensor):
    """Convert a tensor to an ``ma_core.Tensor`` (host float32 copy; :157-168)."""
    if ma_core is None:
        raise ImportError("ma_core needs libma_attn.so, which is not loaded")
    cpu_tensor = tensor.detach().cpu().contiguous()
    mc = ma_core.create_tensor(list(cpu_tensor.shape))
    mc.copy_from_numpy(cpu_tensor.numpy())
    return mc


def ma_core_to_pytorch(mc_tensor, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
    """Convert an ``ma_core.Tensor`` back to torch (:171-181)."""
    out = torch.from_numpy(mc_tensor.to_numpy())
    if out.dtype != dtype:
        out = out.to(dtype)
    return out.to(device) if device.type != "cpu" else out


def pytorch_dense_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            use_causal_mask: bool = False) -> torch.Tensor:
    """PyTorch dense attention with the reference's arithmetic (:184-221):
    scale Q first, Q K^T, causal fill -1e9, softmax, P V."""
    B, S, H, D = query.shape
    query = query * (1.0 / (D ** 0.5))
    qh = query.transpose(1, 2).reshape(B * H, S, D)
    kh = key.transpose(1, 2).reshape(B * H, S, D)
    vh = value.transpose(1, 2).reshape(B * H, S, D)
    scores = torch.matmul(qh, kh.transpose(-2, -1).contiguous())
    if use_causal_mask:
        mask = torch.tril(torch.ones(S, S, device=query.device, dtype=torch.bool))
        scores = scores.masked_fill(~mask, -1e9)
    p = torch.softmax(scores, dim=-1)
    out = torch.matmul(p, vh)
    return out.view(B, H, S, D).transpose(1, 2).contiguous()


def pytorch_sparse_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                             window_size: int = 64) -> torch.Tensor:
    """PyTorch sliding-window attention, keys [max(0,i-w), min(S,i+w+1)) (:224-247).

    Same semantics as the reference's per-(b, i, h) loop (scale Q, scores,
    softmax over the window, weights @ V; an empty window gives zeros), computed
    over query chunks with their key band so it scales past toy sizes.
    Differentiable.
    """
    B, S, H, D = query.shape
    w = int(window_size)
    scale = 1.0 / (D ** 0.5)
    if w < 0:
        return torch.zeros_like(query)
    out = []
    chunk = 256
    for r0 in range(0, S, chunk):
        r1 = min(S, r0 + chunk)
        k0, k1 = max(0, r0 - w), min(S, r1 + w)
        q = (query[:, r0:r1] * scale).transpose(1, 2)        # [B,H,R,D]
        kk = key[:, k0:k1].transpose(1, 2)                   # [B,H,K,D]
        vv = value[:, k0:k1].transpose(1, 2)
        s = torch.matmul(q, kk.transpose(-2, -1).contiguous())
        ii = torch.arange(r0, r1, device=query.device).unsqueeze(1)
        jj = torch.arange(k0, k1, device=query.device).unsqueeze(0)
        band = (jj >= ii - w) & (jj <= ii + w)
        s = s.masked_fill(~band, float("-inf"))
        p = torch.softmax(s, dim=-1)
        out.append(torch.matmul(p, vv).transpose(1, 2))
    return torch.cat(out, dim=1).contiguous()


_PATTERNS = ("sliding", "dense", "block_sparse", "longformer", "index_set")


class MACoreAttention(nn.Module):
    """Drop-in attention module (reference: ma_core_bridge.py:250-330).

    Eval mode (or ``fallback_training=False``) runs the native engine through
    ``MACoreAttentionFunction``; training mode with ``fallback_training=True``
    uses the PyTorch implementations, as the reference does (:317-325).
    """

    def __init__(self, sparse: bool = False, window_size: int = 64,
                 use_causal_mask: bool = False, fallback_training: bool = True, *,
                 pattern: Optional[str] = None, causal: bool = False,
                 window_left: Optional[int] = None, window_right: Optional[int] = None,
                 dilation: int = 1, block_size: int = 64,
                 block_table: Optional[torch.Tensor] = None, num_global_tokens: int = 0,
                 index_set: Optional[object] = None):
        super().__init__()
        self.sparse = sparse
        if self.sparse:
            if not isinstance(window_size, int):
                raise TypeError("window_size must be an integer for sparse attention")
            if window_size <= 0:
                raise ValueError("window_size must be > 0 for sparse attention")
        self.window_size = window_size
        self.use_causal_mask = use_causal_mask
        self.fallback_training = fallback_training
        self.spec = self._resolve(pattern, causal, window_left, window_right, dilation,
                                  block_size, block_table, num_global_tokens, index_set)

    def _resolve(self, pattern, causal, left, right, dilation, block_size, table, num_global, index_set):
        if pattern is None and not causal and left is None and right is None and dilation == 1:
            return None  # reference behaviour
        pattern = pattern or ("sliding" if self.sparse else "dense")
        if pattern not in _PATTERNS:
            raise ValueError(f"Unknown pattern: {pattern}")
        if not isinstance(dilation, int) or dilation < 1:
            raise ValueError("dilation must be an integer >= 1")
        w = int(self.window_size)
        if pattern in ("sliding", "longformer"):
            if left is None:
                left = w - 1 if causal else w
            if right is None:
                right = 0 if causal else w
        if pattern == "block_sparse":
            if table is None:
                raise ValueError("block_sparse pattern needs block_table")
            if isinstance(table, getattr(sparse_attention_cuda, "BlockTable", ())):
                table = table.host  # its checked host copy; the device form is rebuilt per device
            table = torch.as_tensor(table, dtype=torch.int32).cpu()
        if pattern == "index_set" and index_set is None:
            raise ValueError("index_set pattern needs index_set")
        if pattern == "dense":
            causal = causal or self.use_causal_mask
        return PatternSpec(pattern=pattern, left=int(left or 0), right=int(right or 0),
                           dilation=int(dilation), causal=bool(causal),
                           block_size=int(block_size), block_table=table,
                           num_global=int(num_global), index_set=index_set)

    def forward(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
        if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
            raise ValueError("Expected tensors with shape [batch, seq_len, num_heads, head_dim]")
        # Auto-correct a seq_len / num_heads swap in Q and K (:299-304)
        if (query.shape[0] == value.shape[0] and query.shape[1] == value.shape[2]
                and query.shape[2] == value.shape[1] and query.shape[3] == value.shape[3]
                and key.shape == query.shape):
            query = query.transpose(1, 2).contiguous()
            key = key.transpose(1, 2).contiguous()
        if query.shape != key.shape or key.shape != value.shape:
            raise ValueError(
                "Tensor size mismatch: query, key, and value must have identical shapes "
                "[batch, sequence length, num_heads, head_dim]")
        b, s, h, d = query.shape
        if b <= 0 or s <= 0 or h <= 0 or d <= 0:
            raise ValueError("All tensor dimensions must be > 0")
        if self.sparse and (self.window_size <= 0):
            raise ValueError("window_size must be > 0 for sparse attention")

        if self.training and self.fallback_training:
            for t in (query, key, value):
                if t.requires_grad and t.grad_fn is not None:
                    t.retain_grad()
            if self.spec is not None:
                return pytorch_pattern_attention(query, key, value, self.spec)
            if self.sparse:
                return pytorch_sparse_attention(query, key, value, self.window_size)
            return pytorch_dense_attention(query, key, value, self.use_causal_mask)

        return MACoreAttentionFunction.apply(query, key, value, self.sparse, self.window_size,
                                             self.use_causal_mask, self.spec)


def create_attention_layer(attention_type: str = "dense", **kwargs) -> nn.Module:
    """Factory (reference :333-352): "dense", "sparse" or "auto" (= sparse)."""
    if attention_type == "dense":
        return MACoreAttention(sparse=False, **kwargs)
    if attention_type == "sparse":
        return MACoreAttention(sparse=True, **kwargs)
    if attention_type == "auto":
        return MACoreAttention(sparse=True, **kwargs)
    raise ValueError(f"Unknown attention type: {attention_type}")
