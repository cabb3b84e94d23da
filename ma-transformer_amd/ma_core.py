"""MA Transformer Core Engine: the ``ma_core`` module of the reference's
src/csrc, on the MI355X engine.

Same module name, functions, argument names and defaults, classes and error
types as the reference's pybind11 module (/root/reference
src/csrc/main.cpp:10-98), so the reference's unchanged bridge
(src/layers/ma_core_bridge.py:10) and layer (src/layers/sparse_attention.py:9-16)
import it and reach this engine:

    add(a, b)                                               main.cpp:14
    create_tensor(shape, device="cpu")                      main.cpp:17-19
    create_random_tensor(shape, mean=0.0, std=1.0, device="cpu")  :21-23
    create_sliding_window_pattern(seq_len, window_size)     :26-28
    get_pattern_statistics(pattern)                         :30-31
    compute_dense_attention(query, key, value, use_causal_mask=False)  :34-36
    compute_sparse_attention(query, key, value, window_size=64)        :38-40
    SparseTensor, TensorShape, Tensor (copy_from_numpy, to_numpy), Device  :43-97

What runs where:

* ``Tensor`` is a host float32 buffer in the reference's layout
  [batch, seq, heads, head_dim], head_dim fastest (src/csrc/tensor.cpp:108).
* ``compute_sparse_attention`` / ``compute_dense_attention`` stage the three
  host buffers to the current GPU, run the HIP kernels of libma_attn.so
  (``sparse_attention_cuda.forward`` / ``dense_forward``, i.e.
  ma_attn_forward) and copy the output back into a new host ``Tensor``.  The
  reference ran them on a single CPU thread (src/csrc/ma_core.cpp:66-246).
  There is no CPU arithmetic path: without a visible GPU they raise
  RuntimeError, and without libma_attn.so the import fails.
* ``create_sliding_window_pattern`` enumerates the pattern with the engine's
  closed forms in one C-ABI call (ma_attn_pattern_csr): the entries of
  src/csrc/ma_core.cpp:34-48, in the same (row, col) order.

A value head_dim different from the query's is accepted, as the reference
does (its output takes the value's, ma_core.cpp:84-90, :178-183): the kernels
take Q, K and V of one head_dim, so the narrower operands are zero-padded to
the wider one on the device and the scale is passed as 1/sqrtf(query
head_dim).  Zero columns add exact zeros to every dot product and give zero
output columns, which are sliced off.  K and V may carry more batches or heads
than Q (the reference indexes them with their own shapes and reads only Q's
range); fewer raise RuntimeError, where the reference would read past them.
"""
from __future__ import annotations

import enum
import operator
from typing import Sequence

import numpy as np
import torch

import ma_attn as _ma

_INT64_MIN, _INT64_MAX = -(2 ** 63), 2 ** 63 - 1


def _as_int64(x, what: str) -> int:
    """An integer argument as pybind11 converts it for int64_t: ints (and
    objects with __index__) only, TypeError for floats, strings and values
    outside the int64 range."""
    if isinstance(x, float):
        raise TypeError(f"{what}: incompatible function argument (float given, int expected)")
    try:
        v = operator.index(x)
    except TypeError:
        raise TypeError(f"{what}: incompatible function argument ({type(x).__name__} given, "
                        "int expected)") from None
    if not _INT64_MIN <= v <= _INT64_MAX:
        raise TypeError(f"{what}: integer argument outside the int64 range")
    return v


def add(a, b) -> int:
    """A function which adds two numbers (int64; reference main.cpp:14, ma_core.cpp:10-12)."""
    s = _as_int64(a, "add") + _as_int64(b, "add")
    return (s + 2 ** 63) % 2 ** 64 - 2 ** 63  # int64 wraparound


class Device(enum.Enum):
    """Device enumeration (src/csrc/attention_types.hpp:16-21)."""

    CPU = 0
    MPS = 1
    CUDA = 2
    ROCm = 3

    def __int__(self) -> int:
        return self.value


class TensorShape:
    """[batch, seq, heads, head_dim] sizes (src/csrc/attention_types.hpp:61-73)."""

    __slots__ = ("_b", "_s", "_h", "_d")

    def __init__(self, batch_size: int, sequence_length: int, num_heads: int, head_dim: int):
        self._b, self._s, self._h, self._d = (int(batch_size), int(sequence_length), int(num_heads),
                                              int(head_dim))

    batch_size = property(lambda self: self._b)
    sequence_length = property(lambda self: self._s)
    num_heads = property(lambda self: self._h)
    head_dim = property(lambda self: self._d)

    def total_elements(self) -> int:
        return self._b * self._s * self._h * self._d

    def __repr__(self) -> str:
        return (f"TensorShape(batch_size={self._b}, sequence_length={self._s}, "
                f"num_heads={self._h}, head_dim={self._d})")


class Tensor:
    """Owning float32 host tensor [batch, seq, heads, head_dim] (src/csrc/tensor.hpp:16-96)."""

    __slots__ = ("_data",)

    def __init__(self, data: np.ndarray):
        self._data = data  # float32, C-contiguous, 4-D

    def size(self) -> int:
        """Total number of elements."""
        return int(self._data.size)

    def nbytes(self) -> int:
        """Total number of bytes."""
        return int(self._data.nbytes)

    def empty(self) -> bool:
        """Check if tensor is empty."""
        return self._data.size == 0

    def shape(self) -> TensorShape:
        """Get tensor shape."""
        return TensorShape(*self._data.shape)

    def zero(self) -> None:
        """Fill tensor with zeros."""
        self._data.fill(0.0)

    def fill(self, value: float) -> None:
        """Fill tensor with a value."""
        if isinstance(value, (str, bytes)):
            raise TypeError("fill: incompatible function argument (float expected)")
        self._data.fill(np.float32(value))

    def copy_from_numpy(self, array) -> None:
        """Bulk copy from an array of the same element count (cast to float32, C order)."""
        arr = np.ascontiguousarray(array, dtype=np.float32)
        if arr.size * 4 != self._data.nbytes:
            raise RuntimeError("copy_from_numpy: size mismatch")
        self._data.reshape(-1)[:] = arr.reshape(-1)

    def to_numpy(self) -> np.ndarray:
        """A new float32 array [batch, seq, heads, head_dim] with the tensor contents."""
        return self._data.copy()


class SparseTensor:
    """COO sparse pattern (src/csrc/tensor.hpp:101-131): (row, col) entries of value 1."""

    __slots__ = ("_shape", "_rows", "_cols")

    def __init__(self, shape: TensorShape, rows: np.ndarray, cols: np.ndarray):
        self._shape, self._rows, self._cols = shape, rows, cols

    shape = property(lambda self: self._shape)
    device = property(lambda self: Device.CPU)

    def nnz(self) -> int:
        """Number of non-zero elements."""
        return int(self._rows.size)

    def empty(self) -> bool:
        """Check if tensor is empty."""
        return self._rows.size == 0

    @property
    def row_indices(self) -> np.ndarray:
        return self._rows.copy()

    @property
    def col_indices(self) -> np.ndarray:
        return self._cols.copy()


def _shape4(shape: Sequence[int]):
    dims = list(shape)
    if len(dims) != 4:
        raise RuntimeError("Shape must have 4 dimensions: [batch, seq, heads, dim]")
    dims = [_as_int64(x, "create_tensor") for x in dims]
    if any(x < 0 for x in dims):
        raise RuntimeError("Shape dimensions must be >= 0")
    return tuple(dims)


def create_tensor(shape: Sequence[int], device: str = "cpu") -> Tensor:
    """Create a tensor with given shape (zero-filled host buffer)."""
    return Tensor(np.zeros(_shape4(shape), dtype=np.float32))


def create_random_tensor(shape: Sequence[int], mean: float = 0.0, std: float = 1.0,
                         device: str = "cpu") -> Tensor:
    """Create a tensor filled with random values from normal distribution
    (unseeded, as the reference's std::random_device, tensor.cpp:142-154)."""
    dims = _shape4(shape)
    rng = np.random.default_rng()
    return Tensor((rng.standard_normal(dims, dtype=np.float32) * np.float32(std) + np.float32(mean))
                  .astype(np.float32))


def create_sliding_window_pattern(seq_len: int, window_size: int) -> SparseTensor:
    """Create a sliding window sparse attention pattern: entries (i, j) for
    j in [max(0, i-w), min(seq_len, i+w+1)), row after row (ma_core.cpp:34-48);
    shape (1, seq_len, head_dim=1, num_heads=seq_len) as the reference builds it."""
    n = _as_int64(seq_len, "create_sliding_window_pattern")
    w = _as_int64(window_size, "create_sliding_window_pattern")
    shape = TensorShape(1, n, n, 1)
    if n <= 0:
        return SparseTensor(shape, np.zeros(0, np.int64), np.zeros(0, np.int64))
    desc = _ma.make_desc(1, n, 1, 1, _ma.F32, _ma.SLIDING, left=w, right=w, dilation=1)
    offsets, keys = _ma.pattern_csr(desc)
    rows = np.repeat(np.arange(n, dtype=np.int64), np.diff(offsets.numpy()))
    return SparseTensor(shape, rows, keys.numpy().astype(np.int64))


def get_pattern_statistics(pattern: SparseTensor) -> str:
    """Get statistics about a sparse attention pattern (ma_core.cpp:51-63;
    float32 ratio, printed as std::to_string does)."""
    if not isinstance(pattern, SparseTensor):
        raise TypeError("get_pattern_statistics: a SparseTensor is required")
    n = pattern.shape.sequence_length
    total = n * n
    nnz = pattern.nnz()
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.float32(1.0) - np.float32(nnz) / np.float32(total)
    pct = float(ratio * np.float32(100.0))
    return ("Pattern Statistics:\n"
            f"  Total elements: {total}\n"
            f"  Non-zero elements: {nnz}\n"
            f"  Sparsity ratio: {pct:f}%\n")


def _check_qkv(query, key, value):
    for t in (query, key, value):
        if not isinstance(t, Tensor):
            raise TypeError("incompatible function arguments: query, key and value must be ma_core.Tensor")
    qs, ks, vs = query._data.shape, key._data.shape, value._data.shape
    # the reference's two checks, with its messages (ma_core.cpp:72-80)
    if not (qs[1] == ks[1] == vs[1]):
        raise RuntimeError("Query, key, and value must have same sequence length")
    if qs[3] != ks[3]:
        raise RuntimeError("Query and key must have same head dimension")
    # the reference reads K and V at Q's (batch, head) range with their own
    # strides (tensor.cpp:104-114): fewer batches or heads than Q is out of range
    if min(ks[0], vs[0]) < qs[0] or min(ks[2], vs[2]) < qs[2]:
        raise RuntimeError("Key and value must have at least the query's batch size and number of heads")


def _on_engine(query: Tensor, key: Tensor, value: Tensor, run) -> Tensor:
    """Stage Q, K, V to the current GPU, run the kernels, copy O back.

    O is [batch, seq, heads, value head_dim].  run(ext, q, k, v, scale) gets
    device tensors of one shape and scale None (1/sqrtf(head_dim)) or, when
    the head_dims were padded, the query head_dim's 1/sqrtf (ma_core.cpp:188)."""
    B, N, H, D = query._data.shape
    Dv = value._data.shape[3]
    if B * N * H * Dv == 0:
        return Tensor(np.zeros((B, N, H, Dv), dtype=np.float32))
    if not torch.cuda.is_available():
        raise RuntimeError("ma_core: attention runs on the MI355X engine (libma_attn.so); no GPU is visible")
    import sparse_attention_cuda as ext
    dev = torch.device("cuda", torch.cuda.current_device())

    def staged(t: Tensor, width: int) -> torch.Tensor:
        x = t._data[:B, :, :H, :]  # Q's (batch, head) range
        if x.shape[3] == width:
            return torch.from_numpy(np.ascontiguousarray(x)).to(dev)
        y = torch.zeros((B, N, H, width), dtype=torch.float32, device=dev)
        y[..., :x.shape[3]] = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
        return y

    width = max(D, Dv)
    tq, tk, tv = staged(query, width), staged(key, width), staged(value, width)
    scale = None if D == width else float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = run(ext, tq, tk, tv, scale)
    if Dv != width:
        out = out[..., :Dv]
    return Tensor(np.ascontiguousarray(out.cpu().numpy()))


def compute_dense_attention(query: Tensor, key: Tensor, value: Tensor,
                            use_causal_mask: bool = False) -> Tensor:
    """Compute dense attention (Q@K^T, softmax, @V): ma_core.cpp:66-157 on the GPU
    (keys [0, S), or [0, i] with the causal mask)."""
    _check_qkv(query, key, value)
    causal = bool(use_causal_mask)
    return _on_engine(query, key, value,
                      lambda ext, q, k, v, scale: ext.dense_forward(q, k, v, causal, scale=scale))


def compute_sparse_attention(query: Tensor, key: Tensor, value: Tensor, window_size: int = 64) -> Tensor:
    """Compute sparse attention with sliding window: keys [max(0,i-w), min(S,i+w+1)),
    ma_core.cpp:160-246 on the GPU (w = 0 gives O = V, w < 0 an all-zero O)."""
    _check_qkv(query, key, value)
    w = _as_int64(window_size, "compute_sparse_attention")
    return _on_engine(query, key, value,
                      lambda ext, q, k, v, scale: ext.sliding_forward(q, k, v, w, w, 1, scale=scale))


__all__ = ["add", "create_tensor", "create_random_tensor", "create_sliding_window_pattern",
           "get_pattern_statistics", "compute_dense_attention", "compute_sparse_attention",
           "SparseTensor", "TensorShape", "Tensor", "Device"]
