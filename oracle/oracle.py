"""CPU oracle for the sparse-attention forward and backward -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only as the checker / the timed CPU baseline.  The
product (``ma-transformer_amd/``) never imports it.

Independent statements of the same semantics live here:

* ``forward`` -- ctypes over ``liboracle.so`` (oracle.c), the op-for-op
  restatement of ``ma_core::compute_sparse_attention``
  (/root/reference src/csrc/ma_core.cpp:160-246) generalised to explicit key
  lists.
* ``forward_f64`` -- a float64 dense-masked softmax(Q K^T * scale) V written
  with numpy (textbook attention; the masking mirrors the reference PyTorch
  golden ``pytorch_sparse_attention``, src/layers/ma_core_bridge.py:224-247).
* ``member`` -- a brute-force membership predicate per pattern, used on tiny
  shapes to pin ``row_keys`` (the closed forms) bit-exactly.
* ``backward`` -- oracle.c's restatement of the reference's backward kernel
  (src/cuda/sparse_attention_kernel.cu:265-346) over the same key lists,
  pinned by float64 autograd and by finite differences of ``forward_f64``.

``ref_*`` wrap ``_ref/libma_core_ref.so``: the reference's own ma_core.cpp and
tensor.cpp compiled unchanged (see Makefile).  It exists only where it was
built; callers must handle ``ref_available() is False``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libma_core_ref.so")

PATTERNS = {"sliding": 0, "dense": 1, "block_sparse": 2, "longformer": 3, "index_set": 4}


class _Spec(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int64), ("N", ctypes.c_int64), ("H", ctypes.c_int64), ("D", ctypes.c_int64),
        ("pattern", ctypes.c_int32), ("causal", ctypes.c_int32),
        ("left", ctypes.c_int64), ("right", ctypes.c_int64), ("dilation", ctypes.c_int64),
        ("block_size", ctypes.c_int64), ("table", ctypes.POINTER(ctypes.c_int32)),
        ("bpr", ctypes.c_int64), ("num_global", ctypes.c_int64),
        ("offsets", ctypes.POINTER(ctypes.c_int64)), ("keys", ctypes.POINTER(ctypes.c_int32)),
        ("nnz", ctypes.c_int64),
    ]


_lib = None
_ref = None


def build() -> None:
    """Compile liboracle.so (and _ref/ when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if os.path.isdir("/root/reference/src/csrc"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        lib = ctypes.CDLL(LIB_PATH)
        lib.oracle_row_keys.restype = ctypes.c_int64
        lib.oracle_row_keys.argtypes = [ctypes.POINTER(_Spec), ctypes.c_int64,
                                        ctypes.POINTER(ctypes.c_int64), ctypes.c_int64]
        lib.oracle_forward_f32.restype = ctypes.c_int
        lib.oracle_forward_f32.argtypes = [ctypes.POINTER(_Spec)] + [ctypes.c_void_p] * 4 + \
            [ctypes.c_int64] * 4
        lib.oracle_backward_f32.restype = ctypes.c_int
        lib.oracle_backward_f32.argtypes = [ctypes.POINTER(_Spec)] + [ctypes.c_void_p] * 7
        lib.oracle_block_table.restype = ctypes.c_int
        lib.oracle_block_table.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.POINTER(ctypes.c_int32)]
        _lib = lib
    return _lib


class Spec:
    """Pattern parameters (same meaning as ma_attn_desc)."""

    def __init__(self, B, N, H, D, pattern="sliding", left=0, right=0, dilation=1,
                 causal=False, block_size=64, table=None, num_global=0, offsets=None, keys=None):
        """offsets, keys: the INDEX_SET pattern's CSR rows (int64 [N+1], int32 [nnz])."""
        self.B, self.N, self.H, self.D = int(B), int(N), int(H), int(D)
        self.pattern = pattern
        self.left, self.right, self.dilation = int(left), int(right), int(dilation)
        self.causal = bool(causal)
        self.block_size = int(block_size)
        self.table = None if table is None else np.ascontiguousarray(table, dtype=np.int32)
        self.num_global = int(num_global)
        self.offsets = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.int64)
        self.keys = None if keys is None else np.ascontiguousarray(keys, dtype=np.int32)

    def _c(self):
        s = _Spec()
        s.B, s.N, s.H, s.D = self.B, self.N, self.H, self.D
        s.pattern = PATTERNS[self.pattern]
        s.causal = int(self.causal)
        s.left, s.right, s.dilation = self.left, self.right, self.dilation
        s.block_size = self.block_size
        if self.table is not None:
            s.table = self.table.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
            s.bpr = self.table.shape[1]
        else:
            s.table = ctypes.POINTER(ctypes.c_int32)()
            s.bpr = 0
        s.num_global = self.num_global
        if self.offsets is not None:
            s.offsets = self.offsets.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))
            keys = self.keys if self.keys is not None and self.keys.size else np.zeros(1, np.int32)
            self._keys_c = keys  # kept alive with the struct
            s.keys = keys.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
            s.nnz = 0 if self.keys is None else int(self.keys.size)
        return s


def row_keys(spec: Spec, i: int) -> np.ndarray:
    """Ascending key list of query row i (closed forms of oracle.c)."""
    lib = _load()
    s = spec._c()
    cap = max(spec.N, 1)
    buf = (ctypes.c_int64 * cap)()
    n = lib.oracle_row_keys(ctypes.byref(s), int(i), buf, cap)
    if n < 0:
        raise ValueError("invalid spec")
    return np.frombuffer(buf, dtype=np.int64, count=n).copy()


def forward(spec: Spec, q, k, v, heads=None, rows=None) -> np.ndarray:
    """fp32 oracle forward on float32 arrays [B,N,H,D] (restated ma_core.cpp:160-246).

    heads/rows: optional (lo, hi) ranges to compute a bounded sample; rows
    outside the ranges are returned as NaN.
    """
    lib = _load()
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    o = np.full(q.shape, np.nan, dtype=np.float32)
    h_lo, h_hi = heads if heads is not None else (0, spec.H)
    i_lo, i_hi = rows if rows is not None else (0, spec.N)
    s = spec._c()
    rc = lib.oracle_forward_f32(ctypes.byref(s), q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                o.ctypes.data, h_lo, h_hi, i_lo, i_hi)
    if rc != 0:
        raise ValueError("oracle_forward_f32 rejected the spec")
    return o


def forward_value_dim(spec: Spec, q, k, v) -> np.ndarray:
    """``forward`` for V with a head_dim Dv of its own (q, k [B,N,H,D], v
    [B,N,H,Dv] -> o [B,N,H,Dv]), as ma_core.cpp:160-246 computes it: scores
    and scale from D (:188), one weighted sum per value column (:232-239).  V
    runs through ``forward`` in blocks of D columns (the last one zero-padded);
    a column's sum does not depend on the other columns, so each block gives
    its columns' exact values."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, N, H, D = q.shape
    Dv = v.shape[3]
    o = np.empty((B, N, H, Dv), dtype=np.float32)
    for c0 in range(0, Dv, max(D, 1)):
        c1 = min(Dv, c0 + D)
        vb = np.zeros(q.shape, dtype=np.float32)
        vb[..., :c1 - c0] = v[..., c0:c1]
        o[..., c0:c1] = forward(spec, q, k, vb)[..., :c1 - c0]
    return o


def backward(spec: Spec, q, k, v, dout):
    """fp32 oracle backward (restated sparse_attention_kernel.cu:265-346) -> (dq, dk, dv)."""
    lib = _load()
    q, k, v, dout = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v, dout))
    dq, dk, dv = (np.empty(q.shape, dtype=np.float32) for _ in range(3))
    s = spec._c()
    rc = lib.oracle_backward_f32(ctypes.byref(s), q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                 dout.ctypes.data, dq.ctypes.data, dk.ctypes.data, dv.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_backward_f32 rejected the spec")
    return dq, dk, dv


def block_table(seed: int, num_blocks: int, random_per_row: int) -> np.ndarray:
    """Seeded int32 [nb, 2+extra] block table (oracle.c:oracle_block_table)."""
    lib = _load()
    out = np.empty((num_blocks, 2 + random_per_row), dtype=np.int32)
    rc = lib.oracle_block_table(ctypes.c_uint64(seed & (2**64 - 1)), num_blocks, random_per_row,
                                out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
    if rc != 0:
        raise ValueError("bad block table request")
    return out


# ---------------------------------------------------------------- independent checks

def member(spec: Spec, i: int, j: int) -> bool:
    """Brute-force membership j in S_i, written from the set definitions."""
    N = spec.N
    if not (0 <= i < N and 0 <= j < N):
        return False
    if spec.pattern == "sliding":
        diff = j - i
        if diff % spec.dilation != 0:
            return False
        t = diff // spec.dilation
        return -spec.left <= t <= spec.right
    if spec.pattern == "dense":
        return (j <= i) if spec.causal else True
    if spec.pattern == "block_sparse":
        r = i // spec.block_size
        return any(c >= 0 and c * spec.block_size <= j < (c + 1) * spec.block_size
                   for c in spec.table[r])
    if spec.pattern == "longformer":
        G = spec.num_global
        if i < G:
            return True
        return j < G or (i - spec.left <= j <= i + spec.right)
    if spec.pattern == "index_set":
        return bool(np.any(spec.keys[spec.offsets[i]:spec.offsets[i + 1]] == j))
    raise ValueError(spec.pattern)


def mask_dense(spec: Spec) -> np.ndarray:
    """[N, N] boolean mask from ``member`` (tiny N only)."""
    N = spec.N
    m = np.zeros((N, N), dtype=bool)
    for i in range(N):
        for j in range(N):
            m[i, j] = member(spec, i, j)
    return m


def forward_f64(q, k, v, mask: np.ndarray) -> np.ndarray:
    """float64 dense-masked attention; rows with an empty mask give zeros."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, N, H, D = q.shape
    scale = 1.0 / np.sqrt(np.float32(D)).astype(np.float64)
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(H):
            s = (q[b, :, h, :] @ k[b, :, h, :].T) * scale
            s = np.where(mask, s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            e = np.where(mask, np.exp(s - mx), 0.0)
            den = e.sum(axis=1, keepdims=True)
            p = np.divide(e, den, out=np.zeros_like(e), where=den > 0)
            out[b, :, h, :] = p @ v[b, :, h, :]
    return out


# ---------------------------------------------------------------- bf16 / fp16 helpers

def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    r = ((u + rounding) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16, returned as float32."""
    return bf16_bits_to_f32(to_bf16_bits(x))


# ---------------------------------------------------------------- the reference's own engine

def _load_ref():
    global _ref
    if _ref is None:
        if not os.path.exists(REF_PATH):
            return None
        lib = ctypes.CDLL(REF_PATH)
        for name in ("ref_sparse_forward", "ref_dense_forward"):
            getattr(lib, name).restype = ctypes.c_int
        lib.ref_sparse_forward.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_void_p] * 4
        lib.ref_dense_forward.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int] + [ctypes.c_void_p] * 4
        lib.ref_sparse_forward_v.restype = ctypes.c_int
        lib.ref_sparse_forward_v.argtypes = [ctypes.c_int64] * 6 + [ctypes.c_void_p] * 4
        lib.ref_dense_forward_v.restype = ctypes.c_int
        lib.ref_dense_forward_v.argtypes = [ctypes.c_int64] * 5 + [ctypes.c_int] + [ctypes.c_void_p] * 4
        lib.ref_sliding_pattern.restype = ctypes.c_int64
        lib.ref_sliding_pattern.argtypes = [ctypes.c_int64, ctypes.c_int64,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.ref_pattern_statistics.restype = ctypes.c_int64
        lib.ref_pattern_statistics.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_char_p, ctypes.c_int64]
        _ref = lib
    return _ref


def ref_available() -> bool:
    return _load_ref() is not None


def ref_sparse_forward(q, k, v, window: int) -> np.ndarray:
    """The reference's ma_core::compute_sparse_attention (ma_core.cpp:160-246), unchanged."""
    lib = _load_ref()
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    o = np.empty_like(q)
    B, N, H, D = q.shape
    if lib.ref_sparse_forward(B, N, H, D, int(window), q.ctypes.data, k.ctypes.data,
                              v.ctypes.data, o.ctypes.data) != 0:
        raise RuntimeError("reference compute_sparse_attention raised")
    return o


def ref_dense_forward(q, k, v, causal: bool) -> np.ndarray:
    """The reference's ma_core::compute_dense_attention (ma_core.cpp:66-157), unchanged."""
    lib = _load_ref()
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    o = np.empty_like(q)
    B, N, H, D = q.shape
    if lib.ref_dense_forward(B, N, H, D, int(bool(causal)), q.ctypes.data, k.ctypes.data,
                             v.ctypes.data, o.ctypes.data) != 0:
        raise RuntimeError("reference compute_dense_attention raised")
    return o


def ref_forward_v(q, k, v, window=None, causal: bool = False) -> np.ndarray:
    """The reference's compute_sparse_attention (window given) or
    compute_dense_attention (window None) with a value head_dim of its own:
    q, k [B,N,H,D], v [B,N,H,Dv] -> o [B,N,H,Dv] (ma_core.cpp:84-90, :178-183)."""
    lib = _load_ref()
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    B, N, H, D = q.shape
    Dv = v.shape[3]
    o = np.empty((B, N, H, Dv), dtype=np.float32)
    if window is None:
        rc = lib.ref_dense_forward_v(B, N, H, D, Dv, int(bool(causal)), q.ctypes.data, k.ctypes.data,
                                     v.ctypes.data, o.ctypes.data)
    else:
        rc = lib.ref_sparse_forward_v(B, N, H, D, Dv, int(window), q.ctypes.data, k.ctypes.data,
                                      v.ctypes.data, o.ctypes.data)
    if rc != 0:
        raise RuntimeError("reference attention raised")
    return o


def ref_sliding_pattern(N: int, w: int):
    """(rows, cols) COO lists of the reference's create_sliding_window_pattern."""
    lib = _load_ref()
    cap = N * N
    rows = np.empty(max(cap, 1), dtype=np.int64)
    cols = np.empty(max(cap, 1), dtype=np.int64)
    n = lib.ref_sliding_pattern(N, w, rows.ctypes.data, cols.ctypes.data, cap)
    if n < 0:
        raise RuntimeError("reference create_sliding_window_pattern raised")
    return rows[:n], cols[:n]


def ref_pattern_statistics(N: int, w: int) -> str:
    """The reference's get_pattern_statistics of create_sliding_window_pattern(N, w)."""
    lib = _load_ref()
    buf = ctypes.create_string_buffer(1024)
    n = lib.ref_pattern_statistics(N, w, buf, 1024)
    if n < 0 or n >= 1024:
        raise RuntimeError("reference get_pattern_statistics raised")
    return buf.value.decode()
