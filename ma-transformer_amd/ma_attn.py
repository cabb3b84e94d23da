"""ctypes binding of libma_attn.so (the C-ABI declared in include/ma_attn.h).

This is the only place Python touches the native engine.  ``torch`` is
imported before the library is opened so that the HIP runtime torch bundles
(soname libamdhip64.so.7) is the one the engine binds to: tensors, streams and
kernels then share one runtime.  Missing library => ImportError; there is no
fallback path.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede loading the HIP library)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MA_ATTN_LIB", os.path.join(_HERE, "libma_attn.so"))

F32, BF16, F16 = 0, 1, 2
SLIDING, DENSE, BLOCK_SPARSE, LONGFORMER, INDEX_SET = 0, 1, 2, 3, 4
ABI_VERSION = 10

DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}


class TileHeader(ctypes.Structure):
    """Mirror of ``ma_attn_tile_header`` (include/ma_attn.h)."""

    _fields_ = [(n, ctypes.c_int64) for n in (
        "seq_len", "num_tiles", "num_entries", "seg", "num_q_items", "num_q_split", "num_q_partials",
        "num_k_items", "num_k_split", "num_k_partials", "off_blk", "off_mask", "off_kmask", "off_tile",
        "off_kentry", "off_q_items", "off_q_split", "off_k_items", "off_k_split", "total_bytes", "num_masked")]


class Desc(ctypes.Structure):
    """Mirror of ``ma_attn_desc`` (include/ma_attn.h)."""

    _fields_ = [
        ("batch", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("num_heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("pattern", ctypes.c_int32),
        ("left", ctypes.c_int64),
        ("right", ctypes.c_int64),
        ("dilation", ctypes.c_int64),
        ("causal", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("block_size", ctypes.c_int64),
        ("block_table", ctypes.c_void_p),
        ("blocks_per_row", ctypes.c_int64),
        ("num_global", ctypes.c_int64),
        ("scale", ctypes.c_float),
        ("reserved1", ctypes.c_int32),
        ("index_offsets", ctypes.c_void_p),
        ("index_keys", ctypes.c_void_p),
        ("num_indices", ctypes.c_int64),
        ("index_t_offsets", ctypes.c_void_p),
        ("index_t_queries", ctypes.c_void_p),
        ("tile_header", ctypes.c_void_p),
        ("tile_plan", ctypes.c_void_p),
    ]


class EncoderLayer(ctypes.Structure):
    """Mirror of ``ma_encoder_layer`` (include/ma_encoder.h)."""

    _fields_ = [
        ("batch", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("d_model", ctypes.c_int64),
        ("d_ff", ctypes.c_int64),
        ("window", ctypes.c_int64),
        ("ln_eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
        ("norm1_weight", ctypes.c_void_p),
        ("norm1_bias", ctypes.c_void_p),
        ("linear1_weight", ctypes.c_void_p),
        ("linear1_bias", ctypes.c_void_p),
        ("linear2_weight", ctypes.c_void_p),
        ("linear2_bias", ctypes.c_void_p),
        ("norm2_weight", ctypes.c_void_p),
        ("norm2_bias", ctypes.c_void_p),
    ]


def _open():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libma_attn.so not found at {LIB_PATH}; build it with "
            "`python setup.py build_ext` (hipcc --offload-arch=gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    lib.ma_attn_abi_version.restype = ctypes.c_int
    lib.ma_attn_last_error.restype = ctypes.c_char_p
    lib.ma_attn_validate.restype = ctypes.c_int
    lib.ma_attn_validate.argtypes = [ctypes.POINTER(Desc)]
    lib.ma_attn_workspace_size.restype = ctypes.c_size_t
    lib.ma_attn_workspace_size.argtypes = [ctypes.POINTER(Desc)]
    lib.ma_attn_forward.restype = ctypes.c_int
    lib.ma_attn_forward.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 5 + \
        [ctypes.c_size_t, ctypes.c_void_p]
    lib.ma_attn_backward_workspace_size.restype = ctypes.c_size_t
    lib.ma_attn_backward_workspace_size.argtypes = [ctypes.POINTER(Desc)]
    lib.ma_attn_backward.restype = ctypes.c_int
    lib.ma_attn_backward.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 8 + \
        [ctypes.c_size_t, ctypes.c_void_p]
    lib.ma_attn_forward_timed.restype = ctypes.c_int
    lib.ma_attn_forward_timed.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 5 + \
        [ctypes.c_size_t] + [ctypes.c_void_p] * 3
    lib.ma_attn_backward_timed.restype = ctypes.c_int
    lib.ma_attn_backward_timed.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 8 + \
        [ctypes.c_size_t] + [ctypes.c_void_p] * 3
    lib.ma_attn_forward_lse.restype = ctypes.c_int
    lib.ma_attn_forward_lse.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 6 + \
        [ctypes.c_size_t, ctypes.c_void_p]
    lib.ma_attn_forward_lse_timed.restype = ctypes.c_int
    lib.ma_attn_forward_lse_timed.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 6 + \
        [ctypes.c_size_t] + [ctypes.c_void_p] * 3
    lib.ma_attn_backward_saved.restype = ctypes.c_int
    lib.ma_attn_backward_saved.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 10 + \
        [ctypes.c_size_t, ctypes.c_void_p]
    lib.ma_attn_backward_saved_timed.restype = ctypes.c_int
    lib.ma_attn_backward_saved_timed.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 10 + \
        [ctypes.c_size_t] + [ctypes.c_void_p] * 3
    lib.ma_attn_block_table.restype = ctypes.c_int
    lib.ma_attn_block_table.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_void_p]
    lib.ma_attn_row_keys.restype = ctypes.c_int64
    lib.ma_attn_row_keys.argtypes = [ctypes.POINTER(Desc), ctypes.c_void_p, ctypes.c_int64,
                                     ctypes.c_void_p, ctypes.c_int64]
    lib.ma_attn_pattern_csr.restype = ctypes.c_int64
    lib.ma_attn_pattern_csr.argtypes = [ctypes.POINTER(Desc), ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_int64]
    lib.ma_attn_forward_noalloc.restype = ctypes.c_int
    lib.ma_attn_forward_noalloc.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 5
    lib.ma_encoder_layer_forward.restype = ctypes.c_int
    lib.ma_encoder_layer_forward.argtypes = [ctypes.POINTER(EncoderLayer)] + [ctypes.c_void_p] * 4
    lib.ma_attn_tile_plan.restype = ctypes.c_int
    lib.ma_attn_tile_plan.argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.POINTER(TileHeader), ctypes.c_void_p, ctypes.c_size_t]
    lib.ma_attn_copy_probe_timed.restype = ctypes.c_int
    lib.ma_attn_copy_probe_timed.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 7
    lib.ma_attn_backward_copy_probe_timed.restype = ctypes.c_int
    lib.ma_attn_backward_copy_probe_timed.argtypes = [ctypes.POINTER(Desc)] + [ctypes.c_void_p] * 10
    lib.ma_attn_reload_options.restype = None
    lib.ma_attn_reload_options.argtypes = []
    if lib.ma_attn_abi_version() != ABI_VERSION:
        raise ImportError("libma_attn.so ABI version mismatch; rebuild it")
    return lib


LIB = _open()


def last_error() -> str:
    return (LIB.ma_attn_last_error() or b"").decode()


def make_desc(B, N, H, D, dtype_code, pattern, left=0, right=0, dilation=1, causal=False,
              block_size=64, block_table_ptr=0, blocks_per_row=0, num_global=0,
              scale=0.0, index_offsets_ptr=0, index_keys_ptr=0, num_indices=0, index_t_offsets_ptr=0,
              index_t_queries_ptr=0, tile_header_ptr=0, tile_plan_ptr=0) -> Desc:
    d = Desc()
    d.batch, d.seq_len, d.num_heads, d.head_dim = int(B), int(N), int(H), int(D)
    d.dtype, d.pattern = int(dtype_code), int(pattern)
    d.left, d.right, d.dilation = int(left), int(right), int(dilation)
    d.causal = int(bool(causal))
    d.block_size = int(block_size)
    d.block_table = int(block_table_ptr) or None
    d.blocks_per_row = int(blocks_per_row)
    d.num_global = int(num_global)
    d.scale = float(scale)
    d.index_offsets = int(index_offsets_ptr) or None
    d.index_keys = int(index_keys_ptr) or None
    d.num_indices = int(num_indices)
    d.index_t_offsets = int(index_t_offsets_ptr) or None
    d.index_t_queries = int(index_t_queries_ptr) or None
    d.tile_header = int(tile_header_ptr) or None
    d.tile_plan = int(tile_plan_ptr) or None
    return d


def validate(desc: Desc) -> None:
    if LIB.ma_attn_validate(ctypes.byref(desc)) != 0:
        raise RuntimeError(last_error())


def workspace_size(desc: Desc) -> int:
    return int(LIB.ma_attn_workspace_size(ctypes.byref(desc)))


def forward_raw(desc: Desc, q_ptr: int, k_ptr: int, v_ptr: int, o_ptr: int,
                ws_ptr: int = 0, ws_bytes: int = 0, stream: int = 0, events=None) -> None:
    """Launch on ``stream`` (a hipStream_t as int).  Raises RuntimeError on rejection.

    events: optional (start, stop) hipEvent_t handles (ints) stamped on the
    call's first and last kernel (ma_attn_forward_timed)."""
    if events:
        rc = LIB.ma_attn_forward_timed(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, o_ptr, ws_ptr or None,
                                       ws_bytes, stream or None, events[0] or None, events[1] or None)
    else:
        rc = LIB.ma_attn_forward(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, o_ptr, ws_ptr or None,
                                 ws_bytes, stream or None)
    if rc != 0:
        raise RuntimeError(last_error())


def backward_workspace_size(desc: Desc) -> int:
    return int(LIB.ma_attn_backward_workspace_size(ctypes.byref(desc)))


def backward_raw(desc: Desc, q_ptr: int, k_ptr: int, v_ptr: int, g_ptr: int, dq_ptr: int,
                 dk_ptr: int, dv_ptr: int, ws_ptr: int, ws_bytes: int, stream: int = 0, events=None) -> None:
    """Launch the backward on ``stream``.  Raises RuntimeError on rejection."""
    if events:
        rc = LIB.ma_attn_backward_timed(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, g_ptr, dq_ptr, dk_ptr, dv_ptr,
                                        ws_ptr or None, ws_bytes, stream or None, events[0] or None,
                                        events[1] or None)
    else:
        rc = LIB.ma_attn_backward(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, g_ptr, dq_ptr, dk_ptr, dv_ptr,
                                  ws_ptr or None, ws_bytes, stream or None)
    if rc != 0:
        raise RuntimeError(last_error())


def forward_lse_raw(desc: Desc, q_ptr: int, k_ptr: int, v_ptr: int, o_ptr: int, lse_ptr: int,
                    ws_ptr: int = 0, ws_bytes: int = 0, stream: int = 0, events=None) -> None:
    """ma_attn_forward_lse: the forward plus each row's softmax statistic
    (float32 [B*N*H]) for backward_saved_raw; events as for forward_raw.
    Raises RuntimeError on rejection."""
    if events:
        rc = LIB.ma_attn_forward_lse_timed(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, o_ptr, lse_ptr,
                                           ws_ptr or None, ws_bytes, stream or None, events[0] or None,
                                           events[1] or None)
    else:
        rc = LIB.ma_attn_forward_lse(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, o_ptr, lse_ptr, ws_ptr or None,
                                     ws_bytes, stream or None)
    if rc != 0:
        raise RuntimeError(last_error())


def backward_saved_raw(desc: Desc, q_ptr: int, k_ptr: int, v_ptr: int, o_ptr: int, lse_ptr: int, g_ptr: int,
                       dq_ptr: int, dk_ptr: int, dv_ptr: int, ws_ptr: int, ws_bytes: int, stream: int = 0,
                       events=None) -> None:
    """ma_attn_backward_saved: the backward from the forward's O and
    statistics.  Raises RuntimeError on rejection."""
    if events:
        rc = LIB.ma_attn_backward_saved_timed(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, o_ptr, lse_ptr, g_ptr,
                                              dq_ptr, dk_ptr, dv_ptr, ws_ptr or None, ws_bytes, stream or None,
                                              events[0] or None, events[1] or None)
    else:
        rc = LIB.ma_attn_backward_saved(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, o_ptr, lse_ptr, g_ptr, dq_ptr,
                                        dk_ptr, dv_ptr, ws_ptr or None, ws_bytes, stream or None)
    if rc != 0:
        raise RuntimeError(last_error())


def block_table(seed: int, num_blocks: int, random_per_row: int = 2) -> torch.Tensor:
    """Seeded int32 [num_blocks, 2 + random_per_row] table (CPU tensor)."""
    out = torch.empty((max(num_blocks, 0), 2 + random_per_row), dtype=torch.int32)
    rc = LIB.ma_attn_block_table(ctypes.c_uint64(int(seed) & (2**64 - 1)), int(num_blocks),
                                 int(random_per_row), out.data_ptr() if num_blocks > 0 else None)
    if rc != 0:
        raise ValueError(last_error())
    return out


def row_keys(desc: Desc, i: int, host_table: torch.Tensor | None = None) -> list:
    """Ascending key list S_i from the engine's closed forms (host side)."""
    cap = max(int(desc.seq_len), 1)
    buf = (ctypes.c_int64 * cap)()
    tptr = None
    if host_table is not None:
        host_table = host_table.to(torch.int32).contiguous()
        tptr = host_table.data_ptr()
    n = LIB.ma_attn_row_keys(ctypes.byref(desc), tptr, int(i), buf, cap)
    if n < 0:
        raise ValueError(last_error())
    return list(buf[:n])


def pattern_csr(desc: Desc, host_table: torch.Tensor | None = None):
    """Every row's key list of desc as CSR (host int64 offsets [N+1], int32
    keys), from the engine's closed forms in one call (ma_attn_pattern_csr)."""
    N = int(desc.seq_len)
    offsets = torch.empty(N + 1, dtype=torch.int64)
    tptr = None
    if host_table is not None:
        host_table = host_table.to(torch.int32).contiguous()
        tptr = host_table.data_ptr()
    nnz = LIB.ma_attn_pattern_csr(ctypes.byref(desc), tptr, offsets.data_ptr(), None, 0)
    if nnz < 0:
        raise ValueError(last_error())
    keys = torch.empty(max(int(nnz), 1), dtype=torch.int32)
    got = LIB.ma_attn_pattern_csr(ctypes.byref(desc), tptr, None, keys.data_ptr(), int(nnz))
    if got != nnz:
        raise ValueError(last_error())
    return offsets, keys[:nnz]


def tile_header_of(offsets: torch.Tensor, keys: torch.Tensor, seq_len: int, seg: int = 0) -> TileHeader:
    """Sizes of a CSR key set's tile plan (ma_attn_tile_plan without the plan)."""
    off = offsets.to(torch.int64).contiguous()
    kk = keys.to(torch.int32).contiguous()
    hdr = TileHeader()
    if LIB.ma_attn_tile_plan(int(seq_len), off.data_ptr(), kk.data_ptr() if kk.numel() else None, int(seg),
                             ctypes.byref(hdr), None, 0) != 0:
        raise ValueError(last_error())
    return hdr


def tile_plan(offsets: torch.Tensor, keys: torch.Tensor, seq_len: int, seg: int = 0):
    """The 64x64-tile plan of a CSR key set (host int64 offsets, int32 keys):
    (TileHeader, host uint8 tensor of header.total_bytes).  ma_attn_tile_plan."""
    off = offsets.to(torch.int64).contiguous()
    kk = keys.to(torch.int32).contiguous()
    hdr = TileHeader()
    kptr = kk.data_ptr() if kk.numel() else None
    if LIB.ma_attn_tile_plan(int(seq_len), off.data_ptr(), kptr, int(seg), ctypes.byref(hdr), None, 0) != 0:
        raise ValueError(last_error())
    blob = torch.empty(int(hdr.total_bytes), dtype=torch.uint8)
    if LIB.ma_attn_tile_plan(int(seq_len), off.data_ptr(), kptr, int(seg), ctypes.byref(hdr), blob.data_ptr(),
                             blob.numel()) != 0:
        raise ValueError(last_error())
    return hdr, blob


def forward_noalloc_raw(desc: Desc, q_ptr: int, k_ptr: int, v_ptr: int, o_ptr: int, stream: int = 0) -> None:
    """ma_attn_forward_noalloc: no workspace, no allocation (the library's
    static scratch).  Raises RuntimeError on rejection."""
    rc = LIB.ma_attn_forward_noalloc(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, o_ptr, stream or None)
    if rc != 0:
        raise RuntimeError(last_error())


def encoder_layer_forward_raw(layer: EncoderLayer, src_ptr: int, attn_ptr: int, out_ptr: int,
                              stream: int = 0) -> None:
    """ma_encoder_layer_forward (attn_ptr 0: the kernel computes the attention).
    Raises RuntimeError on rejection."""
    rc = LIB.ma_encoder_layer_forward(ctypes.byref(layer), src_ptr, attn_ptr or None, out_ptr, stream or None)
    if rc != 0:
        raise RuntimeError(last_error())


def copy_probe_raw(desc: Desc, q_ptr: int, k_ptr: int, v_ptr: int, o_ptr: int, stream: int = 0,
                   events=None) -> None:
    """ma_attn_copy_probe(_timed): a forward kernel's traffic without its arithmetic
    (SLIDING: the stream kernel's; BLOCK_SPARSE: the block-row kernel's)."""
    e0, e1 = events if events else (None, None)
    if LIB.ma_attn_copy_probe_timed(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, o_ptr, stream or None, e0 or None,
                                    e1 or None) != 0:
        raise RuntimeError(last_error())


def backward_copy_probe_raw(desc: Desc, q_ptr: int, k_ptr: int, v_ptr: int, dout_ptr: int, dq_ptr: int,
                            dk_ptr: int, dv_ptr: int, stream: int = 0, events=None) -> None:
    """ma_attn_backward_copy_probe(_timed): the fused backward's traffic without
    its arithmetic (dq = q xor dout, dk = k, dv = v bitwise)."""
    e0, e1 = events if events else (None, None)
    if LIB.ma_attn_backward_copy_probe_timed(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, dout_ptr, dq_ptr, dk_ptr,
                                             dv_ptr, stream or None, e0 or None, e1 or None) != 0:
        raise RuntimeError(last_error())


def reload_options() -> None:
    """Re-read the MA_ATTN_* kernel-selection switches from the environment."""
    LIB.ma_attn_reload_options()


NOALLOC_SCRATCH_BYTES = 8 << 20  # MA_ATTN_NOALLOC_SCRATCH_BYTES


def default_scale(D: int) -> float:
    """1.0f / sqrtf((float)D) in float32, as src/csrc/ma_core.cpp:188."""
    import numpy as np
    return float(np.float32(1.0) / np.sqrt(np.float32(D)))


__all__ = ["LIB", "Desc", "make_desc", "forward_raw", "forward_noalloc_raw", "validate", "workspace_size",
           "block_table", "row_keys", "pattern_csr", "copy_probe_raw", "backward_copy_probe_raw", "tile_plan", "tile_header_of", "TileHeader", "reload_options", "last_error", "EncoderLayer", "encoder_layer_forward_raw", "DTYPES", "default_scale",
           "SLIDING", "DENSE", "BLOCK_SPARSE", "LONGFORMER", "INDEX_SET", "F32", "BF16", "F16"]
