"""Drop-in for the reference's GPU extension module ``sparse_attention_cuda``.

Same import name, functions, signatures and defaults as the reference's
pybind module (/root/reference src/cuda/sparse_attention_kernel.cu:501-510):

    forward(query, key, value, window_size=64) -> Tensor
    dense_forward(query, key, value, use_causal_mask=False) -> Tensor
    backward(query, key, value, grad_out, window_size=64) -> [dQ, dK, dV]
    dense_backward(query, key, value, grad_out, use_causal_mask=False) -> [dQ, dK, dV]

and the same input contract as its TORCH_CHECKs (:427-432): device tensors,
one dtype, contiguous, identical 4-D [B, S, H, D] shapes, else RuntimeError.
The dtype set is widened from float32 to float32 / bfloat16 / float16; the
output has the input dtype.  Kernels run asynchronously on the current HIP
stream (torch.cuda.current_stream(), as :450 uses the current CUDA stream).

New pattern entry points (not in the reference; the benchmark patterns):

    sliding_forward(q, k, v, left, right, dilation=1)
    block_sparse_forward(q, k, v, block_table, block_size=64)
    BlockTable(block_table, seq_len, block_size=64)   (checked once, on the device)
    longformer_forward(q, k, v, left, right=0, num_global=16)
    longformer_backward(q, k, v, grad_out, left, right=0, num_global=16, out=, lse=)
    make_block_table(seed, num_blocks, random_per_row=2)
    index_set_forward(q, k, v, index_set)              (explicit key set per query row)
    IndexSet(offsets, keys, seq_len), IndexSet.from_coo(rows, cols, seq_len)

Forward and backward are hand-written HIP kernels (libma_attn.so).  The
backward recomputes the softmax from q, k, v as the reference's does, for the
sliding and dense patterns, in the input dtype (index sets, block-sparse and
Longformer have backward entry points of their own: index_set_backward,
longformer_backward):

    sliding_backward(q, k, v, grad_out, left, right, dilation=1) -> [dQ, dK, dV]
"""
from __future__ import annotations

import ctypes
from typing import List

import torch

import ma_attn as _ma

__all__ = ["forward", "dense_forward", "backward", "dense_backward", "sliding_forward",
           "sliding_backward", "block_sparse_forward", "longformer_forward", "longformer_backward",
           "make_block_table", "BlockTable", "IndexSet", "index_set_forward", "index_set_backward",
           "pattern_index_set"]


def _check(*ts: torch.Tensor) -> None:
    """The reference's TORCH_CHECKs (sparse_attention_kernel.cu:427-432) as RuntimeError."""
    # one pass for the common valid call; any failure takes the ordered checks below
    try:
        t0 = ts[0]
        dt, shape, dev = t0.dtype, t0.shape, t0.get_device()
        ok = dt in _ma.DTYPES and len(shape) == 4 and dev >= 0
        for t in ts:
            ok = ok and t.get_device() == dev and t.dtype == dt and t.shape == shape and t.is_contiguous()
        if ok and all(isinstance(t, torch.Tensor) for t in ts):
            return
    except (AttributeError, TypeError):
        pass
    for t in ts:
        if not isinstance(t, torch.Tensor):
            raise RuntimeError("Inputs must be tensors")
    if not all(t.is_cuda for t in ts):
        raise RuntimeError("Inputs must be CUDA (HIP) device tensors")
    dt = ts[0].dtype
    if dt not in _ma.DTYPES or any(t.dtype != dt for t in ts):
        raise RuntimeError("Inputs must share one dtype among float32, bfloat16, float16")
    if not all(t.is_contiguous() for t in ts):
        raise RuntimeError("Inputs must be contiguous")
    if any(t.shape != ts[0].shape for t in ts):
        raise RuntimeError("Q,K,V must have same shape")
    if ts[0].dim() != 4:
        raise RuntimeError("Expected shape [B, S, H, D]")
    dev = ts[0].device
    if any(t.device != dev for t in ts):
        raise RuntimeError("Inputs must be on one device")


# (start, stop) torch.cuda.Event pair for the next launch, set by kernel_events()
_events = None


class kernel_events:
    """Context manager: the forward / backward calls inside it stamp the
    kernels' own start and stop on two torch.cuda.Event(enable_timing=True)
    (already recorded once, so that they exist), without adding commands
    between launches.  ``start.elapsed_time(stop)`` is then the kernels'
    execution time of the last call inside the block."""

    def __init__(self, start: torch.cuda.Event, stop: torch.cuda.Event):
        self.pair = (start.cuda_event, stop.cuda_event)

    def __enter__(self):
        global _events
        _events = self.pair
        return self

    def __exit__(self, *exc):
        global _events
        _events = None
        return False


# Host path per call: descriptors (and their workspace sizes) are cached per
# call signature; the launch stream is read as a raw handle, and the device
# is switched only when the inputs are not on the current one.
_desc_cache: dict = {}
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_current_device = getattr(torch._C, "_cuda_getDevice", None)


def _desc_of(B, N, H, D, dtype, pattern, kw, backward=False):
    key = (B, N, H, D, dtype, pattern, backward, tuple(sorted(kw.items())))
    hit = _desc_cache.get(key)
    if hit is None:
        if len(_desc_cache) > 512:
            _desc_cache.clear()
        desc = _ma.make_desc(B, N, H, D, _ma.DTYPES[dtype], pattern, **kw)
        nbytes = _ma.backward_workspace_size(desc) if backward else _ma.workspace_size(desc)
        hit = _desc_cache[key] = (desc, nbytes)
    return hit


def _on_device(dev: int, fn):
    """Run fn(stream) with dev current and its current stream's raw handle."""
    if _raw_stream is not None and _current_device is not None and _current_device() == dev:
        return fn(_raw_stream(dev))
    with torch.cuda.device(dev):
        return fn(torch.cuda.current_stream(dev).cuda_stream)


def _launch(q, k, v, pattern, return_lse: bool = False, **kw):
    _check(q, k, v)
    B, N, H, D = q.shape
    out = torch.empty_like(q)
    desc, nbytes = _desc_of(B, N, H, D, q.dtype, pattern, kw)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    if return_lse:
        lse = torch.empty((B, N, H), dtype=torch.float32, device=q.device)
        _on_device(q.get_device(), lambda stream: _ma.forward_lse_raw(
            desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
            ws.data_ptr() if ws is not None else 0, nbytes, stream, _events))
        return out, lse
    _on_device(q.get_device(), lambda stream: _ma.forward_raw(
        desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), ws.data_ptr() if ws is not None else 0,
        nbytes, stream, _events))
    return out


def forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
            window_size: int = 64) -> torch.Tensor:
    """Sliding-window forward over keys [max(0,i-w), min(S,i+w+1)).

    Reference: sparse_forward_cuda (sparse_attention_kernel.cu:423-458).
    w = 0 gives O = V; w < 0 gives an empty window and O = 0 (:232-238).
    """
    w = int(window_size)
    return _launch(query, key, value, _ma.SLIDING, left=w, right=w, dilation=1)


def _scale_kw(scale) -> dict:
    """The descriptor's softmax scale: None keeps 1/sqrtf(head_dim)."""
    if scale is None:
        return {}
    s = float(scale)
    if not (s > 0.0 and s != float("inf")):
        raise RuntimeError("scale must be finite and > 0")
    return {"scale": s}


def dense_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                  use_causal_mask: bool = False, return_lse: bool = False, scale=None):
    """Dense (optionally causal) forward.  Reference: dense_forward_cuda (:348-382).
    return_lse: also return each row's softmax statistic (float32 [B, S, H])
    for dense_backward(..., out=, lse=); head_dim 64.
    scale: softmax scale (None: 1/sqrtf(head_dim), as the reference)."""
    return _launch(query, key, value, _ma.DENSE, return_lse, causal=bool(use_causal_mask), **_scale_kw(scale))


def sliding_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                    left: int, right: int, dilation: int = 1, scale=None) -> torch.Tensor:
    """Keys {i + dilation*t : -left <= t <= right} inside [0, S).

    causal window w: left=w-1, right=0; the reference's symmetric w: left=right=w.
    scale: softmax scale (None: 1/sqrtf(head_dim)).
    """
    return _launch(query, key, value, _ma.SLIDING, left=int(left), right=int(right),
                   dilation=int(dilation), **_scale_kw(scale))


def make_block_table(seed: int, num_blocks: int, random_per_row: int = 2) -> torch.Tensor:
    """Seeded int32 [num_blocks, 2 + random_per_row] block table (host tensor)."""
    return _ma.block_table(seed, num_blocks, random_per_row)


def _validated_table(block_table: torch.Tensor, nb: int) -> torch.Tensor:
    """Host int32 copy of block_table after the layout checks the kernels rely on."""
    if not isinstance(block_table, torch.Tensor):
        raise RuntimeError("block_table must be a tensor")
    if block_table.dim() != 2 or block_table.shape[0] != nb:
        raise RuntimeError(f"block_table must be [ceil(S/block_size)={nb}, width]")
    if block_table.shape[1] < 1 or block_table.shape[1] > 64:
        raise RuntimeError("block_table width must be in [1, 64]")
    tab_cpu = block_table.detach().to("cpu", torch.int32)
    if (tab_cpu >= nb).any() or (tab_cpu < -1).any():
        raise RuntimeError("block_table entries must be -1 or in [0, num_blocks)")
    valid = tab_cpu >= 0
    # padding last: once an entry is -1, every later entry of the row is -1
    if (valid[:, 1:] & ~valid[:, :-1]).any():
        raise RuntimeError("block_table rows must hold their -1 padding after the valid entries")
    # strictly ascending among valid entries
    if ((tab_cpu[:, 1:] <= tab_cpu[:, :-1]) & valid[:, 1:]).any():
        raise RuntimeError("block_table rows must be strictly ascending")
    return tab_cpu.contiguous()


class BlockTable:
    """A block table checked once and kept on the device, for repeated calls.

    block_sparse_forward checks a plain tensor table on the host at every
    call (a device-to-host copy and a few host reductions); a BlockTable
    carries the checked device copy, so a call with it only launches.
    """

    def __init__(self, block_table: torch.Tensor, seq_len: int, block_size: int = 64, device=None):
        self.seq_len = int(seq_len)
        self.block_size = int(block_size)
        if self.block_size < 1:
            raise RuntimeError("block_size must be >= 1")
        nb = (self.seq_len + self.block_size - 1) // self.block_size
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.host = _validated_table(block_table, nb)  # checked host copy (index enumeration)
        self.tensor = self.host.to(dev)
        self._index_set = None  # the table's key sets as an IndexSet, built on first use

    @property
    def width(self) -> int:
        return int(self.tensor.shape[1])


def block_sparse_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                         block_table, block_size: int = 64, return_lse: bool = False):
    """Query block r attends the key blocks listed in block_table[r] (ascending, -1 padded).

    block_table: an int tensor [ceil(S/block_size), width] (checked at every
    call), or a BlockTable made for this sequence length and block size.
    return_lse: also return each row's softmax statistic (float32 [B, S, H],
    ma_attn_forward_lse) for index_set_backward(..., out=, lse=); block size 64,
    head_dim 64.
    """
    _check(query, key, value)
    B, N, H, D = query.shape
    bs = int(block_size)
    if bs < 1:
        raise RuntimeError("block_size must be >= 1")
    nb = (N + bs - 1) // bs
    if isinstance(block_table, BlockTable):
        if block_table.seq_len != N or block_table.block_size != bs:
            raise RuntimeError(f"BlockTable was made for S={block_table.seq_len}, block_size="
                               f"{block_table.block_size}; called with S={N}, block_size={bs}")
        if block_table.tensor.device != query.device:
            raise RuntimeError("BlockTable is on another device than the inputs")
        tab = block_table.tensor
    else:
        # Allocated on the current stream; the caching allocator reuses its
        # memory only for later work on that same stream, i.e. after the
        # kernel read it.
        tab = _validated_table(block_table, nb).to(query.device)
    return _launch(query, key, value, _ma.BLOCK_SPARSE, return_lse, block_size=bs,
                   block_table_ptr=tab.data_ptr(), blocks_per_row=tab.shape[1])


def longformer_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                       left: int, right: int = 0, num_global: int = 16, return_lse: bool = False):
    """Rows i < G attend all keys; others attend [i-left, i+right] U [0, G).
    return_lse as for block_sparse_forward (1 <= G <= 16, head_dim 64)."""
    return _launch(query, key, value, _ma.LONGFORMER, return_lse, left=int(left), right=int(right),
                   num_global=int(num_global))


def _validated_index_set(offsets, keys, seq_len: int):
    """Host int64 offsets and int32 keys after the layout checks of an index set:
    offsets [S+1] non-decreasing from 0 to len(keys); keys in [0, S), strictly
    ascending within each row."""
    if not isinstance(offsets, torch.Tensor) or not isinstance(keys, torch.Tensor):
        raise RuntimeError("index set offsets and keys must be tensors")
    off = offsets.detach().to("cpu", torch.int64).contiguous()
    kk = keys.detach().to("cpu", torch.int64).contiguous()
    N = int(seq_len)
    if off.dim() != 1 or off.numel() != N + 1:
        raise RuntimeError(f"index set offsets must be [S+1={N + 1}]")
    if kk.dim() != 1:
        raise RuntimeError("index set keys must be 1-D")
    nnz = kk.numel()
    if int(off[0]) != 0 or int(off[-1]) != nnz or bool((off[1:] < off[:-1]).any()):
        raise RuntimeError("index set offsets must run non-decreasing from 0 to len(keys)")
    if nnz and (bool((kk < 0).any()) or bool((kk >= N).any())):
        raise RuntimeError(f"index set keys must lie in [0, S={N})")
    if nnz > 1:
        bad = kk[1:] <= kk[:-1]
        starts = off[1:N]
        starts = starts[(starts > 0) & (starts < nnz)]
        bad[starts - 1] = False  # a new row may restart low
        if bool(bad.any()):
            raise RuntimeError("index set rows must be strictly ascending (each key once)")
    return off, kk.to(torch.int32)


class IndexSet:
    """An explicit key set per query row (CSR), checked once and kept on the device.

    Row i attends keys[offsets[i]:offsets[i+1]] in every (batch, head): the
    reference's generic COO attention (src/csrc/sparse_attention.cpp:11-152)
    with one pattern for all of them.  ``from_coo`` takes the reference's
    (row, col) entry lists and drops repeated entries.
    """

    def __init__(self, offsets: torch.Tensor, keys: torch.Tensor, seq_len: int, device=None, tiles="auto",
                 tile_seg: int = 0):
        """tiles: "auto" builds the set's 64x64 tile plan (the tiled MFMA
        kernels, head_dim 64) when the set's keys cluster in blocks -- at
        least 1/16 of each touched 64x64 block on average; True always
        builds it, False never (the gather kernels).  tile_seg: blocks per
        work item of the tiled kernels (0: the library's default)."""
        self.seq_len = int(seq_len)
        off, kk = _validated_index_set(offsets, keys, self.seq_len)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.tile_header = self.tile_plan = None
        if tiles and self.seq_len > 0:
            hdr = _ma.tile_header_of(off, kk, self.seq_len, tile_seg)
            dense_work = hdr.num_entries * 4096
            if tiles is True or (dense_work <= 16 * max(int(kk.numel()), 1) and hdr.total_bytes <= (512 << 20)):
                self.tile_header, blob = _ma.tile_plan(off, kk, self.seq_len, tile_seg)
                self.tile_plan = blob.to(dev)
        self.offsets = off.to(dev)
        self.keys = (kk if kk.numel() else torch.zeros(1, dtype=torch.int32)).to(dev)
        self.num_indices = int(kk.numel())
        # the transposed set (for each key, the queries that list it, ascending),
        # which the backward's dK/dV pass walks
        N = self.seq_len
        rows = torch.repeat_interleave(torch.arange(N, dtype=torch.int64), off[1:] - off[:-1])
        order = torch.sort(kk.long(), stable=True).indices
        t_off = torch.zeros(N + 1, dtype=torch.int64)
        t_off[1:] = torch.cumsum(torch.bincount(kk.long(), minlength=N)[:N], 0) if kk.numel() else 0
        t_q = rows[order].to(torch.int32)
        self.t_offsets = t_off.to(dev)
        self.t_queries = (t_q if t_q.numel() else torch.zeros(1, dtype=torch.int32)).to(dev)

    def _tile_kw(self) -> dict:
        if self.tile_plan is None:
            return {}
        return dict(tile_header_ptr=ctypes.addressof(self.tile_header), tile_plan_ptr=self.tile_plan.data_ptr())

    @staticmethod
    def from_coo(rows, cols, seq_len: int, device=None) -> "IndexSet":
        r = torch.as_tensor(rows, dtype=torch.int64).reshape(-1)
        c = torch.as_tensor(cols, dtype=torch.int64).reshape(-1)
        N = int(seq_len)
        if r.numel() != c.numel():
            raise RuntimeError("rows and cols must have the same length")
        if r.numel() and (bool((r < 0).any()) or bool((r >= N).any())):
            raise RuntimeError(f"rows must lie in [0, S={N})")
        pairs = torch.unique(r * max(N, 1) + c) if r.numel() else r  # sorted by (row, col), repeats dropped
        rr, cc = pairs // max(N, 1), pairs % max(N, 1)
        offsets = torch.zeros(N + 1, dtype=torch.int64)
        offsets[1:] = torch.cumsum(torch.bincount(rr, minlength=N)[:N], 0)
        return IndexSet(offsets, cc, N, device)


_pattern_sets: dict = {}


def _enumerated_set(code: int, seq_len: int, device, host_table=None, **kw) -> "IndexSet":
    tptr = host_table.data_ptr() if host_table is not None else 0  # host pointer: enumeration only
    if host_table is not None:
        kw["blocks_per_row"] = int(host_table.shape[1])
    desc = _ma.make_desc(1, seq_len, 1, 64, _ma.F32, code, block_table_ptr=tptr, **kw)
    offsets, keys = _ma.pattern_csr(desc, host_table)
    return IndexSet(offsets, keys, seq_len, device)


def pattern_index_set(pattern: str, seq_len: int, device, **kw) -> IndexSet:
    """The key sets of a closed-form pattern ("block_sparse" with block_table=
    and block_size=, "longformer" with left=, right=, num_global=) as an
    IndexSet, from the engine's own enumerator (ma_attn_pattern_csr), so its
    backward (index_set_backward) is the exact gradient of that pattern's
    forward.  A BlockTable keeps its set (built on first use, no host transfer
    after that); Longformer sets are cached per geometry and device; a plain
    tensor table is copied to the host at every call (from the device, a
    synchronising copy) and its set is cached on the table's contents."""
    if pattern == "block_sparse":
        table = kw.pop("block_table")
        bs = int(kw.pop("block_size", 64))
        if isinstance(table, BlockTable):
            if table.seq_len != seq_len or table.block_size != bs:
                raise RuntimeError("BlockTable was made for another sequence length or block size")
            hit = table._index_set
            if hit is None or hit.offsets.device != torch.device(device):
                hit = table._index_set = _enumerated_set(_ma.BLOCK_SPARSE, seq_len, device, table.host,
                                                         block_size=bs)
            return hit
        nb = (int(seq_len) + bs - 1) // bs
        host = _validated_table(torch.as_tensor(table), nb)
        key = ("block_sparse", int(seq_len), bs, str(device), tuple(host.shape), host.numpy().tobytes())
        hit = _pattern_sets.get(key)
        if hit is None:
            if len(_pattern_sets) > 16:
                _pattern_sets.clear()
            hit = _pattern_sets[key] = _enumerated_set(_ma.BLOCK_SPARSE, seq_len, device, host, block_size=bs)
        return hit
    if pattern != "longformer":
        raise ValueError(f"no closed-form index set for pattern {pattern!r}")
    key = (int(seq_len), str(device), tuple(sorted(kw.items())))
    hit = _pattern_sets.get(key)
    if hit is None:
        if len(_pattern_sets) > 16:
            _pattern_sets.clear()
        hit = _pattern_sets[key] = _enumerated_set(_ma.LONGFORMER, seq_len, device, **kw)
    return hit


def index_set_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                      index_set, return_lse: bool = False):
    """Query i attends exactly the keys of row i of index_set (an IndexSet, or
    an (offsets, keys) pair checked at every call).  Empty rows give zeros.
    return_lse as for block_sparse_forward (a set with a tile plan)."""
    _check(query, key, value)
    B, N, H, D = query.shape
    if not isinstance(index_set, IndexSet):
        offsets, keys = index_set
        index_set = IndexSet(offsets, keys, N, query.device)
    if index_set.seq_len != N:
        raise RuntimeError(f"IndexSet was made for S={index_set.seq_len}; called with S={N}")
    if index_set.offsets.device != query.device:
        raise RuntimeError("IndexSet is on another device than the inputs")
    return _launch(query, key, value, _ma.INDEX_SET, return_lse, index_offsets_ptr=index_set.offsets.data_ptr(),
                   index_keys_ptr=index_set.keys.data_ptr(), num_indices=index_set.num_indices,
                   **index_set._tile_kw())


def index_set_backward(query, key, value, grad_out, index_set, out=None, lse=None) -> List[torch.Tensor]:
    """dQ, dK, dV of index_set_forward (tiled kernels with a tile plan, gather
    kernels otherwise at head_dim 64, row kernels at other head_dims; the
    reference's generic COO path has no backward).  index_set as for
    index_set_forward.

    out, lse: the forward's output and statistics (a forward with
    return_lse=True over the same key sets: index_set_forward, or
    block_sparse_forward / longformer_forward for their pattern_index_set).
    With both, a set with a tile plan skips recomputing the softmax
    statistics (ma_attn_backward_saved); without a plan they are ignored."""
    _check(query, key, value, grad_out)
    N = query.shape[1]
    if not isinstance(index_set, IndexSet):
        offsets, keys = index_set
        index_set = IndexSet(offsets, keys, N, query.device)
    if index_set.seq_len != N:
        raise RuntimeError(f"IndexSet was made for S={index_set.seq_len}; called with S={N}")
    if index_set.offsets.device != query.device:
        raise RuntimeError("IndexSet is on another device than the inputs")
    kw = dict(index_offsets_ptr=index_set.offsets.data_ptr(), index_keys_ptr=index_set.keys.data_ptr(),
              num_indices=index_set.num_indices, index_t_offsets_ptr=index_set.t_offsets.data_ptr(),
              index_t_queries_ptr=index_set.t_queries.data_ptr(), **index_set._tile_kw())
    if out is not None and lse is not None and index_set.tile_plan is not None:
        _check(query, out)
        _check_lse(lse, query)
        return _backward_saved(query, key, value, out, lse, grad_out, _ma.INDEX_SET, **kw)
    return _backward(query, key, value, grad_out, _ma.INDEX_SET, **kw)


# ---------------------------------------------------------------- backward (HIP kernels)

def _check_lse(lse, query) -> None:
    B, N, H, _ = query.shape
    if not (isinstance(lse, torch.Tensor) and lse.dtype == torch.float32 and lse.is_contiguous()
            and tuple(lse.shape) == (B, N, H) and lse.device == query.device):
        raise RuntimeError(f"lse must be a contiguous float32 [{B}, {N}, {H}] tensor on the inputs' device")


def _backward_saved(q, k, v, out, lse, grad_out, pattern, **kw) -> List[torch.Tensor]:
    B, N, H, D = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    desc, nbytes = _desc_of(B, N, H, D, q.dtype, pattern, kw, backward=True)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    _on_device(q.get_device(), lambda stream: _ma.backward_saved_raw(
        desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(), grad_out.data_ptr(),
        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), nbytes, stream, _events))
    return [dq, dk, dv]


def _backward(q, k, v, grad_out, pattern, **kw) -> List[torch.Tensor]:
    _check(q, k, v, grad_out)
    B, N, H, D = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    desc, nbytes = _desc_of(B, N, H, D, q.dtype, pattern, kw, backward=True)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    _on_device(q.get_device(), lambda stream: _ma.backward_raw(
        desc, q.data_ptr(), k.data_ptr(), v.data_ptr(), grad_out.data_ptr(), dq.data_ptr(), dk.data_ptr(),
        dv.data_ptr(), ws.data_ptr(), nbytes, stream, _events))
    return [dq, dk, dv]


def longformer_fused_applies(query, left: int, right: int, num_global: int) -> bool:
    """Whether longformer_backward's one-pass kernel (ma_attn_backward_saved on
    a LONGFORMER descriptor) takes this call: bf16/fp16, head_dim 64, window
    [i-left, i] with left <= 127, 1 to 16 global tokens, 16-byte aligned tensors."""
    return (query.dtype in (torch.bfloat16, torch.float16) and query.dim() == 4 and query.shape[3] == 64
            and int(right) == 0 and 0 <= int(left) < 128 and 1 <= int(num_global) <= 16)


def longformer_backward(query, key, value, grad_out, left: int, right: int = 0, num_global: int = 16,
                        out=None, lse=None) -> List[torch.Tensor]:
    """dQ, dK, dV of longformer_forward.

    For a window [i-left, i] (left <= 127, 1 to 16 global tokens, 16-bit,
    head_dim 64, 16-byte aligned tensors) one pass over the sequence
    (bwd_lf_kernel):
    - with out and lse (longformer_forward(..., return_lse=True)): from the
      forward's output and statistics, delta = dO . O with the 16-bit O
      (ma_attn_backward_saved);
    - without them: ma_attn_backward on the LONGFORMER descriptor, which runs
      the forward first for each row's statistic and
      delta = sum_j P_ij dP_ij (dP_ij = dO_i . V_j, fp32; no O written), then
      the same pass.
    Otherwise the tiled kernels over the pattern's key sets (index_set_backward
    on pattern_index_set)."""
    _check(query, key, value, grad_out)
    N = query.shape[1]
    kw = dict(left=int(left), right=int(right), num_global=int(num_global))
    if longformer_fused_applies(query, left, right, num_global) and all(
            t.data_ptr() % 16 == 0 for t in (query, key, value, grad_out)):
        if out is None or lse is None:
            return _backward(query, key, value, grad_out, _ma.LONGFORMER, **kw)
        if out.data_ptr() % 16 == 0:
            _check(query, out)
            _check_lse(lse, query)
            return _backward_saved(query, key, value, out, lse, grad_out, _ma.LONGFORMER, **kw)
    iset = pattern_index_set("longformer", N, query.device, **kw)
    return index_set_backward(query, key, value, grad_out, iset, out=out, lse=lse)


def backward(query, key, value, grad_out, window_size: int = 64) -> List[torch.Tensor]:
    """dQ, dK, dV of forward(); reference sparse_backward_cuda (.cu:459-497, kernel :265-346)."""
    w = int(window_size)
    return _backward(query, key, value, grad_out, _ma.SLIDING, left=w, right=w, dilation=1)


def dense_backward(query, key, value, grad_out, use_causal_mask: bool = False, out=None,
                   lse=None) -> List[torch.Tensor]:
    """dQ, dK, dV of dense_forward(); reference dense_backward_cuda (.cu:383-418, kernel :104-175).
    out, lse: the forward's output and statistics (dense_forward(return_lse=True));
    with both, the dQ pass skips recomputing the statistics (ma_attn_backward_saved)."""
    if out is not None and lse is not None:
        _check(query, key, value, grad_out, out)
        _check_lse(lse, query)
        return _backward_saved(query, key, value, out, lse, grad_out, _ma.DENSE, causal=bool(use_causal_mask))
    return _backward(query, key, value, grad_out, _ma.DENSE, causal=bool(use_causal_mask))


def sliding_backward(query, key, value, grad_out, left: int, right: int,
                     dilation: int = 1) -> List[torch.Tensor]:
    """dQ, dK, dV of sliding_forward() (keys {i + dilation*t : -left <= t <= right})."""
    return _backward(query, key, value, grad_out, _ma.SLIDING, left=int(left), right=int(right),
                     dilation=int(dilation))
