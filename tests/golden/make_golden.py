"""Write the golden vectors under tests/golden/ (run in the build container).

Outputs come from the reference's own CPU engine, ma_core.cpp + tensor.cpp
compiled unchanged into oracle/_ref/libma_core_ref.so (see oracle/Makefile),
so the committed numbers are the reference's bits, not this repo's:

  ref_sparse_s10_w2.npz   test_cpu_attention_cpp.py:42-56 case: torch.manual_seed(1),
                          B,S,H,D,W = 1,10,2,4,2, ma_core.compute_sparse_attention
  ref_sparse_s256_w64.npz (1,256,4,16) W=64, numpy PCG64 seed 7
  ref_sparse_s33_w0.npz   (2,33,2,16) W=0 (O must equal V)
  ref_dense_s32.npz       (1,32,2,16) causal and non-causal compute_dense_attention
  ref_value_dim.npz       a value head_dim of its own: q, k (1,40,2,16), v_<Dv> (1,40,2,Dv)
                          for Dv in 8, 24, 40 (numpy PCG64 seed 10); o_sparse_<Dv> from
                          compute_sparse_attention(w=5), o_dense_<Dv> / o_causal_<Dv> from
                          compute_dense_attention
  ref_patterns.npz        nnz of create_sliding_window_pattern for
                          (4,4), (4,10), (16,3), (2,1), (1024,64), and the (row, col)
                          entries for the small (N, w) cases listed in `small`
  ref_pattern_stats.json  get_pattern_statistics strings of sliding patterns
  block_table_seed1234_nb256_r2.bin  int32 [256,4]: the frozen block table of the
                          block-sparse config (seed 1234, 2 random blocks per row),
                          from oracle.block_table (SplitMix64 spec in oracle.c)
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import oracle as O  # noqa: E402


def main():
    O.build()
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libma_core_ref.so not built (needs /root/reference)")
    import torch

    torch.manual_seed(1)
    q = torch.randn(1, 10, 2, 4, dtype=torch.float32).numpy()
    k = torch.randn(1, 10, 2, 4, dtype=torch.float32).numpy()
    v = torch.randn(1, 10, 2, 4, dtype=torch.float32).numpy()
    np.savez(os.path.join(HERE, "ref_sparse_s10_w2.npz"), q=q, k=k, v=v, w=np.int64(2),
             o=O.ref_sparse_forward(q, k, v, 2))

    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, 256, 4, 16), dtype=np.float32) for _ in range(3))
    np.savez(os.path.join(HERE, "ref_sparse_s256_w64.npz"), q=q, k=k, v=v, w=np.int64(64),
             o=O.ref_sparse_forward(q, k, v, 64))

    rng = np.random.default_rng(8)
    q, k, v = (rng.standard_normal((2, 33, 2, 16), dtype=np.float32) for _ in range(3))
    np.savez(os.path.join(HERE, "ref_sparse_s33_w0.npz"), q=q, k=k, v=v, w=np.int64(0),
             o=O.ref_sparse_forward(q, k, v, 0))

    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((1, 32, 2, 16), dtype=np.float32) for _ in range(3))
    np.savez(os.path.join(HERE, "ref_dense_s32.npz"), q=q, k=k, v=v,
             o_full=O.ref_dense_forward(q, k, v, False), o_causal=O.ref_dense_forward(q, k, v, True))

    write_value_dim()

    cases = np.array([(4, 4), (4, 10), (16, 3), (2, 1), (1024, 64)], dtype=np.int64)
    nnz = np.array([len(O.ref_sliding_pattern(int(n), int(w))[0]) for n, w in cases], dtype=np.int64)
    # the COO entries themselves, in the reference's order, for the small cases
    small = np.array([(4, 4), (4, 10), (16, 3), (2, 1), (8, 2), (5, 0), (6, -1)], dtype=np.int64)
    coo = {}
    for n, w in small:
        r, c = O.ref_sliding_pattern(int(n), int(w))
        coo[f"rows_{n}_{w}"], coo[f"cols_{n}_{w}"] = r, c
    np.savez(os.path.join(HERE, "ref_patterns.npz"), cases=cases, nnz=nnz, small=small, **coo)

    # get_pattern_statistics strings (ma_core.cpp:51-63) of create_sliding_window_pattern
    stats = {f"{n},{w}": O.ref_pattern_statistics(n, w)
             for n, w in ((16, 3), (4, 4), (8, 1), (1024, 64), (7, 2), (100, 10))}
    with open(os.path.join(HERE, "ref_pattern_stats.json"), "w") as f:
        json.dump(stats, f, indent=1, sort_keys=True)

    O.block_table(1234, 256, 2).astype("<i4").tofile(
        os.path.join(HERE, "block_table_seed1234_nb256_r2.bin"))
    print("golden vectors written to", HERE)


def write_value_dim():
    """ref_value_dim.npz: the reference's outputs when V's head_dim differs from Q's."""
    rng = np.random.default_rng(10)
    q, k = (rng.standard_normal((1, 40, 2, 16), dtype=np.float32) for _ in range(2))
    out = dict(q=q, k=k, w=np.int64(5))
    for dv in (8, 24, 40):
        v = rng.standard_normal((1, 40, 2, dv), dtype=np.float32)
        out[f"v_{dv}"] = v
        out[f"o_sparse_{dv}"] = O.ref_forward_v(q, k, v, window=5)
        out[f"o_dense_{dv}"] = O.ref_forward_v(q, k, v, causal=False)
        out[f"o_causal_{dv}"] = O.ref_forward_v(q, k, v, causal=True)
    np.savez(os.path.join(HERE, "ref_value_dim.npz"), **out)


if __name__ == "__main__":
    main()
