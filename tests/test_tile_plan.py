"""The 64x64-tile plan of an explicit key set (ma_attn_tile_plan, host side):
entries, row and column masks, full flags and work items against a
brute-force construction from the set's (row, key) pairs."""
import numpy as np
import pytest
import torch

FULL = 1 << 30


def _csr(rng, N, density, full_rows=0, full_cols=0):
    m = rng.random((N, N)) < density
    if full_rows:
        m[rng.choice(N, full_rows, replace=False)] = True
    if full_cols:
        m[:, rng.choice(N, full_cols, replace=False)] = True
    off = np.zeros(N + 1, np.int64)
    off[1:] = np.cumsum(m.sum(1))
    return m, off, np.nonzero(m)[1].astype(np.int32)


def _plan(N, off, keys, seg=0):
    import ma_attn
    hdr, blob = ma_attn.tile_plan(torch.from_numpy(off), torch.from_numpy(keys), N, seg)
    b = blob.numpy()
    arr = lambda o, n, dt: np.frombuffer(b[o:o + n * np.dtype(dt).itemsize].tobytes(), dtype=dt)
    ne = hdr.num_entries
    return hdr, dict(blk=arr(hdr.off_blk, ne, np.int32), mask=arr(hdr.off_mask, 64 * ne, np.uint64).reshape(ne, 64),
                     kmask=arr(hdr.off_kmask, 64 * ne, np.uint64).reshape(ne, 64), tile=arr(hdr.off_tile, ne, np.int32),
                     kentry=arr(hdr.off_kentry, ne, np.int32),
                     q_items=arr(hdr.off_q_items, 4 * hdr.num_q_items, np.int32).reshape(-1, 4),
                     q_split=arr(hdr.off_q_split, 4 * hdr.num_q_split, np.int32).reshape(-1, 4),
                     k_items=arr(hdr.off_k_items, 4 * hdr.num_k_items, np.int32).reshape(-1, 4),
                     k_split=arr(hdr.off_k_split, 4 * hdr.num_k_split, np.int32).reshape(-1, 4))


def _check_items(items, split, ids, nt, seg, ranges, nparts):
    """Every tile (key block) has its entry range covered exactly once, in
    runs of at most seg; split ones through consecutive partial slots."""
    seen_slots = []
    by_id = {}
    for it in items:
        by_id.setdefault(int(it[0]), []).append(it)
    assert sorted(by_id) == list(range(nt))
    sp = {int(s[0]): s for s in split}
    for t in range(nt):
        its = by_id[t]
        a, b = ranges[t]
        if len(its) == 1 and t not in sp:
            assert (its[0][1], its[0][2], its[0][3]) == (a, b, -1)
            assert b - a <= seg
        else:
            s = sp[t]
            assert s[2] == len(its) and all(b_ - a_ <= seg for _, a_, b_, _ in its)
            assert [int(i[3]) for i in its] == list(range(s[1], s[1] + s[2]))
            seen_slots += [int(i[3]) for i in its]
        assert its[0][1] == a and its[-1][2] == b
        assert all(its[j][2] == its[j + 1][1] for j in range(len(its) - 1))
    assert sorted(seen_slots) == list(range(nparts))


@pytest.mark.parametrize("N,density,fr,fc,seg", [(200, 0.05, 0, 0, 0), (130, 0.3, 3, 3, 2), (64, 1.0, 0, 0, 0),
                                                 (700, 0.02, 4, 4, 3), (1, 1.0, 0, 0, 0), (65, 0.0, 0, 0, 0)])
def test_tile_plan_matches_brute_force(N, density, fr, fc, seg):
    rng = np.random.default_rng(N + fr)
    m, off, keys = _csr(rng, N, density, fr, fc)
    hdr, p = _plan(N, off, keys, seg)
    nt = (N + 63) // 64
    assert hdr.seq_len == N and hdr.num_tiles == nt and hdr.seg == (seg or 32)
    # entries: exactly the (tile, block) pairs with a key, ordered by tile then block
    pairs = sorted({(i // 64, j // 64) for i, j in zip(*np.nonzero(m))})
    blk = p["blk"] & (FULL - 1)
    assert list(zip(p["tile"].tolist(), blk.tolist())) == pairs
    for e, (t, c) in enumerate(pairs):
        sub = np.zeros((64, 64), bool)
        r1, k1 = min(N, 64 * t + 64) - 64 * t, min(N, 64 * c + 64) - 64 * c
        sub[:r1, :k1] = m[64 * t:64 * t + r1, 64 * c:64 * c + k1]
        rows = np.array([sum(1 << int(k) for k in np.nonzero(sub[r])[0]) for r in range(64)], dtype=np.uint64)
        cols = np.array([sum(1 << int(r) for r in np.nonzero(sub[:, k])[0]) for k in range(64)], dtype=np.uint64)
        assert np.array_equal(p["mask"][e], rows) and np.array_equal(p["kmask"][e], cols), e
        assert bool(p["blk"][e] & FULL) == bool(sub.all() and r1 == 64 and k1 == 64), e
    # the header counts the entries that are not full (the kernels' mask-free variant needs 0)
    n_full = sum(bool(m[64 * t:64 * t + 64, 64 * c:64 * c + 64].all()) and 64 * t + 64 <= N and 64 * c + 64 <= N
                 for t, c in pairs)
    assert hdr.num_masked == len(pairs) - n_full
    # key-block order of the entries
    assert [(int(blk[e]), int(p["tile"][e])) for e in p["kentry"]] == sorted((c, t) for t, c in pairs)
    # work items
    t_first = np.searchsorted(p["tile"], np.arange(nt + 1))
    _check_items(p["q_items"], p["q_split"], None, nt, hdr.seg, [(t_first[t], t_first[t + 1]) for t in range(nt)],
                 hdr.num_q_partials)
    kblk = blk[p["kentry"]]
    k_first = np.searchsorted(kblk, np.arange(nt + 1))
    _check_items(p["k_items"], p["k_split"], None, nt, hdr.seg, [(k_first[c], k_first[c + 1]) for c in range(nt)],
                 hdr.num_k_partials)


def test_tile_plan_rejects_malformed_sets():
    import ma_attn
    off = torch.tensor([0, 2, 3], dtype=torch.int64)
    for keys in ([1, 0, 1], [0, 0, 1], [0, 2, 1], [-1, 0, 1]):
        with pytest.raises(ValueError):
            ma_attn.tile_plan(off, torch.tensor(keys, dtype=torch.int32), 2)
    with pytest.raises(ValueError):
        ma_attn.tile_plan(torch.tensor([0, 3, 2]), torch.tensor([0, 1, 1], dtype=torch.int32), 2)


def test_index_set_builds_plan_when_keys_cluster():
    """IndexSet(tiles="auto"): a windowed set gets a plan, a scattered one not."""
    import sparse_attention_cuda as ext
    N = 2048
    i = np.arange(N)
    lo = np.maximum(i - 63, 0)
    off = np.zeros(N + 1, np.int64)
    off[1:] = np.cumsum(i - lo + 1)
    keys = np.concatenate([np.arange(a, b + 1) for a, b in zip(lo, i)]).astype(np.int32)
    s = ext.IndexSet(torch.from_numpy(off), torch.from_numpy(keys), N, device="cpu")
    assert s.tile_plan is not None and s.tile_header.num_entries == 2 * (N // 64) - 1
    rng = np.random.default_rng(0)
    m, off2, keys2 = _csr(rng, N, 0.002)
    s2 = ext.IndexSet(torch.from_numpy(off2), torch.from_numpy(keys2), N, device="cpu")
    assert s2.tile_plan is None
    s3 = ext.IndexSet(torch.from_numpy(off2), torch.from_numpy(keys2), N, device="cpu", tiles=False)
    assert s3.tile_plan is None
