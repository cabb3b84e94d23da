"""C-ABI library checks that need no GPU: load, exported symbols, host-side
validation, the engine's closed-form index sets and block table vs the oracle."""
import ctypes
import os
import re

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(REPO, "include", h) for h in ("ma_attn.h", "ma_features.h", "ma_encoder.h")]


def _declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(ma_(?:attn|tick|encoder)_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    import ma_attn
    names = _declared_functions()
    assert len(names) >= 11 and "ma_tick_features" in names and "ma_encoder_layer_forward" in names
    lib = ctypes.CDLL(ma_attn.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
    assert ma_attn.LIB.ma_attn_abi_version() == ma_attn.ABI_VERSION


def test_desc_layout_matches_header(tmp_path):
    """Every field of the ctypes Desc sits at the offset the C compiler gives
    the header's struct (gcc on include/ma_attn.h), and the sizes agree."""
    import subprocess
    import ma_attn
    names = [f[0] for f in ma_attn.Desc._fields_]
    src = tmp_path / "probe.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "ma_attn.h"\nint main(void) {\n'
                   + "".join(f'  printf("{n} %zu\\n", offsetof(ma_attn_desc, {n}));\n' for n in names)
                   + '  printf("sizeof %zu\\n", sizeof(ma_attn_desc));\n  return 0;\n}\n')
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                       text=True).stdout.splitlines())
    for n in names:
        assert int(got[n]) == getattr(ma_attn.Desc, n).offset, n
    assert int(got["sizeof"]) == ctypes.sizeof(ma_attn.Desc)


@pytest.mark.parametrize("kw,msg", [
    (dict(dtype_code=7), "dtype"),
    (dict(pattern=9), "pattern"),
    (dict(dilation=0), "dilation"),
    (dict(D=(1 << 24) + 1), "head_dim"),
    (dict(N=-1), "negative"),
])
def test_validate_rejects(kw, msg):
    import ma_attn
    args = dict(B=1, N=8, H=1, D=16, dtype_code=ma_attn.F32, pattern=ma_attn.SLIDING)
    args.update(kw)
    d = ma_attn.make_desc(**args)
    with pytest.raises(RuntimeError, match=msg):
        ma_attn.validate(d)


def test_validate_accepts_wide_heads():
    """Any head_dim up to the 2^24 sanity bound (the reference loops over any)."""
    import ma_attn
    for D in (513, 1000, 4096, 1 << 24):
        ma_attn.validate(ma_attn.make_desc(1, 8, 1, D, ma_attn.F32, ma_attn.SLIDING, left=2, right=2))


def test_forward_rejects_before_launch():
    """Invalid descriptors fail on the host; nothing touches a device."""
    import ma_attn
    d = ma_attn.make_desc(1, 8, 1, 16, ma_attn.F32, ma_attn.BLOCK_SPARSE, blocks_per_row=2)
    with pytest.raises(RuntimeError, match="block_table"):
        ma_attn.forward_raw(d, 1, 1, 1, 1)
    d = ma_attn.make_desc(0, 8, 1, 16, ma_attn.F32, ma_attn.SLIDING)  # empty problem: no-op
    ma_attn.forward_raw(d, 0, 0, 0, 0)


def _engine_vs_oracle_keys(oracle, N, pattern, table=None, **kw):
    import ma_attn
    import torch
    code = {"sliding": ma_attn.SLIDING, "dense": ma_attn.DENSE, "block_sparse": ma_attn.BLOCK_SPARSE,
            "longformer": ma_attn.LONGFORMER}[pattern]
    # block_table_ptr only has to be non-null: host enumeration reads the host table argument
    d = ma_attn.make_desc(1, N, 1, 1, ma_attn.F32, code,
                          blocks_per_row=0 if table is None else table.shape[1],
                          block_table_ptr=0 if table is None else 1, **kw)
    s = oracle.Spec(1, N, 1, 1, pattern=pattern, table=table, **kw)
    ht = None if table is None else torch.from_numpy(table)
    for i in range(N):
        assert ma_attn.row_keys(d, i, ht) == oracle.row_keys(s, i).tolist(), (pattern, kw, i)


@pytest.mark.parametrize("pattern,kw", [
    ("sliding", dict(left=63, right=0)), ("sliding", dict(left=32, right=31)),
    ("sliding", dict(left=63, right=0, dilation=4)), ("sliding", dict(left=2, right=7, dilation=3)),
    ("sliding", dict(left=-1, right=-1)), ("sliding", dict(left=-3, right=5)),
    ("dense", dict(causal=True)), ("dense", dict(causal=False)),
    ("longformer", dict(left=127, right=0, num_global=16)), ("longformer", dict(left=3, right=2, num_global=5)),
])
@pytest.mark.parametrize("N", [1, 7, 150])
def test_engine_index_sets_match_oracle(oracle, pattern, kw, N):
    _engine_vs_oracle_keys(oracle, N, pattern, **kw)


def test_engine_block_index_sets_match_oracle(oracle):
    for N, bs in ((150, 16), (64, 64), (129, 64)):
        nb = (N + bs - 1) // bs
        _engine_vs_oracle_keys(oracle, N, "block_sparse", table=oracle.block_table(4, nb, 2), block_size=bs)


def test_engine_block_table_bitexact(oracle):
    import ma_attn
    for seed, nb, extra in ((1234, 256, 2), (0, 1, 2), (7, 2, 2), (99, 1000, 5), (2**63 + 5, 17, 3)):
        assert np.array_equal(ma_attn.block_table(seed, nb, extra).numpy(), oracle.block_table(seed, nb, extra))
    fix = np.fromfile(os.path.join(REPO, "tests", "golden", "block_table_seed1234_nb256_r2.bin"),
                      dtype="<i4").reshape(256, 4)
    assert np.array_equal(ma_attn.block_table(1234, 256, 2).numpy(), fix)
