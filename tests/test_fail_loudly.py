"""No silent fallback: without libma_attn.so the engine modules refuse to
import, and on a machine with a GPU so does the layer bridge (device tensors
never reach a PyTorch substitute).  Each case runs in a child interpreter
with MA_ATTN_LIB pointing at a missing file."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "ma-transformer_amd")


def _run(code: str):
    env = dict(os.environ, MA_ATTN_LIB=os.path.join(REPO, "no-such-dir", "libma_attn.so"),
               PYTHONPATH=os.pathsep.join([PKG, REPO, os.environ.get("PYTHONPATH", "")]))
    return subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)


@pytest.mark.parametrize("module", ["ma_attn", "sparse_attention_cuda", "ma_core"])
def test_engine_modules_refuse_without_library(module):
    r = _run(f"import {module}")
    assert r.returncode != 0
    assert "ImportError" in r.stderr and "libma_attn.so" in r.stderr


def test_bridge_on_a_host_without_gpu_keeps_cpu_path():
    """Without a GPU the bridge imports (CPU tensors use the PyTorch path, as
    the reference's CPU branch does) and says the engine is absent."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible here")
    r = _run("from layers import ma_core_bridge as b\n"
             "assert b.sparse_attention_cuda is None and not b._HAS_SPARSE_CUDA\n"
             "print('ok')")
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip().endswith("ok")


@pytest.mark.gpu
def test_bridge_on_a_gpu_host_refuses_without_library():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    r = _run("import torch\n"
             "assert torch.cuda.is_available()\n"
             "from layers import ma_core_bridge")
    assert r.returncode != 0
    assert "ImportError" in r.stderr and "libma_attn.so" in r.stderr
