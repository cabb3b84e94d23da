"""Build and install the MI355X sparse-attention engine.

    python setup.py build_ext --inplace   # libma_attn.so next to the modules (in-tree use)
    pip install .                         # modules + library into site-packages

The native part is one C-ABI shared library compiled by hipcc for gfx950
(ma-transformer_amd/build_ext.py); Python binds it with ctypes, so no torch
extension machinery and no hipify step is involved.  The import name of the
Python module is the reference's, `sparse_attention_cuda`.
"""
import importlib.util
import os
import shutil

from setuptools import setup
from setuptools.command.build_ext import build_ext as _build_ext
from setuptools.command.build_py import build_py as _build_py

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(HERE, "ma-transformer_amd")


def _hip_build():
    spec = importlib.util.spec_from_file_location("ma_build_ext", os.path.join(PKG, "build_ext.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build()


class build_hip(_build_ext):
    """Compile libma_attn.so with hipcc --offload-arch=gfx950 (always in-tree)."""

    def run(self):
        lib = _hip_build()
        if not self.inplace:
            os.makedirs(self.build_lib, exist_ok=True)
            shutil.copy2(lib, os.path.join(self.build_lib, os.path.basename(lib)))


class build_py(_build_py):
    """Build the library before the modules, so installs carry it."""

    def run(self):
        self.run_command("build_ext")
        super().run()


setup(
    name="ma-sparse-mi355x",
    version="0.1.0",
    description="MI355X sparse-attention forward (drop-in for ma-transformer's sparse_attention_cuda)",
    package_dir={"": "ma-transformer_amd"},
    py_modules=["sparse_attention_cuda", "ma_attn", "ma_core", "model", "tick_features"],
    packages=["layers"],
    cmdclass={"build_ext": build_hip, "build_py": build_py},
    python_requires=">=3.9",
)
