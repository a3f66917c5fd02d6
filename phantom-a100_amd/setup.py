"""pip install -e phantom-a100_amd   -> builds libphantom_attn.so (hipcc, gfx950) and installs cuda_attn.

Replaces the reference's CUDAExtension build (/root/reference/setup.py:8-34): the kernels are
plain HIP behind a C ABI, so the build is one hipcc invocation (build_native.py), not a torch
extension.
"""
import os
import sys

from setuptools import setup
from setuptools.command.build_py import build_py

HERE = os.path.dirname(os.path.abspath(__file__))


class BuildWithHip(build_py):
    def run(self):
        sys.path.insert(0, HERE)
        import build_native
        build_native.build()
        super().run()


setup(
    name="cuda_attn",
    version="0.1.0",
    description="Attention forward kernels for AMD MI355X (gfx950) behind the cuda_attn API",
    packages=["cuda_attn"],
    package_data={"cuda_attn": ["libphantom_attn.so"]},
    cmdclass={"build_py": BuildWithHip},
    python_requires=">=3.9",
)
