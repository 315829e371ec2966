"""Installable package: `pip install --no-build-isolation .` compiles the gfx950
HIP library (flash_spacetime_amd.build, hipcc from ROCm) and ships it inside
the package, so `import flash_spacetime_amd` works outside the source tree.

The reference packages its Python sources only (pyproject.toml; Triton JIT-
compiles at run time); here the kernels are ahead-of-time HIP, so the build
step runs hipcc. FST_OFFLOAD_ARCH (default gfx950) and HIPCC are honoured.
"""

import importlib.util
from pathlib import Path

from setuptools import setup
from setuptools.command.build_py import build_py

ROOT = Path(__file__).resolve().parent


class BuildWithKernels(build_py):
    """Compile libflash_spacetime.so before the package files are copied."""

    def run(self):
        spec = importlib.util.spec_from_file_location("fst_build", ROOT / "flash_spacetime_amd" / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
        super().run()


setup(
    name="flash-spacetime-amd",
    version="0.3.0",
    description="flash-spacetime attention on MI355X (gfx950): hand-written HIP kernels behind the "
                "reference's operator API",
    long_description=(ROOT / "README.md").read_text(),
    long_description_content_type="text/markdown",
    python_requires=">=3.10",
    install_requires=["torch>=2.4"],
    extras_require={"dev": ["pytest>=7"]},
    packages=["flash_spacetime_amd"],
    package_data={"flash_spacetime_amd": ["libflash_spacetime.so"]},
    cmdclass={"build_py": BuildWithKernels},
    zip_safe=False,
)
