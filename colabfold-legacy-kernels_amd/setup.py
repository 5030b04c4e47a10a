"""Wheel of the gfx950 kernel library with the reference's package layout.

    cd colabfold-legacy-kernels_amd && pip wheel --no-deps --no-build-isolation -w dist .

Like the reference's packaging (setup.py:1-25, pyproject.toml:31-34), the wheel carries the
prebuilt shared library as package data under colabfold_legacy_kernels/kernels/<arch>/ and is
tagged py3-none-<platform> (not pure: it holds machine code, but no Python extension ABI).
build_py compiles the library first (build.py, hipcc for gfx950) unless CLK_SKIP_KERNEL_BUILD=1
and the library is already in the tree.
"""

import os
import re
import sys
from pathlib import Path

from setuptools import setup
from setuptools.command.build_py import build_py as _build_py
from setuptools.dist import Distribution

try:
    from setuptools.command.bdist_wheel import bdist_wheel as _bdist_wheel
except ImportError:
    from wheel.bdist_wheel import bdist_wheel as _bdist_wheel

HERE = Path(__file__).resolve().parent
PKG = HERE / "colabfold_legacy_kernels"
LIB = PKG / "kernels" / "gfx950" / "libclk_gfx950.so"


def _version():
    text = (PKG / "__init__.py").read_text()
    return re.search(r'^__version__ = "([^"]+)"', text, re.M).group(1)


class build_py(_build_py):
    def run(self):
        if not (os.environ.get("CLK_SKIP_KERNEL_BUILD") == "1" and LIB.is_file()):
            sys.path.insert(0, str(HERE))
            import build as kernel_build  # colabfold-legacy-kernels_amd/build.py
            kernel_build.build()
        super().run()


class BinaryDistribution(Distribution):
    def has_ext_modules(self):
        return True


class bdist_wheel(_bdist_wheel):
    def finalize_options(self):
        _bdist_wheel.finalize_options(self)
        self.root_is_pure = False

    def get_tag(self):
        _python, _abi, plat = _bdist_wheel.get_tag(self)
        return "py3", "none", plat


setup(
    name="colabfold-legacy-kernels",
    version=_version(),
    description="MI355X (gfx950) HIP kernels for ColabFold's Evoformer hot path: attention with "
                "pair bias, LayerNorm, gated dual projection.",
    python_requires=">=3.8",
    license="MIT",
    packages=["colabfold_legacy_kernels"],
    package_data={"colabfold_legacy_kernels": ["kernels/*/*.so"]},
    include_package_data=True,
    distclass=BinaryDistribution,
    cmdclass={"build_py": build_py, "bdist_wheel": bdist_wheel},
)
