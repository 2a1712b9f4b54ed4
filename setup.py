"""Wheel packaging of skmetal_amd with libskmetal_hip.so (gfx950 code objects inside).

``pip wheel . --no-build-isolation`` (or ``python setup.py bdist_wheel``) compiles
the HIP sources with hipcc for gfx950 (skmetal_amd/_build.py) and ships the
library as package data next to the ctypes loader that finds it
(skmetal_amd/_bridge.py).  ROCm's hipcc is required at build time; at run time
only the HIP runtime (libamdhip64) and an MI355X are.
"""

from pathlib import Path

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

ROOT = Path(__file__).resolve().parent


def _version() -> str:
    ns: dict = {}
    exec((ROOT / "skmetal_amd" / "_about.py").read_text(), ns)
    return ns["__version__"]


class BuildWithHip(build_py):
    """Compile libskmetal_hip.so in-tree before the package files are copied."""

    def run(self):
        import sys

        sys.path.insert(0, str(ROOT))
        from skmetal_amd import _build

        _build.build(verbose=True)
        super().run()


class BinaryDistribution(Distribution):
    """The package carries a native library: the wheel is platform-specific."""

    def has_ext_modules(self):
        return True


setup(
    name="skmetal-amd",
    version=_version(),
    description="MI355X (gfx950) KMeans Lloyd path behind skmetal's accelerate() API",
    packages=["skmetal_amd", "skmetal_amd.estimators"],
    package_data={"skmetal_amd": ["libskmetal_hip.so", "csrc/*.hip", "csrc/*.h"]},
    python_requires=">=3.10",
    install_requires=["numpy", "scikit-learn"],
    cmdclass={"build_py": BuildWithHip},
    distclass=BinaryDistribution,
    zip_safe=False,
)
