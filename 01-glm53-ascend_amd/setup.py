"""Package build of sgl-glm53-ascend-ops for AMD MI355X (gfx950).

``pip install ./01-glm53-ascend_amd`` (from a checkout of this repository; the
C-ABI header lives in its ``include/``) compiles both native libraries with
``kda_build.py`` (hipcc for gfx950, g++ against the installed torch) into the
build tree and packages them with the Python sources. The build needs torch
and ROCm at build time, so with no package index use
``pip install --no-build-isolation ./01-glm53-ascend_amd``.
"""

import os
import sys

from setuptools import setup
from setuptools.command.build_py import build_py
from setuptools.dist import Distribution

HERE = os.path.dirname(os.path.abspath(__file__))


class BuildWithKernels(build_py):
    """build_py that also compiles the gfx950 libraries into the package."""

    def run(self):
        super().run()
        sys.path.insert(0, HERE)
        import kda_build

        kda_build.build(verbose=self.verbose > 1,
                        out_dir=os.path.join(self.build_lib, "sgl_glm53_ascend_ops"))


class BinaryDistribution(Distribution):
    """The wheel carries native libraries: a platform wheel, not a pure one."""

    def has_ext_modules(self):
        return True


setup(
    name="sgl-glm53-ascend-ops",
    version="0.2.0",
    description=("KDA (Kimi Delta Attention) operators for SGLang's GLM-5.3 backend on AMD "
                 "MI355X (gfx950)"),
    python_requires=">=3.10",
    packages=["sgl_glm53_ascend_ops", "sgl_glm53_ascend_ops.ops"],
    cmdclass={"build_py": BuildWithKernels},
    distclass=BinaryDistribution,
    zip_safe=False,
)
