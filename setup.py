"""Wheel build for ROCm (the reference's setup.py compiles its Metal and
Objective-C++ sources; here hipcc compiles the gfx950 kernels).

    pip wheel . --no-build-isolation --no-deps -w dist/

The build step runs mtlattn_amd/build.py in the source tree: libmtlattn_hip.so
(hipcc --offload-arch=gfx950, override with MTLATTN_ARCH) and the _C torch
binding (g++ against the torch found in the build environment, hence no build
isolation). Both land in the mtlattn_amd package of the wheel, which is
platform-specific; include/mtlattn_capi.h is installed under <prefix>/include.
"""

import importlib.util
import os

from setuptools import Distribution, setup
from setuptools.command.build_py import build_py

ROOT = os.path.dirname(os.path.abspath(__file__))


class BuildWithHip(build_py):
    def run(self):
        # build.py stands alone (the package itself refuses to import until
        # the native parts exist)
        spec = importlib.util.spec_from_file_location("_mtlattn_hip_build",
                                                      os.path.join(ROOT, "mtlattn_amd", "build.py"))
        hip_build = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(hip_build)
        hip_build.build_lib(verbose=True)
        hip_build.build_ext(verbose=True)
        super().run()


class BinaryDistribution(Distribution):
    """The wheel carries compiled libraries: tag it for this platform."""

    def has_ext_modules(self):
        return True


setup(
    name="mtlattn",
    version="0.4.0+mi355x",
    description="Fused variable-length flash attention (forward + backward, additive masks, split-KV and "
                "paged decode) for AMD Instinct MI355X (gfx950) and PyTorch-ROCm",
    long_description=open(os.path.join(ROOT, "README.md")).read(),
    long_description_content_type="text/markdown",
    python_requires=">=3.10",
    install_requires=["torch"],
    packages=["mtlattn", "mtlattn_amd"],
    package_data={"mtlattn_amd": ["*.so", "csrc/*.hip", "csrc/*.h", "csrc/*.cpp"]},
    data_files=[("include", ["include/mtlattn_capi.h"])],
    entry_points={"console_scripts": ["mtlattn-bench = mtlattn.bench:main"]},
    classifiers=[
        "Programming Language :: Python :: 3",
        "Operating System :: POSIX :: Linux",
        "Environment :: GPU",
        "Topic :: Scientific/Engineering :: Artificial Intelligence",
    ],
    cmdclass={"build_py": BuildWithHip},
    distclass=BinaryDistribution,
)
