"""Builds libshadowkv_amd.so (gfx950 HIP kernels behind a C ABI) in place:

    python setup.py build_ext --inplace
"""
from setuptools import Command, setup


class BuildHipLibrary(Command):
    description = "compile shadowkv_amd/csrc/*.hip for gfx950 into shadowkv_amd/libshadowkv_amd.so"
    user_options = [("inplace", "i", "build in place (always the case)")]

    def initialize_options(self):
        self.inplace = True

    def finalize_options(self):
        pass

    def run(self):
        from shadowkv_amd.build import build
        build(verbose=True)


setup(
    name="shadowkv_amd",
    version="0.1.0",
    packages=["shadowkv_amd", "shadowkv_amd.kernels", "shadowkv_amd.models", "shadowkv_amd.models.kvcache",
              "shadowkv_amd.models.attention"],
    package_data={"shadowkv_amd": ["libshadowkv_amd.so"]},
    cmdclass={"build_ext": BuildHipLibrary},
)
