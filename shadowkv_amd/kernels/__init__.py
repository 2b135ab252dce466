"""Native kernel module: `from shadowkv_amd.kernels import shadowkv` mirrors the reference's
`from kernels import shadowkv` (models/kvcache/shadow.py:23)."""
from . import shadowkv  # noqa: F401
