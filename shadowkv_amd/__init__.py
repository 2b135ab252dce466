"""shadowkv_amd — MI355X (gfx950) HIP kernels for the ShadowKV sparse decode step.

`shadowkv_amd.kernels.shadowkv` is the drop-in for the reference's native module,
`shadowkv_amd.models.kvcache` / `shadowkv_amd.models.attention` the drop-in for its
ShadowKV cache and attention classes. The compute runs only in libshadowkv_amd.so.
"""
__version__ = "0.1.0"
