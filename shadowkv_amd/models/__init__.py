"""Host-side mirror of the reference's ShadowKV cache and attention interfaces
(models/kvcache/shadow.py, models/attention/shadow.py, models/tensor_op.py)."""
