"""CPU oracle for the ShadowKV sparse decode step — TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithms on the CPU (numpy for index/byte work,
torch-CPU for the bf16/fp32 arithmetic the reference itself does in torch) so that the HIP
kernels can be checked against it. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the checker or the timed CPU baseline; the
product path (shadowkv_amd) never imports or calls it.

Each function names the reference file:line it follows and the checks that pin it
(tests/test_oracle_*.py). See shadowkv_oracle.py.
"""
from .shadowkv_oracle import *  # noqa: F401,F403
