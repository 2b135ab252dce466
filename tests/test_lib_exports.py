"""The C-ABI library loads on a CPU-only host and exports every function the header declares."""
import ctypes

from shadowkv_amd import _lib


def test_header_and_binding_agree():
    declared = _lib.header_functions()
    assert len(declared) >= 17
    assert sorted(declared) == sorted(_lib.SIGNATURES), "ctypes signatures must cover the header exactly"


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in _lib.header_functions():
        assert hasattr(lib, name), name
    assert lib.skv_version().decode().startswith("shadowkv_amd")


def test_argument_errors_are_reported_without_a_gpu():
    lib = _lib.lib()
    # Null pointers and unsupported sizes are rejected on the host before any launch.
    rc = lib.skv_reorder_keys_and_compute_offsets(None, None, None, None, 1, 8, 256, None)
    assert rc == 1 and "null pointer" in _lib.last_error()
    p = ctypes.c_void_p(16)
    rc = lib.skv_reorder_keys_and_compute_offsets(p, p, p, p, 1, 8, 4096, None)
    assert rc == 2 and "map_size" in _lib.last_error()
    rc = lib.skv_topk_gather(p, 100, p, 100, 4, 100, 200, p, None)
    assert rc == 1 and "k=200" in _lib.last_error()
    rc = lib.skv_batch_gemm_softmax(p, p, p, p, p, p, 1, 4, 10, 64, 1.0, 0.0, None)
    assert rc == 2 and "k=64" in _lib.last_error()
    assert lib.skv_sparse_attn_workspace_bytes(8, 32, 2600) == 8 * 32 * 21 * 130 * 4  # 128-key splits
