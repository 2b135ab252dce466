"""ctypes binding of libshadowkv_amd.so (the C ABI declared in include/shadowkv_amd.h).

The library is loaded lazily and never replaced by a fallback: if it is missing or a call
fails, a RuntimeError names the entry point and the library's own error text.
"""
from __future__ import annotations

import ctypes
import re
import threading
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libshadowkv_amd.so"
HEADER_PATH = PKG_DIR.parent / "include" / "shadowkv_amd.h"

_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> (restype, argtypes); must cover every function declared in the header.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "skv_version": (ctypes.c_char_p, []),
    "skv_last_error": (ctypes.c_char_p, []),
    "skv_host_device_pointer": (_i32, [_p, ctypes.POINTER(_p)]),
    "skv_reorder_keys_and_compute_offsets": (_i32, [_p, _p, _p, _p, _i32, _i32, _i32, _p]),
    "skv_gather_copy_with_offsets": (_i32, [_p, _p, _p, _p, _i32, _i32, _i64, _i64, _i64, _i64, _i32, _i32, _p]),
    "skv_gather_copy_misses_with_offsets": (_i32, [_p, _p, _p, _p, _i32, _i32, _i64, _i64, _i64, _i64, _i32, _i32,
                                                    _p]),
    "skv_gather_copy_d2d_with_offsets": (_i32, [_p, _p, _p, _i32, _i32, _i64, _i64, _i64, _i32, _i32, _p]),
    "skv_gather_copy": (_i32, [_p, _p, _p, _i32, _i32, _i64, _i64, _i32, _i32, _p]),
    "skv_apply_rotary_pos_emb_new": (
        _i32, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64,
               _p]),
    "skv_apply_rotary_pos_emb_push_cache_opt": (
        _i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
               _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i64, _p]),
    "skv_apply_rotary_pos_emb_push_cache_opt_glm": (
        _i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
               _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i64, _p]),
    "skv_apply_rotary_pos_emb": (
        _i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
               _i64, _p]),
    "skv_apply_rotary_pos_emb_new_v2": (
        _i32, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i64,
               _p]),
    "skv_apply_rotary_pos_emb_push_cache": (
        _i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
               _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i64, _p]),
    "skv_batch_gather_gemm": (_i32, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p]),
    "skv_rebuild_k_rope": (
        _i32, [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _i64, _i32,
               _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "skv_batch_gemm_softmax": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _f32, _f32, _p]),
    "skv_score_gqa_max": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _f32, _p]),
    "skv_score_logits": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _f32, _p]),
    "skv_softmax_gqa_max": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _p]),
    "skv_select_chunks": (_i32, [_p, _p, _p, _i32, _i32, _i32, _p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p]),
    "skv_select_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "skv_select_chunks_ws": (_i32, [_p, _p, _p, _i32, _i32, _i32, _p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p,
                                    _i64, _p]),
    "skv_select_chunks_compact": (_i32, [_p, _p, _p, _i32, _i32, _i32, _p, _i64, _i32, _i32, _p, _p, _p, _p, _p,
                                         _p, _i64, _p, _p, _i64, _i64, _i32, _p]),
    "skv_topk_gather": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _i32, _p, _p]),
    "skv_sparse_attn_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "skv_sparse_attn_xcd_check": (_i32, [_p, _p, _p]),
    "skv_rmsnorm": (_i32, [_p, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _i32, _i32, _f32, _p]),
    "skv_silu_and_mul": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _p]),
    "skv_linear": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _p]),
    "skv_linear_silu_mul": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _p]),
    "skv_linear_gate_up_silu": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _p]),
    "skv_linear_bias": (_i32, [_p, _i64, _p, _i64, _p, _p, _i64, _i32, _i32, _i32, _p]),
    "skv_chunk_stats": (_i32, [_p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _p, _p, _p]),
    "skv_select_outliers": (_i32, [_p, _i32, _i32, _i32, _p, _p, _p]),
    "skv_gather_rows": (_i32, [_p, _i32, _i32, _p, _i32, _p, _p]),
    "skv_pool_assign": (_i32, [_p, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "skv_gather_copy_misses_to_slots": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _i64, _i64, _i64, _i32, _i32, _i32,
                                                _p]),
    "skv_rebuild_k_rope_slots": (_i32, [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64,
                                         _i32, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                         _p]),
    "skv_fetch_misses_rebuild_k_rope_slots": (
        _i32, [_p, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64,
               _i32, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "skv_sparse_attn_decode_paged": (_i32, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
                                             _p, _f32, _p, _i64, _p, _i64, _i64, _p, _i32, _i32, _i32, _i32, _p]),
    "skv_sparse_attn_decode_vstore": (_i32, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
                                              _p, _f32, _p, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i32, _i32,
                                              _i32, _p]),
    "skv_rope_qk_append": (
        _i32, [_p, _i64, _i32, _i32, _i32, _i32, _p, _p, _i64, _i64, _i32, _p, _i64, _p, _p, _i64, _i64, _i64, _p,
               _i64, _p]),
    "skv_linear_qkv_rope_append": (
        _i32, [_p, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32, _p, _p, _i64, _i64, _i32, _p, _i64, _p, _p, _i64, _i64,
               _i64, _p, _i64, _p]),
    "skv_fetch_misses_rebuild_k_rope": (
        _i32, [_p, _p, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _p,
               _i64, _i64, _i32, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "skv_hbm_read_probe": (_i32, [_p, _i64, _i32, _i32, _p, _i64, _p]),
    "skv_mfma_peak_probe": (_i32, [_i32, _i32, _p, _i64, _p]),
    "skv_mfma_peak_probe_flops": (_i64, [_i32, _i32]),
    "skv_sparse_attn_noalloc_max_bytes": (_i64, []),
    "skv_sparse_attn_decode_noalloc": (
        _i32, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p, _f32, _p, _i64, _i64, _p]),
    "skv_sparse_attn_decode": (
        _i32, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p, _f32, _p, _i64, _p,
               _i64, _i64, _p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def header_functions() -> list[str]:
    """Names of the functions declared in include/shadowkv_amd.h."""
    text = HEADER_PATH.read_text()
    return re.findall(r"^\s*(?:const\s+char\s*\*|int64_t|int)\s+(skv_\w+)\s*\(", text, flags=re.M)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} is not built: run `python -m shadowkv_amd.build` "
                        "(or __graft_entry__.build()) first; there is no non-HIP fallback")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().skv_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise RuntimeError on a nonzero status."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed with status {rc}: {last_error()}")


def host_device_pointer(host_ptr: int) -> int:
    out = ctypes.c_void_p()
    call("skv_host_device_pointer", ctypes.c_void_p(host_ptr), ctypes.byref(out))
    return int(out.value or 0)
