"""The C-ABI library loads on a CPU-only host and exports every function the header declares."""
import ctypes

from shadowkv_amd import _lib


def test_header_and_binding_agree():
    declared = _lib.header_functions()
    assert len(declared) >= 17
    assert sorted(declared) == sorted(_lib.SIGNATURES), "ctypes signatures must cover the header exactly"


def _header_argument_kinds():
    """{name: (return kind, [argument kinds])} parsed from the header's declarations, a kind being
    "p" (any pointer), "i64", "i32" or "f32"."""
    import re
    text = re.sub(r"/\*.*?\*/", "", _lib.HEADER_PATH.read_text(), flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"^\s*(const\s+char\s*\*|int64_t|int)\s+(skv_\w+)\s*\(([^;]*?)\)\s*;",
                                        text, flags=re.M):
        kinds = []
        for prm in params.split(","):
            prm = " ".join(prm.split())
            if not prm or prm == "void":
                continue
            kinds.append("p" if "*" in prm else "i64" if prm.startswith("int64_t") else
                         "f32" if prm.startswith("float") else "i32" if prm.startswith("int ") else prm)
        out[name] = ("p" if "*" in ret else "i64" if ret == "int64_t" else "i32", kinds)
    return out


def test_header_argument_types_match_bindings():
    """Every ctypes signature has the header's arity and argument kinds (a missing or extra
    argument would shift every later one at the call)."""
    import ctypes as C
    kind = {C.c_void_p: "p", C.c_char_p: "p", C.c_int64: "i64", C.c_int32: "i32", C.c_float: "f32"}
    decl = _header_argument_kinds()
    assert sorted(decl) == sorted(_lib.SIGNATURES)
    for name, (ret, args) in _lib.SIGNATURES.items():
        want_ret, want_args = decl[name]
        got = ["p" if isinstance(a, type) and issubclass(a, C._Pointer) else kind.get(a, str(a)) for a in args]
        assert got == want_args, f"{name}: binding {got} vs header {want_args}"
        assert kind.get(ret, str(ret)) == want_ret, f"{name}: return type"


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
    # the arrival counters (4096 rows x 4 bytes), then the partials of 64-key splits (the shorter choice)
    assert lib.skv_sparse_attn_workspace_bytes(8, 32, 2600) == 16384 + 8 * 32 * 41 * 130 * 4


def test_selection_workspace_plan():
    """The selection workspace covers the slice histograms, counts and winners of the plan the
    library uses (about 256 / rows slices of at most 4096 keys per row) and the softmax kernel's
    per-workgroup key histograms, and bad sizes give 0."""
    lib = _lib.lib()
    assert lib.skv_select_workspace_bytes(0, 100, 10) == 0
    assert lib.skv_select_workspace_bytes(8, 0, 10) == 0
    for rows, n, S in ((8, 130680, 2048), (8, 32712, 256), (32, 15304, 256), (1, 1000, 7), (4, 1001, 7)):
        target = max(1, min(64, 256 // rows))
        part_len = max(256, min(4096, -(-(-(-n // target)) // 256) * 256))
        parts = -(-n // part_len)
        align = lambda b: -(-b // 256) * 256
        want = 2 * align(rows * parts * 256 * 4) + align(rows * parts * 8) + align(rows * 16) + align(rows * S * 8)
        # the softmax kernel's per-workgroup key histograms: 8, 4 or 2 columns per thread of 256,
        # the widest giving >= 512 workgroups (n % 8 == 0 rows only)
        cpt = 8
        while cpt > 2 and rows * -(-n // (256 * cpt)) < 512:
            cpt //= 2
        sparts = -(-n // (256 * cpt)) if n % 8 == 0 else 0
        want += align(rows * sparts * 256 * 4)
        assert lib.skv_select_workspace_bytes(rows, n, S) == want, (rows, n, S)
    # select_chunks_ws rejects a null workspace and a short one on the host
    p = ctypes.c_void_p(16)
    rc = lib.skv_select_chunks_ws(p, p, p, 8, 4, 130680, p, 130680, 2048, 131000, p, p, p, p, None, None, 0, None)
    assert rc == 1 and "null workspace" in _lib.last_error()
    rc = lib.skv_select_chunks_ws(p, p, p, 8, 4, 130680, p, 130680, 2048, 131000, p, p, p, p, None, p, 1, None)
    assert rc == 1 and "workspace of 1 bytes" in _lib.last_error()


def test_selection_only_needs_an_output():
    """Selection without previous slots (null position_ids, offsets, cnts) writes only the ids in
    top-k order, so out_selected must be given; a half-given reorder triple is rejected too."""
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    rc = lib.skv_select_chunks(p, p, p, 8, 4, 1000, p, 1000, 256, 1100, None, None, None, p, None, None)
    assert rc == 1 and "null pointer" in _lib.last_error()
    rc = lib.skv_select_chunks(p, p, p, 8, 4, 1000, p, 1000, 256, 1100, p, None, p, p, None, None)
    assert rc == 1 and "null pointer" in _lib.last_error()


def test_build_rejects_kernels_that_use_scratch():
    """The build's scan of hipcc's resource-usage remarks names every kernel with scratch."""
    from shadowkv_amd import build
    remarks = "\n".join([
        "x.hip:1:1: remark: Function Name: k_ok [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark: Function Name: k_spills [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 320 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build.scratch_kernels(remarks) == [("k_spills", 320)]
