"""CPU-side checks of the C ABI: the library builds for gfx950, loads, and
exports every function include/moe_amd.h declares; the Python binding maps
the same names.  No compute call runs here (there is no GPU)."""
import ctypes
import os
import subprocess

import pytest

from helpers import PKG_DIR, header_functions, load_pkg


@pytest.fixture(scope="module")
def lib_path():
    path = os.path.join(PKG_DIR, "libmoe_amd.so")
    if not os.path.exists(path):
        subprocess.run(["python", os.path.join(PKG_DIR, "build.py")], check=True)
    return path


def test_header_declares_the_boundary():
    names = header_functions()
    for n in ("moe_sgemm_nt", "moe_sgemm_nn", "moe_gate_logits", "moe_route",
              "moe_permute", "moe_expert_ffn_grouped", "moe_combine",
              "moe_layer_forward", "moe_ctx_create", "moe_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol(lib_path):
    lib = ctypes.CDLL(lib_path)
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(header_functions()) <= exported


def test_binding_covers_the_header(lib_path):
    pkg = load_pkg()
    assert set(pkg.EXPORTS) == set(header_functions())
    lib = pkg.load_library()
    assert lib.moe_version().decode().endswith("gfx950")


def test_library_is_built_for_gfx950(lib_path):
    # the offload bundle ids of the library's device code name the target
    with open(lib_path, "rb") as f:
        blob = f.read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob


def test_errors_without_context(lib_path):
    pkg = load_pkg()
    lib = pkg.load_library()
    rc = lib.moe_sgemm_nt(None, None, None, None, None, 1, 1, 1, None)
    assert rc == pkg.ERR_INVALID
    assert "moe_ctx" in lib.moe_last_error().decode()
    rc = lib.moe_route(None, None, None, 4, 8, 2, 0, 1e-3, 2e-2, None, None, None)
    assert rc == pkg.ERR_INVALID


def test_rope_table_is_the_oracles_libm_table(lib_path, orc):
    # moe_rope_table is host code (no device work): its float libm calls must
    # give the oracle's table bit for bit, since RoPE's parity rests on it
    import numpy as np
    lib = load_pkg().load_library()
    for theta, hd, pos in ((10000.0, 64, 513), (500000.0, 128, 40), (10000.0, 2, 7)):
        t = np.empty((pos, hd // 2, 2), np.float32)
        assert lib.moe_rope_table(theta, hd, pos, t.ctypes.data_as(ctypes.c_void_p)) == 0
        assert np.array_equal(t, orc.rope_table(theta, hd, pos))
    t = np.empty(4, np.float32)
    assert lib.moe_rope_table(10000.0, 3, 1, t.ctypes.data_as(ctypes.c_void_p)) == \
        load_pkg().ERR_INVALID


def test_every_entry_point_rejects_a_null_context(lib_path):
    # each call taking a context checks it before any device work, so a null
    # one is an invalid-argument error (with the reason) even without a GPU
    import ctypes as ct
    pkg = load_pkg()
    lib = pkg.load_library()
    skip = {"moe_ctx_create", "moe_rope_table", "moe_last_error", "moe_version"}
    checked = []
    for name in header_functions():
        if name in skip:
            continue
        fn = getattr(lib, name)
        args = []
        for t in fn.argtypes:
            if t in (ct.c_float, ct.c_double):
                args.append(0.0)
            elif t in (ct.c_int, ct.c_int32, ct.c_int64, ct.c_uint, ct.c_uint32, ct.c_uint64):
                args.append(1)
            else:
                args.append(None)
        rc = fn(*args)
        if name == "moe_ctx_destroy":
            assert rc in (pkg.OK, pkg.ERR_INVALID), name
            continue
        if name == "moe_ctx_kernel_times":  # a count, or minus the status
            rc = -rc
        assert rc == pkg.ERR_INVALID, f"{name} returned {rc}"
        assert lib.moe_last_error().decode(), name
        checked.append(name)
    assert len(checked) >= 30
