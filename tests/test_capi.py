"""The C ABI library loads without a GPU, exports every symbol the header
declares, and rejects bad arguments on the host before any launch."""
import ctypes
import os
import re

import pytest

from dw_tpu_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "dwtpu_moe.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dwm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_entry_points():
    names = declared_functions()
    assert names, "no declarations parsed"
    assert sorted(_lib.SIGNATURES) == names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_empty_error():
    lib = _lib.load()
    assert lib.dwm_version() >= 100
    assert lib.dwm_last_error() == b""


def _rc(name, *args):
    lib = _lib.load()
    return getattr(lib, name)(*args), lib.dwm_last_error().decode()


def test_gmm_argument_checks_need_no_gpu():
    null = None
    # K not a multiple of 64 -> unsupported (fail-closed fallback)
    rc, msg = _rc("dwm_gmm_fp4", null, 8, 192, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 0, null)
    assert rc == _lib.ERR_UNSUPPORTED and "K" in msg
    rc, msg = _rc("dwm_gmm_fp4", null, 8, 128, null, null, null, 4, null, 4, 64, null, 7, 0, 0, null)
    assert rc == _lib.ERR_INVALID and "dtype" in msg
    rc, msg = _rc("dwm_gmm_fp4", null, 8, 128, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 0, null)
    assert rc == _lib.ERR_INVALID and "null" in msg
    rc, _ = _rc("dwm_gmm_fp4", null, 0, 128, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 0, null)
    assert rc == _lib.OK  # M == 0: nothing to do
    rc, msg = _rc("dwm_gmm_fp4", null, 8, 128, null, null, null, 2000, null, 4, 64, null, _lib.BF16, 0, 0, null)
    assert rc == _lib.ERR_UNSUPPORTED and "groups" in msg
    rc, msg = _rc("dwm_gmm_fp4", null, 8, 128, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 5, null)
    assert rc == _lib.ERR_INVALID and "fuse_act" in msg
    rc, msg = _rc("dwm_gmm_fp4", null, 8, 128, null, null, null, 4, null, 4, 80, null, _lib.BF16, 0,
                  _lib.ACT_SILU_MUL_CLAMP, null)
    assert rc == _lib.ERR_UNSUPPORTED and "fuse_act" in msg
    rc, msg = _rc("dwm_gmm_fp4_prepack_gate_up", null, 0, null, _lib.U8, 1, 128, 80, null, null, null, null)
    assert rc == _lib.ERR_UNSUPPORTED and "64" in msg
    # the fused-gather entry: its own checks, then the gmm's
    g = "dwm_gmm_fp4_gather"
    rc, msg = _rc(g, null, 10, null, 8, 128, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 0, null)
    assert rc == _lib.ERR_INVALID and "row_idx" in msg
    rc, msg = _rc(g, null, -1, null, 8, 128, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 0, null)
    assert rc == _lib.ERR_INVALID and "lhs_rows" in msg
    idx = (ctypes.c_int32 * 8)()
    rc, msg = _rc(g, null, 10, idx, 8, 192, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 0, null)
    assert rc == _lib.ERR_UNSUPPORTED and "K" in msg
    rc, msg = _rc(g, ctypes.c_void_p(16), 1 << 20, idx, 8, 4096, ctypes.c_void_p(16), ctypes.c_void_p(16),
                  ctypes.c_void_p(16), 4, null, 4, 64, ctypes.c_void_p(16), _lib.BF16, 0, 0, null)
    assert rc == _lib.ERR_UNSUPPORTED and "too large" in msg  # 32-bit lhs row offsets
    rc, _ = _rc(g, null, 0, null, 0, 128, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 0, null)
    assert rc == _lib.OK  # M == 0: nothing to do


def test_prepack_size_query():
    wb, sb = ctypes.c_int64(), ctypes.c_int64()
    rc, _ = _rc("dwm_gmm_fp4_prepack_size", 32, 7168, 4096, ctypes.byref(wb), ctypes.byref(sb))
    assert rc == _lib.OK
    assert wb.value == 32 * 7168 * 4096 // 2
    assert sb.value == 32 * (4096 // 64) * (7168 // 128) * 256
    rc, _ = _rc("dwm_gmm_fp4_prepack_size", 2, 256, 80, ctypes.byref(wb), ctypes.byref(sb))
    assert rc == _lib.OK
    assert wb.value == 2 * 128 * 256 // 2  # N padded to 128 columns
    assert sb.value == 2 * 2 * 2 * 256
    rc, _ = _rc("dwm_gmm_fp4_prepack_size", 1, 192, 64, ctypes.byref(wb), ctypes.byref(sb))
    assert rc == _lib.ERR_UNSUPPORTED


def test_dispatch_and_combine_argument_checks():
    ws = ctypes.c_int64()
    rc, _ = _rc("dwm_moe_dispatch_workspace_size", 65536, 32, ctypes.byref(ws))
    assert rc == _lib.OK and ws.value == 64 * 33 * 4
    rc, _ = _rc("dwm_moe_dispatch_workspace_size", 10, 4096, ctypes.byref(ws))
    assert rc == _lib.ERR_UNSUPPORTED
    rc, _ = _rc("dwm_moe_dispatch", None, 4, 0, 8, None, None, None, None, None, None, None, None)
    assert rc == _lib.ERR_INVALID
    rc, _ = _rc("dwm_moe_combine", None, 5, 4, 8, None, None, _lib.F32, 2, 2, None, _lib.BF16, None)
    assert rc == _lib.ERR_INVALID
    rc, _ = _rc("dwm_row_gather", None, 4, 16, None, 0, None, None)
    assert rc == _lib.OK  # zero rows
    rc, _ = _rc("dwm_fp4_decode", None, 0, 3, None, None, None, None)
    assert rc == _lib.ERR_INVALID  # odd count


def test_checkpoint_format_argument_checks():
    null = None
    st = ctypes.c_void_p(8)  # never dereferenced: the checks fail before any launch
    rc, msg = _rc("dwm_mxfp4_requant", null, null, 2, 128, 96, 0, null, null, st, null)
    assert rc == _lib.ERR_UNSUPPORTED and "K" in msg
    rc, msg = _rc("dwm_mxfp4_requant", null, null, 2, 96, 128, 0, null, null, st, null)
    assert rc == _lib.ERR_UNSUPPORTED and "N" in msg
    rc, msg = _rc("dwm_mxfp4_requant", null, null, 2, 64, 128, 1, null, null, st, null)
    assert rc == _lib.ERR_UNSUPPORTED and "interleave" in msg
    rc, msg = _rc("dwm_mxfp4_requant", null, null, 2, 64, 128, 0, null, null, null, null)
    assert rc == _lib.ERR_INVALID and "status" in msg
    rc, msg = _rc("dwm_mxfp4_requant", null, null, -1, 64, 128, 0, null, null, st, null)
    assert rc == _lib.ERR_INVALID and "sizes" in msg
    rc, msg = _rc("dwm_fp8_block_requant", null, null, 256, 192, 1, null, null, st, null)
    assert rc == _lib.ERR_UNSUPPORTED and "N" in msg
    rc, msg = _rc("dwm_fp8_block_requant", null, null, 200, 256, 1, null, null, st, null)
    assert rc == _lib.ERR_UNSUPPORTED and "K" in msg
    rc, msg = _rc("dwm_fp8_block_requant", null, null, 256, 256, 1, null, null, null, null)
    assert rc == _lib.ERR_INVALID and "status" in msg


def test_router_argument_checks():
    null = None
    p = ctypes.c_void_p(8)  # never dereferenced: the checks fail before any launch
    rc, msg = _rc("dwm_route_topk", p, _lib.F32, 4, 8, 9, 0, null, null, 0, null, p, _lib.F32, p, null)
    assert rc == _lib.ERR_INVALID and "topk" in msg
    rc, msg = _rc("dwm_route_topk", p, _lib.F32, 4, 2048, 8, 0, null, null, 0, null, p, _lib.F32, p, null)
    assert rc == _lib.ERR_UNSUPPORTED and "E <= 1024" in msg
    rc, msg = _rc("dwm_route_topk", p, _lib.F32, 4, 64, 8, 7, null, null, 0, null, p, _lib.F32, p, null)
    assert rc == _lib.ERR_INVALID and "score_fn" in msg
    rc, msg = _rc("dwm_route_topk", null, _lib.F32, 4, 64, 8, 0, null, null, 0, null, p, _lib.F32, p, null)
    assert rc == _lib.ERR_INVALID and "null" in msg
    rc, _ = _rc("dwm_route_topk", null, _lib.F32, 0, 64, 8, 0, null, null, 0, null, null, _lib.F32, null, null)
    assert rc == _lib.OK  # no tokens: nothing to do
    rc, msg = _rc("dwm_dedupe_topk", p, p, 4, 65, 256, p, p, null)
    assert rc == _lib.ERR_UNSUPPORTED and "topk" in msg


def test_python_layer_rejects_host_tensors():
    import torch
    from dw_tpu_amd import e2m1_to_codes
    with pytest.raises(ValueError):
        e2m1_to_codes(torch.zeros(4, dtype=torch.uint8))


def test_missing_library_is_loud(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(_lib.LibraryMissing):
        _lib.load()


def test_last_error_is_per_thread():
    import threading
    lib = _lib.load()
    null = None
    # this thread fails an argument check ...
    assert lib.dwm_gmm_fp4(null, 8, 192, null, null, null, 4, null, 4, 64, null, _lib.BF16, 0, 0, null) \
        == _lib.ERR_UNSUPPORTED
    mine = lib.dwm_last_error()
    assert mine
    seen = {}

    def other():
        seen["fresh"] = lib.dwm_last_error()
        lib.dwm_gmm_fp4(null, 8, 128, null, null, null, 4, null, 4, 64, null, 7, 0, 0, null)  # bad dtype
        seen["own"] = lib.dwm_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    # ... another thread starts clean, sees only its own failure, and leaves ours alone
    assert seen["fresh"] == b""
    assert b"dtype" in seen["own"]
    assert lib.dwm_last_error() == mine


@pytest.mark.parametrize("compiler,std", [("gcc", "-std=c99"), ("g++", "-std=c++11")])
def test_header_is_plain_c(tmp_path, compiler, std):
    """include/dwtpu_moe.h is a C header (no torch or HIP types): it compiles
    as strict C99 and as C++, and a C program can link against the library."""
    import shutil
    import subprocess
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not installed")
    src = tmp_path / "use.c"
    src.write_text('#include "dwtpu_moe.h"\nint main(void) { return dwm_version() > 0 ? 0 : 1; }\n')
    cmd = [compiler, std, "-Wall", "-Wextra", "-Werror", "-I", os.path.dirname(HEADER)]
    if compiler == "gcc":  # C: compile and link
        cmd += ["-pedantic", str(src), "-o", str(tmp_path / "use"), _lib.LIB_PATH]
    else:  # C++: the same header compiles
        cmd += ["-fsyntax-only", "-x", "c++", str(src)]
    r = subprocess.run(cmd, capture_output=True, timeout=120)
    assert r.returncode == 0, r.stderr.decode(errors="replace")
