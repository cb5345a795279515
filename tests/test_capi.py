"""CPU checks of the C-ABI boundary: libtcc_swtcf.so loads without a GPU and
exports every function declared in include/*.h (no compute call is made)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "tcc_amd", "libtcc_swtcf.so")


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "tcc_*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names.update(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(tcc_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_headers_declare_the_boundary():
    names = declared_functions()
    for must in ("tcc_swtcf_convert", "tcc_swtcf_spmm", "tcc_swtcf_spmm_quantized", "tcc_bcsr_spmm",
                 "tcc_bcsc_spmm", "tcc_spmm_cnic_forward", "tcc_spmm_cnic_forward_mixed", "tcc_coo_to_bcsr"):
        assert must in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build with python -m tcc_amd.build"
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_signatures_cover_the_headers():
    from tcc_amd import _lib

    assert set(declared_functions()) <= set(_lib.SIGNATURES)


def test_host_side_argument_errors_without_gpu():
    """Argument validation runs on the host before any HIP call."""
    from tcc_amd import _lib

    L = _lib.lib()
    m = _lib.SWTCFMatrix()
    assert L.tcc_swtcf_alloc_matrix(ctypes.byref(m), 4, 0, 4, 16) == 1  # cols == 0
    assert b"invalid SWTCF allocation size" in L.tcc_last_error()
    assert L.tcc_swtcf_alloc_matrix(ctypes.byref(m), 4, 8, 4, 33) == 1  # S > 32
    ws = _lib.SWTCFWorkspace()
    assert L.tcc_swtcf_alloc_workspace(ctypes.byref(ws), 0, 8, 16) == 1
    assert L.tcc_swtcf_spmm(None, None, None, 12, None) == 1
    m.superWindowSize = 8
    m.numSuperWindows = 1
    assert L.tcc_swtcf_spmm(ctypes.byref(m), ctypes.c_void_p(16), ctypes.c_void_p(16), 12, None) == 3
    assert b"superWindowSize=16" in L.tcc_last_error()
    # feature rows are addressed with 32-bit byte offsets: F below 2^30
    assert L.tcc_tf32_pack(ctypes.c_void_p(16), 4, 1 << 30, ctypes.c_void_p(16), None) == 1
    assert b"invalid TF32 pack arguments" in L.tcc_last_error()
    assert L.tcc_tf32_pack(ctypes.c_void_p(16), 4, 0, ctypes.c_void_p(16), None) == 1


def test_packed_bytes_follow_the_documented_layout():
    """tcc_tf32_packed_bytes = rows x the row stride of the packed layout of
    include/tcc_spmm_cnic.h: 256-feature chunks of 640 bytes, the last padded
    to 16 bytes, rows of more than one chunk padded to 128 (host-only call)."""
    from tcc_amd import _lib

    L = _lib.lib()
    for F, stride in [(1, 16), (2, 16), (7, 32), (100, 256), (128, 320), (256, 640), (257, 768), (300, 768),
                      (512, 1280), (513, 1408), (602, 1536)]:
        assert L.tcc_tf32_packed_bytes(1, F) == stride, F
        assert L.tcc_tf32_packed_bytes(37, F) == 37 * stride, F
