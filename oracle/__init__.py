"""CPU oracle for the SWTCF / spmm_cnic path — TEST INFRASTRUCTURE ONLY.

Thin numpy wrappers over ``oracle/oracle.c`` (a plain-C restatement of the
reference algorithms; every C function cites the reference file:line it
follows).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker / the timed CPU baseline — never as a product code path.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
c_u32, c_i32, c_i64, c_int = ctypes.c_uint32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int
vp = ctypes.c_void_p

INVALID_SLOT = 0xFFFFFFFF
INVALID_CACHE = 0xFF
CACHE_SIZE = 32


def build() -> None:
    """Compile oracle.c with gcc (called by __graft_entry__.build())."""
    subprocess.run(["bash", os.path.join(_HERE, "build.sh")], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_tf32_bits.restype = c_u32
        L.oracle_tf32_bits.argtypes = [c_u32]
        L.oracle_tf32_array.argtypes = [f32p, f32p, c_i64]
        L.oracle_swtcf_convert.restype = c_int
        L.oracle_swtcf_convert.argtypes = [u32p, u32p, c_u32, c_u32, c_u32, c_u32, u32p, u32p, u32p,
                                           u8p, u32p, u8p, u32p, u64p, u32p]
        L.oracle_validate_swtcf.restype = c_int
        L.oracle_validate_swtcf.argtypes = [u32p, u32p, c_u32, c_u32, c_u32, c_u32, u32p, u32p, u32p,
                                            u32p, u64p]
        L.oracle_validate_repeat_cache.restype = c_int
        L.oracle_validate_repeat_cache.argtypes = [c_u32, c_u32, c_u32, u32p, u32p, u32p, u64p, u8p,
                                                   u32p, u8p]
        L.oracle_csr_spmm.argtypes = [c_u32, i64p, u32p, vp, f32p, c_u32, c_int, c_int, f64p]
        L.oracle_swtcf_spmm.argtypes = [c_u32, c_u32, u32p, u32p, u32p, u32p, u64p, f32p, c_u32, c_u32,
                                        c_u32, f64p]
        L.oracle_kat_source_a.restype = ctypes.c_float
        L.oracle_kat_source_a.argtypes = [c_u32]
        L.oracle_kat_source_b.restype = ctypes.c_float
        L.oracle_kat_source_b.argtypes = [c_u32]
        L.oracle_kat_fill_x.argtypes = [c_u32, c_u32, f32p]
        L.oracle_kat_expected.argtypes = [u32p, u32p, c_u32, c_u32, c_u32, f64p]
        L.oracle_bcsr_count.restype = c_i64
        L.oracle_bcsr_count.argtypes = [c_u32, i64p, u32p]
        L.oracle_bcsr_build.argtypes = [c_u32, i64p, u32p, vp, u32p, u32p, u32p, u64p, f32p]
        L.oracle_bcsc_count.restype = c_i64
        L.oracle_bcsc_count.argtypes = [c_u32, i64p, u32p]
        L.oracle_bcsc_build.argtypes = [c_u32, i64p, u32p, vp, u32p, u32p, u32p, u64p, f32p]
        L.oracle_bcsr_spmm.argtypes = [c_u32, u32p, u32p, u32p, u64p, vp, c_u32, f32p, c_u32, f64p]
        L.oracle_bcsc_spmm.argtypes = [c_u32, u32p, u32p, u32p, u64p, vp, c_u32, c_u32, f32p, c_u32,
                                       f64p]
        L.oracle_bcsc_transpose_spmm.argtypes = [c_u32, u32p, u32p, u32p, u64p, vp, c_u32, f32p, c_u32,
                                                 f64p]
        L.oracle_resolve_features.restype = c_int
        L.oracle_resolve_features.argtypes = [c_u32, i32p, i32p, f32p, c_i32, f32p, c_i64, c_u32, f32p]
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _ptr_or_none(a):
    return None if a is None else a.ctypes.data_as(vp)


# ---------------------------------------------------------------- TF32
def tf32(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().oracle_tf32_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def tf32_bits(b: int) -> int:
    return int(lib().oracle_tf32_bits(b))


# ---------------------------------------------------------------- SWTCF
def swtcf_dims(cols: int, S: int):
    cw = (cols + 7) // 8
    sw = (cw + S - 1) // S
    return cw, sw


def swtcf_convert(dst, src, rows: int, cols: int, S: int = 16) -> dict:
    """Canonical SWTCF of a COO (src/swtcf_convert.cu:1754-2342).

    Returns a dict with the reference array names at their allocation
    capacities (nnz = E), plus ``err`` (device error code), ``numGroups``,
    ``numTiles`` (T) and ``numRows`` (U)."""
    dst = _c(dst, np.uint32)
    src = _c(src, np.uint32)
    E = dst.size
    cw, sw = swtcf_dims(cols, S)
    cap = max(E, 1)
    out = dict(
        colWindowOffset=np.zeros(cw + 1, np.uint32),
        superWindowRowOffset=np.zeros(sw + 1, np.uint32),
        superWindowRows=np.zeros(cap, np.uint32),
        superWindowRowCacheSlot=np.zeros(cap, np.uint8),
        superWindowCachedRowSlot=np.zeros(sw * CACHE_SIZE, np.uint32),
        superWindowCachedCount=np.zeros(max(sw, 1), np.uint8),
        tileRowSlot=np.zeros(cap * 8, np.uint32),
        tileLocalBit=np.zeros(cap, np.uint64),
    )
    ng = np.zeros(1, np.uint32)
    err = lib().oracle_swtcf_convert(
        dst, src, E, rows, cols, S, out["colWindowOffset"], out["superWindowRowOffset"],
        out["superWindowRows"], out["superWindowRowCacheSlot"], out["superWindowCachedRowSlot"],
        out["superWindowCachedCount"], out["tileRowSlot"], out["tileLocalBit"], ng)
    out.update(err=int(err), numGroups=int(ng[0]), numColWindows=cw, numSuperWindows=sw,
               superWindowSize=S, rows=rows, cols=cols)
    out["numTiles"] = int(out["colWindowOffset"][cw])
    out["numRows"] = int(out["superWindowRowOffset"][sw])
    return out


def swtcf_valid_extents(m: dict) -> dict:
    """The arrays restricted to the extents the reference defines (A.1 step 6)."""
    T, U = m["numTiles"], m["numRows"]
    return dict(
        colWindowOffset=m["colWindowOffset"],
        superWindowRowOffset=m["superWindowRowOffset"],
        tileLocalBit=m["tileLocalBit"][:T],
        tileRowSlot=m["tileRowSlot"][:T * 8],
        superWindowRows=m["superWindowRows"][:U],
        superWindowRowCacheSlot=m["superWindowRowCacheSlot"][:U],
        superWindowCachedRowSlot=m["superWindowCachedRowSlot"],
        superWindowCachedCount=m["superWindowCachedCount"][:m["numSuperWindows"]],
    )


def validate_swtcf(dst, src, numSrc: int, m: dict) -> int:
    """validateSWTCF (src/swtcf_convert_main.cu:36-130): 0 = PASS."""
    dst = _c(dst, np.uint32)
    src = _c(src, np.uint32)
    return int(lib().oracle_validate_swtcf(
        dst, src, dst.size, numSrc, m["superWindowSize"], m["numColWindows"],
        _c(m["colWindowOffset"], np.uint32), _c(m["superWindowRowOffset"], np.uint32),
        _c(m["superWindowRows"], np.uint32), _c(m["tileRowSlot"], np.uint32),
        _c(m["tileLocalBit"], np.uint64)))


def validate_repeat_cache(m: dict) -> int:
    """validateRepeatCacheMetadata (src/swtcf_convert_main.cu:132-310): 0 = PASS."""
    return int(lib().oracle_validate_repeat_cache(
        m["superWindowSize"], m["numColWindows"], m["numSuperWindows"],
        _c(m["colWindowOffset"], np.uint32), _c(m["superWindowRowOffset"], np.uint32),
        _c(m["tileRowSlot"], np.uint32), _c(m["tileLocalBit"], np.uint64),
        _c(m["superWindowRowCacheSlot"], np.uint8), _c(m["superWindowCachedRowSlot"], np.uint32),
        _c(m["superWindowCachedCount"], np.uint8)))


# ---------------------------------------------------------------- SpMM
def csr_spmm(rowptr, colind, vals, X, use_tf32: bool = True, threads: int = 0) -> np.ndarray:
    rowptr = _c(rowptr, np.int64)
    colind = _c(colind, np.uint32)
    X = _c(X, np.float32)
    rows = rowptr.size - 1
    F = X.shape[1]
    vals = None if vals is None else _c(vals, np.float32)
    Y = np.empty((rows, F), np.float64)
    lib().oracle_csr_spmm(rows, rowptr, colind, _ptr_or_none(vals), X, F, int(use_tf32), threads, Y)
    return Y


def swtcf_spmm(m: dict, X, tc: int = 12, rows: int | None = None, Y=None) -> np.ndarray:
    X = _c(X, np.float32)
    F = X.shape[1]
    if Y is None:
        Y = np.zeros((rows if rows is not None else m["rows"], F), np.float64)
    lib().oracle_swtcf_spmm(
        m["numColWindows"], m["superWindowSize"], _c(m["colWindowOffset"], np.uint32),
        _c(m["superWindowRowOffset"], np.uint32), _c(m["superWindowRows"], np.uint32),
        _c(m["tileRowSlot"], np.uint32), _c(m["tileLocalBit"], np.uint64), X, m["cols"], F, tc, Y)
    return Y


def kat_source_a(s: int) -> float:
    return float(lib().oracle_kat_source_a(s))


def kat_source_b(s: int) -> float:
    return float(lib().oracle_kat_source_b(s))


def kat_fill_x(numSrc: int, F: int = 128) -> np.ndarray:
    X = np.empty((numSrc, F), np.float32)
    lib().oracle_kat_fill_x(numSrc, F, X)
    return X


def kat_expected(dst, src, numDst: int, F: int = 128) -> np.ndarray:
    dst = _c(dst, np.uint32)
    src = _c(src, np.uint32)
    Y = np.empty((numDst, F), np.float64)
    lib().oracle_kat_expected(dst, src, dst.size, numDst, F, Y)
    return Y


# ---------------------------------------------------------------- BCSR / BCSC
def coo_to_csr(rows_idx, cols_idx, n_rows: int, vals=None):
    """Sort a COO by (row, col) into CSR arrays (rowptr int64, colind, vals)."""
    r = np.asarray(rows_idx, dtype=np.int64)
    c = np.asarray(cols_idx, dtype=np.int64)
    order = np.lexsort((c, r))
    rowptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n_rows), out=rowptr[1:])
    v = None if vals is None else np.asarray(vals, np.float32)[order]
    return rowptr, c[order].astype(np.uint32), v


def bcsr_build(n_rows: int, n_cols: int, rowptr, colind, vals=None) -> dict:
    rowptr = _c(rowptr, np.int64)
    colind = _c(colind, np.uint32)
    vals = None if vals is None else _c(vals, np.float32)
    L = lib()
    B = int(L.oracle_bcsr_count(n_rows, rowptr, colind))
    rw = (n_rows + 7) // 8
    d = dict(rowWindowOffset=np.zeros(rw + 1, np.uint32), tcOffset=np.zeros(B + 1, np.uint32),
             sparseA2B=np.zeros(max(B, 1) * 8, np.uint32), tcLocalBit=np.zeros(max(B, 1), np.uint64),
             data=np.zeros(max(colind.size, 1), np.float32))
    L.oracle_bcsr_build(n_rows, rowptr, colind, _ptr_or_none(vals), d["rowWindowOffset"], d["tcOffset"],
                        d["sparseA2B"], d["tcLocalBit"], d["data"])
    d.update(num_rows=n_rows, num_cols=n_cols, nnz=int(colind.size), num_TCBlocks=B, num_rowWindows=rw)
    return d


def bcsc_build(n_rows: int, n_cols: int, colptr, rowind, cvals=None) -> dict:
    colptr = _c(colptr, np.int64)
    rowind = _c(rowind, np.uint32)
    cvals = None if cvals is None else _c(cvals, np.float32)
    L = lib()
    B = int(L.oracle_bcsc_count(n_cols, colptr, rowind))
    cw = (n_cols + 7) // 8
    d = dict(colWindowOffset=np.zeros(cw + 1, np.uint32), tcOffset=np.zeros(B + 1, np.uint32),
             sparseA2C=np.zeros(max(B, 1) * 8, np.uint32), tcLocalBit=np.zeros(max(B, 1), np.uint64),
             data=np.zeros(max(rowind.size, 1), np.float32))
    L.oracle_bcsc_build(n_cols, colptr, rowind, _ptr_or_none(cvals), d["colWindowOffset"], d["tcOffset"],
                        d["sparseA2C"], d["tcLocalBit"], d["data"])
    d.update(num_rows=n_rows, num_cols=n_cols, nnz=int(rowind.size), num_TCBlocks=B, num_colWindows=cw)
    return d


def bcsr_spmm(A: dict, X, use_data: bool = False) -> np.ndarray:
    X = _c(X, np.float32)
    F = X.shape[1]
    Y = np.zeros((A["num_rowWindows"] * 8, F), np.float64)
    data = A["data"] if use_data else None
    lib().oracle_bcsr_spmm(A["num_rowWindows"], A["rowWindowOffset"], A["tcOffset"], A["sparseA2B"],
                           A["tcLocalBit"], _ptr_or_none(data), A["num_cols"], X, F, Y)
    return Y


def bcsc_spmm(A: dict, X, use_data: bool = False, Y=None) -> np.ndarray:
    X = _c(X, np.float32)
    F = X.shape[1]
    if Y is None:
        Y = np.zeros((A["num_rows"], F), np.float64)
    data = A["data"] if use_data else None
    lib().oracle_bcsc_spmm(A["num_colWindows"], A["colWindowOffset"], A["tcOffset"], A["sparseA2C"],
                           A["tcLocalBit"], _ptr_or_none(data), A["num_rows"], A["num_cols"], X, F, Y)
    return Y


def bcsc_transpose_spmm(A: dict, dY, use_data: bool = False) -> np.ndarray:
    dY = _c(dY, np.float32)
    F = dY.shape[1]
    dX = np.zeros((A["num_colWindows"] * 8, F), np.float64)
    data = A["data"] if use_data else None
    lib().oracle_bcsc_transpose_spmm(A["num_colWindows"], A["colWindowOffset"], A["tcOffset"],
                                     A["sparseA2C"], A["tcLocalBit"], _ptr_or_none(data),
                                     A["num_rows"], dY, F, dX)
    return dX


def resolve_features(id_map, cache_search_map, hot, cap: int, cpu, F: int) -> np.ndarray:
    id_map = _c(id_map, np.int32)
    csm = _c(cache_search_map, np.int32)
    hot = _c(hot, np.float32).reshape(-1)
    cpu = _c(cpu, np.float32).reshape(-1)
    X = np.empty((id_map.size, F), np.float32)
    rc = lib().oracle_resolve_features(id_map.size, id_map, csm, hot, cap, cpu, cpu.size, F, X)
    if rc:
        raise ValueError(f"oracle_resolve_features failed ({rc})")
    return X
