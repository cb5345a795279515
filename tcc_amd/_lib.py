"""ctypes binding of libtcc_swtcf.so (the C-ABI in include/tcc_swtcf.h and
include/tcc_spmm_cnic.h).  Loading fails loudly when the library is missing:
there is no CPU fallback for any entry point."""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtcc_swtcf.so")

u32, i32, i64, u64 = ctypes.c_uint32, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64
vp = ctypes.c_void_p
P32 = ctypes.POINTER(ctypes.c_uint32)
P8 = ctypes.POINTER(ctypes.c_uint8)
P64 = ctypes.POINTER(ctypes.c_uint64)
PF = ctypes.POINTER(ctypes.c_float)
PI32 = ctypes.POINTER(ctypes.c_int32)


class SWTCFMatrix(ctypes.Structure):
    """tcc_swtcf_matrix == DeviceSWTCFMatrix (include/swtcf_convert.cuh:13-35)."""
    _fields_ = [
        ("rows", u32), ("cols", u32), ("nnz", u32), ("colWindowWidth", u32), ("tileRows", u32),
        ("superWindowSize", u32), ("numColWindows", u32), ("numSuperWindows", u32),
        ("superWindowRowOffset", vp), ("superWindowRows", vp), ("superWindowRowCacheSlot", vp),
        ("superWindowCachedRowSlot", vp), ("superWindowCachedCount", vp), ("colWindowOffset", vp),
        ("tileRowSlot", vp), ("tileLocalBit", vp),
    ]


class SWTCFWorkspace(ctypes.Structure):
    _fields_ = [
        ("edgeCapacity", u32), ("numColWindows", u32), ("numSuperWindows", u32), ("superWindowSize", u32),
        ("deviceNumGroups", vp), ("deviceError", vp), ("scratch", vp), ("scratchBytes", ctypes.c_size_t),
    ]


class BCSR(ctypes.Structure):
    """tcc_bcsr == BCSR<T> (spmm_cnic/include/class.h:20-37) + value array."""
    _fields_ = [
        ("num_rows", u32), ("num_cols", u32), ("nnz", u32), ("num_TCBlocks", u32), ("num_rowWindows", u32),
        ("rowWindowOffset", vp), ("tcOffset", vp), ("sparseA2B", vp), ("tcLocalBit", vp), ("data", vp),
        ("unitBlocks", u32), ("phases", u32),
    ]


class BCSC(ctypes.Structure):
    """tcc_bcsc == BCSC<T> (spmm_cnic/include/class.h:39-58) + value array."""
    _fields_ = [
        ("num_rows", u32), ("num_cols", u32), ("nnz", u32), ("num_TCBlocks", u32), ("num_colWindows", u32),
        ("colWindowOffset", vp), ("tcOffset", vp), ("sparseA2C", vp), ("tcLocalBit", vp), ("data", vp),
        ("unitBlocks", u32),
    ]


class HubTiles(ctypes.Structure):
    """tcc_hub_tiles: dense 16x16 tiles of the degree-sorted matrix (no reference counterpart)."""
    _fields_ = [
        ("num_rows", u32), ("num_cols", u32), ("nnz", u32), ("group_blocks", u32), ("num_groups", u32),
        ("num_steps", u32), ("num_tiles", u32), ("num_units", u32), ("unit_steps", u32), ("hub_cols", u32),
        ("tile_format", u32),
        ("rowOrder", vp), ("hubColOrder", vp), ("groupStepOffset", vp), ("stepCol", vp), ("tileVals", vp),
        ("units", vp), ("unitOrder", vp),
        ("num_partial_units", u32), ("num_shared_groups", u32), ("unitPartial", vp), ("sharedGroups", vp),
        ("tileMasks", vp), ("rowScale", vp), ("colScale", vp),
    ]


class Hybrid(ctypes.Structure):
    """tcc_hybrid: hub tiles + the remainder's BCSR."""
    _fields_ = [("tiles", HubTiles), ("rest", BCSR), ("tilesAllocation", vp), ("restAllocation", vp),
                ("restRowScale", vp)]


class FeatureSource(ctypes.Structure):
    _fields_ = [
        ("id_map", vp), ("cache_search_map", vp), ("gpu_feature_cache", vp), ("gpu_node_capacity", i32),
        ("cpu_features", vp), ("cpu_feature_len", i64), ("gpu_feature_cache_count", u32), ("row_format", u32),
        ("device_error", vp),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "tcc_last_error": (ctypes.c_char_p, []),
    "tcc_swtcf_alloc_matrix": (ctypes.c_int, [ctypes.POINTER(SWTCFMatrix), u32, u32, u32, u32]),
    "tcc_swtcf_free_matrix": (ctypes.c_int, [ctypes.POINTER(SWTCFMatrix)]),
    "tcc_swtcf_alloc_workspace": (ctypes.c_int, [ctypes.POINTER(SWTCFWorkspace), u32, u32, u32]),
    "tcc_swtcf_free_workspace": (ctypes.c_int, [ctypes.POINTER(SWTCFWorkspace)]),
    "tcc_swtcf_convert": (ctypes.c_int, [vp, vp, u32, ctypes.POINTER(SWTCFMatrix), ctypes.POINTER(SWTCFWorkspace),
                                         vp]),
    "tcc_swtcf_spmm": (ctypes.c_int, [ctypes.POINTER(SWTCFMatrix), vp, vp, u32, vp]),
    "tcc_swtcf_spmm_f": (ctypes.c_int, [ctypes.POINTER(SWTCFMatrix), vp, vp, u32, u32, vp]),
    "tcc_swtcf_spmm_mfma": (ctypes.c_int, [ctypes.POINTER(SWTCFMatrix), vp, vp, u32, u32, u32, vp]),
    "tcc_swtcf_spmm_quantized": (ctypes.c_int, [ctypes.POINTER(SWTCFMatrix), vp, vp, vp, vp, u32, vp]),
    "tcc_swtcf_set_plans": (ctypes.c_int, [u32]),
    "tcc_swtcf_release_plans": (ctypes.c_int, []),
    "tcc_swtcf_plans_built": (u32, []),
    "tcc_hash_arrays": (ctypes.c_int, [vp, vp, u32, vp, vp]),
    "tcc_bcsr_spmm": (ctypes.c_int, [ctypes.POINTER(BCSR), vp, vp, u32, ctypes.c_int, vp]),
    "tcc_bcsr_spmm_mixed": (ctypes.c_int, [ctypes.POINTER(BCSR), ctypes.POINTER(FeatureSource), vp, u32,
                                           ctypes.c_int, vp]),
    "tcc_bcsc_spmm": (ctypes.c_int, [ctypes.POINTER(BCSC), vp, vp, u32, vp]),
    "tcc_bcsc_transpose_spmm": (ctypes.c_int, [ctypes.POINTER(BCSC), vp, vp, u32, ctypes.c_int, vp]),
    "tcc_spmm_cnic_forward": (ctypes.c_int, [ctypes.POINTER(BCSR), ctypes.POINTER(BCSC), vp, vp, u32, vp]),
    "tcc_spmm_cnic_forward_mixed": (ctypes.c_int, [ctypes.POINTER(BCSR), ctypes.POINTER(BCSC),
                                                   ctypes.POINTER(FeatureSource), vp, u32, vp]),
    "tcc_coo_to_bcsr": (ctypes.c_int, [vp, vp, vp, u32, u32, u32, ctypes.POINTER(BCSR), ctypes.POINTER(vp), vp]),
    "tcc_coo_to_bcsr_phased": (ctypes.c_int, [vp, vp, vp, u32, u32, u32, u32, ctypes.POINTER(BCSR),
                                              ctypes.POINTER(vp), vp]),
    "tcc_coo_to_bcsc": (ctypes.c_int, [vp, vp, vp, u32, u32, u32, ctypes.POINTER(BCSC), ctypes.POINTER(vp), vp]),
    "tcc_block_release": (ctypes.c_int, [vp]),
    "tcc_tf32_packed_bytes": (ctypes.c_size_t, [u32, u32]),
    "tcc_tf32_pack": (ctypes.c_int, [vp, u32, u32, vp, vp]),
    "tcc_bcsr_spmm_packed": (ctypes.c_int, [ctypes.POINTER(BCSR), vp, vp, u32, ctypes.c_int, vp]),
    "tcc_coo_to_hybrid": (ctypes.c_int, [vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, u32, ctypes.POINTER(Hybrid),
                                         vp]),
    "tcc_coo_to_hybrid_scaled": (ctypes.c_int, [vp, vp, u32, u32, u32, vp, vp, u32, u32, u32, u32,
                                                 ctypes.POINTER(Hybrid), vp]),
    "tcc_hybrid_release": (ctypes.c_int, [ctypes.POINTER(Hybrid)]),
    "tcc_calibration_atomic": (ctypes.c_int, [vp, u32, u32, ctypes.c_uint64, vp]),
    "tcc_hybrid_from_bcsr": (ctypes.c_int, [ctypes.POINTER(BCSR), ctypes.c_int, u32, u32, ctypes.POINTER(Hybrid),
                                            vp]),
    "tcc_spmm_cnic_forward_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(BCSR), u32]),
    "tcc_spmm_cnic_forward_ws": (ctypes.c_int, [ctypes.POINTER(BCSR), ctypes.POINTER(BCSC), vp, vp, u32, vp,
                                                ctypes.c_size_t, vp]),
    "tcc_hybrid_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Hybrid), u32]),
    "tcc_hub_tiles_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(HubTiles), u32]),
    "tcc_hybrid_spmm": (ctypes.c_int, [ctypes.POINTER(Hybrid), vp, vp, u32, ctypes.c_int, vp, ctypes.c_size_t, vp]),
    "tcc_hub_tiles_spmm": (ctypes.c_int, [ctypes.POINTER(HubTiles), vp, vp, u32, vp, ctypes.c_size_t, vp]),
    "tcc_dense_tn_workspace_bytes": (ctypes.c_size_t, [u32, u32, u32]),
    "tcc_calibration_copy": (ctypes.c_int, [vp, vp, ctypes.c_size_t, vp]),
    "tcc_dense_tn": (ctypes.c_int, [vp, u32, vp, u32, vp, u32, u32, u32, u32, ctypes.c_int, vp, ctypes.c_size_t, vp]),
    "tcc_dense_tn_noalloc": (ctypes.c_int, [vp, u32, vp, u32, vp, u32, u32, u32, u32, ctypes.c_int, vp]),
    "tcc_gcn_relu_forward": (ctypes.c_int, [vp, u32, vp, vp, vp, u32, vp, u32, u32, u32, u32, u32, vp]),
    "tcc_gcn_relu_grad_workspace_bytes": (ctypes.c_size_t, [u32, u32, u32, u32]),
    "tcc_gcn_relu_grad": (ctypes.c_int, [vp, u32, vp, u32, vp, u32, vp, vp, vp, u32, u32, u32, u32, vp, ctypes.c_size_t,
                                         vp]),
}

_lib = None


class TccError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"tcc error {code}: {msg}")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m tcc_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise TccError(rc, lib().tcc_last_error().decode())
