"""Python host API over the C-ABI, for tests, the bench and Python callers.

Device memory and streams come from PyTorch-ROCm; all compute runs in
libtcc_swtcf.so.  Names follow the reference C++ API
(include/swtcf_convert.cuh:74-78, include/swtcf_spmm.cuh:10-25).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import BCSC, BCSR, FeatureSource, Hybrid, SWTCFMatrix, SWTCFWorkspace, check

INVALID_ROW_SLOT = 0xFFFFFFFF
INVALID_CACHE_SLOT = 0xFF
REPEAT_CACHE_SIZE = 32
DEFAULT_TC_THRESHOLD = 12
DEVERR_FEATURE_INDEX = 7  # TCC_DEVERR_FEATURE_INDEX
TILES_FP32, TILES_BF16X2, TILES_BINARY = 0, 1, 2  # TCC_TILES_*
FEATURE_DIM = 128


_hip = None


def _hip_memcpy_d2h(dst: np.ndarray, src_ptr: int) -> None:
    """hipMemcpy(device -> host) into a numpy array (synchronous)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    if dst.nbytes:
        err = _hip.hipMemcpy(dst.ctypes.data, src_ptr, dst.nbytes, 2)  # hipMemcpyDeviceToHost
        if err != 0:
            raise RuntimeError(f"hipMemcpy failed ({err})")


def _download(ptr: int, count: int, dtype) -> np.ndarray:
    out = np.empty(int(count), dtype=dtype)
    if count:
        _hip_memcpy_d2h(out, ptr)
    return out


def _stream(stream=None) -> int:
    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _f32(t: torch.Tensor, name: str) -> torch.Tensor:
    """A contiguous float32 device tensor (the kernels read raw fp32)."""
    if t.dtype != torch.float32 or not t.is_cuda:
        raise TypeError(f"{name} must be a float32 device tensor (got {t.dtype} on {t.device})")
    return t.contiguous()


def _u32(t: torch.Tensor) -> torch.Tensor:
    """int32/uint32 device tensor viewed as u32 storage (contiguous)."""
    if t.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"index tensors must be int32/uint32, got {t.dtype}")
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("index tensors must be contiguous device tensors")
    return t


class DeviceSWTCFMatrix:
    """Owns one SWTCF matrix in device memory (allocateDeviceSWTCF /
    freeDeviceSWTCF, src/swtcf_convert.cu:1113-1303)."""

    def __init__(self, rows: int, cols: int, nnz: int, superWindowSize: int = 16):
        self.m = SWTCFMatrix()
        check(_lib.lib().tcc_swtcf_alloc_matrix(ctypes.byref(self.m), rows, cols, nnz, superWindowSize))

    def free(self) -> None:
        if self.m.superWindowRowOffset:
            check(_lib.lib().tcc_swtcf_free_matrix(ctypes.byref(self.m)))

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def numColWindows(self) -> int:
        return self.m.numColWindows

    @property
    def numSuperWindows(self) -> int:
        return self.m.numSuperWindows

    def to_host(self) -> dict:
        """All arrays at their valid extents (SWTCF semantics, A.1 step 6),
        as numpy, with the reference names."""
        torch.cuda.synchronize()
        m = self.m
        cw, sw = m.numColWindows, m.numSuperWindows
        cwo = _download(m.colWindowOffset, cw + 1, np.uint32)
        swo = _download(m.superWindowRowOffset, sw + 1, np.uint32)
        T, U = int(cwo[-1]), int(swo[-1])
        d = dict(
            colWindowOffset=cwo, superWindowRowOffset=swo,
            tileLocalBit=_download(m.tileLocalBit, T, np.uint64),
            tileRowSlot=_download(m.tileRowSlot, 8 * T, np.uint32),
            superWindowRows=_download(m.superWindowRows, U, np.uint32),
            superWindowRowCacheSlot=_download(m.superWindowRowCacheSlot, U, np.uint8),
            superWindowCachedRowSlot=_download(m.superWindowCachedRowSlot, 32 * sw, np.uint32),
            superWindowCachedCount=_download(m.superWindowCachedCount, sw, np.uint8),
        )
        d.update(numTiles=T, numRows=U, numColWindows=cw, numSuperWindows=sw, superWindowSize=m.superWindowSize,
                 rows=m.rows, cols=m.cols)
        return d


class SWTCFConvertWorkspace:
    """allocateSWTCFConvertWorkspace / freeSWTCFConvertWorkspace
    (src/swtcf_convert.cu:1306-1751)."""

    def __init__(self, edgeCapacity: int, numSrc: int, superWindowSize: int = 16):
        self.ws = SWTCFWorkspace()
        check(_lib.lib().tcc_swtcf_alloc_workspace(ctypes.byref(self.ws), edgeCapacity, numSrc, superWindowSize))

    def free(self) -> None:
        if self.ws.scratch:
            check(_lib.lib().tcc_swtcf_free_workspace(ctypes.byref(self.ws)))

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def device_error(self) -> int:
        """workspace.deviceError after the stream is drained (0 = none)."""
        torch.cuda.synchronize()
        return int(_download(self.ws.deviceError, 1, np.uint32)[0])

    def num_groups(self) -> int:
        torch.cuda.synchronize()
        return int(_download(self.ws.deviceNumGroups, 1, np.uint32)[0])


def convertCOOToSWTCF(dst: torch.Tensor, src: torch.Tensor, numEdges: int, output: DeviceSWTCFMatrix,
                      workspace: SWTCFConvertWorkspace, stream=None) -> None:
    _u32(dst)
    _u32(src)
    check(_lib.lib().tcc_swtcf_convert(dst.data_ptr(), src.data_ptr(), numEdges, ctypes.byref(output.m),
                                       ctypes.byref(workspace.ws), _stream(stream)))


def launchSWTCFSpMM(matrix: DeviceSWTCFMatrix, X: torch.Tensor, Y: torch.Tensor,
                    tcThreshold: int = DEFAULT_TC_THRESHOLD, stream=None) -> None:
    """Y += A X with F = 128 (src/swtcf_spmm.cu:437-466)."""
    check(_lib.lib().tcc_swtcf_spmm(ctypes.byref(matrix.m), X.data_ptr(), Y.data_ptr(), tcThreshold,
                                    _stream(stream)))


def swtcf_spmm(matrix: DeviceSWTCFMatrix, X: torch.Tensor, Y: torch.Tensor,
               tcThreshold: int = DEFAULT_TC_THRESHOLD, stream=None) -> None:
    """Y += A X for any feature width (X: [cols x F], Y: [rows x F])."""
    F = X.shape[1]
    check(_lib.lib().tcc_swtcf_spmm_f(ctypes.byref(matrix.m), X.data_ptr(), Y.data_ptr(), F, tcThreshold,
                                      _stream(stream)))


def swtcf_spmm_mfma(matrix: DeviceSWTCFMatrix, X: torch.Tensor, Y: torch.Tensor,
                    tcThreshold: int = DEFAULT_TC_THRESHOLD, mfmaThreshold: int = 65, stream=None) -> None:
    """Y += A X with tiles of >= max(mfmaThreshold, tcThreshold) entries on
    fp32 MFMA (tcc_swtcf_spmm_mfma; > 64: never)."""
    F = X.shape[1]
    check(_lib.lib().tcc_swtcf_spmm_mfma(ctypes.byref(matrix.m), X.data_ptr(), Y.data_ptr(), F, tcThreshold,
                                         mfmaThreshold, _stream(stream)))


def launchSWTCFSpMMQuantized(matrix: DeviceSWTCFMatrix, quantizedX: torch.Tensor, scales: torch.Tensor,
                             srcGlobal: torch.Tensor, Y: torch.Tensor, tcThreshold: int = DEFAULT_TC_THRESHOLD,
                             stream=None) -> None:
    check(_lib.lib().tcc_swtcf_spmm_quantized(ctypes.byref(matrix.m), quantizedX.data_ptr(), scales.data_ptr(),
                                              srcGlobal.data_ptr(), Y.data_ptr(), tcThreshold, _stream(stream)))


# ---------------------------------------------------------------- BCSR / BCSC


class BlockMatrix:
    """A BCSR or BCSC built on the device by tcc_coo_to_bcsr/bcsc (owns one
    allocation) or wrapping caller tensors (owns nothing)."""

    def __init__(self, kind: str, view, allocation=None, keep=()):
        self.kind = kind
        self.view = view
        self._alloc = allocation
        self._keep = keep

    def release(self) -> None:
        if self._alloc:
            check(_lib.lib().tcc_block_release(self._alloc))
            self._alloc = None

    def set_unit_blocks(self, unit_blocks: int) -> "BlockMatrix":
        """Blocks each wave of work walks (0 = chosen from the block count)."""
        self.view.unitBlocks = int(unit_blocks)
        return self

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    @property
    def num_windows(self) -> int:
        return self.view.num_rowWindows if self.kind == "bcsr" else self.view.num_colWindows

    @property
    def phases(self) -> int:
        return max(1, self.view.phases) if self.kind == "bcsr" else 1

    @property
    def out_windows(self) -> int:
        """8-row windows of the product's output (a phased BCSR has
        `phases` row windows per output window)."""
        return self.num_windows // self.phases

    def to_host(self) -> dict:
        torch.cuda.synchronize()
        v = self.view
        B, W = v.num_TCBlocks, self.num_windows
        woff = "rowWindowOffset" if self.kind == "bcsr" else "colWindowOffset"
        idx = "sparseA2B" if self.kind == "bcsr" else "sparseA2C"
        d = {
            woff: _download(getattr(v, woff), W + 1, np.uint32),
            "tcOffset": _download(v.tcOffset, B + 1, np.uint32),
            idx: _download(getattr(v, idx), 8 * B, np.uint32),
            "tcLocalBit": _download(v.tcLocalBit, B, np.uint64),
            "data": _download(v.data, v.nnz, np.float32) if v.data else None,
        }
        d.update(num_rows=v.num_rows, num_cols=v.num_cols, nnz=v.nnz, num_TCBlocks=B)
        d["num_rowWindows" if self.kind == "bcsr" else "num_colWindows"] = W
        if self.kind == "bcsr":
            d["phases"] = self.phases
        return d


def coo_to_bcsr(row: torch.Tensor, col: torch.Tensor, val: torch.Tensor | None, num_rows: int, num_cols: int,
                stream=None, phases: int = 1) -> BlockMatrix:
    """BCSR of the COO matrix; phases > 1 builds the phased form
    (tcc_coo_to_bcsr_phased), taken by bcsr_spmm and bcsr_spmm_packed."""
    view = BCSR()
    alloc = ctypes.c_void_p()
    check(_lib.lib().tcc_coo_to_bcsr_phased(_u32(row).data_ptr(), _u32(col).data_ptr(), _ptr(val), row.numel(),
                                            num_rows, num_cols, int(phases), ctypes.byref(view), ctypes.byref(alloc),
                                            _stream(stream)))
    return BlockMatrix("bcsr", view, alloc.value)


def coo_to_bcsc(row: torch.Tensor, col: torch.Tensor, val: torch.Tensor | None, num_rows: int, num_cols: int,
                stream=None) -> BlockMatrix:
    view = BCSC()
    alloc = ctypes.c_void_p()
    check(_lib.lib().tcc_coo_to_bcsc(_u32(row).data_ptr(), _u32(col).data_ptr(), _ptr(val), row.numel(), num_rows,
                                     num_cols, ctypes.byref(view), ctypes.byref(alloc), _stream(stream)))
    return BlockMatrix("bcsc", view, alloc.value)


def wrap_bcsr(num_rows, num_cols, nnz, num_TCBlocks, num_rowWindows, rowWindowOffset, tcOffset, sparseA2B,
              tcLocalBit, data=None, phases: int = 1) -> BlockMatrix:
    """View caller-owned device tensors as a BCSR (no copy)."""
    v = BCSR(num_rows, num_cols, nnz, num_TCBlocks, num_rowWindows, _ptr(rowWindowOffset), _ptr(tcOffset),
             _ptr(sparseA2B), _ptr(tcLocalBit), _ptr(data), 0, int(phases))
    return BlockMatrix("bcsr", v, None, keep=(rowWindowOffset, tcOffset, sparseA2B, tcLocalBit, data))


def wrap_bcsc(num_rows, num_cols, nnz, num_TCBlocks, num_colWindows, colWindowOffset, tcOffset, sparseA2C,
              tcLocalBit, data=None) -> BlockMatrix:
    v = BCSC(num_rows, num_cols, nnz, num_TCBlocks, num_colWindows, _ptr(colWindowOffset), _ptr(tcOffset),
             _ptr(sparseA2C), _ptr(tcLocalBit), _ptr(data))
    return BlockMatrix("bcsc", v, None, keep=(colWindowOffset, tcOffset, sparseA2C, tcLocalBit, data))


def host_to_bcsr(d: dict, use_data: bool = False) -> BlockMatrix:
    """Upload a host BCSR dict (numpy arrays, reference names) and wrap it."""
    t = {k: torch.from_numpy(np.ascontiguousarray(d[k]).view(np.int32 if d[k].dtype == np.uint32 else
                                                              (np.int64 if d[k].dtype == np.uint64 else d[k].dtype)))
         .cuda() for k in ("rowWindowOffset", "tcOffset", "sparseA2B", "tcLocalBit", "data")}
    return wrap_bcsr(d["num_rows"], d["num_cols"], d["nnz"], d["num_TCBlocks"], d["num_rowWindows"],
                     t["rowWindowOffset"], t["tcOffset"], t["sparseA2B"], t["tcLocalBit"],
                     t["data"] if use_data else None, d.get("phases", 1))


def host_to_bcsc(d: dict, use_data: bool = False) -> BlockMatrix:
    t = {k: torch.from_numpy(np.ascontiguousarray(d[k]).view(np.int32 if d[k].dtype == np.uint32 else
                                                              (np.int64 if d[k].dtype == np.uint64 else d[k].dtype)))
         .cuda() for k in ("colWindowOffset", "tcOffset", "sparseA2C", "tcLocalBit", "data")}
    return wrap_bcsc(d["num_rows"], d["num_cols"], d["nnz"], d["num_TCBlocks"], d["num_colWindows"],
                     t["colWindowOffset"], t["tcOffset"], t["sparseA2C"], t["tcLocalBit"],
                     t["data"] if use_data else None)


def bcsr_spmm(A: BlockMatrix, X: torch.Tensor, Y: torch.Tensor | None = None, accumulate: bool = False,
              stream=None) -> torch.Tensor:
    """Y[8*W x F] (=|+=) A X, W = A.out_windows."""
    X = _f32(X, "X")
    F = X.shape[1]
    if Y is None:
        Y = torch.empty((A.out_windows * 8, F), dtype=torch.float32, device=X.device)
    check(_lib.lib().tcc_bcsr_spmm(ctypes.byref(A.view), X.data_ptr(), Y.data_ptr(), F, int(accumulate),
                                   _stream(stream)))
    return Y


def tf32_pack(X: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """TF32(X) packed in 2.5 bytes per element (tcc_tf32_pack); a uint8
    device tensor of tcc_tf32_packed_bytes(rows, F) bytes."""
    X = _f32(X, "X")
    rows, F = X.shape
    nbytes = _lib.lib().tcc_tf32_packed_bytes(rows, F)
    if out is None:
        out = torch.empty(nbytes + 16, dtype=torch.uint8, device=X.device)
    base = out.data_ptr()
    shift = (-base) % 16
    packed = out[shift:shift + nbytes]
    check(_lib.lib().tcc_tf32_pack(X.data_ptr(), rows, F, packed.data_ptr(), _stream(stream)))
    return packed


def bcsr_spmm_packed(A: BlockMatrix, packed: torch.Tensor, F: int, Y: torch.Tensor | None = None,
                     accumulate: bool = False, stream=None) -> torch.Tensor:
    """Y[8*W x F] (=|+=) A X with X given by tf32_pack, W = A.out_windows."""
    if Y is None:
        Y = torch.empty((A.out_windows * 8, F), dtype=torch.float32, device=packed.device)
    check(_lib.lib().tcc_bcsr_spmm_packed(ctypes.byref(A.view), packed.data_ptr(), Y.data_ptr(), F,
                                          int(accumulate), _stream(stream)))
    return Y


class HybridMatrix:
    """Dense hub tiles (MFMA) + the remainder's BCSR, built on the device by
    tcc_coo_to_hybrid; owns both allocations."""

    def __init__(self, view: Hybrid):
        self.view = view
        self.rest = BlockMatrix("bcsr", view.rest)  # a view: the allocation stays with the hybrid

    def release(self) -> None:
        if self.view.tilesAllocation or self.view.restAllocation:
            check(_lib.lib().tcc_hybrid_release(ctypes.byref(self.view)))

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    @property
    def out_rows(self) -> int:
        """Rows of Y: 8 per output row window of the remainder's BCSR."""
        return self.rest.out_windows * 8

    def workspace_bytes(self, F: int) -> int:
        return int(_lib.lib().tcc_hybrid_workspace_bytes(ctypes.byref(self.view), F))

    def to_host(self) -> dict:
        torch.cuda.synchronize()
        t = self.view.tiles
        G, NG, S, U = t.group_blocks, t.num_groups, t.num_steps, t.num_units
        NSG = t.num_shared_groups
        d = {
            "rowOrder": _download(t.rowOrder, 16 * G * NG, np.uint32),
            "hubColOrder": _download(t.hubColOrder, t.hub_cols, np.uint32),
            "groupStepOffset": _download(t.groupStepOffset, NG + 1, np.uint32),
            "stepCol": _download(t.stepCol, S, np.uint32),
            "tile_format": t.tile_format,
            "units": _download(t.units, 3 * U, np.uint32).reshape(U, 3),
            "unitOrder": _download(t.unitOrder, U, np.uint32),
            "unitPartial": _download(t.unitPartial, U, np.uint32),
            "sharedGroups": _download(t.sharedGroups, 3 * NSG, np.uint32).reshape(NSG, 3),
            "num_partial_units": t.num_partial_units, "num_shared_groups": NSG,
            "group_blocks": G, "num_groups": NG, "num_steps": S, "num_tiles": t.num_tiles, "num_units": U,
            "hub_cols": t.hub_cols, "tile_nnz": t.nnz, "unit_steps": t.unit_steps,
            "rest": self.rest.to_host(),
        }
        if t.tile_format == TILES_BINARY:
            # sub-step p's 96 G bytes (value masks, then positions; with the zero sub-step after the last)
            d["tileMasks"] = _download(t.tileMasks, 24 * G * (S + 1), np.uint32).view(np.uint8).reshape(S + 1, 96 * G)
            d["rowScale"] = None if not t.rowScale else _download(t.rowScale, 16 * G * NG, np.float32)
            d["colScale"] = None if not t.colScale else _download(t.colScale, t.num_cols, np.float32)
            n8 = (t.num_rows + 7) // 8 * 8
            d["restRowScale"] = None if not self.view.restRowScale else _download(self.view.restRowScale, n8,
                                                                                   np.float32)
        elif t.tile_format == TILES_FP32:
            d["tileVals"] = _download(t.tileVals, 256 * G * S, np.float32).reshape(S, G, 64, 4)
        else:
            d["tileVals"] = _download(t.tileVals, 512 * G * S, np.uint16).reshape(S, G, 2, 16, 16)
        return d


def coo_to_hybrid(row: torch.Tensor, col: torch.Tensor, val: torch.Tensor | None, num_rows: int, num_cols: int,
                  min_tile_nnz: int = 0, group_blocks: int = 0, unit_steps: int = 0, tile_format: int = TILES_BF16X2,
                  phases: int = 1, stream=None) -> HybridMatrix:
    """Dense hub tiles + remainder BCSR of the COO matrix (tcc_coo_to_hybrid)."""
    view = Hybrid()
    check(_lib.lib().tcc_coo_to_hybrid(_u32(row).data_ptr() if row.numel() else None,
                                       _u32(col).data_ptr() if col.numel() else None, _ptr(val), row.numel(),
                                       num_rows, num_cols, int(min_tile_nnz), int(group_blocks), int(unit_steps),
                                       int(tile_format), int(phases), ctypes.byref(view), _stream(stream)))
    return HybridMatrix(view)


def coo_to_hybrid_scaled(row: torch.Tensor, col: torch.Tensor, num_rows: int, num_cols: int,
                         row_scale: torch.Tensor | None = None, col_scale: torch.Tensor | None = None,
                         min_step_nnz: int = 0, group_blocks: int = 0, unit_steps: int = 0, phases: int = 1,
                         stream=None) -> HybridMatrix:
    """Binary hub tiles + pattern remainder of diag(row_scale) P diag(col_scale),
    P the COO's pattern (tcc_coo_to_hybrid_scaled); the scales are copied."""
    rs = None if row_scale is None else _f32(row_scale.reshape(-1), "row_scale")
    cs = None if col_scale is None else _f32(col_scale.reshape(-1), "col_scale")
    if rs is not None and rs.shape[0] != num_rows:
        raise ValueError("row_scale must have num_rows entries")
    if cs is not None and cs.shape[0] != num_cols:
        raise ValueError("col_scale must have num_cols entries")
    view = Hybrid()
    check(_lib.lib().tcc_coo_to_hybrid_scaled(_u32(row).data_ptr() if row.numel() else None,
                                              _u32(col).data_ptr() if col.numel() else None, row.numel(),
                                              num_rows, num_cols, _ptr(rs), _ptr(cs), int(min_step_nnz),
                                              int(group_blocks), int(unit_steps), int(phases), ctypes.byref(view),
                                              _stream(stream)))
    return HybridMatrix(view)


def hybrid_from_bcsr(A: BlockMatrix, use_values: bool = False, min_step_nnz: int = 0, phases: int = 0,
                     stream=None) -> HybridMatrix:
    """The hybrid of a BCSR's own entries (tcc_hybrid_from_bcsr): binary
    tiles over its pattern, or split-TF32 value tiles with use_values."""
    if A.kind != "bcsr":
        raise TypeError("hybrid_from_bcsr takes a BCSR")
    view = Hybrid()
    check(_lib.lib().tcc_hybrid_from_bcsr(ctypes.byref(A.view), int(use_values), int(min_step_nnz), int(phases),
                                          ctypes.byref(view), _stream(stream)))
    return HybridMatrix(view)


def hybrid_spmm(H: HybridMatrix, X: torch.Tensor, Y: torch.Tensor | None = None, accumulate: bool = False,
                workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Y[out_rows x F] (=|+=) A X (tcc_hybrid_spmm); `workspace` (uint8,
    at least H.workspace_bytes(F) + 16 bytes) is allocated when not given."""
    X = _f32(X, "X")
    F = X.shape[1]
    if Y is None:
        Y = torch.empty((H.out_rows, F), dtype=torch.float32, device=X.device)
    need = H.workspace_bytes(F)
    if workspace is None:
        workspace = torch.empty(need + 16, dtype=torch.uint8, device=X.device)
    base = workspace.data_ptr()
    shift = (-base) % 16
    check(_lib.lib().tcc_hybrid_spmm(ctypes.byref(H.view), X.data_ptr(), Y.data_ptr(), F, int(accumulate),
                                     base + shift, workspace.numel() - shift, _stream(stream)))
    return Y


def hub_tiles_spmm(H: HybridMatrix, X: torch.Tensor, Y: torch.Tensor, workspace: torch.Tensor | None = None,
                   stream=None) -> torch.Tensor:
    """Y[out_rows x F] += the hub tiles' share of A X alone
    (tcc_hub_tiles_spmm, without the remainder); `workspace` as hybrid_spmm,
    at least tcc_hub_tiles_workspace_bytes + 16 bytes."""
    X = _f32(X, "X")
    F = X.shape[1]
    need = int(_lib.lib().tcc_hub_tiles_workspace_bytes(ctypes.byref(H.view.tiles), F))
    if workspace is None:
        workspace = torch.empty(need + 16, dtype=torch.uint8, device=X.device)
    base = workspace.data_ptr()
    shift = (-base) % 16
    check(_lib.lib().tcc_hub_tiles_spmm(ctypes.byref(H.view.tiles), X.data_ptr(), Y.data_ptr(), F, base + shift,
                                        workspace.numel() - shift, _stream(stream)))
    return Y


def bcsc_spmm(A: BlockMatrix, X: torch.Tensor, Y: torch.Tensor, stream=None) -> torch.Tensor:
    """Y[num_rows x F] += A X with atomics."""
    X = _f32(X, "X")
    check(_lib.lib().tcc_bcsc_spmm(ctypes.byref(A.view), X.data_ptr(), Y.data_ptr(), X.shape[1], _stream(stream)))
    return Y


def bcsc_transpose_spmm(A: BlockMatrix, dY: torch.Tensor, dX: torch.Tensor | None = None, accumulate: bool = False,
                        stream=None) -> torch.Tensor:
    """dX[8*CW x F] (=|+=) A^T dY."""
    dY = _f32(dY, "dY")
    F = dY.shape[1]
    if dX is None:
        dX = torch.empty((A.view.num_colWindows * 8, F), dtype=torch.float32, device=dY.device)
    check(_lib.lib().tcc_bcsc_transpose_spmm(ctypes.byref(A.view), dY.data_ptr(), dX.data_ptr(), F,
                                             int(accumulate), _stream(stream)))
    return dX


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    """A float32 device matrix whose rows are contiguous (row stride free)."""
    if t.dtype != torch.float32 or not t.is_cuda or t.dim() != 2:
        raise TypeError(f"{name} must be a 2-D float32 device tensor (got {t.dtype} {tuple(t.shape)} on {t.device})")
    if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        t = t.contiguous()
    return t


def dense_tn(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor | None = None, accumulate: bool = False,
             stream=None) -> torch.Tensor:
    """C[M x N] (=|+=) A^T B for A [K x M], B [K x N] (tcc_dense_tn): the
    weight gradient torch.mm(X_out.T, d_output) of the GCN layer backward
    (train/tcgnn_conv_release.py:150), split over K on fp32 MFMA."""
    A, B = _rows(A, "A"), _rows(B, "B")
    K, M = A.shape
    if B.shape[0] != K:
        raise ValueError(f"A and B need the same number of rows (got {K} and {B.shape[0]})")
    N = B.shape[1]
    if C is None:
        C = torch.empty((M, N), dtype=torch.float32, device=A.device)
    elif C.shape != (M, N) or C.dtype != torch.float32 or C.stride(1) != 1:
        raise ValueError(f"C must be a float32 [{M} x {N}] tensor with contiguous rows")
    nbytes = _lib.lib().tcc_dense_tn_workspace_bytes(K, M, N)
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=A.device)
    check(_lib.lib().tcc_dense_tn(A.data_ptr(), A.stride(0), B.data_ptr(), B.stride(0), C.data_ptr(), C.stride(0),
                                  K, M, N, int(accumulate), ws.data_ptr(), nbytes, _stream(stream)))
    return C


def gcn_relu_forward_supported(F: int, Hd: int, C: int) -> bool:
    return F <= 128 and Hd <= 256 and C <= 4


def gcn_relu_forward(AX: torch.Tensor, W1: torch.Tensor, W2: torch.Tensor,
                     stream=None) -> tuple[torch.Tensor, torch.Tensor]:
    """(H, XW) = (relu(AX W1), H W2) in one pass (tcc_gcn_relu_forward), for
    AX [K x F], W1 [F x Hd], W2 [Hd x C]."""
    AX = _rows(AX, "AX")
    W1, W2 = _f32(W1, "W1"), _f32(W2, "W2")
    K, F = AX.shape
    Hd, C = W2.shape
    if W1.shape != (F, Hd):
        raise ValueError(f"shape mismatch: AX {tuple(AX.shape)}, W1 {tuple(W1.shape)}, W2 {tuple(W2.shape)}")
    H = torch.empty((K, Hd), dtype=torch.float32, device=AX.device)
    XW = torch.empty((K, C), dtype=torch.float32, device=AX.device)
    check(_lib.lib().tcc_gcn_relu_forward(AX.data_ptr(), AX.stride(0), W1.data_ptr(), W2.data_ptr(), H.data_ptr(),
                                          Hd, XW.data_ptr(), C, K, F, Hd, C, _stream(stream)))
    return H, XW


def gcn_relu_grad(AX: torch.Tensor, H: torch.Tensor, G: torch.Tensor, W2: torch.Tensor,
                  stream=None) -> tuple[torch.Tensor, torch.Tensor]:
    """(dW1, dW2) of conv_final(relu(conv1(X))) in one pass (tcc_gcn_relu_grad):
    dW1 = AXᵀ((G W2ᵀ) ⊙ [H > 0]), dW2 = Hᵀ G, for AX [K x F], H [K x Hd],
    G [K x C] and W2 [Hd x C]."""
    AX, H, G = _rows(AX, "AX"), _rows(H, "H"), _rows(G, "G")
    W2 = _f32(W2, "W2")
    K, F = AX.shape
    Hd, C = W2.shape
    if H.shape != (K, Hd) or G.shape != (K, C):
        raise ValueError(f"shape mismatch: AX {tuple(AX.shape)}, H {tuple(H.shape)}, G {tuple(G.shape)}, "
                         f"W2 {tuple(W2.shape)}")
    dW1 = torch.empty((F, Hd), dtype=torch.float32, device=AX.device)
    dW2 = torch.empty((Hd, C), dtype=torch.float32, device=AX.device)
    nbytes = _lib.lib().tcc_gcn_relu_grad_workspace_bytes(K, F, Hd, C)
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=AX.device)
    check(_lib.lib().tcc_gcn_relu_grad(AX.data_ptr(), AX.stride(0), H.data_ptr(), H.stride(0), G.data_ptr(),
                                       G.stride(0), W2.data_ptr(), dW1.data_ptr(), dW2.data_ptr(), K, F, Hd, C,
                                       ws.data_ptr(), nbytes, _stream(stream)))
    return dW1, dW2


def spmm_cnic_forward(bcsr: BlockMatrix, bcsc: BlockMatrix, X: torch.Tensor, denseC: torch.Tensor,
                      stream=None) -> torch.Tensor:
    check(_lib.lib().tcc_spmm_cnic_forward(ctypes.byref(bcsr.view), ctypes.byref(bcsc.view), X.data_ptr(),
                                           denseC.data_ptr(), X.shape[1], _stream(stream)))
    return denseC


class FeatureSourceHandle:
    """A tcc_feature_source plus references to the device tensors it points
    into: the struct holds raw addresses, so the tensors must outlive every
    launch that uses it (keep this object alive across those launches)."""

    def __init__(self, struct: FeatureSource, keep: tuple):
        self.struct = struct
        self._keep = keep


# tcc_feature_source.row_format
ROWS_FP32 = 0
ROWS_TF32_PACKED = 1


def feature_source(id_map: torch.Tensor, cache_search_map: torch.Tensor, gpu_cache_ptrs: torch.Tensor,
                   gpu_node_capacity: int, cpu_features_dev_ptr: int, cpu_len: int,
                   row_format: int = ROWS_FP32, device_error: torch.Tensor | None = None) -> FeatureSourceHandle:
    """tcc_feature_source over device tensors; `device_error` (one int32 on
    the device, or None) receives TCC_DEVERR_FEATURE_INDEX when a lookup
    falls outside its table."""
    for t, name in ((id_map, "id_map"), (cache_search_map, "cache_search_map")):
        if t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous int32 device tensor")
    if gpu_cache_ptrs.dtype != torch.int64 or not gpu_cache_ptrs.is_cuda:
        raise TypeError("gpu_cache_ptrs must be an int64 device tensor of device pointers")
    if device_error is not None and (device_error.dtype != torch.int32 or not device_error.is_cuda):
        raise TypeError("device_error must be an int32 device tensor")
    s = FeatureSource(id_map.data_ptr(), cache_search_map.data_ptr(), gpu_cache_ptrs.data_ptr(), gpu_node_capacity,
                      cpu_features_dev_ptr, cpu_len, gpu_cache_ptrs.numel(), row_format,
                      None if device_error is None else device_error.data_ptr())
    return FeatureSourceHandle(s, (id_map, cache_search_map, gpu_cache_ptrs, device_error))


def spmm_cnic_forward_mixed(bcsr: BlockMatrix, bcsc: BlockMatrix, src: FeatureSourceHandle, denseC: torch.Tensor,
                            F: int, stream=None) -> torch.Tensor:
    check(_lib.lib().tcc_spmm_cnic_forward_mixed(ctypes.byref(bcsr.view), ctypes.byref(bcsc.view),
                                                 ctypes.byref(src.struct), denseC.data_ptr(), F, _stream(stream)))
    return denseC


def bcsr_spmm_mixed(A: BlockMatrix, src: FeatureSourceHandle, Y: torch.Tensor, F: int, accumulate: bool = False,
                    stream=None) -> torch.Tensor:
    check(_lib.lib().tcc_bcsr_spmm_mixed(ctypes.byref(A.view), ctypes.byref(src.struct), Y.data_ptr(), F,
                                         int(accumulate), _stream(stream)))
    return Y
