/*
 * tcc_swtcf.h — C-ABI of the MI355X (gfx950) SWTCF sparse path.
 *
 * The SWTCF ("super-window tiled compressed format") stores a binary sparse
 * matrix A (rows = destinations, cols = sources) as:
 *   - column windows of 8 consecutive sources, each split into tiles of
 *     8 destination rows ordered by degree (descending; ties by destination
 *     ascending), with one u64 bitmap per tile (bit r*8+c = row r, column c);
 *   - super-windows of S consecutive column windows, each with a sorted list
 *     of the distinct destinations it touches ("slots") and a repeat-row cache
 *     of up to 32 destinations that occur in more than one of its windows.
 *
 * Every entry point returns 0 on success or a TCC_ERR_* code; the text of the
 * last host-side error is available from tcc_last_error().  Device-side data
 * errors found during a conversion are written asynchronously to
 * workspace->deviceError (codes TCC_DEVERR_*), which the caller reads after
 * synchronising the stream, as with the reference.
 *
 * All array pointers are device pointers unless stated otherwise.  The stream
 * argument is a hipStream_t passed as void* (NULL = default stream).
 *
 * Reference interface replaced: include/swtcf_convert.cuh:13-78 and
 * include/swtcf_spmm.cuh:7-25 of Shixg-cnic/tcc.
 */
#ifndef TCC_SWTCF_H
#define TCC_SWTCF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Format constants — include/swtcf_convert.cuh:7-11, include/swtcf_spmm.cuh:7-8 */
#define TCC_SWTCF_COL_WINDOW_WIDTH 8u
#define TCC_SWTCF_TILE_ROWS 8u
#define TCC_SWTCF_REPEAT_CACHE_SIZE 32u
#define TCC_SWTCF_MAX_SUPER_WINDOW_SIZE 32u
#define TCC_SWTCF_INVALID_CACHE_SLOT 0xFFu
#define TCC_SWTCF_INVALID_ROW_SLOT 0xFFFFFFFFu
#define TCC_SWTCF_FEATURE_DIM 128u
#define TCC_SWTCF_DEFAULT_TC_THRESHOLD 12u

/* Host-side return codes. */
#define TCC_OK 0
#define TCC_ERR_INVALID_ARGUMENT 1 /* bad sizes / arguments (reference: std::runtime_error) */
#define TCC_ERR_HIP 2              /* a HIP runtime call failed */
#define TCC_ERR_UNSUPPORTED 3      /* argument combination the kernel does not support */
#define TCC_ERR_NO_MEMORY 4        /* device allocation failed */

/* Device-side conversion error codes written to workspace->deviceError.
 * 1-4 keep the reference's meaning (src/swtcf_convert.cu:186-196, 582-585,
 * 981-999, 765-775); 5 and 6 are checks the reference does not make (it
 * writes out of range instead). */
#define TCC_DEVERR_DEGREE 1        /* a (window,dst) group has 0 or more than 8 edges */
#define TCC_DEVERR_HASH_FULL 2     /* reference only: never raised (no hash table here) */
#define TCC_DEVERR_HASH_MISS 3     /* reference only: never raised */
#define TCC_DEVERR_OCCURRENCE 4    /* a row occurs in more than 32 windows of a super-window */
#define TCC_DEVERR_SRC_RANGE 5     /* src >= cols */
#define TCC_DEVERR_DST_RANGE 6     /* dst >= rows (only checked when rows > 0) */

/* Same fields, order and meaning as DeviceSWTCFMatrix
 * (include/swtcf_convert.cuh:13-35). */
typedef struct tcc_swtcf_matrix {
    uint32_t rows;
    uint32_t cols;
    uint32_t nnz; /* capacity: edges the arrays were sized for */
    uint32_t colWindowWidth;
    uint32_t tileRows;
    uint32_t superWindowSize;
    uint32_t numColWindows;
    uint32_t numSuperWindows;
    uint32_t* superWindowRowOffset;     /* [numSuperWindows+1] */
    uint32_t* superWindowRows;          /* [nnz] valid: superWindowRowOffset[SW] */
    uint8_t* superWindowRowCacheSlot;   /* [nnz] 0xFF = not cached */
    uint32_t* superWindowCachedRowSlot; /* [numSuperWindows*32] 0xFFFFFFFF = unused */
    uint8_t* superWindowCachedCount;    /* [numSuperWindows] */
    uint32_t* colWindowOffset;          /* [numColWindows+1] tile offsets */
    uint32_t* tileRowSlot;              /* [nnz*8] valid: colWindowOffset[CW]*8 */
    uint64_t* tileLocalBit;             /* [nnz] valid: colWindowOffset[CW] */
} tcc_swtcf_matrix;

/* Conversion scratch.  Only edgeCapacity, numColWindows, numSuperWindows,
 * deviceNumGroups and deviceError are meant for callers; the rest is the
 * sort/scan scratch of this implementation (the reference's hash table and
 * CUB temporaries have no counterpart here). */
typedef struct tcc_swtcf_workspace {
    uint32_t edgeCapacity;
    uint32_t numColWindows;
    uint32_t numSuperWindows;
    uint32_t superWindowSize;
    uint32_t* deviceNumGroups; /* [1] number of (window,dst) groups of the last conversion */
    uint32_t* deviceError;     /* [1] TCC_DEVERR_* of the last conversion, 0 = none */
    void* scratch;             /* one device allocation carved into the buffers below */
    size_t scratchBytes;
} tcc_swtcf_workspace;

/* ---- allocation (src/swtcf_convert.cu:1113-1303, 1306-1751) ---- */

/* allocateDeviceSWTCF: rows, cols, nnz capacity, super-window size in [1,32]. */
int tcc_swtcf_alloc_matrix(tcc_swtcf_matrix* m, uint32_t rows, uint32_t cols,
                           uint32_t nnz, uint32_t superWindowSize);
/* freeDeviceSWTCF: frees the arrays and resets *m to all-zero. */
int tcc_swtcf_free_matrix(tcc_swtcf_matrix* m);
/* allocateSWTCFConvertWorkspace */
int tcc_swtcf_alloc_workspace(tcc_swtcf_workspace* ws, uint32_t edgeCapacity,
                              uint32_t numSrc, uint32_t superWindowSize);
/* freeSWTCFConvertWorkspace */
int tcc_swtcf_free_workspace(tcc_swtcf_workspace* ws);

/* ---- conversion (src/swtcf_convert.cu:1754-2342) ----
 * convertCOOToSWTCF: builds the SWTCF arrays of `m` from a device COO.
 * Asynchronous on `stream`; no host synchronisation.  The output is
 * deterministic: every tie the reference breaks by atomic order is broken by
 * destination (row order within a degree bucket, super-window slots) or slot
 * (repeat-cache ranks) ascending. */
int tcc_swtcf_convert(const uint32_t* dDst, const uint32_t* dSrc, uint32_t numEdges,
                      tcc_swtcf_matrix* m, tcc_swtcf_workspace* ws, void* stream);

/* ---- SpMM (src/swtcf_spmm.cu:437-502) ----
 * launchSWTCFSpMM: Y[rows x 128] += A * X[cols x 128] (row-major fp32).
 * Requires superWindowSize == 16 like the reference.  Tiles with at least
 * tcThreshold nonzeros use TF32-rounded X (the reference's tensor-core path),
 * sparser tiles use X as given (its fp32 path).  The caller zeroes Y.
 * Plans (no reference counterpart, see tcc_swtcf_set_plans): on a matrix of
 * at least 2^18 edges of capacity, with tcThreshold <= 64 and the stream not
 * capturing a graph, the call hashes the matrix's arrays on the device and
 * waits for the hash; from the second call that finds the same matrix on,
 * the product runs through a kept plan with TF32(X) for every entry, exact
 * products and fp32 sums: at 4M edges or more and 64 entries per row on
 * average, the matrix's pattern as binary hub tiles plus a gathered
 * remainder (tcc_coo_to_hybrid_scaled), else the BCSR gather of the pattern
 * (tcc_coo_to_bcsr; over X packed to TF32 rows, tcc_tf32_pack, where rows
 * are gathered 16 times or more on average).  Y keeps exactly rows rows
 * either way.  The call that builds the plan synchronises the stream and
 * allocates the plan's device memory. */
int tcc_swtcf_spmm(const tcc_swtcf_matrix* m, const float* X, float* Y,
                   uint32_t tcThreshold, void* stream);

/* Same as tcc_swtcf_spmm for any feature width F >= 1 and any super-window
 * size (the reference fixes F = 128 and S = 16; this entry point has no
 * reference counterpart). */
int tcc_swtcf_spmm_f(const tcc_swtcf_matrix* m, const float* X, float* Y,
                     uint32_t featureDim, uint32_t tcThreshold, void* stream);

/* tcc_swtcf_spmm_f with tiles of at least max(mfmaThreshold, tcThreshold)
 * entries multiplied on fp32 MFMA (v_mfma_f32_16x16x4f32, two tiles of a
 * window per instruction) instead of the vector ALUs; mfmaThreshold > 64
 * never does.  Same numerics (TF32 X for those tiles), sums in another
 * order.  No reference counterpart: the A/B of the reference's tensor-core
 * split (src/swtcf_spmm.cu:188-241) on this GPU. */
int tcc_swtcf_spmm_mfma(const tcc_swtcf_matrix* m, const float* X, float* Y, uint32_t featureDim,
                        uint32_t tcThreshold, uint32_t mfmaThreshold, void* stream);

/* Plans for repeated products over one matrix (tcc_swtcf_spmm and
 * tcc_swtcf_spmm_f; no reference counterpart).  At most maxPlans plans are
 * kept, the least recently used released first; 0 turns plans off.  The
 * default is 1, or the value of the environment variable TCC_SWTCF_PLANS
 * read at the first SpMM.  A plan holds the hybrid of its matrix (about
 * 0.5 GB at 233k rows and 114M edges) or its BCSR, and a workspace (or
 * packed X) for the last feature width. */
int tcc_swtcf_set_plans(uint32_t maxPlans);
/* Releases every kept plan. */
int tcc_swtcf_release_plans(void);
/* Plans built since the process started. */
uint32_t tcc_swtcf_plans_built(void);

/* Two order-independent 64-bit sums over the 32-bit words of up to 8 device
 * arrays (each bytes[k] a multiple of 4), mixed with their array and index
 * (no reference counterpart): what the plan caches compare to recognise a
 * matrix whose arrays they have seen.  Written in stream order to
 * deviceOut[0 .. TCC_HASH_WORDS-1] as TCC_HASH_WORDS/2 pairs of partial
 * sums (the threads' sums spread over pairs, so that their atomics do not
 * queue on one address): the sums are those of the even and of the odd
 * words, modulo 2^64. */
#define TCC_HASH_WORDS 64u
int tcc_hash_arrays(const void* const* arrays, const uint64_t* bytes, uint32_t count, uint64_t* deviceOut,
                    void* stream);

/* launchSWTCFSpMMQuantized: X[src][f] = q[srcGlobal[src]*128+f] * scales[srcGlobal[src]]
 * (src/swtcf_spmm.cu:317-323), otherwise as tcc_swtcf_spmm, plans included
 * (a plan dequantizes X into a buffer of its own, cols x 128 floats, then
 * runs as for fp32 X). */
int tcc_swtcf_spmm_quantized(const tcc_swtcf_matrix* m, const int8_t* quantizedX,
                             const float* scales, const uint32_t* srcGlobal, float* Y,
                             uint32_t tcThreshold, void* stream);

/* Text of the last host-side error on this thread ("" if none). */
const char* tcc_last_error(void);

/* A plain device copy of `bytes` (a multiple of 16; both pointers 16-byte
 * aligned) by calibration_copy_kernel, whose HBM traffic is known (bytes read,
 * bytes written): the reference run that scales rocprofv3's FETCH_SIZE and
 * WRITE_SIZE into bytes (bench.py --copy-calibration-mib).  No reference
 * counterpart. */
int tcc_calibration_copy(void* dst, const void* src, size_t bytes, void* stream);

/* The L2's fp32 atomic rate for the SpMM's output pattern (no reference
 * counterpart; bench.py --atomic-probe-mib): `waves` waves each add 1.0 to
 * 64 consecutive floats (one 256-byte segment, one per lane) of a
 * pseudo-random row of `rowFloats` floats (a multiple of 64) among `rows`
 * rows of dst, as a tile row's sums go to Y in the SWTCF SpMM. */
int tcc_calibration_atomic(float* dst, uint32_t rows, uint32_t rowFloats, uint64_t waves, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TCC_SWTCF_H */
