/*
 * tcc_spmm_cnic.h — C-ABI of the block-sparse (BCSR / BCSC) SpMM behind the
 * `spmm_cnic` PyTorch extension, for MI355X (gfx950).
 *
 * Block formats (8x8 blocks, one u64 bitmap each, bit r*8+c = block row r,
 * block column c):
 *   BCSR: row window w covers rows 8w..8w+7; its blocks are
 *         [rowWindowOffset[w], rowWindowOffset[w+1]); block b lists the 8
 *         global source columns it covers in sparseA2B[8b..8b+7]
 *         (padding = 0xFFFFFFFF or any value >= num_cols).
 *         Y[8w+r] += sum_c bit(r,c) * v * X[sparseA2B[8b+c]].
 *   BCSC: column window w covers sources 8w..8w+7; its blocks are
 *         [colWindowOffset[w], colWindowOffset[w+1]); block b lists the 8
 *         global destination rows in sparseA2C[8b..8b+7] (padding >= num_rows).
 *         Y[sparseA2C[8b+r]] += sum_c bit(r,c) * v * X[8w+c].
 * Values: when `data` is NULL every stored entry is 1.0 (what the reference
 * kernels do, spmm_cnic/src/core/spmm_kernel.cu:96-102).  Otherwise the value
 * of bit i of block b is data[tcOffset[b] + popcount(bitmap & ((1<<i)-1))]
 * (the layout of the reference's commented-out value load, :88-101).
 * Forward products use TF32-rounded (round-to-nearest, ties away from zero,
 * 10 mantissa bits) X and values with fp32 accumulation, reproducing the
 * reference's mma.m16n8k8 tf32 numerics; the A^T product is plain fp32.
 *
 * Reference interface replaced: spmm_cnic/include/class.h:20-58 (views),
 * spmm_cnic/src/core/spmm_launcher.cu:30-271 (launch_spmm_kernel) and
 * spmm_cnic/src/core/spmm_dispatcher.cu:15-301 (tf32_spmm_bcsr/bcsc and the
 * mixed variants).
 */
#ifndef TCC_SPMM_CNIC_H
#define TCC_SPMM_CNIC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* BCSR<T> (spmm_cnic/include/class.h:20-37) plus the optional value array. */
typedef struct tcc_bcsr {
    uint32_t num_rows;
    uint32_t num_cols;
    uint32_t nnz;
    uint32_t num_TCBlocks;
    uint32_t num_rowWindows;
    const uint32_t* rowWindowOffset; /* [num_rowWindows+1] */
    const uint32_t* tcOffset;        /* [num_TCBlocks+1] value offsets (used only with data) */
    const uint32_t* sparseA2B;       /* [num_TCBlocks*8] */
    const uint64_t* tcLocalBit;      /* [num_TCBlocks] */
    const float* data;               /* [nnz] or NULL */
    /* Blocks per unit of work (no reference counterpart; 0 = automatic).
     * The kernels cut the blocks into units of this many consecutive blocks,
     * one wave each, regardless of window boundaries, so skewed windows are
     * spread over many waves; a window split between units has its partial
     * sums combined with fp32 atomics. */
    uint32_t unitBlocks;
    /* Column phases (no reference counterpart; 0 and 1 = an ordinary BCSR).
     * With P > 1 the arrays hold P row windows per 8 output rows: the
     * matrix's column slices [p*num_cols/P, (p+1)*num_cols/P) stacked
     * vertically, built by tcc_coo_to_bcsr_phased.  num_rowWindows is then P
     * times ceil(num_rows / 8) and window w adds into output window
     * w % (num_rowWindows / P).  Only tcc_bcsr_spmm and tcc_bcsr_spmm_packed
     * take such a matrix (the others return TCC_ERR_UNSUPPORTED); their Y has
     * 8 * num_rowWindows / P rows. */
    uint32_t phases;
} tcc_bcsr;

/* BCSC<T> (spmm_cnic/include/class.h:39-58) plus the optional value array. */
typedef struct tcc_bcsc {
    uint32_t num_rows;
    uint32_t num_cols;
    uint32_t nnz;
    uint32_t num_TCBlocks;
    uint32_t num_colWindows;
    const uint32_t* colWindowOffset; /* [num_colWindows+1] */
    const uint32_t* tcOffset;        /* [num_TCBlocks+1] */
    const uint32_t* sparseA2C;       /* [num_TCBlocks*8] */
    const uint64_t* tcLocalBit;      /* [num_TCBlocks] */
    const float* data;               /* [nnz] or NULL */
    uint32_t unitBlocks;             /* as in tcc_bcsr */
} tcc_bcsc;

/* Where the first GCN layer reads feature row j from
 * (spmm_cnic/src/core/spmm_kernel.cu:129-153): g = cache_search_map[j];
 * g >= 0: hot row (g % cap) of gpu_feature_cache[g / gpu_node_capacity]
 * (device memory); g < 0: cold row id_map[j] of cpu_features, a device
 * pointer to mapped pinned host memory read zero-copy; id_map[j] < 0 reads
 * zeros.  The reference checks neither table bound and reads outside the
 * tables on bad map values; here three lookups are refused instead: a cache
 * index g / cap >= gpu_feature_cache_count (when nonzero), a host row past
 * cpu_feature_len features (when > 0), and a cold row when cpu_features is
 * NULL.  A refused lookup reads zeros and, when device_error is set, writes
 * TCC_DEVERR_FEATURE_INDEX there (device memory, read by the caller after
 * synchronising; it is never cleared by the kernels).  On one GPU the
 * pointer table has one entry.
 * Rows are F floats (row_format TCC_ROWS_FP32, the reference's layout) or,
 * with TCC_ROWS_TF32_PACKED (no reference counterpart), TF32 rows packed by
 * tcc_tf32_pack (tcc_tf32_packed_bytes(1, F) bytes each, tables 16-byte
 * aligned): the products are the same bit for bit, since the first layer's
 * products round X to TF32 anyway, and each row moves 2.5 instead of 4
 * bytes per feature -- across PCIe for the cold rows. */
#define TCC_ROWS_FP32 0u
#define TCC_ROWS_TF32_PACKED 1u
#define TCC_DEVERR_FEATURE_INDEX 7u /* a feature lookup outside its table (read as zeros) */

typedef struct tcc_feature_source {
    const int32_t* id_map;           /* device [num_cols] */
    const int32_t* cache_search_map; /* device [num_cols] */
    const float* const* gpu_feature_cache; /* device array of device pointers */
    int32_t gpu_node_capacity;
    const float* cpu_features;       /* device-visible pointer to pinned host rows */
    int64_t cpu_feature_len;         /* features (rows x F) available at cpu_features (<= 0: unchecked) */
    uint32_t gpu_feature_cache_count; /* entries of gpu_feature_cache (0: unchecked) */
    uint32_t row_format;             /* TCC_ROWS_FP32 (0) or TCC_ROWS_TF32_PACKED */
    uint32_t* device_error;          /* device [1] or NULL: TCC_DEVERR_FEATURE_INDEX on a refused lookup */
} tcc_feature_source;

/* Y[row-window rows x F] (=, or += when accumulate != 0) A_bcsr * X.
 * With accumulate == 0 every row 0..8*num_rowWindows-1 is written (empty
 * windows write zeros).  Y must hold 8*num_rowWindows*F floats.  Here and in
 * every BCSR/BCSC product and tcc_tf32_pack, 1 <= featureDim < 2^30 (rows
 * are addressed with 32-bit byte offsets); larger is an argument error.
 * (tf32_spmm_bcsr, spmm_dispatcher.cu:167-232; kernel spmm_kernel.cu:1560-1842.) */
int tcc_bcsr_spmm(const tcc_bcsr* A, const float* X, float* Y, uint32_t featureDim,
                  int accumulate, void* stream);

/* ---- packed TF32 features (no reference counterpart) ----
 * A TF32 value has 19 significant bits.  tcc_tf32_pack writes TF32(X) of an
 * fp32 [rows x F] matrix in 2.5 bytes per element.  A row is cut into chunks
 * of 256 features; a chunk of n features holds the high 16 bits of each
 * value (sign, exponent, 7 mantissa bits; 2n bytes) followed by the 3 low
 * mantissa bits of element pairs (element 2k in bits 0-2 and 2k+1 in bits
 * 3-5 of byte k; ceil(n/2) bytes).  A full chunk is 640 bytes; the last is
 * padded to 16 bytes; a row of more than one chunk is padded to 128 bytes,
 * a single-chunk row to 16 (tcc_tf32_packed_bytes / rows).  A NaN is stored
 * as a quiet NaN with its top 19 bits (the low payload bits do not fit); all
 * other values, inf included, unpack to TF32(x) exactly.  The gather over
 * packed rows reads 37.5% fewer bytes per gathered row than fp32 X, with
 * bit-identical products, and each 256-feature chunk it loads covers whole
 * 128-byte lines; it pays off when rows are gathered many times
 * (8*num_TCBlocks against num_cols).  The packed buffer must be 16-byte
 * aligned and hold tcc_tf32_packed_bytes(rows, F) bytes. */
size_t tcc_tf32_packed_bytes(uint32_t rows, uint32_t featureDim);
int tcc_tf32_pack(const float* X, uint32_t rows, uint32_t featureDim, void* packed, void* stream);

/* tcc_bcsr_spmm with X given packed by tcc_tf32_pack (rows = num_cols). */
int tcc_bcsr_spmm_packed(const tcc_bcsr* A, const void* packedX, float* Y, uint32_t featureDim,
                         int accumulate, void* stream);

/* Y[num_rows x F] += A_bcsc * X with fp32 atomics (rows >= num_rows skipped).
 * (tf32_spmm_bcsc, spmm_dispatcher.cu:236-301; kernel spmm_kernel.cu:1844-2166.) */
int tcc_bcsc_spmm(const tcc_bcsc* A, const float* X, float* Y, uint32_t featureDim,
                  void* stream);

/* Transposed use of a BCSC for the backward pass: dX = A^T * dY, i.e.
 * dX[8w+c] (=, or +=) sum_b sum_r bit(r,c) * v * dY[sparseA2C[8b+r]] — a
 * gather (atomics only where a window is split between units).
 * dX must hold 8*num_colWindows*F floats.  The reference computes this
 * product with torch.sparse.mm (train/tcgnn_conv_release.py:152); this is its
 * block-sparse replacement, with the same plain fp32 products (no TF32
 * rounding). */
int tcc_bcsc_transpose_spmm(const tcc_bcsc* A, const float* dY, float* dX,
                            uint32_t featureDim, int accumulate, void* stream);

/* launch_spmm_kernel, non-first-layer form (spmm_launcher.cu:203-271):
 * denseC[(num_rowWindows+1)*8*F] = A_bcsr*X + A_bcsc*X.  The BCSR part writes
 * every row (replacing the reference's memset), the BCSC part then adds with
 * atomics, both on `stream`. */
int tcc_spmm_cnic_forward(const tcc_bcsr* bcsr, const tcc_bcsc* bcsc, const float* X,
                          float* denseC, uint32_t featureDim, void* stream);

/* tcc_spmm_cnic_forward with a caller-owned workspace (no reference
 * counterpart; the spmm_cnic extension's forward_tensorcore uses it): when
 * the BCSR gathers each input row at least 16 times on average, X is first
 * packed to exact TF32 rows in the workspace (tcc_tf32_pack) and the BCSR
 * part gathers those (the same products, fewer bytes: config 3, 36.7 ->
 * 21.5 ms).  tcc_spmm_cnic_forward_workspace_bytes gives the bytes that
 * enable it (0: packing would not pay); a smaller or NULL workspace takes
 * the fp32 gather.  The workspace must not be shared with a concurrent call. */
size_t tcc_spmm_cnic_forward_workspace_bytes(const tcc_bcsr* bcsr, uint32_t featureDim);
int tcc_spmm_cnic_forward_ws(const tcc_bcsr* bcsr, const tcc_bcsc* bcsc, const float* X, float* denseC,
                             uint32_t featureDim, void* workspace, size_t workspaceBytes, void* stream);

/* launch_spmm_kernel, first-layer (mixed memory) form
 * (spmm_launcher.cu:30-112 with the mixed kernels of spmm_kernel.cu:7-794):
 * as tcc_spmm_cnic_forward, with feature rows resolved through `src`. */
int tcc_spmm_cnic_forward_mixed(const tcc_bcsr* bcsr, const tcc_bcsc* bcsc,
                                const tcc_feature_source* src, float* denseC,
                                uint32_t featureDim, void* stream);

/* The BCSR part of the mixed form alone (for hot/cold measurements). */
int tcc_bcsr_spmm_mixed(const tcc_bcsr* A, const tcc_feature_source* src, float* Y,
                        uint32_t featureDim, int accumulate, void* stream);

/* ---- construction ----
 * The reference receives these arrays from ipc_service (called at
 * train/tcgnn_conv_release.py:295-296), which is not part of its tree; these
 * builders produce the layout its kernels consume from a device COO
 * (row = destination, col = source, no duplicate pairs; dVal may be NULL).
 *   BCSR: per 8-row window, its distinct columns ascending, 8 per block.
 *   BCSC: per 8-source window, its rows by (degree desc, dst asc), 8 per
 *         block (the SWTCF row order with one window per super-window).
 * Each synchronises `stream` (to size the output), places all arrays in one
 * device allocation returned in *allocation (free it with tcc_block_release)
 * and fills *out with views into it.  `data` is set only when dVal != NULL.
 * nnz = 0 gives empty windows and no blocks (dRow, dCol may then be NULL). */
int tcc_coo_to_bcsr(const uint32_t* dRow, const uint32_t* dCol, const float* dVal, uint32_t nnz,
                    uint32_t numRows, uint32_t numCols, tcc_bcsr* out, void** allocation, void* stream);
int tcc_coo_to_bcsc(const uint32_t* dRow, const uint32_t* dCol, const float* dVal, uint32_t nnz,
                    uint32_t numRows, uint32_t numCols, tcc_bcsc* out, void** allocation, void* stream);
/* A phased BCSR (see tcc_bcsr.phases; no reference counterpart): the same
 * product as tcc_coo_to_bcsr's, with the blocks ordered column phase first,
 * so that the waves of one gather in flight together read rows of one phase
 * of the columns, which the L2 and the last-level cache then hold.  Worth it
 * where windows are long (hundreds of blocks per window); every window is
 * then added into Y with atomics.  phases 0 or 1 = tcc_coo_to_bcsr. */
int tcc_coo_to_bcsr_phased(const uint32_t* dRow, const uint32_t* dCol, const float* dVal, uint32_t nnz,
                           uint32_t numRows, uint32_t numCols, uint32_t phases, tcc_bcsr* out,
                           void** allocation, void* stream);
int tcc_block_release(void* allocation);

/* ---- dense hub tiles + sparse remainder (no reference counterpart) ----
 * The product tf32_spmm_bcsr computes, for graphs with a dense core (R-MAT
 * hubs).  Rows and columns are ranked by degree (descending, ties by index)
 * and the reordered matrix is cut into 16x16 tiles; tiles holding at least
 * minTileNnz entries are stored densely (TF32-rounded values, zeros
 * included) and multiplied with fp32 MFMA (v_mfma_f32_16x16x4f32), the other
 * entries form an ordinary or phased BCSR (`rest`) for the gather kernels.
 * Row blocks (16 rows) are grouped G at a time; a step of a group is a
 * column block where at least one of its G tiles is dense, and holds all G
 * (zeros for the tiles that are not), so that one load of the step's 16
 * feature rows serves G tiles.
 *   rowOrder[16(G g + j) + i]: original row of row i of row block j of group
 *     g (0xFFFFFFFF past num_rows); hubColOrder[r]: original column of column
 *     rank r < hub_cols;
 *   group g's steps are [groupStepOffset[g], groupStepOffset[g+1]); step p
 *     covers column ranks 16*stepCol[p] .. +15;
 *   tileVals[256(G p + j) + 4l + s] = A(row l%16, column 4s + l/16) of the
 *     tile of row block j at step p (the MFMA A operand of lane l at step s);
 *   units[3u .. 3u+2] = group, first step, end step (at most unit_steps
 *     steps); a group held by more than one unit (a shared group) has its
 *     units' sums stored in the workspace and added into Y by a reduction
 *     pass (no atomics: the sum order is fixed);
 *   unitPartial[u]: the workspace slot of unit u's partial sum (the units
 *     of shared groups, numbered in unit order), 0xFFFFFFFF for a unit that
 *     holds its whole group; sharedGroups[3s .. 3s+2] = group, slot of its
 *     first unit, number of units (consecutive units and slots), for the
 *     num_shared_groups shared groups;
 *   unitOrder[i]: the unit the SpMM launches i-th, the units sorted by the
 *     column block of their first step (stable), so that units running at
 *     the same time read the same feature rows; for binary tiles first by
 *     size, in buckets of 128 steps, the largest first (a long unit
 *     launched last would hold the grid's tail); NULL launches them in
 *     index order (the products do not depend on it).
 * Binary tiles (TCC_TILES_BINARY, tcc_coo_to_hybrid_scaled) hold the
 * pattern of A only, with A = diag(rowScale) P diag(colScale) (the scales
 * NULL for ones).  Their step is a group's G row blocks by a pair of
 * 16-column blocks (32 column ranks, 32*stepCol[p] .. +31); a step is
 * chosen when its tiles together hold at least minStepNnz entries, and then
 * every entry of the step is stored, as operands of the 2:4 sparse MFMA
 * (v_smfmac_f32_32x32x32_f16 / _bf16) over 32-row tiles (row blocks 2t and
 * 2t+1).  Lane l of the SpMM's wave covers row l%32 of each tile and, with
 * c = l/32, columns 8c..8c+7 of both 16-column blocks, as four groups of
 * four columns (k = 0, 1: columns 8c + 4k..+3 of block 0; k = 2, 3:
 * columns 8c + 4(k-2)..+3 of block 1); group k's entries take value slots
 * 2k and 2k+1, two at most, so a step in which some group holds three or
 * four entries takes two sub-steps of the same columns (layer 0: each
 * group's lowest two entries, layer 1: the rest).  Sub-steps are what
 * groupStepOffset, stepCol, units and num_steps count:
 *   tileMasks, sub-step p's 96*G bytes at byte 96*G*p: at byte
 *     l*(G/2) + t the value mask of lane l in tile t (bit j: slot j is 1,
 *     else 0), and at byte 32*G + l*G + 2t the slots' positions in their
 *     groups (2 bits a slot, slot j in bits 2j..2j+1, increasing within a
 *     group; a slot without an entry has value 0 and an unused position);
 *   rowScale[16(G g + j) + i]: the scale of row i of row block j of group g
 *     (rowOrder's order, 0 past num_rows); colScale[c]: the scale of column
 *     c (original order).
 * The products multiply 2^e TF32(colScale[c] * X[c]), with one power of two
 * e per 32-feature slice chosen from the slice's largest magnitude, by the
 * pattern: on the f16 form for a (column-block pair, slice) whose values
 * are all fp16 values, and as two exact bf16 halves on the bf16 form for
 * any other; each row's fp32 sum is then scaled by 2^-e and rowScale.  Both
 * forms are exact, so the sums are those of the TF32 values.  A zero value
 * slot multiplies the column its position names: an Inf or NaN in a hub
 * column's feature row can reach rows without an entry in that column. */
#define TCC_TILES_FP32 0u   /* tileVals in the fp32 MFMA's A-operand order (above) */
#define TCC_TILES_BF16X2 1u /* each tile 256 bf16 hi then 256 bf16 lo, row-major: hi + lo = the TF32 value */
#define TCC_TILES_BINARY 2u /* the pattern as sparse-MFMA operands (tileMasks); values from rowScale and colScale */

typedef struct tcc_hub_tiles {
    uint32_t num_rows;
    uint32_t num_cols;
    uint32_t nnz;                    /* entries held in the tiles */
    uint32_t group_blocks;           /* G: row blocks per group, 1, 2, 4 or 8 */
    uint32_t num_groups;             /* ceil(ceil(num_rows / 16) / G) */
    uint32_t num_steps;
    uint32_t num_tiles;              /* dense tiles (at most G * num_steps) */
    uint32_t num_units;
    uint32_t unit_steps;
    uint32_t hub_cols;               /* column ranks the tiles cover: [0, hub_cols) */
    uint32_t tile_format;            /* TCC_TILES_FP32, TCC_TILES_BF16X2 or TCC_TILES_BINARY */
    const uint32_t* rowOrder;        /* [16*G*num_groups] */
    const uint32_t* hubColOrder;     /* [hub_cols] */
    const uint32_t* groupStepOffset; /* [num_groups+1] */
    const uint32_t* stepCol;         /* [num_steps] */
    const float* tileVals;           /* [256*G*(num_steps+1)] (1 KB a tile; FP32, BF16X2): the last step zeros */
    const uint32_t* units;           /* [3*num_units] */
    const uint32_t* unitOrder;       /* [num_units] or NULL */
    uint32_t num_partial_units;      /* units of shared groups (workspace partial sums) */
    uint32_t num_shared_groups;
    const uint32_t* unitPartial;     /* [num_units] */
    const uint32_t* sharedGroups;    /* [3*num_shared_groups] */
    const uint32_t* tileMasks;       /* BINARY: [24*G*(num_steps+1)] words, the last sub-step zeros; else NULL */
    const float* rowScale;           /* BINARY: [16*G*num_groups] or NULL (ones) */
    const float* colScale;           /* BINARY: [num_cols] or NULL (ones) */
} tcc_hub_tiles;

typedef struct tcc_hybrid {
    tcc_hub_tiles tiles;
    tcc_bcsr rest;                  /* every entry outside the dense tiles */
    void* tilesAllocation;          /* device allocations (tcc_hybrid_release) */
    void* restAllocation;
    /* BINARY: the row scales in row order for the remainder's gather
     * ([8*ceil(num_rows/8)], 0 past num_rows), or NULL (ones); the
     * remainder's columns take tiles.colScale. */
    const float* restRowScale;
} tcc_hybrid;

/* Build the hybrid of a device COO (row = destination, col = source, no
 * duplicate pairs; dVal may be NULL).  minTileNnz 0 = 16 (at most 256),
 * groupBlocks 0 = 8 (1, 2, 4 or 8), unitSteps 0 = 128 (at most 256), tileFormat
 * TCC_TILES_FP32 (products on v_mfma_f32_16x16x4f32) or TCC_TILES_BF16X2
 * (each TF32 operand as two bf16, four exact bf16 products on
 * v_mfma_f32_16x16x32_bf16, fp32 accumulation), phases
 * as tcc_coo_to_bcsr_phased for the remainder (whose unitBlocks is set to
 * 64; a caller may change it).  Synchronises `stream`; free with
 * tcc_hybrid_release. */
int tcc_coo_to_hybrid(const uint32_t* dRow, const uint32_t* dCol, const float* dVal, uint32_t nnz,
                      uint32_t numRows, uint32_t numCols, uint32_t minTileNnz, uint32_t groupBlocks,
                      uint32_t unitSteps, uint32_t tileFormat, uint32_t phases, tcc_hybrid* out, void* stream);

/* The hybrid of the matrix diag(rowScale) P diag(colScale), P the pattern
 * of a device COO (row = destination, col = source, no duplicate pairs;
 * dRowScale [numRows] and dColScale [numCols] device arrays, either NULL
 * for ones), with binary tiles (TCC_TILES_BINARY): steps of at least
 * minStepNnz entries (0 = 40), groupBlocks 8 or 16 (0 = 16), unitSteps
 * 0 = 1024 (any number: the SpMM reads a unit's step list 256 steps at a
 * time), phases as tcc_coo_to_hybrid.  The remainder holds the pattern
 * (data NULL); its gather reads the column-scaled packed rows and scales
 * its row sums.  The scales are copied.  Synchronises `stream`; free with
 * tcc_hybrid_release. */
int tcc_coo_to_hybrid_scaled(const uint32_t* dRow, const uint32_t* dCol, uint32_t nnz, uint32_t numRows,
                             uint32_t numCols, const float* dRowScale, const float* dColScale, uint32_t minStepNnz,
                             uint32_t groupBlocks, uint32_t unitSteps, uint32_t phases, tcc_hybrid* out,
                             void* stream);
int tcc_hybrid_release(tcc_hybrid* H);

/* The hybrid of a BCSR's own entries (no reference counterpart: a per-graph
 * plan for callers that hold the reference's BCSR arrays and multiply by the
 * same graph many times, such as full-graph training).  With useValues = 0
 * the entries count as 1.0, as the reference's kernels read them
 * (spmm_kernel.cu:96-102): binary tiles (tcc_coo_to_hybrid_scaled without
 * scales, minStepNnz 0 = 40); else the values of `data` (value of bit i of
 * block b = data[tcOffset[b] + rank]) in split-TF32 tiles (tcc_coo_to_hybrid,
 * TCC_TILES_BF16X2, minTileNnz 16, groups of 8).  Bits in padding columns
 * (>= num_cols) or rows (>= num_rows) are ignored, as the gather ignores
 * them.  phases as tcc_coo_to_hybrid (0: when windows hold at least 64
 * blocks on average, 2 for binary tiles and 4 for value tiles, else 1).  Synchronises `stream`; the BCSR may be freed
 * afterwards (the hybrid holds its own arrays); free with tcc_hybrid_release. */
int tcc_hybrid_from_bcsr(const tcc_bcsr* A, int useValues, uint32_t minStepNnz, uint32_t phases, tcc_hybrid* out,
                         void* stream);

/* Bytes of device workspace tcc_hybrid_spmm needs for F features: the
 * remainder's packed TF32 rows and tcc_hub_tiles_workspace_bytes. */
size_t tcc_hybrid_workspace_bytes(const tcc_hybrid* H, uint32_t featureDim);

/* Bytes of device workspace tcc_hub_tiles_spmm needs for F features: the hub
 * columns' TF32 rows (roundup(hub_cols, 16) x roundup(F, 64) floats), one
 * 16G-row partial sum per unit of a shared group (num_partial_units x 16G x
 * roundup(F, 64) floats) and, for binary tiles, the half records' slice
 * maxima, scales and flags (64 + 2 words per 32-feature slice and one byte
 * per (16-column block, slice)). */
size_t tcc_hub_tiles_workspace_bytes(const tcc_hub_tiles* T, uint32_t featureDim);

/* Y (=, or += when accumulate != 0) A X for fp32 X [num_cols x F].  Value
 * tiles, or accumulate: the remainder's gather (which writes or adds every
 * row of Y), then the tiles added into Y.  Binary tiles without
 * accumulate: the tiles first, storing their rows (and zeros in every row
 * no tile group covers), then the remainder added into Y.  Y holds
 * 8*ceil(num_rows/8) rows of F floats (as for the remainder's BCSR);
 * workspace 16-byte aligned, at least tcc_hybrid_workspace_bytes(H, F)
 * bytes, not shared with a concurrent call. */
int tcc_hybrid_spmm(const tcc_hybrid* H, const float* X, float* Y, uint32_t featureDim, int accumulate,
                    void* workspace, size_t workspaceBytes, void* stream);

/* The tiles' part alone: Y[num_rows x F] += A_tiles X (workspace 16-byte
 * aligned, at least tcc_hub_tiles_workspace_bytes(T, F) bytes). */
int tcc_hub_tiles_spmm(const tcc_hub_tiles* T, const float* X, float* Y, uint32_t featureDim, void* workspace,
                       size_t workspaceBytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TCC_SPMM_CNIC_H */
