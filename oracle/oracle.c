/*
 * oracle.c — CPU restatement of the reference's SWTCF / spmm_cnic algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (tcc_amd/, include/)
 * links, loads or calls this file.  It is the checker used by tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the Shixg-cnic/tcc tree).  Where the reference breaks ties by atomic order
 * (nondeterministic), this file fixes the canonical choice the HIP converter
 * reproduces bit for bit:
 *   - rows of a column window: degree descending, destination ascending
 *     (reference: atomicAdd rank, src/swtcf_convert.cu:345-349);
 *   - slots of a super-window: destination ascending
 *     (reference: atomicAdd slot, src/swtcf_convert.cu:615-621);
 *   - repeat-cache ranks: occurrence descending, slot ascending
 *     (reference: atomicAdd rank, src/swtcf_convert.cu:851-856).
 *
 * Built by oracle/build.sh into oracle/_build/liboracle.so (gcc, OpenMP).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define CW_WIDTH 8u
#define TILE_ROWS 8u
#define CACHE_SIZE 32u
#define MAX_SW 32u
#define INVALID_SLOT 0xFFFFFFFFu
#define INVALID_CACHE 0xFFu

/* ------------------------------------------------------------------ */
/* TF32 rounding: cvt.rna.tf32.f32 (include/mma_tf32.cuh:17-22,       */
/* spmm_cnic/include/ptx_tf32.h:67-72).  Round to nearest, ties away   */
/* from zero, keep 10 explicit mantissa bits; inf/NaN pass through.    */
/* ------------------------------------------------------------------ */
uint32_t oracle_tf32_bits(uint32_t b) {
    if ((b & 0x7F800000u) == 0x7F800000u) return b; /* inf / NaN */
    /* Adding half an ulp of the 10-bit mantissa to the magnitude bits and
     * truncating rounds ties away from zero (sign bit is untouched because
     * the magnitude add can at most carry into the exponent, giving inf). */
    return (b + 0x1000u) & 0xFFFFE000u;
}

float oracle_tf32(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    b = oracle_tf32_bits(b);
    float y;
    memcpy(&y, &b, 4);
    return y;
}

void oracle_tf32_array(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_tf32(in[i]);
}

static int popcount8(uint32_t v) { return __builtin_popcount(v & 0xFFu); }

/* ------------------------------------------------------------------ */
/* Canonical COO -> SWTCF (src/swtcf_convert.cu:1754-2342).            */
/* ------------------------------------------------------------------ */
typedef struct {
    uint64_t key; /* (window << 32) | dst — buildEdgeKeysKernel :104-144 */
    uint32_t lc;  /* src & 7 */
} edge_t;

/* Stable LSD radix sort of edges by key, 8 bits per pass, as the
 * reference's CUB SortPairs over bits 0-64 (swtcf_convert.cu:1951-1966);
 * passes whose byte is the same for every key are skipped.  Stable, so
 * equal keys keep their input order. */
static void sort_edges(edge_t* e, uint32_t n) {
    if (n < 2) return;
    edge_t* tmp = (edge_t*)malloc(sizeof(edge_t) * (size_t)n);
    edge_t* src = e;
    edge_t* dst = tmp;
    for (int shift = 0; shift < 64; shift += 8) {
        size_t count[257] = {0};
        for (uint32_t i = 0; i < n; ++i) count[((src[i].key >> shift) & 0xFFu) + 1]++;
        int single = 0;
        for (int d = 0; d < 256; ++d)
            if (count[d + 1] == n) single = 1;
        if (single) continue;
        for (int d = 0; d < 256; ++d) count[d + 1] += count[d];
        for (uint32_t i = 0; i < n; ++i) dst[count[(src[i].key >> shift) & 0xFFu]++] = src[i];
        edge_t* t = src;
        src = dst;
        dst = t;
    }
    if (src != e) memcpy(e, src, sizeof(edge_t) * (size_t)n);
    free(tmp);
}

typedef struct {
    uint32_t window, dst, count, bits;
} group_t;

typedef struct {
    uint32_t dst, occ;
} swrow_t;

static int cmp_u32(const void* a, const void* b) {
    uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

/* Returns 0, or the device error code the HIP converter reports:
 * 1 group degree > 8 (:186-196), 5 src >= cols, 6 dst >= rows (rows > 0).
 * Output capacities follow allocateDeviceSWTCF (:1166-1262) with nnz = E;
 * fills follow the memsets of convertCOOToSWTCF (:1827-1910). */
int oracle_swtcf_convert(const uint32_t* dst, const uint32_t* src, uint32_t E, uint32_t rows,
                         uint32_t cols, uint32_t S, uint32_t* colWindowOffset,
                         uint32_t* superWindowRowOffset, uint32_t* superWindowRows,
                         uint8_t* superWindowRowCacheSlot, uint32_t* superWindowCachedRowSlot,
                         uint8_t* superWindowCachedCount, uint32_t* tileRowSlot,
                         uint64_t* tileLocalBit, uint32_t* numGroupsOut) {
    const uint32_t CW = (cols + CW_WIDTH - 1) / CW_WIDTH; /* :1150-1156 */
    const uint32_t SW = (CW + S - 1) / S;                 /* :1158-1164 */
    int err = 0;

    memset(tileLocalBit, 0, sizeof(uint64_t) * (size_t)E);               /* :1827-1837 */
    memset(superWindowRowCacheSlot, 0xFF, (size_t)E);                    /* :1875-1885 */
    memset(superWindowCachedRowSlot, 0xFF, sizeof(uint32_t) * (size_t)SW * CACHE_SIZE); /* :1887-1898 */
    memset(superWindowCachedCount, 0, (size_t)SW);                       /* :1900-1910 */
    for (size_t i = 0; i < (size_t)E * TILE_ROWS; ++i) tileRowSlot[i] = INVALID_SLOT;

    for (uint32_t e = 0; e < E; ++e) {
        if (src[e] >= cols) return 5;
        if (rows > 0 && dst[e] >= rows) return 6;
    }

    /* 1-3: key = (src>>3, dst), sort, run-length encode (:1925-2007). */
    edge_t* edges = (edge_t*)malloc(sizeof(edge_t) * (size_t)(E ? E : 1));
    for (uint32_t e = 0; e < E; ++e) {
        edges[e].key = ((uint64_t)(src[e] >> 3) << 32) | dst[e];
        edges[e].lc = src[e] & 7u;
    }
    sort_edges(edges, E);
    group_t* groups = (group_t*)malloc(sizeof(group_t) * (size_t)(E ? E : 1));
    uint32_t G = 0;
    for (uint32_t e = 0; e < E;) {
        uint32_t f = e;
        uint32_t bits = 0;
        while (f < E && edges[f].key == edges[e].key) {
            bits |= 1u << edges[f].lc; /* buildTileBitmapsKernel :416-428 */
            ++f;
        }
        groups[G].window = (uint32_t)(edges[e].key >> 32);
        groups[G].dst = (uint32_t)edges[e].key;
        groups[G].count = f - e; /* degree = edges in the run, duplicates included */
        groups[G].bits = bits;
        if (f - e > CW_WIDTH) err = 1; /* countWindowDegreesKernel :186-196 */
        ++G;
        e = f;
    }
    free(edges);
    *numGroupsOut = G;
    if (err) {
        free(groups);
        return err;
    }

    /* 4-5: per-window degree buckets, degree 8 first (:216-265), tile scan (:2059-2085). */
    uint32_t* degCount = (uint32_t*)calloc((size_t)CW * 8, sizeof(uint32_t));
    uint32_t* degBase = (uint32_t*)calloc((size_t)CW * 8, sizeof(uint32_t));
    uint32_t* degCursor = (uint32_t*)calloc((size_t)CW * 8, sizeof(uint32_t));
    uint32_t* activeRows = (uint32_t*)calloc(CW ? CW : 1, sizeof(uint32_t));
    for (uint32_t g = 0; g < G; ++g) degCount[(size_t)groups[g].window * 8 + groups[g].count - 1]++;
    uint32_t tiles = 0;
    for (uint32_t w = 0; w < CW; ++w) {
        uint32_t running = 0;
        for (int d = 7; d >= 0; --d) {
            degBase[(size_t)w * 8 + d] = running;
            running += degCount[(size_t)w * 8 + d];
        }
        activeRows[w] = running;
        colWindowOffset[w] = tiles;
        tiles += (running + TILE_ROWS - 1) / TILE_ROWS;
    }
    colWindowOffset[CW] = tiles; /* setOffsetTailKernel :268-289 */

    /* 6-7: row location and bitmaps (:292-456).  Groups of a window are in
     * dst-ascending order here, so the bucket cursor gives the canonical rank. */
    uint32_t* groupTile = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(G ? G : 1));
    for (uint32_t g = 0; g < G; ++g) {
        const size_t bucket = (size_t)groups[g].window * 8 + groups[g].count - 1;
        const uint32_t reordered = degBase[bucket] + degCursor[bucket]++;
        const uint32_t tile = colWindowOffset[groups[g].window] + reordered / TILE_ROWS;
        const uint32_t lr = reordered & (TILE_ROWS - 1);
        groupTile[g] = tile * TILE_ROWS + lr;
        tileLocalBit[tile] |= (uint64_t)groups[g].bits << (lr * 8);
    }

    /* 8-10: distinct (superWindow, dst) rows, slots, occurrence (:459-681).
     * Canonical slot order: dst ascending. */
    uint32_t U = 0;
    uint32_t* swDst = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(G ? G : 1));
    uint32_t* occ = (uint32_t*)calloc(G ? G : 1, sizeof(uint32_t));
    uint32_t g0 = 0;
    for (uint32_t s = 0; s < SW; ++s) {
        superWindowRowOffset[s] = U;
        uint32_t g1 = g0;
        while (g1 < G && groups[g1].window / S == s) ++g1;
        const uint32_t n = g1 - g0;
        uint32_t* tmp = (uint32_t*)malloc(sizeof(uint32_t) * (n ? n : 1));
        for (uint32_t i = 0; i < n; ++i) tmp[i] = groups[g0 + i].dst;
        qsort(tmp, n, sizeof(uint32_t), cmp_u32);
        for (uint32_t i = 0; i < n;) {
            uint32_t j = i;
            while (j < n && tmp[j] == tmp[i]) ++j;
            swDst[U] = tmp[i];
            occ[U] = j - i; /* one group per window: run length = windows containing dst */
            superWindowRows[U] = tmp[i];
            ++U;
            i = j;
        }
        free(tmp);
        /* 12-13: group -> slot (lookupGroupSlotsKernel :898-1000, :1003-1048). */
        const uint32_t base = superWindowRowOffset[s];
        for (uint32_t g = g0; g < g1; ++g) {
            uint32_t lo = base, hi = U;
            while (lo < hi) {
                uint32_t mid = lo + (hi - lo) / 2;
                if (swDst[mid] < groups[g].dst) lo = mid + 1; else hi = mid;
            }
            tileRowSlot[groupTile[g]] = lo - base;
        }
        g0 = g1;
    }
    superWindowRowOffset[SW] = U;

    /* 11: repeat cache per super-window (buildRepeatCacheMetadataKernel :699-895).
     * Order: occurrence descending (S..2), then slot ascending; first 32 cached. */
    for (uint32_t s = 0; s < SW; ++s) {
        const uint32_t b = superWindowRowOffset[s], e = superWindowRowOffset[s + 1];
        uint32_t cache = 0;
        for (int o = (int)MAX_SW; o >= 2; --o) {
            for (uint32_t u = b; u < e && cache < CACHE_SIZE; ++u) {
                if (occ[u] == (uint32_t)o) {
                    superWindowRowCacheSlot[u] = (uint8_t)cache;
                    superWindowCachedRowSlot[(size_t)s * CACHE_SIZE + cache] = u - b;
                    ++cache;
                }
            }
        }
        for (uint32_t u = b; u < e; ++u)
            if (occ[u] > MAX_SW) err = 4; /* :765-775 (unreachable for S <= 32) */
        superWindowCachedCount[s] = (uint8_t)cache;
    }

    /* padding rows keep tileRowSlot = INVALID and bits 0 (:1051-1107). */
    free(groups);
    free(degCount);
    free(degBase);
    free(degCursor);
    free(activeRows);
    free(groupTile);
    free(swDst);
    free(occ);
    return err;
}

/* ------------------------------------------------------------------ */
/* validateSWTCF (src/swtcf_convert_main.cu:36-130).  Returns 0 = PASS, */
/* otherwise a code naming the failed check.                           */
/* ------------------------------------------------------------------ */
static int cmp_u64(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

int oracle_validate_swtcf(const uint32_t* dst, const uint32_t* src, uint32_t E, uint32_t numSrc,
                          uint32_t S, uint32_t CW, const uint32_t* colWindowOffset,
                          const uint32_t* superWindowRowOffset, const uint32_t* superWindowRows,
                          const uint32_t* tileRowSlot, const uint64_t* tileLocalBit) {
    uint64_t* expected = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(E ? E : 1));
    size_t recCap = (size_t)E + 64, recN = 0;
    uint64_t* rec = (uint64_t*)malloc(sizeof(uint64_t) * recCap);
    int rc = 0;
    for (uint32_t e = 0; e < E; ++e) expected[e] = ((uint64_t)dst[e] << 32) | src[e];
    for (uint32_t w = 0; w < CW && !rc; ++w) {
        const uint32_t s = w / S;
        const uint32_t sb = superWindowRowOffset[s], se = superWindowRowOffset[s + 1];
        uint32_t prevDeg = 9;
        for (uint32_t t = colWindowOffset[w]; t < colWindowOffset[w + 1] && !rc; ++t) {
            const uint64_t bm = tileLocalBit[t];
            for (uint32_t lr = 0; lr < TILE_ROWS; ++lr) {
                const uint32_t rb = (uint32_t)((bm >> (lr * 8)) & 0xFFu);
                const uint32_t slot = tileRowSlot[(size_t)t * TILE_ROWS + lr];
                if (rb == 0) {
                    if (slot != INVALID_SLOT) { rc = 1; break; } /* padding slot not INVALID */
                    continue;
                }
                const uint32_t deg = (uint32_t)popcount8(rb);
                if (deg > prevDeg) { rc = 2; break; } /* not degree descending */
                prevDeg = deg;
                if (slot >= se - sb) { rc = 3; break; } /* invalid row slot */
                const uint32_t gdst = superWindowRows[sb + slot];
                for (uint32_t c = 0; c < 8; ++c) {
                    if (!(rb & (1u << c))) continue;
                    const uint32_t gsrc = w * 8 + c;
                    if (gsrc >= numSrc) { rc = 4; break; } /* src exceeds numSrc */
                    if (recN == recCap) {
                        recCap *= 2;
                        rec = (uint64_t*)realloc(rec, sizeof(uint64_t) * recCap);
                    }
                    rec[recN++] = ((uint64_t)gdst << 32) | gsrc;
                }
                if (rc) break;
            }
        }
    }
    if (!rc) {
        if (recN != E) rc = 5; /* edge count mismatch */
        else {
            qsort(expected, E, sizeof(uint64_t), cmp_u64);
            qsort(rec, recN, sizeof(uint64_t), cmp_u64);
            if (memcmp(expected, rec, sizeof(uint64_t) * (size_t)E) != 0) rc = 6; /* COO mismatch */
        }
    }
    free(expected);
    free(rec);
    return rc;
}

/* validateRepeatCacheMetadata (src/swtcf_convert_main.cu:132-310). */
int oracle_validate_repeat_cache(uint32_t S, uint32_t CW, uint32_t SW, const uint32_t* colWindowOffset,
                                 const uint32_t* superWindowRowOffset, const uint32_t* tileRowSlot,
                                 const uint64_t* tileLocalBit, const uint8_t* rowCacheSlot,
                                 const uint32_t* cachedRowSlot, const uint8_t* cachedCount) {
    for (uint32_t s = 0; s < SW; ++s) {
        const uint32_t rb = superWindowRowOffset[s], re = superWindowRowOffset[s + 1];
        const uint32_t n = re - rb;
        uint32_t* occ = (uint32_t*)calloc(n ? n : 1, sizeof(uint32_t));
        uint8_t* isCached = (uint8_t*)calloc(n ? n : 1, 1);
        uint8_t seen[CACHE_SIZE];
        memset(seen, 0, sizeof(seen));
        int rc = 0;
        const uint32_t wb = s * S, we = (wb + S < CW) ? wb + S : CW;
        for (uint32_t w = wb; w < we && !rc; ++w)
            for (uint32_t t = colWindowOffset[w]; t < colWindowOffset[w + 1] && !rc; ++t)
                for (uint32_t lr = 0; lr < TILE_ROWS; ++lr) {
                    if (((tileLocalBit[t] >> (lr * 8)) & 0xFFu) == 0) continue;
                    const uint32_t slot = tileRowSlot[(size_t)t * TILE_ROWS + lr];
                    if (slot >= n) { rc = 11; break; }
                    occ[slot]++;
                }
        uint32_t repeated = 0;
        for (uint32_t i = 0; i < n && !rc; ++i) {
            if (occ[i] == 0) rc = 12; /* unused row */
            else if (occ[i] > 1) ++repeated;
        }
        const uint32_t expected = repeated < CACHE_SIZE ? repeated : CACHE_SIZE;
        const uint32_t cc = cachedCount[s];
        if (!rc && cc != expected) rc = 13;
        uint32_t minCached = 0xFFFFFFFFu, maxUncached = 0;
        for (uint32_t c = 0; c < CACHE_SIZE && !rc; ++c) {
            const uint32_t slot = cachedRowSlot[(size_t)s * CACHE_SIZE + c];
            if (c < cc) {
                if (slot >= n) { rc = 14; break; }
                if (occ[slot] <= 1) { rc = 15; break; }
                if (isCached[slot]) { rc = 16; break; }
                if (seen[c]) { rc = 17; break; }
                isCached[slot] = 1;
                seen[c] = 1;
                if (rowCacheSlot[rb + slot] != (uint8_t)c) { rc = 18; break; }
                if (occ[slot] < minCached) minCached = occ[slot];
            } else if (slot != INVALID_SLOT) {
                rc = 19;
                break;
            }
        }
        for (uint32_t i = 0; i < n && !rc; ++i) {
            const uint8_t c = rowCacheSlot[rb + i];
            if (isCached[i]) {
                if (c >= CACHE_SIZE) rc = 20;
            } else {
                if (c != INVALID_CACHE) rc = 21;
                if (occ[i] > 1 && occ[i] > maxUncached) maxUncached = occ[i];
            }
        }
        if (!rc && repeated > CACHE_SIZE && minCached < maxUncached) rc = 22; /* top-H priority */
        free(occ);
        free(isCached);
        if (rc) return rc;
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* SpMM oracles.  Y is fp64.                                           */
/* ------------------------------------------------------------------ */

/* CSR SpMM: Y[r] = sum_k v_k * X[col_k] in fp64, with v and X rounded to TF32
 * when tf32 != 0 (the numerics of the reference's mma.m16n8k8 tf32 path,
 * include/mma_tf32.cuh:16-27).  vals == NULL means every value is 1.0
 * (spmm_cnic/src/core/spmm_kernel.cu:96-102).  Parallel over rows with
 * `threads` OpenMP threads (0 = runtime default). */
void oracle_csr_spmm(uint32_t rows, const int64_t* rowptr, const uint32_t* colind, const float* vals,
                     const float* X, uint32_t F, int tf32, int threads, double* Y) {
    if (threads > 0) {
#pragma omp parallel for schedule(dynamic, 64) num_threads(threads)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            double* y = Y + (size_t)r * F;
            for (uint32_t f = 0; f < F; ++f) y[f] = 0.0;
            for (int64_t k = rowptr[r]; k < rowptr[r + 1]; ++k) {
                const float v = vals ? (tf32 ? oracle_tf32(vals[k]) : vals[k]) : 1.0f;
                const float* x = X + (size_t)colind[k] * F;
                for (uint32_t f = 0; f < F; ++f)
                    y[f] += (double)v * (double)(tf32 ? oracle_tf32(x[f]) : x[f]);
            }
        }
    } else {
#pragma omp parallel for schedule(dynamic, 64)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            double* y = Y + (size_t)r * F;
            for (uint32_t f = 0; f < F; ++f) y[f] = 0.0;
            for (int64_t k = rowptr[r]; k < rowptr[r + 1]; ++k) {
                const float v = vals ? (tf32 ? oracle_tf32(vals[k]) : vals[k]) : 1.0f;
                const float* x = X + (size_t)colind[k] * F;
                for (uint32_t f = 0; f < F; ++f)
                    y[f] += (double)v * (double)(tf32 ? oracle_tf32(x[f]) : x[f]);
            }
        }
    }
}

/* SWTCF SpMM semantics (src/swtcf_spmm.cu:142-264): for every tile of every
 * column window, each nonzero row r adds sum_c bit(r,c) X[8w+c] to
 * Y[superWindowRows[off(s) + tileRowSlot]]; tiles with popcount >= tc use
 * TF32-rounded X (tensor-core path :188-221), sparser tiles fp32 X (:222-241).
 * Y (fp64, rows x F) is accumulated into, like the kernel's Y += A X. */
void oracle_swtcf_spmm(uint32_t CW, uint32_t S, const uint32_t* colWindowOffset,
                       const uint32_t* superWindowRowOffset, const uint32_t* superWindowRows,
                       const uint32_t* tileRowSlot, const uint64_t* tileLocalBit, const float* X,
                       uint32_t cols, uint32_t F, uint32_t tc, double* Y) {
    for (uint32_t w = 0; w < CW; ++w) {
        const uint32_t base = superWindowRowOffset[w / S];
        for (uint32_t t = colWindowOffset[w]; t < colWindowOffset[w + 1]; ++t) {
            const uint64_t bm = tileLocalBit[t];
            const int useTf32 = (uint32_t)__builtin_popcountll(bm) >= tc;
            for (uint32_t lr = 0; lr < TILE_ROWS; ++lr) {
                const uint32_t rb = (uint32_t)((bm >> (lr * 8)) & 0xFFu);
                const uint32_t slot = tileRowSlot[(size_t)t * TILE_ROWS + lr];
                if (rb == 0 || slot == INVALID_SLOT) continue;
                double* y = Y + (size_t)superWindowRows[base + slot] * F;
                for (uint32_t c = 0; c < 8; ++c) {
                    if (!(rb & (1u << c))) continue;
                    const uint32_t col = w * 8 + c;
                    if (col >= cols) continue; /* staged as 0 (:154-158) */
                    const float* x = X + (size_t)col * F;
                    for (uint32_t f = 0; f < F; ++f)
                        y[f] += (double)(useTf32 ? oracle_tf32(x[f]) : x[f]);
                }
            }
        }
    }
}

/* Known-answer input of src/swtcf_spmm_main.cu:33-45. */
float oracle_kat_source_a(uint32_t s) { return (float)((s * 17u + 13u) % 97u) * 0.001f; }
float oracle_kat_source_b(uint32_t s) { return (float)((s * 29u + 7u) % 89u) * 0.00001f; }

/* initializeXKernel (:47-56): X[s][f] = a(s) + b(s) * f in fp32. */
void oracle_kat_fill_x(uint32_t numSrc, uint32_t F, float* X) {
    for (uint32_t s = 0; s < numSrc; ++s) {
        const float a = oracle_kat_source_a(s), b = oracle_kat_source_b(s);
        for (uint32_t f = 0; f < F; ++f) X[(size_t)s * F + f] = a + b * (float)f;
    }
}

/* validateOutput's reference (:58-85): Y[r][f] = sum a(src) + f * sum b(src), fp64. */
void oracle_kat_expected(const uint32_t* dst, const uint32_t* src, uint32_t E, uint32_t numDst,
                         uint32_t F, double* Y) {
    double* sa = (double*)calloc(numDst ? numDst : 1, sizeof(double));
    double* sb = (double*)calloc(numDst ? numDst : 1, sizeof(double));
    for (uint32_t e = 0; e < E; ++e) {
        sa[dst[e]] += (double)oracle_kat_source_a(src[e]);
        sb[dst[e]] += (double)oracle_kat_source_b(src[e]);
    }
    for (uint32_t r = 0; r < numDst; ++r)
        for (uint32_t f = 0; f < F; ++f) Y[(size_t)r * F + f] = sa[r] + sb[r] * (double)f;
    free(sa);
    free(sb);
}

/* ------------------------------------------------------------------ */
/* Canonical BCSR / BCSC builders.  The reference's producer            */
/* (ipc_service) is absent; these fix the layout its kernels consume:  */
/* spmm_cnic/src/core/spmm_kernel.cu:87-121 (BCSR bitmap, sparseA2B),   */
/* :521-524, :600-615, :689-690 (BCSC), :88-101 (value order).          */
/* Input: CSR (row = destination, col = source) without duplicates.    */
/* ------------------------------------------------------------------ */

/* Number of BCSR blocks: per row window, distinct columns chunked by 8. */
int64_t oracle_bcsr_count(uint32_t rows, const int64_t* rowptr, const uint32_t* colind) {
    const uint32_t RW = (rows + 7) / 8;
    int64_t blocks = 0;
    for (uint32_t w = 0; w < RW; ++w) {
        const uint32_t r0 = w * 8, r1 = (r0 + 8 < rows) ? r0 + 8 : rows;
        const int64_t n = rowptr[r1] - rowptr[r0];
        uint32_t* tmp = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(n ? n : 1));
        memcpy(tmp, colind + rowptr[r0], sizeof(uint32_t) * (size_t)n);
        qsort(tmp, (size_t)n, sizeof(uint32_t), cmp_u32);
        int64_t u = 0;
        for (int64_t i = 0; i < n; ++i)
            if (i == 0 || tmp[i] != tmp[i - 1]) ++u;
        blocks += (u + 7) / 8;
        free(tmp);
    }
    return blocks;
}

/* Fills rowWindowOffset[RW+1], tcOffset[B+1], sparseA2B[8B] (padding
 * 0xFFFFFFFF), tcLocalBit[B], and data[nnz] (value of each set bit in
 * ascending bit order; vals == NULL gives 1.0).  Columns of a row window are
 * its distinct columns in ascending order, 8 per block. */
void oracle_bcsr_build(uint32_t rows, const int64_t* rowptr, const uint32_t* colind, const float* vals,
                       uint32_t* rowWindowOffset, uint32_t* tcOffset, uint32_t* sparseA2B,
                       uint64_t* tcLocalBit, float* data) {
    const uint32_t RW = (rows + 7) / 8;
    uint32_t b = 0, v = 0;
    for (uint32_t w = 0; w < RW; ++w) {
        rowWindowOffset[w] = b;
        const uint32_t r0 = w * 8, r1 = (r0 + 8 < rows) ? r0 + 8 : rows;
        const int64_t n = rowptr[r1] - rowptr[r0];
        uint32_t* tmp = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(n ? n : 1));
        memcpy(tmp, colind + rowptr[r0], sizeof(uint32_t) * (size_t)n);
        qsort(tmp, (size_t)n, sizeof(uint32_t), cmp_u32);
        int64_t u = 0;
        for (int64_t i = 0; i < n; ++i)
            if (i == 0 || tmp[i] != tmp[u - 1]) tmp[u++] = tmp[i];
        const uint32_t nb = (uint32_t)((u + 7) / 8);
        float* vv = (float*)calloc((size_t)nb * 64 + 1, sizeof(float));
        for (uint32_t k = 0; k < nb; ++k) {
            tcLocalBit[b + k] = 0;
            for (uint32_t c = 0; c < 8; ++c) {
                const int64_t idx = (int64_t)k * 8 + c;
                sparseA2B[(size_t)(b + k) * 8 + c] = idx < u ? tmp[idx] : INVALID_SLOT;
            }
        }
        for (uint32_t r = r0; r < r1; ++r)
            for (int64_t q = rowptr[r]; q < rowptr[r + 1]; ++q) {
                int64_t lo = 0, hi = u; /* position of the column in the compacted list */
                while (lo < hi) {
                    int64_t mid = (lo + hi) / 2;
                    if (tmp[mid] < colind[q]) lo = mid + 1; else hi = mid;
                }
                const uint32_t k = (uint32_t)(lo / 8);
                const uint32_t bit = (r - r0) * 8 + (uint32_t)(lo % 8);
                tcLocalBit[b + k] |= 1ull << bit;
                vv[(size_t)k * 64 + bit] = vals ? vals[q] : 1.0f;
            }
        for (uint32_t k = 0; k < nb; ++k) {
            const uint64_t bm = tcLocalBit[b + k];
            tcOffset[b + k] = v;
            for (int i = 0; i < 64; ++i)
                if (bm >> i & 1ull) data[v++] = vv[(size_t)k * 64 + i];
        }
        b += nb;
        free(vv);
        free(tmp);
    }
    rowWindowOffset[RW] = b;
    tcOffset[b] = v;
}

/* Number of BCSC blocks: per column window (8 sources), distinct destination
 * rows chunked by 8.  Needs the CSR transposed view: colptr/rowind over
 * sources (CSC of A). */
int64_t oracle_bcsc_count(uint32_t cols, const int64_t* colptr, const uint32_t* rowind) {
    const uint32_t CWn = (cols + 7) / 8;
    int64_t blocks = 0;
    for (uint32_t w = 0; w < CWn; ++w) {
        const uint32_t c0 = w * 8, c1 = (c0 + 8 < cols) ? c0 + 8 : cols;
        const int64_t n = colptr[c1] - colptr[c0];
        uint32_t* tmp = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(n ? n : 1));
        memcpy(tmp, rowind + colptr[c0], sizeof(uint32_t) * (size_t)n);
        qsort(tmp, (size_t)n, sizeof(uint32_t), cmp_u32);
        int64_t u = 0;
        for (int64_t i = 0; i < n; ++i)
            if (i == 0 || tmp[i] != tmp[i - 1]) ++u;
        blocks += (u + 7) / 8;
        free(tmp);
    }
    return blocks;
}

typedef struct {
    uint32_t dst, deg, bits;
    float v[8];
} bcsc_row_t;

typedef struct {
    uint32_t dst, c;
    float v;
} bcsc_entry_t;

static int cmp_bcsc_entry(const void* a, const void* b) {
    const bcsc_entry_t* x = (const bcsc_entry_t*)a;
    const bcsc_entry_t* y = (const bcsc_entry_t*)b;
    if (x->dst != y->dst) return x->dst < y->dst ? -1 : 1;
    return x->c < y->c ? -1 : (x->c > y->c ? 1 : 0);
}

static int cmp_bcsc_row(const void* a, const void* b) {
    const bcsc_row_t* x = (const bcsc_row_t*)a;
    const bcsc_row_t* y = (const bcsc_row_t*)b;
    if (x->deg != y->deg) return x->deg > y->deg ? -1 : 1; /* degree descending */
    return x->dst < y->dst ? -1 : (x->dst > y->dst ? 1 : 0); /* dst ascending */
}

/* BCSC canonical form = the SWTCF row order with one window per super-window:
 * rows of a column window sorted by (degree desc, dst asc), 8 per block,
 * padding rows 0xFFFFFFFF.  Input is the CSC of A (colptr over sources,
 * rowind = destinations, cvals aligned with rowind; NULL = all 1.0). */
void oracle_bcsc_build(uint32_t cols, const int64_t* colptr, const uint32_t* rowind, const float* cvals,
                       uint32_t* colWindowOffset, uint32_t* tcOffset, uint32_t* sparseA2C,
                       uint64_t* tcLocalBit, float* data) {
    const uint32_t CWn = (cols + 7) / 8;
    uint32_t b = 0, v = 0;
    for (uint32_t w = 0; w < CWn; ++w) {
        colWindowOffset[w] = b;
        const uint32_t c0 = w * 8, c1 = (c0 + 8 < cols) ? c0 + 8 : cols;
        const int64_t n = colptr[c1] - colptr[c0];
        bcsc_entry_t* ent = (bcsc_entry_t*)malloc(sizeof(bcsc_entry_t) * (size_t)(n ? n : 1));
        int64_t m = 0;
        for (uint32_t c = c0; c < c1; ++c)
            for (int64_t q = colptr[c]; q < colptr[c + 1]; ++q) {
                ent[m].dst = rowind[q];
                ent[m].c = c - c0;
                ent[m].v = cvals ? cvals[q] : 1.0f;
                ++m;
            }
        qsort(ent, (size_t)m, sizeof(bcsc_entry_t), cmp_bcsc_entry);
        bcsc_row_t* rowsv = (bcsc_row_t*)calloc((size_t)(m ? m : 1), sizeof(bcsc_row_t));
        int64_t u = 0;
        for (int64_t i = 0; i < m; ++i) {
            if (i == 0 || ent[i].dst != ent[i - 1].dst) rowsv[u++].dst = ent[i].dst;
            bcsc_row_t* rr = &rowsv[u - 1];
            rr->deg++;
            rr->bits |= 1u << ent[i].c;
            rr->v[ent[i].c] = ent[i].v;
        }
        free(ent);
        qsort(rowsv, (size_t)u, sizeof(bcsc_row_t), cmp_bcsc_row);
        const uint32_t nb = (uint32_t)((u + 7) / 8);
        for (uint32_t k = 0; k < nb; ++k) {
            uint64_t bm = 0;
            for (uint32_t r = 0; r < 8; ++r) {
                const int64_t idx = (int64_t)k * 8 + r;
                sparseA2C[(size_t)(b + k) * 8 + r] = idx < u ? rowsv[idx].dst : INVALID_SLOT;
                if (idx < u) bm |= (uint64_t)rowsv[idx].bits << (r * 8);
            }
            tcLocalBit[b + k] = bm;
            tcOffset[b + k] = v;
            for (uint32_t i = 0; i < 64; ++i)
                if (bm >> i & 1ull) data[v++] = rowsv[(int64_t)k * 8 + i / 8].v[i % 8];
        }
        b += nb;
        free(rowsv);
    }
    colWindowOffset[CWn] = b;
    tcOffset[b] = v;
}

static double block_value(const float* data, const uint32_t* tcOffset, uint32_t blk, uint64_t bm,
                          uint32_t bit) {
    if (!data) return 1.0;
    const uint64_t below = bit ? (bm & ((1ull << bit) - 1ull)) : 0ull;
    return (double)oracle_tf32(data[tcOffset[blk] + (uint32_t)__builtin_popcountll(below)]);
}

/* BCSR SpMM as the kernel consumes it (spmm_kernel.cu:1560-1842):
 * Y[8w+r] += sum_b sum_c bit(r,c) * v * tf32(X[sparseA2B[8b+c]]), padding
 * columns (>= num_cols) skipped.  Y is fp64 [8*RW x F], accumulated into. */
void oracle_bcsr_spmm(uint32_t RW, const uint32_t* rowWindowOffset, const uint32_t* tcOffset,
                      const uint32_t* sparseA2B, const uint64_t* tcLocalBit, const float* data,
                      uint32_t num_cols, const float* X, uint32_t F, double* Y) {
    for (uint32_t w = 0; w < RW; ++w)
        for (uint32_t b = rowWindowOffset[w]; b < rowWindowOffset[w + 1]; ++b) {
            const uint64_t bm = tcLocalBit[b];
            for (uint32_t bit = 0; bit < 64; ++bit) {
                if (!(bm >> bit & 1ull)) continue;
                const uint32_t r = bit / 8, c = bit % 8;
                const uint32_t col = sparseA2B[(size_t)b * 8 + c];
                if (col >= num_cols) continue;
                const double v = block_value(data, tcOffset, b, bm, bit);
                double* y = Y + ((size_t)w * 8 + r) * F;
                const float* x = X + (size_t)col * F;
                for (uint32_t f = 0; f < F; ++f) y[f] += v * (double)oracle_tf32(x[f]);
            }
        }
}

/* BCSC SpMM (spmm_kernel.cu:1844-2166): Y[sparseA2C[8b+r]] += sum_c bit(r,c)
 * * v * tf32(X[8w+c]); rows >= num_rows and sources >= num_cols skipped.
 * Y is fp64 [num_rows x F], accumulated into. */
void oracle_bcsc_spmm(uint32_t CWn, const uint32_t* colWindowOffset, const uint32_t* tcOffset,
                      const uint32_t* sparseA2C, const uint64_t* tcLocalBit, const float* data,
                      uint32_t num_rows, uint32_t num_cols, const float* X, uint32_t F, double* Y) {
    for (uint32_t w = 0; w < CWn; ++w)
        for (uint32_t b = colWindowOffset[w]; b < colWindowOffset[w + 1]; ++b) {
            const uint64_t bm = tcLocalBit[b];
            for (uint32_t bit = 0; bit < 64; ++bit) {
                if (!(bm >> bit & 1ull)) continue;
                const uint32_t r = bit / 8, c = bit % 8;
                const uint32_t row = sparseA2C[(size_t)b * 8 + r];
                const uint32_t col = w * 8 + c;
                if (row >= num_rows || col >= num_cols) continue;
                const double v = block_value(data, tcOffset, b, bm, bit);
                double* y = Y + (size_t)row * F;
                const float* x = X + (size_t)col * F;
                for (uint32_t f = 0; f < F; ++f) y[f] += v * (double)oracle_tf32(x[f]);
            }
        }
}

/* Transposed BCSC use: dX[8w+c] += sum_b sum_r bit(r,c) * v * dY[sparseA2C[8b+r]],
 * rows >= num_rows skipped.  dX is fp64 [8*CW x F], accumulated into.  This is
 * A^T * dY of train/tcgnn_conv_release.py:152, where torch.sparse.mm
 * multiplies the fp32 operands as given (no TF32 rounding of dY or v). */
void oracle_bcsc_transpose_spmm(uint32_t CWn, const uint32_t* colWindowOffset, const uint32_t* tcOffset,
                                const uint32_t* sparseA2C, const uint64_t* tcLocalBit,
                                const float* data, uint32_t num_rows, const float* dY, uint32_t F,
                                double* dX) {
    for (uint32_t w = 0; w < CWn; ++w)
        for (uint32_t b = colWindowOffset[w]; b < colWindowOffset[w + 1]; ++b) {
            const uint64_t bm = tcLocalBit[b];
            for (uint32_t bit = 0; bit < 64; ++bit) {
                if (!(bm >> bit & 1ull)) continue;
                const uint32_t r = bit / 8, c = bit % 8;
                const uint32_t row = sparseA2C[(size_t)b * 8 + r];
                if (row >= num_rows) continue;
                double v = 1.0;
                if (data) {
                    const uint64_t below = bit ? (bm & ((1ull << bit) - 1ull)) : 0ull;
                    v = (double)data[tcOffset[b] + (uint32_t)__builtin_popcountll(below)];
                }
                double* x = dX + ((size_t)w * 8 + c) * F;
                const float* y = dY + (size_t)row * F;
                for (uint32_t f = 0; f < F; ++f) x[f] += v * (double)y[f];
            }
        }
}

/* Feature-row resolution of the first GCN layer (spmm_kernel.cu:129-153),
 * single-GPU slice: g = cache_search_map[j]; g >= 0 -> hot[g % cap] (the
 * clique index g / cap must be 0 on one GPU), else cpu[id_map[j]] or zeros
 * when id_map[j] < 0.  Writes the resolved dense X [cols x F]. */
int oracle_resolve_features(uint32_t cols, const int32_t* id_map, const int32_t* cache_search_map,
                            const float* hot, int32_t cap, const float* cpu, int64_t cpu_len,
                            uint32_t F, float* X) {
    for (uint32_t j = 0; j < cols; ++j) {
        float* x = X + (size_t)j * F;
        const int32_t g = cache_search_map[j];
        const float* srcRow = NULL;
        if (g >= 0) {
            if (g / cap != 0) return 1;
            srcRow = hot + (size_t)(g % cap) * F;
        } else if (id_map[j] >= 0) {
            if ((int64_t)id_map[j] * F + F > cpu_len) return 2;
            srcRow = cpu + (size_t)id_map[j] * F;
        }
        for (uint32_t f = 0; f < F; ++f) x[f] = srcRow ? srcRow[f] : 0.0f;
    }
    return 0;
}
