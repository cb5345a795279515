// Tall-skinny transposed products C = A^T B of the GCN layer backward, for
// gfx950 (reference: torch.mm(X_out.T, d_output),
// TAC_training_backend/train/tcgnn_conv_release.py:150).
//
// A [K x M] and B [K x N] are row-major with K = graph nodes (millions) and
// M, N = layer widths (hundreds or less).  K is split over workgroups; each
// accumulates the product of its rows for one block of C with
// v_mfma_f32_16x16x4f32 (fp32 products and sums) and writes it to a partial
// buffer, and a second kernel sums the partials in a fixed order.
//
// MFMA operand layout (16x16x4, fp32): lane l supplies A(i = l%16, k = l/16)
// and B(k = l/16, j = l%16), and holds D(4*(l/16) + v, l%16) in accumulator
// register v.  For C = A^T B the A operand of a 16x16 tile at (m0, n0) and
// rows k..k+3 is A[k + l/16][m0 + l%16] and the B operand B[k + l/16][n0 + l%16]:
// both are 16 consecutive floats of one input row per lane quarter, so the
// operands are loaded straight from global memory without a transpose.
// Columns past M (N) are clamped to the last one: they only feed rows
// (columns) of C that are never stored.  Rows past K are zero.
#include <algorithm>
#include <mutex>

#include "../../include/tcc_gcn.h"
#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "primitives.hpp"

namespace tcc {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct TnArgs {
    const float* A;
    const float* B;
    float* partial;  // [splits][M][N]
    std::uint32_t lda, ldb;
    std::uint32_t K, M, N;
    std::uint32_t rowsPerSplit;
    std::uint32_t blocksM;  // blocks of C along M
    // Relu-gradient form only (see tn_partial_kernel): G [K x C] with row
    // stride ldg, W2 [N x C], and the H^T G partials [splits][N][C].
    const float* G;
    const float* W2;
    float* partial2;
    std::uint32_t ldg, C;
};

__device__ __forceinline__ std::uint32_t tn_uniform(std::uint32_t v) {
    return static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

// Workgroup = WM x WN waves; a wave owns TM x TN tiles of 16x16, so a
// workgroup covers a (16*TM*WM) x (16*TN*WN) block of C.  Each iteration
// takes U steps of 4 rows; the next iteration's operands are loaded while
// the current one is multiplied.
//
// CT > 0 is the GCN relu-gradient form: B holds H (the relu output of the
// layer, [K x N]) and the B operand is formed in registers as
// (G W2^T) (.) [H > 0] from G [K x C] and W2 [N x C] (C <= CT), while H^T G
// is summed beside it into partial2 -- the layer-1 weight gradient and the
// layer-2 weight gradient of a two-layer GCN in one pass over its rows.
template <int TM, int TN, int WM, int WN, int U, int CT, bool VB = false, bool VA = false>
__global__ void __launch_bounds__(kWave * WM * WN) tn_partial_kernel(TnArgs a) {
    static_assert(!VB || TN % 4 == 0, "a float4 of B feeds four N tiles");
    constexpr int TA = VA ? TM / 4 : 0;  // groups of four M tiles fed by one float4 of A
    constexpr int BM = 16 * TM * WM, BN = 16 * TN * WN;
    constexpr int GC = CT > 0 ? CT : 1;  // G columns held per row
    constexpr std::uint32_t kStep = 4 * U;
    const unsigned lane = __lane_id();
    const unsigned wave = tn_uniform(threadIdx.x / kWave);
    const unsigned wm = wave % WM, wn = wave / WM;
    const std::uint32_t cbm = blockIdx.y % a.blocksM, cbn = blockIdx.y / a.blocksM;
    const std::uint32_t m0 = cbm * BM + wm * 16 * TM, n0 = cbn * BN + wn * 16 * TN;
    const std::uint32_t k0 = blockIdx.x * a.rowsPerSplit;
    const std::uint32_t k1 = min(a.K, k0 + a.rowsPerSplit);
    const unsigned li = lane & 15u, lk = lane >> 4;
    // Column of N tile u on this lane: 16u + l%16; with VB, tile u = 4g + t
    // takes column 64g + 4(l%16) + t, so that one float4 load from a row of B
    // feeds four tiles (a quarter of the load instructions, each costing the
    // same address-processing time whatever its width).
    const auto ncol = [&](int u) -> std::uint32_t {
        return VB ? n0 + 64 * (u / 4) + 4 * li + (u % 4) : n0 + 16 * u + li;
    };
    // Row r of M tile t: 16t + r, or with VA, for the first 4*TA tiles
    // (t = 4h + e), 64h + 4r + e (one float4 of an A row feeds four tiles).
    const auto mrow = [&](int t, unsigned r) -> std::uint32_t {
        return t < 4 * TA ? m0 + 64 * (t / 4) + 4 * r + (t % 4) : m0 + 16 * t + r;
    };

    // Per-lane element offsets inside a 4-row step (row lk, clamped column;
    // with VB the float4's start, clamped to the row's last 4 columns: a
    // clamped float4 only feeds columns past N, which are never stored).
    std::uint32_t offA[TM], offB[TN];
#pragma unroll
    for (int t = 0; t < TM; ++t)
        offA[t] = t < 4 * TA ? lk * a.lda + min(m0 + 64 * (t / 4) + 4 * li, a.M - 4) : lk * a.lda + min(mrow(t, li), a.M - 1);
#pragma unroll
    for (int t = 0; t < TN; ++t)
        offB[t] = VB ? lk * a.ldb + min(n0 + 64 * (t / 4) + 4 * li, a.N - 4) : lk * a.ldb + min(ncol(t), a.N - 1);
    // Relu-gradient form: this lane's W2 rows, G column offsets (clamped).
    float w2[TN][GC];
    float dw2[TN][GC];
    std::uint32_t offG[GC];
#pragma unroll
    for (int j = 0; j < GC; ++j) offG[j] = CT > 0 ? lk * a.ldg + min<std::uint32_t>(j, a.C - 1) : 0u;
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int j = 0; j < GC; ++j) {
            dw2[t][j] = 0.0f;
            w2[t][j] = 0.0f;
            if (CT > 0 && static_cast<std::uint32_t>(j) < a.C)
                w2[t][j] = a.W2[static_cast<std::uint64_t>(min(ncol(t), a.N - 1)) * a.C + j];
        }

    f32x4 acc[TM][TN];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u) acc[t][u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto load_full = [&](std::uint32_t k, float (&xa)[U][TM], float (&xb)[U][TN], float (&xg)[U][GC]) {
#pragma unroll
        for (int s = 0; s < U; ++s) {
            const float* ra = a.A + static_cast<std::uint64_t>(k + 4 * s) * a.lda;
            const float* rb = a.B + static_cast<std::uint64_t>(k + 4 * s) * a.ldb;
#pragma unroll
            for (int h = 0; h < TA; ++h) {
                const float4 v = *reinterpret_cast<const float4*>(ra + offA[4 * h]);
                xa[s][4 * h] = v.x;
                xa[s][4 * h + 1] = v.y;
                xa[s][4 * h + 2] = v.z;
                xa[s][4 * h + 3] = v.w;
            }
#pragma unroll
            for (int t = 4 * TA; t < TM; ++t) xa[s][t] = ra[offA[t]];
            if constexpr (VB) {
#pragma unroll
                for (int g = 0; g < TN / 4; ++g) {
                    const float4 v = *reinterpret_cast<const float4*>(rb + offB[4 * g]);
                    xb[s][4 * g] = v.x;
                    xb[s][4 * g + 1] = v.y;
                    xb[s][4 * g + 2] = v.z;
                    xb[s][4 * g + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int t = 0; t < TN; ++t) xb[s][t] = rb[offB[t]];
            }
            if constexpr (CT > 0) {
                const float* rg = a.G + static_cast<std::uint64_t>(k + 4 * s) * a.ldg;
#pragma unroll
                for (int j = 0; j < GC; ++j) xg[s][j] = rg[offG[j]];
            }
        }
    };
    auto multiply = [&](const float (&xa)[U][TM], const float (&xb)[U][TN], const float (&xg)[U][GC]) {
#pragma unroll
        for (int s = 0; s < U; ++s) {
            float b[TN];
#pragma unroll
            for (int u = 0; u < TN; ++u) {
                if constexpr (CT > 0) {
                    // dOut1 = (G W2^T) (.) [H > 0]; dW2 += H^T G (columns past C have w2 = 0
                    // and are never stored)
                    float d = 0.0f;
#pragma unroll
                    for (int j = 0; j < GC; ++j) {
                        d = fmaf(xg[s][j], w2[u][j], d);
                        dw2[u][j] = fmaf(xb[s][u], xg[s][j], dw2[u][j]);
                    }
                    b[u] = xb[s][u] > 0.0f ? d : 0.0f;
                } else {
                    b[u] = xb[s][u];
                }
            }
#pragma unroll
            for (int t = 0; t < TM; ++t)
#pragma unroll
                for (int u = 0; u < TN; ++u)
                    acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[s][t], b[u], acc[t][u], 0, 0, 0);
        }
    };

    // Two operand buffers in turn; loads are unconditional (past the last
    // full iteration they repeat in-bounds rows and are not used), so the
    // loads of one buffer stay in flight while the other is multiplied.
    // (sched_barrier keeps the scheduler from sinking the loads to their
    // uses, which it does to lower register pressure.)
    const std::uint32_t rows = k1 > k0 ? k1 - k0 : 0u;
    const std::uint32_t nFull = rows / kStep;
    float ca[U][TM], cb[U][TN], cg[U][GC], na[U][TM], nb[U][TN], ng[U][GC];
#pragma unroll
    for (int s = 0; s < U; ++s)
#pragma unroll
        for (int j = 0; j < GC; ++j) cg[s][j] = ng[s][j] = 0.0f;
    if (nFull > 0) load_full(k0, ca, cb, cg);
    std::uint32_t i = 0;
    for (; i + 1 < nFull; i += 2) {
        const std::uint32_t k = k0 + i * kStep;
        load_full(k + kStep, na, nb, ng);
        __builtin_amdgcn_sched_barrier(0);
        multiply(ca, cb, cg);
        __builtin_amdgcn_sched_barrier(0);
        load_full(i + 2 < nFull ? k + 2 * kStep : k + kStep, ca, cb, cg);
        __builtin_amdgcn_sched_barrier(0);
        multiply(na, nb, ng);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (i < nFull) multiply(ca, cb, cg);
    const std::uint32_t kt = k0 + nFull * kStep;
    if (kt < k1) {  // last rows of the split: zeros past k1
#pragma unroll
        for (int s = 0; s < U; ++s) {
            const bool in = kt + 4 * s + lk < k1;
            const float* ra = a.A + static_cast<std::uint64_t>(kt + 4 * s) * a.lda;
            const float* rb = a.B + static_cast<std::uint64_t>(kt + 4 * s) * a.ldb;
#pragma unroll
            for (int h = 0; h < TA; ++h) {
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (in) v = *reinterpret_cast<const float4*>(ra + offA[4 * h]);
                ca[s][4 * h] = v.x;
                ca[s][4 * h + 1] = v.y;
                ca[s][4 * h + 2] = v.z;
                ca[s][4 * h + 3] = v.w;
            }
#pragma unroll
            for (int t = 4 * TA; t < TM; ++t) ca[s][t] = in ? ra[offA[t]] : 0.0f;
            if constexpr (VB) {
#pragma unroll
                for (int g = 0; g < TN / 4; ++g) {
                    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (in) v = *reinterpret_cast<const float4*>(rb + offB[4 * g]);
                    cb[s][4 * g] = v.x;
                    cb[s][4 * g + 1] = v.y;
                    cb[s][4 * g + 2] = v.z;
                    cb[s][4 * g + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int t = 0; t < TN; ++t) cb[s][t] = in ? rb[offB[t]] : 0.0f;
            }
            if constexpr (CT > 0) {
                const float* rg = a.G + static_cast<std::uint64_t>(kt + 4 * s) * a.ldg;
#pragma unroll
                for (int j = 0; j < GC; ++j) cg[s][j] = in ? rg[offG[j]] : 0.0f;
            }
        }
        multiply(ca, cb, cg);
    }

    // Tile (t, u): accumulator v of lane l is C(mrow(t, 4*(l/16) + v), ncol(u)).
    float* out = a.partial + static_cast<std::uint64_t>(blockIdx.x) * a.M * a.N;
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u) {
            const std::uint32_t n = ncol(u);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const std::uint32_t m = mrow(t, 4 * lk + v);
                if (m < a.M && n < a.N) out[static_cast<std::uint64_t>(m) * a.N + n] = acc[t][u][v];
            }
        }
    if constexpr (CT > 0) {
        // H^T G of this split: column n = ncol(u) summed over the 4 row
        // quarters; one block row of C (cbm == 0, first wave row) writes it.
        float* out2 = a.partial2 + static_cast<std::uint64_t>(blockIdx.x) * a.N * a.C;
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
            for (int j = 0; j < GC; ++j) {
                float v = dw2[u][j];
                v += __shfl_xor(v, 16);
                v += __shfl_xor(v, 32);
                const std::uint32_t n = ncol(u);
                if (cbm == 0 && wm == 0 && lk == 0 && n < a.N && static_cast<std::uint32_t>(j) < a.C)
                    out2[static_cast<std::uint64_t>(n) * a.C + j] = v;
            }
    }
}

// ---------------------------------------------------------------- forward
// H = relu(AX W1) [K x Hd] and XW = H W2 [K x C] in one pass over the rows
// of AX (the first layer's transform, its activation and the second layer's
// transform of a two-layer GCN; tcgnn_conv_release.py:134 and :243-247).
//
// A wave computes 16 rows x 256 hidden units (16 tiles of 16x16) over
// F <= 16*KB inputs with v_mfma_f32_16x16x4f32.  Lane (q = l/16, i = l%16)
// loads AX[row0 + i][16b + 4q .. +3] as one float4 per block b of 16 inputs,
// and MFMA step s of block b takes input 16b + 4q + s on lane quarter q: the
// sum over the 16 inputs is the same in any order, so the four steps come
// from one float4 instead of four strided loads.  The matching B operands,
// W1[16b + 4q + s][16u + i] for s = 0..3, are one ds_read_b128 from W1^T
// held in LDS (row pitch 16*KB + 4 floats: conflict-free b128 reads).
// Relu, the store of H and the row sums of H W2 (a 16-lane butterfly) follow
// in registers.  Workgroups (one per CU for the LDS copy of W1^T, 12 waves:
// 1.44 ms for 2.45M x 100 x 256 against 1.59-1.68 ms with 8, before the
// interleaved MFMA steps below) are persistent
// over 16-row tiles.
struct ReluFwdArgs {
    const float* AX;
    const float* W1;  // [F x Hd]
    const float* W2;  // [Hd x C]
    float* H;
    float* XW;
    std::uint32_t ldax, ldh, ldxw;
    std::uint32_t K, F, Hd, C;
    std::uint32_t tiles;  // ceil(K / 16)
    int vec;              // AX rows allow float4 loads
};

constexpr unsigned kFwdWaves = 12;  // waves per workgroup (one workgroup per CU: the LDS copy of W1^T)
constexpr int kFwdTiles = 16;       // 16 tiles of 16 hidden units per wave

template <int KB>
__device__ __forceinline__ void fwd_load_rows(const ReluFwdArgs& a, std::uint32_t tile, float4 (&x)[KB]) {
    const unsigned lane = __lane_id();
    const std::uint32_t row = tile * 16 + (lane & 15u);
    const unsigned q = lane >> 4;
#pragma unroll
    for (int b = 0; b < KB; ++b) {
        const std::uint32_t k = 16 * b + 4 * q;
        x[b] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (row >= a.K || tile >= a.tiles) continue;
        const float* p = a.AX + static_cast<std::uint64_t>(row) * a.ldax + k;
        if (a.vec && k + 3 < a.F) {
            x[b] = *reinterpret_cast<const float4*>(p);
        } else {
            if (k < a.F) x[b].x = p[0];
            if (k + 1 < a.F) x[b].y = p[1];
            if (k + 2 < a.F) x[b].z = p[2];
            if (k + 3 < a.F) x[b].w = p[3];
        }
    }
}

// PF: load the next tile's rows during the current tile's products (with 12
// waves per CU measured no faster than without, 1.44-1.57 ms for
// 2.45M x 100 x 256, and 28 VGPRs more).
template <int KB, int CT, unsigned W = kFwdWaves, bool PF = false>
__global__ void __launch_bounds__(kWave * W) gcn_relu_forward_kernel(ReluFwdArgs a) {
    constexpr int KP = 16 * KB + 4;  // LDS row pitch of W1^T (floats)
    extern __shared__ float w1t[];   // [256][KP], then W2 [256][CT]
    const unsigned lane = __lane_id();
    const unsigned i = lane & 15u, q = lane >> 4;
    const unsigned wave = tn_uniform(threadIdx.x / kWave);

    // W1^T into LDS, zeros past F and Hd.
    for (std::uint32_t e = threadIdx.x; e < 256u * KP; e += blockDim.x) {
        const std::uint32_t n = e / KP, k = e - n * KP;
        w1t[e] = (n < a.Hd && k < a.F) ? a.W1[static_cast<std::uint64_t>(k) * a.Hd + n] : 0.0f;
    }
    // W2 [256][CT] after it, zeros past Hd and C.
    float* w2 = w1t + 256 * KP;
    for (std::uint32_t e = threadIdx.x; e < 256u * CT; e += blockDim.x) {
        const std::uint32_t n = e / CT, j = e - n * CT;
        w2[e] = (n < a.Hd && j < a.C) ? a.W2[static_cast<std::uint64_t>(n) * a.C + j] : 0.0f;
    }
    __syncthreads();

    const std::uint32_t stride = gridDim.x * W;
    std::uint32_t tile = blockIdx.x * W + wave;
    float4 x[KB];
    if (PF) fwd_load_rows<KB>(a, tile, x);
    for (; tile < a.tiles; tile += stride) {
        float4 nx[KB];
        if (PF) {
            fwd_load_rows<KB>(a, tile + stride, nx);  // past the last tile: zeros, no loads
        } else {
            fwd_load_rows<KB>(a, tile, x);
        }
        __builtin_amdgcn_sched_barrier(0);
        f32x4 acc[kFwdTiles];
#pragma unroll
        for (int u = 0; u < kFwdTiles; ++u) acc[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // W1^T rows as float4 (KP % 4 == 0): ds_read_b128.  Each step s runs
        // over 8 accumulators before the next, so no MFMA waits on the one
        // before it.
        const float4* w1t4 = reinterpret_cast<const float4*>(w1t);
#pragma unroll
        for (int b = 0; b < KB; ++b) {
#pragma unroll
            for (int h = 0; h < kFwdTiles; h += 8) {
                float4 w[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) w[t] = w1t4[(16 * (h + t) + i) * (KP / 4) + 4 * b + q];
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[h + t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[b].x, w[t].x, acc[h + t], 0, 0, 0);
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[h + t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[b].y, w[t].y, acc[h + t], 0, 0, 0);
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[h + t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[b].z, w[t].z, acc[h + t], 0, 0, 0);
#pragma unroll
                for (int t = 0; t < 8; ++t) acc[h + t] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[b].w, w[t].w, acc[h + t], 0, 0, 0);
            }
        }
        // Lane holds H(row0 + 4q + v, 16u + i): relu (NaN kept, as clamp_min),
        // store, and this lane's part of the row sums of H W2.
        const std::uint32_t row0 = tile * 16 + 4 * q;
        float xw[4][CT];
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int j = 0; j < CT; ++j) xw[v][j] = 0.0f;
#pragma unroll
        for (int u = 0; u < kFwdTiles; ++u) {
            const std::uint32_t n = 16 * u + i;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float h = acc[u][v] < 0.0f ? 0.0f : acc[u][v];
                if (row0 + v < a.K && n < a.Hd) a.H[static_cast<std::uint64_t>(row0 + v) * a.ldh + n] = h;
#pragma unroll
                for (int j = 0; j < CT; ++j) xw[v][j] = fmaf(h, w2[n * CT + j], xw[v][j]);
            }
        }
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int j = 0; j < CT; ++j) {
                float t = xw[v][j];
                t += __shfl_xor(t, 1);
                t += __shfl_xor(t, 2);
                t += __shfl_xor(t, 4);
                t += __shfl_xor(t, 8);
                if (i == 0 && row0 + v < a.K && static_cast<std::uint32_t>(j) < a.C)
                    a.XW[static_cast<std::uint64_t>(row0 + v) * a.ldxw + j] = t;
            }
        if (PF) {
#pragma unroll
            for (int b = 0; b < KB; ++b) x[b] = nx[b];
        }
    }
}

template <int KB, int CT, unsigned W = kFwdWaves>
void relu_forward_launch(const ReluFwdArgs& a, hipStream_t st) {
    const std::uint32_t lds = 256u * (16 * KB + 4 + CT) * sizeof(float);
    const std::uint32_t grid = std::min<std::uint32_t>(device_cus(), (a.tiles + W - 1) / W);
    hipLaunchKernelGGL((gcn_relu_forward_kernel<KB, CT, W>), dim3(std::max<std::uint32_t>(grid, 1)), dim3(kWave * W),
                       lds, st, a);
}

// C[m][n] (=|+=) sum over splits of partial[s][m][n], splits added in a fixed
// order: 16 elements per workgroup, 16 interleaved groups of splits summed
// per thread, then the 16 group sums in order.
// With `transposed` the partials hold C^T (an M x N block of C^T is C's
// N x M block): element (m, n) of the partials goes to C[n][m].
__global__ void __launch_bounds__(256) tn_reduce_kernel(const float* __restrict__ partial, std::uint32_t splits,
                                                        std::uint32_t M, std::uint32_t N, float* __restrict__ C,
                                                        std::uint32_t ldc, int accumulate, int transposed) {
    __shared__ float part[16][17];
    const std::uint64_t MN = static_cast<std::uint64_t>(M) * N;
    const unsigned col = threadIdx.x & 15u, grp = threadIdx.x >> 4;
    const std::uint64_t e = static_cast<std::uint64_t>(blockIdx.x) * 16 + col;
    float s = 0.0f;
    if (e < MN)
        for (std::uint32_t sp = grp; sp < splits; sp += 16) s += partial[sp * MN + e];
    part[grp][col] = s;
    __syncthreads();
    if (threadIdx.x < 16 && e < MN) {
        float t = 0.0f;
#pragma unroll
        for (int g = 0; g < 16; ++g) t += part[g][col];
        const std::uint32_t m = static_cast<std::uint32_t>(e / N), n = static_cast<std::uint32_t>(e % N);
        float* c = transposed ? C + static_cast<std::uint64_t>(n) * ldc + m : C + static_cast<std::uint64_t>(m) * ldc + n;
        *c = accumulate ? *c + t : t;
    }
}

// Wave shapes by output shape (measured on MI355X, K = 2.45M rows):
//  - anything wide: 4 waves side by side along N, each with TM x 4 tiles
//    (TM = 4, 7 or 8, the fewest that cover M, so that a 100-wide layer does
//    not multiply a 128-wide tile column); 4 tiles along N reuse each A
//    operand 4 times from registers: 100x256 runs at ~110 TFLOP/s, against
//    ~50 with 8 waves of 7x2 tiles.  These waves hold ~340 registers (one
//    wave per SIMD); limiting them to 256 for two waves per SIMD measured
//    1.6-1.9x slower.  Six 4-row steps per buffer (24 rows in flight ahead
//    of the multiply) measured 1.14 ms against 1.23-1.32 with four; the
//    relu-gradient form, at 256 VGPRs, keeps four;
//  - N <= 16 (a class-width gradient): 4 waves along M with 4 x 1 tiles,
//    eight workgroups per CU for memory parallelism (~5 TB/s for 256x2);
//    M <= 16 the same along N.
enum class TnShape { Wide4, Wide7, Wide8, NarrowN, NarrowM };

struct TnPlan {
    TnShape shape;
    std::uint32_t step;  // rows per iteration (4*U)
    std::uint32_t BM, BN;
    std::uint32_t blocksM, blocksN;
    std::uint32_t splits, rowsPerSplit;
};

// Shape chosen from (M, N); block counts from (realM, realN) and the rows per
// iteration from `step` when given.
TnPlan tn_plan(std::uint32_t K, std::uint32_t M, std::uint32_t N, std::uint32_t realM = 0, std::uint32_t realN = 0,
               std::uint32_t step = 0, std::uint64_t splitCap = 0) {
    TnPlan p{};
    if (N <= 16) {
        p.shape = TnShape::NarrowN;  // TM=4, TN=1, WM=4, WN=1, U=8
        p.step = 32, p.BM = 256, p.BN = 16;
    } else if (M <= 16) {
        p.shape = TnShape::NarrowM;  // TM=1, TN=4, WM=1, WN=4, U=8
        p.step = 32, p.BM = 16, p.BN = 256;
    } else {
        // TM in {4, 7, 8}, TN=4, WM=1, WN=4, U=6 (U=4 for the relu-gradient form)
        p.shape = M <= 64 ? TnShape::Wide4 : M <= 112 ? TnShape::Wide7 : TnShape::Wide8;
        p.step = 24, p.BN = 256;
        p.BM = p.shape == TnShape::Wide4 ? 64 : p.shape == TnShape::Wide7 ? 112 : 128;
    }
    if (realM != 0) M = realM;
    if (realN != 0) N = realN;
    if (step != 0) p.step = step;
    p.blocksM = (M + p.BM - 1) / p.BM;
    p.blocksN = (N + p.BN - 1) / p.BN;
    const std::uint64_t blocks = static_cast<std::uint64_t>(p.blocksM) * p.blocksN;
    // About two (Wide*) or eight workgroups per compute unit in all.
    const bool narrow = p.shape == TnShape::NarrowN || p.shape == TnShape::NarrowM;
    const std::uint64_t target = static_cast<std::uint64_t>(device_cus()) * (narrow ? 8 : 2);
    const std::uint64_t maxSplits = std::max<std::uint64_t>(1, (K + p.step - 1) / p.step);
    std::uint64_t splits = std::min<std::uint64_t>(maxSplits, std::max<std::uint64_t>(1, (target + blocks - 1) / blocks));
    if (splitCap != 0) splits = std::min(splits, splitCap);
    std::uint64_t rps = (K + splits - 1) / splits;
    rps = std::max<std::uint64_t>(p.step, (rps + p.step - 1) / p.step * p.step);
    splits = std::max<std::uint64_t>(1, (K + rps - 1) / rps);
    p.splits = static_cast<std::uint32_t>(splits);
    p.rowsPerSplit = static_cast<std::uint32_t>(rps);
    return p;
}

// C = A^T B or, when N is the narrow side of a wide product (17..128 and
// below M), C^T = B^T A: the wide tiles lay 4 waves of 64 columns along N,
// so a narrow N would leave waves multiplying padding (602 x 64 ran at 10 ms
// as C, 2.5x torch.mm).
inline bool tn_swapped(std::uint32_t M, std::uint32_t N) { return M > 16 && N > 16 && N <= 128 && N < M; }

template <int TM, int TN, int WM, int WN, int U, int CT = 0, bool VB = false, bool VA = false>
void tn_launch(const TnArgs& a, const TnPlan& p, hipStream_t st) {
    hipLaunchKernelGGL((tn_partial_kernel<TM, TN, WM, WN, U, CT, VB, VA>), dim3(p.splits, p.blocksM * p.blocksN),
                       dim3(kWave * WM * WN), 0, st, a);
}

// The relu-gradient form always takes the wide shapes (N is the hidden width)
// with 16 rows per iteration (4 steps of 4; 8-class tiles take 2 x 4).
TnPlan relu_grad_plan(std::uint32_t K, std::uint32_t F, std::uint32_t Hd) {
    return tn_plan(K, std::max<std::uint32_t>(F, 17), std::max<std::uint32_t>(Hd, 17), F, Hd, 16);
}

}  // namespace
}  // namespace tcc

using namespace tcc;

extern "C" {

size_t tcc_dense_tn_workspace_bytes(std::uint32_t K, std::uint32_t M, std::uint32_t N) {
    if (K == 0 || M == 0 || N == 0) return 0;
    const TnPlan p = tn_swapped(M, N) ? tn_plan(K, N, M) : tn_plan(K, M, N);
    return static_cast<size_t>(p.splits) * M * N * sizeof(float);
}

}  // extern "C"

namespace tcc {
namespace {

// C = A^T B (or +=) with the partial products in `workspace`; splitCap
// bounds the split of K (0 = none) so that the partials fit a fixed buffer.
int dense_tn_impl(const float* A, std::uint32_t lda, const float* B, std::uint32_t ldb, float* C, std::uint32_t ldc,
                  std::uint32_t K, std::uint32_t M, std::uint32_t N, int accumulate, void* workspace,
                  size_t workspaceBytes, std::uint64_t splitCapBytes, hipStream_t st) {
    TCC_REQUIRE(C && M >= 1 && N >= 1 && lda >= M && ldb >= N && ldc >= N, TCC_ERR_INVALID_ARGUMENT,
                "invalid dense A^T B arguments");
    TCC_REQUIRE(lda < (1u << 28) && ldb < (1u << 28) && ldc < (1u << 28), TCC_ERR_UNSUPPORTED,
                "dense A^T B row strides must be below 2^28");
    if (K == 0) {
        if (accumulate) return TCC_OK;
        for (std::uint32_t m = 0; m < M; ++m)  // C rows may be strided: clear row by row
            TCC_HIP_CHECK(fill<float>(C + static_cast<std::uint64_t>(m) * ldc, N, 0.0f, st));
        return TCC_OK;
    }
    TCC_REQUIRE(A && B && workspace, TCC_ERR_INVALID_ARGUMENT, "invalid dense A^T B arguments");
    const bool swapped = tn_swapped(M, N);
    if (swapped) {  // C^T = B^T A
        std::swap(A, B);
        std::swap(lda, ldb);
        std::swap(M, N);
    }
    const std::uint64_t splitBytes = static_cast<std::uint64_t>(M) * N * sizeof(float);
    const TnPlan p = tn_plan(K, M, N, 0, 0, 0, splitCapBytes ? splitCapBytes / splitBytes : 0);
    TCC_REQUIRE(workspaceBytes >= static_cast<size_t>(p.splits) * M * N * sizeof(float), TCC_ERR_INVALID_ARGUMENT,
                "dense A^T B workspace too small (tcc_dense_tn_workspace_bytes)");
    TCC_REQUIRE(static_cast<std::uint64_t>(p.blocksM) * p.blocksN <= 65535, TCC_ERR_UNSUPPORTED,
                "dense A^T B output too large");
    TnArgs a{};
    a.A = A;
    a.B = B;
    a.partial = static_cast<float*>(workspace);
    a.lda = lda;
    a.ldb = ldb;
    a.K = K;
    a.M = M;
    a.N = N;
    a.rowsPerSplit = p.rowsPerSplit;
    a.blocksM = p.blocksM;
    // B rows as float4 feeding four interleaved N tiles (as the relu-gradient
    // form) when they allow 16-byte loads
    const bool vb = N % 4 == 0 && ldb % 4 == 0 && reinterpret_cast<std::uintptr_t>(B) % 16 == 0;
    // and A rows likewise feeding four interleaved M tiles
    const bool va = vb && M % 4 == 0 && lda % 4 == 0 && reinterpret_cast<std::uintptr_t>(A) % 16 == 0;
    switch (p.shape) {
        case TnShape::NarrowN: tn_launch<4, 1, 4, 1, 8>(a, p, st); break;
        case TnShape::NarrowM: tn_launch<1, 4, 1, 4, 8>(a, p, st); break;
        case TnShape::Wide4:
            if (va) tn_launch<4, 4, 1, 4, 6, 0, true, true>(a, p, st);
            else vb ? tn_launch<4, 4, 1, 4, 6, 0, true>(a, p, st) : tn_launch<4, 4, 1, 4, 6>(a, p, st);
            break;
        case TnShape::Wide7:
            if (va) tn_launch<7, 4, 1, 4, 6, 0, true, true>(a, p, st);
            else vb ? tn_launch<7, 4, 1, 4, 6, 0, true>(a, p, st) : tn_launch<7, 4, 1, 4, 6>(a, p, st);
            break;
        default:
            if (va) tn_launch<8, 4, 1, 4, 6, 0, true, true>(a, p, st);
            else vb ? tn_launch<8, 4, 1, 4, 6, 0, true>(a, p, st) : tn_launch<8, 4, 1, 4, 6>(a, p, st);
            break;
    }
    TCC_LAUNCH_CHECK();
    const std::uint64_t MN = static_cast<std::uint64_t>(M) * N;
    hipLaunchKernelGGL(tn_reduce_kernel, dim3(grid_for(MN, 16)), dim3(256), 0, st,
                       static_cast<const float*>(workspace), p.splits, M, N, C, ldc, accumulate, swapped ? 1 : 0);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

// Scratch of tcc_dense_tn_noalloc: the partial products, in device memory of
// the library's code object (one copy per GPU, held until the process ends).
constexpr std::size_t kTnScratchBytes = static_cast<std::size_t>(TCC_DENSE_TN_NOALLOC_SCRATCH_BYTES);
__device__ __align__(256) float tn_scratch[kTnScratchBytes / sizeof(float)];

// Device address of tn_scratch on the current device, looked up once per
// device (host code must not pass the symbol itself to a kernel: in host
// code it names a host-side stand-in).
int tn_scratch_address(float** out) {
    static std::mutex mu;
    static float* addr[64] = {};
    int dev = 0;
    TCC_HIP_CHECK(hipGetDevice(&dev));
    TCC_REQUIRE(dev >= 0 && dev < 64, TCC_ERR_UNSUPPORTED, "device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        void* p = nullptr;
        TCC_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(tn_scratch)));
        TCC_REQUIRE(p != nullptr, TCC_ERR_HIP, "no device address for the dense A^T B scratch");
        addr[dev] = static_cast<float*>(p);
    }
    *out = addr[dev];
    return TCC_OK;
}

}  // namespace
}  // namespace tcc

extern "C" {

int tcc_dense_tn(const float* A, std::uint32_t lda, const float* B, std::uint32_t ldb, float* C, std::uint32_t ldc,
                 std::uint32_t K, std::uint32_t M, std::uint32_t N, int accumulate, void* workspace,
                 size_t workspaceBytes, void* stream) {
    clear_last_error();
    return dense_tn_impl(A, lda, B, ldb, C, ldc, K, M, N, accumulate, workspace, workspaceBytes, 0,
                         as_stream(stream));
}

int tcc_dense_tn_noalloc(const float* A, std::uint32_t lda, const float* B, std::uint32_t ldb, float* C,
                         std::uint32_t ldc, std::uint32_t K, std::uint32_t M, std::uint32_t N, int accumulate,
                         void* stream) {
    clear_last_error();
    TCC_REQUIRE(static_cast<std::uint64_t>(M) * N * sizeof(float) <= kTnScratchBytes, TCC_ERR_UNSUPPORTED,
                "dense A^T B without allocation: M x N above the 16 MiB scratch (4M floats)");
    float* scratch = nullptr;
    if (K > 0) {
        const int rc = tn_scratch_address(&scratch);
        if (rc) return rc;
    }
    return dense_tn_impl(A, lda, B, ldb, C, ldc, K, M, N, accumulate, scratch, kTnScratchBytes, kTnScratchBytes,
                         as_stream(stream));
}

int tcc_gcn_relu_forward(const float* AX, std::uint32_t ldax, const float* W1, const float* W2, float* H,
                         std::uint32_t ldh, float* XW, std::uint32_t ldxw, std::uint32_t K, std::uint32_t F,
                         std::uint32_t Hd, std::uint32_t C, void* stream) {
    clear_last_error();
    TCC_REQUIRE(W1 && W2 && H && XW && F >= 1 && Hd >= 1 && C >= 1 && ldax >= F && ldh >= Hd && ldxw >= C,
                TCC_ERR_INVALID_ARGUMENT, "invalid GCN relu-forward arguments");
    TCC_REQUIRE(F <= 128 && Hd <= 256 && C <= 4, TCC_ERR_UNSUPPORTED,
                "GCN relu-forward supports F <= 128, hidden <= 256 and at most 4 classes");
    if (K == 0) return TCC_OK;
    TCC_REQUIRE(AX != nullptr, TCC_ERR_INVALID_ARGUMENT, "invalid GCN relu-forward arguments");
    ReluFwdArgs a{};
    a.AX = AX;
    a.W1 = W1;
    a.W2 = W2;
    a.H = H;
    a.XW = XW;
    a.ldax = ldax;
    a.ldh = ldh;
    a.ldxw = ldxw;
    a.K = K;
    a.F = F;
    a.Hd = Hd;
    a.C = C;
    a.tiles = (K + 15) / 16;
    a.vec = (ldax % 4 == 0) && (reinterpret_cast<std::uintptr_t>(AX) % 16 == 0);
    const hipStream_t st = as_stream(stream);
    const bool two = C <= 2;
    if (F <= 64) two ? relu_forward_launch<4, 2>(a, st) : relu_forward_launch<4, 4>(a, st);
    else if (F <= 112) two ? relu_forward_launch<7, 2>(a, st) : relu_forward_launch<7, 4>(a, st);
    else two ? relu_forward_launch<8, 2>(a, st) : relu_forward_launch<8, 4>(a, st);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

size_t tcc_gcn_relu_grad_workspace_bytes(std::uint32_t K, std::uint32_t F, std::uint32_t Hd, std::uint32_t C) {
    if (K == 0 || F == 0 || Hd == 0 || C == 0) return 0;
    const TnPlan p = relu_grad_plan(K, F, Hd);
    return static_cast<size_t>(p.splits) * (static_cast<size_t>(F) * Hd + static_cast<size_t>(Hd) * C) *
           sizeof(float);
}

int tcc_gcn_relu_grad(const float* AX, std::uint32_t ldax, const float* H, std::uint32_t ldh, const float* G,
                      std::uint32_t ldg, const float* W2, float* dW1, float* dW2, std::uint32_t K, std::uint32_t F,
                      std::uint32_t Hd, std::uint32_t C, void* workspace, size_t workspaceBytes, void* stream) {
    clear_last_error();
    TCC_REQUIRE(dW1 && dW2 && W2 && F >= 1 && Hd >= 1 && C >= 1 && ldax >= F && ldh >= Hd && ldg >= C,
                TCC_ERR_INVALID_ARGUMENT, "invalid GCN relu-gradient arguments");
    TCC_REQUIRE(C <= 8, TCC_ERR_UNSUPPORTED, "GCN relu-gradient supports at most 8 classes");
    TCC_REQUIRE(ldax < (1u << 28) && ldh < (1u << 28) && ldg < (1u << 28), TCC_ERR_UNSUPPORTED,
                "GCN relu-gradient row strides must be below 2^28");
    const hipStream_t st = as_stream(stream);
    if (K == 0) {
        TCC_HIP_CHECK(fill<float>(dW1, static_cast<std::uint64_t>(F) * Hd, 0.0f, st));
        TCC_HIP_CHECK(fill<float>(dW2, static_cast<std::uint64_t>(Hd) * C, 0.0f, st));
        return TCC_OK;
    }
    TCC_REQUIRE(AX && H && G && workspace, TCC_ERR_INVALID_ARGUMENT, "invalid GCN relu-gradient arguments");
    const TnPlan p = relu_grad_plan(K, F, Hd);
    const size_t need1 = static_cast<size_t>(p.splits) * F * Hd * sizeof(float);
    const size_t need2 = static_cast<size_t>(p.splits) * Hd * C * sizeof(float);
    TCC_REQUIRE(workspaceBytes >= need1 + need2, TCC_ERR_INVALID_ARGUMENT,
                "GCN relu-gradient workspace too small (tcc_gcn_relu_grad_workspace_bytes)");
    TCC_REQUIRE(static_cast<std::uint64_t>(p.blocksM) * p.blocksN <= 65535, TCC_ERR_UNSUPPORTED,
                "GCN relu-gradient output too large");
    TnArgs a{};
    a.A = AX;
    a.B = H;
    a.partial = static_cast<float*>(workspace);
    a.lda = ldax;
    a.ldb = ldh;
    a.K = K;
    a.M = F;
    a.N = Hd;
    a.rowsPerSplit = p.rowsPerSplit;
    a.blocksM = p.blocksM;
    a.G = G;
    a.W2 = W2;
    a.partial2 = reinterpret_cast<float*>(static_cast<char*>(workspace) + need1);
    a.ldg = ldg;
    a.C = C;
    // C <= 2: the wide tiles; up to 8 classes: 8 waves of TM x 2 tiles and 2
    // steps per iteration, to hold the G rows in registers (same blocks).
    const bool two = C <= 2;
    // H rows as float4 when they allow 16-byte loads (4 | Hd, 4 | ldh, H aligned)
    const bool vb = Hd % 4 == 0 && ldh % 4 == 0 && reinterpret_cast<std::uintptr_t>(H) % 16 == 0;
    const bool va = two && vb && F % 4 == 0 && ldax % 4 == 0 && reinterpret_cast<std::uintptr_t>(AX) % 16 == 0;
    switch (p.shape) {
        case TnShape::Wide4:
            if (va) tn_launch<4, 4, 1, 4, 4, 2, true, true>(a, p, st);
            else if (two && vb) tn_launch<4, 4, 1, 4, 4, 2, true>(a, p, st);
            else two ? tn_launch<4, 4, 1, 4, 4, 2>(a, p, st) : tn_launch<4, 2, 1, 8, 2, 8>(a, p, st);
            break;
        case TnShape::Wide7:
            if (va) tn_launch<7, 4, 1, 4, 4, 2, true, true>(a, p, st);
            else if (two && vb) tn_launch<7, 4, 1, 4, 4, 2, true>(a, p, st);
            else two ? tn_launch<7, 4, 1, 4, 4, 2>(a, p, st) : tn_launch<7, 2, 1, 8, 2, 8>(a, p, st);
            break;
        default:
            if (va) tn_launch<8, 4, 1, 4, 4, 2, true, true>(a, p, st);
            else if (two && vb) tn_launch<8, 4, 1, 4, 4, 2, true>(a, p, st);
            else two ? tn_launch<8, 4, 1, 4, 4, 2>(a, p, st) : tn_launch<8, 2, 1, 8, 2, 8>(a, p, st);
            break;
    }
    TCC_LAUNCH_CHECK();
    hipLaunchKernelGGL(tn_reduce_kernel, dim3(grid_for(static_cast<std::uint64_t>(F) * Hd, 16)), dim3(256), 0, st,
                       a.partial, p.splits, F, Hd, dW1, Hd, 0, 0);
    TCC_LAUNCH_CHECK();
    hipLaunchKernelGGL(tn_reduce_kernel, dim3(grid_for(static_cast<std::uint64_t>(Hd) * C, 16)), dim3(256), 0, st,
                       a.partial2, p.splits, Hd, C, dW2, C, 0, 0);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

}  // extern "C"
