// Plans for repeated SWTCF SpMMs over one matrix (no reference counterpart;
// the product is launchSWTCFSpMM's, src/swtcf_spmm.cu:437-466).
//
// The SWTCF SpMM adds every tile row's partial sums into Y with atomics: at
// 233k rows and 114M edges (F = 128) that is 815.9M 64-byte atomic requests,
// at 0.86 of the rate a probe reaches, 46.6 ms.  A caller that multiplies
// by the same matrix again and again (the reference's own timing loop,
// src/swtcf_spmm_main.cu:203-247; a training loop) can be served by the
// binary hybrid of the same pattern instead (hub_tiles.hip: degree-ordered
// binary tiles on the sparse MFMA plus a gather of the rest), which writes
// each output row once per phase.
//
// A sparser or smaller matrix is served by the BCSR gather of its pattern
// (bcsr_spmm.hip), which also writes each output row once: on a 169k-row,
// 1.17M-edge R-MAT graph at F = 128 the kernel takes 0.61 ms, the plan
// 0.12 ms (the gather 0.09 ms, the rest the hash and the wait for it).
//
// Every call of tcc_swtcf_spmm / tcc_swtcf_spmm_f on a matrix of at least
// kGatherPlanMinEdges edges of capacity hashes the arrays that define the
// product (colWindowOffset, superWindowRowOffset, tileLocalBit, tileRowSlot,
// superWindowRows at their valid extents; two order-independent sums of
// mixed words) on the device and reads the hash back.  The second call
// that finds the same hash and dimensions decodes the matrix into a COO,
// builds the plan and keeps it; that call and the later ones run the plan:
// the hybrid for at least kPlanMinEdges edges and 64 entries per row on
// average, else the gather (over X packed to TF32 rows where rows are
// gathered 16 times or more).  A matrix changed in place hashes differently
// and is multiplied afresh.  Plans need tcThreshold <= 64: they multiply
// TF32(X) everywhere, where the reference uses X as given for tiles below
// the threshold (tcThreshold > 64 asks for the fp32 path throughout).
#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "../../include/tcc_spmm_cnic.h"
#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "gather_ops.hpp"
#include "primitives.hpp"
#include "swtcf_plan.hpp"

namespace tcc {
namespace {

constexpr unsigned kThreads = 256;
constexpr std::uint64_t kGatherPlanMinEdges = 1u << 18;  // any plan
constexpr std::uint64_t kPlanMinEdges = 4u << 20;         // the hybrid (with the degree)
constexpr std::uint32_t kPlanMinRowDegree = 64;
// Gathers per source row (8 per block column) from which X is packed.
constexpr std::uint64_t kPlanPackMinGathers = 16;
constexpr unsigned kHashBlocks = 2048;
// The blocks add their sums into kHashSlots pairs of words (block b into
// pair b % kHashSlots), which the host adds up: 2048 atomics on one address
// are performed one after another past the L2 (about 45 us).
constexpr unsigned kHashSlots = TCC_HASH_WORDS / 2;
constexpr unsigned kHashWords = 2 * kHashSlots + 2;

// MurmurHash3's 32-bit finalizer (Appleby): a bijective mix of 32 bits
__device__ __forceinline__ std::uint32_t fmix32(std::uint32_t h) {
    h ^= h >> 16;
    h *= 0x85EBCA6Bu;
    h ^= h >> 13;
    h *= 0xC2B2AE35u;
    h ^= h >> 16;
    return h;
}

// Word j of array `salt`, mixed two ways into the two sums.
__device__ __forceinline__ void hash_word(std::uint32_t w, std::uint64_t j, std::uint32_t salt, std::uint64_t& s0,
                                          std::uint64_t& s1) {
    const std::uint32_t k = static_cast<std::uint32_t>(j) ^ (static_cast<std::uint32_t>(j >> 32) * 0x27D4EB2Fu);
    const std::uint32_t a = fmix32(w + k * 0x9E3779B9u + salt);
    s0 += a;
    s1 += fmix32(a ^ (k + 0x5BD1E995u * salt));
}

// The words of one array, 16 bytes a thread when the array is 16-byte
// aligned (as tcc_swtcf_alloc_matrix carves them), else one word a thread.
__device__ __forceinline__ void hash_array(const std::uint32_t* p, std::uint64_t words, std::uint32_t salt,
                                           std::uint64_t& s0, std::uint64_t& s1) {
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    const std::uint64_t quads = (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0 ? words / 4 : 0;
    for (std::uint64_t q = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < quads; q += stride) {
        const vu4 v = load_global<vu4>(p + 4 * q);
        hash_word(v.x, 4 * q, salt, s0, s1);
        hash_word(v.y, 4 * q + 1, salt, s0, s1);
        hash_word(v.z, 4 * q + 2, salt, s0, s1);
        hash_word(v.w, 4 * q + 3, salt, s0, s1);
    }
    for (std::uint64_t j = 4 * quads + static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < words;
         j += stride)
        hash_word(p[j], j, salt, s0, s1);
}

// out[2k], out[2k + 1] (k < kHashSlots): two sums of mixed (array, index,
// word) over the arrays that define the product, slot k's share of them;
// out[2 kHashSlots] = tiles, out[2 kHashSlots + 1] = super-window rows.
// The sums over the slots do not depend on the order in which the threads
// add them.
__global__ void __launch_bounds__(kThreads) swtcf_hash_kernel(tcc_swtcf_matrix m, std::uint64_t* __restrict__ out) {
    const std::uint64_t T = m.colWindowOffset[m.numColWindows], U = m.superWindowRowOffset[m.numSuperWindows];
    std::uint64_t s0 = 0, s1 = 0;
    hash_array(m.colWindowOffset, m.numColWindows + 1ull, 1, s0, s1);
    hash_array(m.superWindowRowOffset, m.numSuperWindows + 1ull, 2, s0, s1);
    hash_array(reinterpret_cast<const std::uint32_t*>(m.tileLocalBit), 2 * T, 3, s0, s1);
    hash_array(m.tileRowSlot, 8 * T, 4, s0, s1);
    hash_array(m.superWindowRows, U, 5, s0, s1);
    __shared__ std::uint64_t r0[kThreads / kWave], r1[kThreads / kWave];
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        s0 += __shfl_xor(s0, d, kWave);
        s1 += __shfl_xor(s1, d, kWave);
    }
    if (__lane_id() == 0) {
        r0[threadIdx.x / kWave] = s0;
        r1[threadIdx.x / kWave] = s1;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (unsigned w = 1; w < kThreads / kWave; ++w) {
            s0 += r0[w];
            s1 += r1[w];
        }
        std::uint64_t* slot = out + 2 * (blockIdx.x % kHashSlots);
        atomicAdd(reinterpret_cast<unsigned long long*>(&slot[0]), static_cast<unsigned long long>(s0));
        atomicAdd(reinterpret_cast<unsigned long long*>(&slot[1]), static_cast<unsigned long long>(s1));
        if (blockIdx.x == 0) {
            out[2 * kHashSlots] = T;
            out[2 * kHashSlots + 1] = U;
        }
    }
}

// Up to kMaxSpans device arrays of 32-bit words, hashed as hash_array does.
constexpr unsigned kMaxSpans = 8;
struct HashSpans {
    const std::uint32_t* p[kMaxSpans];
    std::uint64_t words[kMaxSpans];
    std::uint32_t n;
};

// out[2k], out[2k + 1] (k < kHashSlots): slot k's share of the two sums.
__global__ void __launch_bounds__(kThreads) hash_spans_kernel(HashSpans s, std::uint64_t* __restrict__ out) {
    std::uint64_t s0 = 0, s1 = 0;
    for (std::uint32_t k = 0; k < s.n; ++k) hash_array(s.p[k], s.words[k], k + 1, s0, s1);
    __shared__ std::uint64_t r0[kThreads / kWave], r1[kThreads / kWave];
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        s0 += __shfl_xor(s0, d, kWave);
        s1 += __shfl_xor(s1, d, kWave);
    }
    if (__lane_id() == 0) {
        r0[threadIdx.x / kWave] = s0;
        r1[threadIdx.x / kWave] = s1;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (unsigned w = 1; w < kThreads / kWave; ++w) {
            s0 += r0[w];
            s1 += r1[w];
        }
        std::uint64_t* slot = out + 2 * (blockIdx.x % kHashSlots);
        atomicAdd(reinterpret_cast<unsigned long long*>(&slot[0]), static_cast<unsigned long long>(s0));
        atomicAdd(reinterpret_cast<unsigned long long*>(&slot[1]), static_cast<unsigned long long>(s1));
    }
}

__global__ void swtcf_tile_counts_kernel(const std::uint64_t* __restrict__ bits, std::uint32_t T,
                                         std::uint32_t* __restrict__ counts) {
    const std::uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < T) counts[t] = static_cast<std::uint32_t>(__popcll(bits[t]));
}

// The COO of the matrix: tile t of column window w (the last w with
// colWindowOffset[w] <= t) holds bit 8r + c for the edge (row
// superWindowRows[superWindowRowOffset[w / S] + tileRowSlot[8t + r]],
// column 8w + c).  Bits of padding rows or past the matrix (a converted
// matrix has none) are counted in `dropped`; the matrix then gets no plan.
__global__ void swtcf_decode_kernel(tcc_swtcf_matrix m, std::uint32_t T, const std::uint32_t* __restrict__ offset,
                                    std::uint32_t* __restrict__ dst, std::uint32_t* __restrict__ src,
                                    std::uint32_t* __restrict__ dropped) {
    const std::uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    std::uint32_t lo = 0, hi = m.numColWindows;  // colWindowOffset[lo] <= t < colWindowOffset[hi]
    while (hi - lo > 1) {
        const std::uint32_t mid = lo + (hi - lo) / 2;
        if (m.colWindowOffset[mid] <= t) lo = mid;
        else hi = mid;
    }
    const std::uint32_t w = lo, base = m.superWindowRowOffset[w / m.superWindowSize];
    const std::uint32_t rowsU = m.superWindowRowOffset[m.numSuperWindows];
    std::uint64_t b = m.tileLocalBit[t];
    std::uint32_t k = offset[t], bad = 0;
    while (b) {
        const unsigned i = static_cast<unsigned>(__builtin_ctzll(b));
        b &= b - 1;
        const std::uint32_t slot = m.tileRowSlot[8ull * t + i / 8];
        const std::uint32_t col = 8 * w + i % 8;
        const std::uint32_t row = slot < rowsU - base ? m.superWindowRows[base + slot] : 0xFFFFFFFFu;
        if (row < m.rows && col < m.cols) {
            dst[k] = row;
            src[k] = col;
        } else {
            dst[k] = 0;
            src[k] = 0;
            ++bad;
        }
        ++k;
    }
    if (bad) atomicAdd(dropped, bad);
}

// X[src][f] = q[srcGlobal[src] * F + f] * scales[srcGlobal[src]]
// (src/swtcf_spmm.cu:317-323), four features a thread.
__global__ void dequantize_kernel(const std::int8_t* __restrict__ q, const float* __restrict__ scales,
                                  const std::uint32_t* __restrict__ srcGlobal, std::uint32_t cols, std::uint32_t F,
                                  float* __restrict__ X) {
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::uint32_t quads = F / 4;
    if (i >= static_cast<std::uint64_t>(cols) * quads) return;
    const std::uint32_t src = static_cast<std::uint32_t>(i / quads), f = 4 * static_cast<std::uint32_t>(i % quads);
    const std::uint32_t g = srcGlobal[src];
    const float sc = scales[g];
    const std::int8_t* r = q + static_cast<std::uint64_t>(g) * F + f;
    *reinterpret_cast<vf4*>(X + static_cast<std::uint64_t>(src) * F + f) =
        vf4{r[0] * sc, r[1] * sc, r[2] * sc, r[3] * sc};
}

struct Plan {
    int device = -1;
    std::uint32_t rows = 0, cols = 0, S = 0, CW = 0, SW = 0;
    std::uint64_t h0 = 0, h1 = 0, T = 0, U = 0;
    std::uint64_t lastUse = 0;
    bool built = false;
    bool unplannable = false;  // bits outside the rows or columns: always the SWTCF kernel
    bool hybrid = false;       // the binary hybrid, else the BCSR gather
    tcc_hybrid H{};
    tcc_bcsr B{};
    void* bAlloc = nullptr;    // B's arrays (tcc_block_release)
    bool packs = false;        // the gather reads X packed to TF32 rows (in ws)
    void* ws = nullptr;        // the hybrid's workspace or the packed X
    std::size_t wsBytes = 0;
    std::uint32_t wsF = 0;
    float* xq = nullptr;  // the dequantized X of the int8 entry point ([cols x 128])

    void release() {
        if (built && hybrid) tcc_hybrid_release(&H);
        if (bAlloc) (void)tcc_block_release(bAlloc);
        if (ws) (void)hipFree(ws);
        if (xq) (void)hipFree(xq);
        built = false;
        bAlloc = nullptr;
        ws = nullptr;
        wsBytes = 0;
        wsF = 0;
        xq = nullptr;
    }
};

struct PlanCache {
    std::mutex mu;
    bool init = false;
    std::uint32_t maxPlans = 1;
    std::uint64_t clock = 0;
    std::uint32_t builtCount = 0;
    std::vector<Plan> plans;                 // seen matrices, built or not
    struct HashBuf {
        int device;
        std::uint64_t* dev;   // kHashWords u64 on the device
        std::uint64_t* host;  // their pinned host copy
    };
    std::vector<HashBuf> hashBuf;

    void configure() {
        if (init) return;
        init = true;
        if (const char* e = std::getenv("TCC_SWTCF_PLANS")) maxPlans = static_cast<std::uint32_t>(std::strtoul(e, nullptr, 10));
    }
    const HashBuf* buffer(int device) {
        for (auto& b : hashBuf)
            if (b.device == device) return &b;
        HashBuf b{device, nullptr, nullptr};
        if (hipMalloc(&b.dev, kHashWords * sizeof(std::uint64_t)) != hipSuccess) return nullptr;
        if (hipHostMalloc(&b.host, kHashWords * sizeof(std::uint64_t), hipHostMallocDefault) != hipSuccess) {
            (void)hipFree(b.dev);
            return nullptr;
        }
        hashBuf.push_back(b);
        return &hashBuf.back();
    }
    // keep at most maxPlans built plans and 2 maxPlans + 2 entries, dropping the least recently used
    void trim() {
        auto lru = [&](bool builtOnly) {
            std::size_t best = plans.size();
            for (std::size_t i = 0; i < plans.size(); ++i)
                if ((!builtOnly || plans[i].built) && (best == plans.size() || plans[i].lastUse < plans[best].lastUse))
                    best = i;
            return best;
        };
        for (;;) {
            std::uint32_t built = 0;
            for (auto& p : plans) built += p.built ? 1 : 0;
            if (built <= maxPlans) break;
            const std::size_t i = lru(true);
            plans[i].release();
        }
        while (plans.size() > 2ull * maxPlans + 2) {
            const std::size_t i = lru(false);
            plans[i].release();
            plans.erase(plans.begin() + static_cast<std::ptrdiff_t>(i));
        }
    }
};

PlanCache& cache() {
    static PlanCache c;
    return c;
}

// The hybrid of the matrix's pattern (binary tiles, no scales), or the BCSR
// of its pattern.  Two column phases for the hybrid's remainder: a phased
// remainder adds only the rows it touches, so Y needs no rows past m.rows
// (the gather takes a row limit instead).  A matrix with bits outside its
// rows or columns (the SWTCF kernel skips them) is marked unplannable.
int build_plan(const tcc_swtcf_matrix* m, Plan& P, hipStream_t st) {
    const std::uint32_t T = static_cast<std::uint32_t>(P.T);
    struct Bufs {
        void* p = nullptr;
        ~Bufs() {
            if (p) (void)hipFree(p);
        }
    } scratch;
    const std::uint64_t Tn = std::max<std::uint64_t>(T, 1);
    const std::size_t a = (4 * (Tn + 1) + 255) / 256 * 256;
    const std::size_t tempBytes = (4 * scan_temp_elems(Tn + 1) + 255) / 256 * 256;
    TCC_HIP_CHECK(hipMalloc(&scratch.p, 2 * a + tempBytes + 256));
    auto* counts = static_cast<std::uint32_t*>(scratch.p);
    auto* offset = reinterpret_cast<std::uint32_t*>(static_cast<char*>(scratch.p) + a);
    auto* temp = reinterpret_cast<std::uint32_t*>(static_cast<char*>(scratch.p) + 2 * a);
    auto* small = reinterpret_cast<std::uint32_t*>(static_cast<char*>(scratch.p) + 2 * a + tempBytes);
    TCC_HIP_CHECK(fill<std::uint32_t>(small, 4, 0u, st));
    if (T > 0) {
        hipLaunchKernelGGL(swtcf_tile_counts_kernel, dim3(grid_for(T, kThreads)), dim3(kThreads), 0, st, m->tileLocalBit,
                           T, counts);
        TCC_LAUNCH_CHECK();
    }
    TCC_HIP_CHECK(exclusive_scan(counts, offset, T, small, temp, st));
    std::uint32_t nnz = 0;
    TCC_HIP_CHECK(hipMemcpyAsync(&nnz, small, 4, hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    Bufs coo;
    const std::uint64_t En = std::max<std::uint32_t>(nnz, 1);
    TCC_HIP_CHECK(hipMalloc(&coo.p, 8 * En));
    auto* dst = static_cast<std::uint32_t*>(coo.p);
    auto* src = dst + En;
    if (T > 0) {
        hipLaunchKernelGGL(swtcf_decode_kernel, dim3(grid_for(T, kThreads)), dim3(kThreads), 0, st, *m, T, offset, dst,
                           src, small + 1);
        TCC_LAUNCH_CHECK();
    }
    std::uint32_t dropped = 0;
    TCC_HIP_CHECK(hipMemcpyAsync(&dropped, small + 1, 4, hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    if (dropped) {
        P.unplannable = true;
        return TCC_OK;
    }
    if (P.hybrid) {
        const int rc =
            tcc_coo_to_hybrid_scaled(dst, src, nnz, m->rows, m->cols, nullptr, nullptr, 0, 0, 0, 2, &P.H, st);
        if (rc) return rc;
    } else {
        const int rc = tcc_coo_to_bcsr(dst, src, nullptr, nnz, m->rows, m->cols, &P.B, &P.bAlloc, st);
        if (rc) return rc;
        P.packs = 8ull * P.B.num_TCBlocks >= kPlanPackMinGathers * m->cols;
    }
    P.built = true;
    return TCC_OK;
}

}  // namespace

int swtcf_plan_spmm(const tcc_swtcf_matrix* m, const float* X, float* Y, std::uint32_t F, std::uint32_t tc,
                    void* stream, bool* used, const SwtcfQuantX* quant) {
    *used = false;
    PlanCache& C = cache();
    std::lock_guard<std::mutex> lock(C.mu);
    C.configure();
    if (C.maxPlans == 0 || tc > 64 || m->nnz < kGatherPlanMinEdges || m->rows == 0) return TCC_OK;
    const bool hybrid = m->nnz >= kPlanMinEdges &&
                        static_cast<std::uint64_t>(m->nnz) >= static_cast<std::uint64_t>(kPlanMinRowDegree) * m->rows;
    const hipStream_t st = as_stream(stream);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return TCC_OK;
    int device = 0;
    TCC_HIP_CHECK(hipGetDevice(&device));
    const PlanCache::HashBuf* hb = C.buffer(device);
    TCC_REQUIRE(hb, TCC_ERR_NO_MEMORY, "out of memory for the SWTCF plan hash");
    TCC_HIP_CHECK(fill<std::uint64_t>(hb->dev, kHashWords, 0ull, st));
    hipLaunchKernelGGL(swtcf_hash_kernel, dim3(kHashBlocks), dim3(kThreads), 0, st, *m, hb->dev);
    TCC_LAUNCH_CHECK();
    TCC_HIP_CHECK(hipMemcpyAsync(hb->host, hb->dev, kHashWords * sizeof(std::uint64_t), hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    std::uint64_t h[4] = {0, 0, hb->host[2 * kHashSlots], hb->host[2 * kHashSlots + 1]};
    for (unsigned k = 0; k < kHashSlots; ++k) {
        h[0] += hb->host[2 * k];
        h[1] += hb->host[2 * k + 1];
    }
    Plan* P = nullptr;
    for (auto& p : C.plans)
        if (p.device == device && p.rows == m->rows && p.cols == m->cols && p.S == m->superWindowSize &&
            p.CW == m->numColWindows && p.SW == m->numSuperWindows && p.h0 == h[0] && p.h1 == h[1] && p.T == h[2] &&
            p.U == h[3])
            P = &p;
    ++C.clock;
    if (!P) {
        // first sighting: remember it, multiply with the SWTCF kernel
        Plan q;
        q.device = device;
        q.rows = m->rows;
        q.cols = m->cols;
        q.S = m->superWindowSize;
        q.CW = m->numColWindows;
        q.SW = m->numSuperWindows;
        q.h0 = h[0];
        q.h1 = h[1];
        q.T = h[2];
        q.U = h[3];
        q.hybrid = hybrid;
        q.lastUse = C.clock;
        C.plans.push_back(q);
        C.trim();
        return TCC_OK;
    }
    P->lastUse = C.clock;
    if (P->unplannable) return TCC_OK;
    if (!P->built) {
        // a plan that cannot be built (device memory, an odd matrix) leaves
        // the product to the SWTCF kernel, now and on later calls
        if (build_plan(m, *P, st) != TCC_OK || !P->built) {
            P->release();
            P->unplannable = true;
            clear_last_error();
            (void)hipGetLastError();
            return TCC_OK;
        }
        ++C.builtCount;
    }
    if (P->wsF != F) {
        if (P->ws) (void)hipFree(P->ws);
        P->ws = nullptr;
        P->wsF = 0;
        P->wsBytes = P->hybrid ? tcc_hybrid_workspace_bytes(&P->H, F) + 16
                               : (P->packs ? tcc_tf32_packed_bytes(m->cols, F) + 16 : 0);
        if (P->wsBytes && hipMalloc(&P->ws, P->wsBytes) != hipSuccess) {  // no room for this F: the kernel
            P->ws = nullptr;
            P->wsBytes = 0;
            (void)hipGetLastError();
            return TCC_OK;
        }
        P->wsF = F;
    }
    if (quant) {
        if (!P->xq && hipMalloc(&P->xq, 4ull * m->cols * F) != hipSuccess) {
            P->xq = nullptr;
            (void)hipGetLastError();
            return TCC_OK;
        }
        const std::uint64_t n = static_cast<std::uint64_t>(m->cols) * (F / 4);
        hipLaunchKernelGGL(dequantize_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, st, quant->q,
                           quant->scales, quant->srcGlobal, m->cols, F, P->xq);
        TCC_LAUNCH_CHECK();
        X = P->xq;
    }
    int rc;
    if (P->hybrid) {
        rc = tcc_hybrid_spmm(&P->H, X, Y, F, 1, P->ws, P->wsBytes, stream);
    } else {
        // Y holds m.rows rows: a last window cut short takes the row limit
        const std::uint32_t limit = m->rows % 8 ? m->rows : 0;
        if (P->packs) {
            rc = tf32_pack_scaled(X, m->cols, F, nullptr, P->ws, st);
            if (rc == TCC_OK) rc = bcsr_spmm_packed_scaled(&P->B, P->ws, Y, F, 1, nullptr, st, limit);
        } else {
            rc = bcsr_spmm_scaled(&P->B, X, Y, F, 1, nullptr, st, limit);
        }
    }
    if (rc) return rc;
    *used = true;
    C.trim();  // after the last use of P: trimming may move the entries
    return TCC_OK;
}

}  // namespace tcc

using namespace tcc;

extern "C" {

int tcc_swtcf_set_plans(std::uint32_t maxPlans) {
    clear_last_error();
    PlanCache& C = cache();
    std::lock_guard<std::mutex> lock(C.mu);
    C.init = true;
    C.maxPlans = maxPlans;
    C.trim();
    return TCC_OK;
}

int tcc_swtcf_release_plans(void) {
    clear_last_error();
    PlanCache& C = cache();
    std::lock_guard<std::mutex> lock(C.mu);
    for (auto& p : C.plans) p.release();
    C.plans.clear();
    return TCC_OK;
}

int tcc_hash_arrays(const void* const* arrays, const std::uint64_t* bytes, std::uint32_t count,
                    std::uint64_t* deviceOut, void* stream) {
    clear_last_error();
    TCC_REQUIRE(deviceOut && count <= kMaxSpans && (count == 0 || (arrays && bytes)), TCC_ERR_INVALID_ARGUMENT,
                "tcc_hash_arrays: at most 8 arrays and an output");
    HashSpans s{};
    s.n = count;
    for (std::uint32_t k = 0; k < count; ++k) {
        TCC_REQUIRE(bytes[k] % 4 == 0 && (bytes[k] == 0 || arrays[k]), TCC_ERR_INVALID_ARGUMENT,
                    "tcc_hash_arrays: arrays of whole 32-bit words");
        s.p[k] = static_cast<const std::uint32_t*>(arrays[k]);
        s.words[k] = bytes[k] / 4;
    }
    const hipStream_t st = as_stream(stream);
    TCC_HIP_CHECK(fill<std::uint64_t>(deviceOut, 2 * kHashSlots, 0ull, st));
    hipLaunchKernelGGL(hash_spans_kernel, dim3(kHashBlocks), dim3(kThreads), 0, st, s, deviceOut);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

uint32_t tcc_swtcf_plans_built(void) {
    PlanCache& C = cache();
    std::lock_guard<std::mutex> lock(C.mu);
    return C.builtCount;
}

}  // extern "C"
