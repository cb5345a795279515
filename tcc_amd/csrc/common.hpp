// Shared helpers for the gfx950 kernels of libtcc_swtcf.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace tcc {

// ---------------------------------------------------------------- errors
void set_last_error(const std::string& msg);
void clear_last_error();

// Returns TCC_ERR_HIP (2) from the enclosing C-ABI function on failure.
#define TCC_HIP_CHECK(call)                                                              \
    do {                                                                                 \
        const hipError_t tcc_err__ = (call);                                             \
        if (tcc_err__ != hipSuccess) {                                                   \
            ::tcc::set_last_error(std::string("HIP error: ") + hipGetErrorString(tcc_err__) + \
                                  " at " + __FILE__ + ":" + std::to_string(__LINE__));   \
            return 2;                                                                    \
        }                                                                                \
    } while (0)

#define TCC_REQUIRE(cond, code, msg)        \
    do {                                    \
        if (!(cond)) {                      \
            ::tcc::set_last_error(msg);     \
            return (code);                  \
        }                                   \
    } while (0)

#define TCC_LAUNCH_CHECK() TCC_HIP_CHECK(hipGetLastError())

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kWave = 64;

inline unsigned grid_for(std::uint64_t n, unsigned threads) {
    return static_cast<unsigned>((n + threads - 1) / threads);
}

// Compute units of the current device (cached per device).
inline std::uint32_t device_cus() {
    static std::uint32_t cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = static_cast<std::uint32_t>(n);
    }
    return cache[dev];
}

// ---------------------------------------------------------------- numerics
// cvt.rna.tf32.f32 restated from its definition: round to nearest with ties
// away from zero, keeping 10 explicit mantissa bits; inf and NaN unchanged.
// (Reference use: include/mma_tf32.cuh:17-22.)  The add-and-mask maps +-inf
// to themselves and carries the largest finite values into inf, as rounding
// does, so only NaN (whose payload could carry into the sign) is passed
// through: 4 instructions.
__device__ __forceinline__ float tf32_rna(float x) {
    const std::uint32_t b = __float_as_uint(x);
    const std::uint32_t r = __builtin_isnan(x) ? b : ((b + 0x1000u) & 0xFFFFE000u);
    return __uint_as_float(r);
}

// ---------------------------------------------------------------- loads
// A load through a global-address-space pointer.  Row pointers rebuilt from
// integers (v_readlane of a pointer table) are generic to the compiler and
// would become flat loads, which also count against the LDS/scalar wait
// counter, so every wait for a scalar load would wait for them too.
// T is a scalar or a clang vector type (vf2, vf4, vu2, vu4).
using vf2 = float __attribute__((ext_vector_type(2)));
using vf4 = float __attribute__((ext_vector_type(4)));
using vu2 = std::uint32_t __attribute__((ext_vector_type(2)));
using vu4 = std::uint32_t __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ T load_global(const void* p) {
    // through an integer: a direct cast of a generic pointer stays flat
    return *(const __attribute__((address_space(1))) T*)(reinterpret_cast<std::uintptr_t>(p));
}

// ---------------------------------------------------------------- wave64
__device__ __forceinline__ unsigned lane_id() { return __lane_id(); }

__device__ __forceinline__ std::uint64_t lanemask_lt() {
    const unsigned l = __lane_id();
    return (l == 0) ? 0ull : ((~0ull) >> (64 - l));
}

// Lanes of the wave (among `active`) whose `key` (nbits wide) equals this
// lane's key.  Used for stable wave-level multisplit ranks.
template <int NBITS>
__device__ __forceinline__ std::uint64_t match_peers(unsigned key, bool active) {
    std::uint64_t peers = __ballot(active);
#pragma unroll
    for (int b = 0; b < NBITS; ++b) {
        const bool bit = (key >> b) & 1u;
        const std::uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return active ? peers : 0ull;
}

// counter[idx] += 1 for every calling lane, one atomic per distinct index
// in the wave: sorted inputs put many lanes of a wave on the same few
// counters, where per-lane atomics serialise.
__device__ __forceinline__ void aggregated_increment(std::uint32_t* counter, std::uint32_t idx) {
    std::uint64_t todo = __ballot(true);
    while (todo) {
        const int leader = __builtin_ctzll(todo);
        const std::uint32_t lidx =
            static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(idx), leader));
        const std::uint64_t same = __ballot(idx == lidx) & todo;
        if (static_cast<int>(__lane_id()) == leader) atomicAdd(&counter[lidx], static_cast<std::uint32_t>(__popcll(same)));
        todo &= ~same;
    }
}

// fp32 atomic add to global memory (hardware global_atomic_add_f32; the
// library is compiled with -munsafe-fp-atomics for coarse-grained memory).
__device__ __forceinline__ void atomic_add_f32(float* p, float v) { unsafeAtomicAdd(p, v); }

}  // namespace tcc
