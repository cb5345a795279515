// swtcf_spmm_run <dst_local.bin> <src_local.bin> [tc_threshold=12] [repeat=20]
//
// Converts a raw u32 COO to SWTCF (S = 16), fills X [cols x 128] with
// X[s][f] = a(s) + b(s)*f, times launchSWTCFSpMM, and checks Y against the
// closed form Y[d][f] = sum_{s in N(d)} a(s) + f * sum b(s) — the driver of
// src/swtcf_spmm_main.cu:116-280 over this library, with its tolerances
// (atol = rtol = 1e-2 while tiles take the TF32 path, 2e-4/1e-4 when
// tc > 64 keeps every tile in fp32).  Exit codes: 0 pass, 1 usage,
// 2 converter device error, 3 check failed.
#include <cmath>
#include <cstdlib>

#include "cli_common.hpp"

using namespace tcc_cli;

int run(int argc, char** argv) {
    if (argc < 3) {
        std::cerr << "usage:\n" << argv[0] << " <dst_local.bin> <src_local.bin> [tc_threshold=12] [repeat=20]\n";
        return 1;
    }
    const IndexType tc = argc > 3 ? static_cast<IndexType>(std::stoul(argv[3])) : SWTCF_DEFAULT_TC_THRESHOLD;
    const int repeat = argc > 4 ? std::stoi(argv[4]) : 20;
    constexpr IndexType S = 16;
    constexpr IndexType F = SWTCF_FEATURE_DIM;
    const auto dst = read_raw<IndexType>(argv[1]);
    const auto src = read_raw<IndexType>(argv[2]);
    if (dst.empty() || dst.size() != src.size()) throw std::runtime_error("invalid COO");
    const IndexType E = static_cast<IndexType>(dst.size());
    const IndexType numDst = *std::max_element(dst.begin(), dst.end()) + 1;
    const IndexType numSrc = *std::max_element(src.begin(), src.end()) + 1;
    std::cout << "rows / dst: " << numDst << '\n'
              << "cols / src: " << numSrc << '\n'
              << "edges: " << E << '\n'
              << "super window size: " << S << '\n'
              << "repeat cache size: " << SWTCF_REPEAT_CACHE_SIZE << '\n'
              << "TC threshold: " << tc << '\n';

    IndexType* dDst = to_device(dst);
    IndexType* dSrc = to_device(src);
    DeviceSWTCFMatrix m;
    SWTCFConvertWorkspace ws;
    allocateDeviceSWTCF(m, numDst, numSrc, E, S);
    allocateSWTCFConvertWorkspace(ws, E, numSrc, S);
    convertCOOToSWTCF(dDst, dSrc, E, m, ws);
    hip_check(hipDeviceSynchronize(), "conversion");
    const IndexType err = to_host(ws.deviceError, 1)[0];
    if (err != 0) {
        std::cerr << "converter error: " << err << '\n';
        return 2;
    }

    std::vector<ValueType> hx(std::size_t(numSrc) * F);
    for (IndexType s = 0; s < numSrc; ++s)
        for (IndexType f = 0; f < F; ++f) hx[std::size_t(s) * F + f] = feature_a(s) + feature_b(s) * float(f);
    ValueType* dX = to_device(hx);
    ValueType* dY = nullptr;
    const std::size_t ny = std::size_t(numDst) * F;
    hip_check(hipMalloc(reinterpret_cast<void**>(&dY), ny * sizeof(ValueType)), "hipMalloc");

    hip_check(hipMemset(dY, 0, ny * sizeof(ValueType)), "hipMemset");
    for (int i = 0; i < 5; ++i) launchSWTCFSpMM(m, dX, dY, tc);
    hip_check(hipDeviceSynchronize(), "warm-up");
    hip_check(hipMemset(dY, 0, ny * sizeof(ValueType)), "hipMemset");
    hipEvent_t t0, t1;
    hip_check(hipEventCreate(&t0), "hipEventCreate");
    hip_check(hipEventCreate(&t1), "hipEventCreate");
    hip_check(hipEventRecord(t0, 0), "hipEventRecord");
    for (int i = 0; i < repeat; ++i) launchSWTCFSpMM(m, dX, dY, tc);
    hip_check(hipEventRecord(t1, 0), "hipEventRecord");
    hip_check(hipEventSynchronize(t1), "hipEventSynchronize");
    float ms = 0.0f;
    hip_check(hipEventElapsedTime(&ms, t0, t1), "hipEventElapsedTime");
    ms /= static_cast<float>(std::max(repeat, 1));
    std::cout << "kernel time: " << ms << " ms\n"
              << "effective performance: " << 2.0 * double(E) * F / (double(ms) * 1.0e6) << " GFLOPS\n";

    // one clean launch for the check
    hip_check(hipMemset(dY, 0, ny * sizeof(ValueType)), "hipMemset");
    launchSWTCFSpMM(m, dX, dY, tc);
    hip_check(hipDeviceSynchronize(), "SpMM");
    const std::vector<ValueType> y = to_host(dY, ny);
    std::vector<double> sa(numDst, 0.0), sb(numDst, 0.0);
    for (std::size_t e = 0; e < dst.size(); ++e) {
        sa[dst[e]] += feature_a(src[e]);
        sb[dst[e]] += feature_b(src[e]);
    }
    const double atol = tc > 64 ? 2.0e-4 : 1.0e-2, rtol = tc > 64 ? 1.0e-4 : 1.0e-2;
    double maxAbs = 0.0, maxRel = 0.0, sumAbs = 0.0;
    std::uint64_t bad = 0;
    for (IndexType d = 0; d < numDst; ++d)
        for (IndexType f = 0; f < F; ++f) {
            const double want = sa[d] + sb[d] * f, got = y[std::size_t(d) * F + f];
            const double ae = std::fabs(got - want);
            maxAbs = std::max(maxAbs, ae);
            maxRel = std::max(maxRel, ae / std::max(std::fabs(want), 1.0e-8));
            sumAbs += ae;
            if (ae > atol + rtol * std::fabs(want)) ++bad;
        }
    std::cout << "max abs error: " << maxAbs << '\n'
              << "mean abs error: " << sumAbs / double(ny) << '\n'
              << "max relative error: " << maxRel << '\n'
              << "failed elements: " << bad << " / " << ny << '\n'
              << "tolerance: atol=" << atol << " rtol=" << rtol << '\n'
              << "SpMM validation: " << (bad == 0 ? "PASS" : "FAIL") << '\n';

    hip_check(hipEventDestroy(t0), "hipEventDestroy");
    hip_check(hipEventDestroy(t1), "hipEventDestroy");
    hip_check(hipFree(dX), "hipFree");
    hip_check(hipFree(dY), "hipFree");
    freeSWTCFConvertWorkspace(ws);
    freeDeviceSWTCF(m);
    hip_check(hipFree(dDst), "hipFree");
    hip_check(hipFree(dSrc), "hipFree");
    return bad == 0 ? 0 : 3;
}

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << '\n';
        return 4;
    }
}
