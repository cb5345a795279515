// swtcf_convert_run <dst_local.bin> <src_local.bin> [super_window_size=16] [repeat=20]
//
// Converts a raw u32 COO to SWTCF on the GPU, times the conversion, and
// checks the structure and the repeat cache — the driver of
// src/swtcf_convert_main.cu:314-546 over this library.  Exit codes: 0 both
// checks pass, 1 usage, 2 converter device error, 3 a check failed.
#include <chrono>
#include <cstdlib>

#include "cli_common.hpp"

using namespace tcc_cli;

int run(int argc, char** argv) {
    if (argc < 3) {
        std::cerr << "usage:\n"
                  << argv[0] << " <dst_local.bin> <src_local.bin> [super_window_size=16] [repeat=20]\n";
        return 1;
    }
    const IndexType S = argc > 3 ? static_cast<IndexType>(std::stoul(argv[3])) : 16;
    const int repeat = argc > 4 ? std::stoi(argv[4]) : 20;
    const auto dst = read_raw<IndexType>(argv[1]);
    const auto src = read_raw<IndexType>(argv[2]);
    if (dst.empty() || dst.size() != src.size()) throw std::runtime_error("invalid COO input");
    const IndexType E = static_cast<IndexType>(dst.size());
    const IndexType numDst = *std::max_element(dst.begin(), dst.end()) + 1;
    const IndexType numSrc = *std::max_element(src.begin(), src.end()) + 1;
    std::cout << "rows / dst: " << numDst << '\n'
              << "cols / src: " << numSrc << '\n'
              << "edges: " << E << '\n'
              << "super window size: " << S << '\n'
              << "repeat cache size: " << SWTCF_REPEAT_CACHE_SIZE << '\n';

    IndexType* dDst = to_device(dst);
    IndexType* dSrc = to_device(src);
    DeviceSWTCFMatrix m;
    SWTCFConvertWorkspace ws;
    allocateDeviceSWTCF(m, numDst, numSrc, E, S);
    allocateSWTCFConvertWorkspace(ws, E, numSrc, S);
    for (int i = 0; i < 5; ++i) convertCOOToSWTCF(dDst, dSrc, E, m, ws);
    hip_check(hipDeviceSynchronize(), "warm-up");
    hipEvent_t t0, t1;
    hip_check(hipEventCreate(&t0), "hipEventCreate");
    hip_check(hipEventCreate(&t1), "hipEventCreate");
    hip_check(hipEventRecord(t0, 0), "hipEventRecord");
    for (int i = 0; i < repeat; ++i) convertCOOToSWTCF(dDst, dSrc, E, m, ws);
    hip_check(hipEventRecord(t1, 0), "hipEventRecord");
    hip_check(hipEventSynchronize(t1), "hipEventSynchronize");
    float ms = 0.0f;
    hip_check(hipEventElapsedTime(&ms, t0, t1), "hipEventElapsedTime");
    ms /= static_cast<float>(std::max(repeat, 1));
    std::cout << "conversion time: " << ms << " ms\n"
              << "throughput: " << double(E) / ms / 1.0e6 << " GEdges/s\n";

    const IndexType err = to_host(ws.deviceError, 1)[0];
    const IndexType groups = to_host(ws.deviceNumGroups, 1)[0];
    if (err != 0) {
        std::cerr << "converter device error: " << err << '\n';
        return 2;
    }
    const HostSWTCF h = download(m);
    std::cout << "active window rows / groups: " << groups << '\n'
              << "col windows: " << m.numColWindows << '\n'
              << "super windows: " << m.numSuperWindows << '\n'
              << "tiles: " << h.colWindowOffset.back() << '\n'
              << "super-window unique rows: " << h.superWindowRowOffset.back() << '\n';
    const bool structure = check_structure(dst, src, numSrc, S, h);
    std::cout << "SWTCF validation: " << (structure ? "PASS" : "FAIL") << '\n';
    const bool cache = structure && check_repeat_cache(S, h);
    std::cout << "repeat-cache validation: " << (cache ? "PASS" : "FAIL") << '\n';

    hip_check(hipEventDestroy(t0), "hipEventDestroy");
    hip_check(hipEventDestroy(t1), "hipEventDestroy");
    freeSWTCFConvertWorkspace(ws);
    freeDeviceSWTCF(m);
    hip_check(hipFree(dDst), "hipFree");
    hip_check(hipFree(dSrc), "hipFree");
    return structure && cache ? 0 : 3;
}

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << '\n';
        return 4;
    }
}
