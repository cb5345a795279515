"""The reference's C++ API (include/tcc_swtcf.hpp over the C-ABI): a program
written against the reference's names compiles with g++, links
libtcc_swtcf.so and gets its defaults and host-side errors (thrown
std::runtime_error, as src/swtcf_convert.cu:1120-1130 throws) without a GPU."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "tcc_amd")

PROGRAM = r"""
#include "tcc_swtcf.hpp"
#include <cstdio>
#include <cstring>

static int expect_throw(const char* what, void (*fn)(), const char* needle) {
    try {
        fn();
    } catch (const std::runtime_error& e) {
        if (std::strstr(e.what(), needle) == nullptr) {
            std::printf("%s: message '%s' lacks '%s'\n", what, e.what(), needle);
            return 1;
        }
        return 0;
    }
    std::printf("%s: no exception\n", what);
    return 1;
}

int main() {
    int bad = 0;
    DeviceSWTCFMatrix m;
    SWTCFConvertWorkspace ws;
    if (m.colWindowWidth != 8 || m.tileRows != 8 || m.superWindowSize != 0 || m.tileLocalBit != nullptr) bad++;
    if (ws.edgeCapacity != 0 || ws.deviceError != nullptr) bad++;
    static_assert(SWTCF_FEATURE_DIM == 128 && SWTCF_DEFAULT_TC_THRESHOLD == 12, "constants");
    static_assert(SWTCF_REPEAT_CACHE_SIZE == 32 && SWTCF_MAX_SUPER_WINDOW_SIZE == 32, "constants");
    static_assert(sizeof(IndexType) == 4 && sizeof(BitmapType) == 8, "types");
    bad += expect_throw("cols == 0", [] { DeviceSWTCFMatrix a; allocateDeviceSWTCF(a, 4, 0, 4, 16); },
                        "invalid SWTCF allocation size");
    bad += expect_throw("S > 32", [] { DeviceSWTCFMatrix a; allocateDeviceSWTCF(a, 4, 8, 4, 33); },
                        "allocateDeviceSWTCF");
    bad += expect_throw("edges == 0", [] { SWTCFConvertWorkspace w; allocateSWTCFConvertWorkspace(w, 0, 8, 16); },
                        "allocateSWTCFConvertWorkspace");
    bad += expect_throw("S != 16", [] {
        DeviceSWTCFMatrix a;
        a.superWindowSize = 8;
        a.numSuperWindows = 1;
        launchSWTCFSpMM(a, reinterpret_cast<const float*>(16), reinterpret_cast<float*>(16));
    }, "superWindowSize=16");
    std::printf(bad ? "FAIL\n" : "OK\n");
    return bad;
}
"""


def test_cpp_api_compiles_links_and_throws(tmp_path):
    lib = os.path.join(PKG, "libtcc_swtcf.so")
    if not os.path.exists(lib):
        pytest.fail("build with python -m tcc_amd.build")
    src = tmp_path / "api.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "api"
    cmd = ["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__=1", f"-I{os.path.join(ROOT, 'include')}",
           "-I/opt/rocm/include", str(src), "-o", str(exe), f"-L{PKG}", "-ltcc_swtcf", f"-Wl,-rpath,{PKG}",
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "OK" in r.stdout, r.stdout + r.stderr
