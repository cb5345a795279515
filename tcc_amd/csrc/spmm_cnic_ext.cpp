// `spmm_cnic` PyTorch extension for ROCm: the drop-in for the reference's
// pybind module (spmm_cnic/src/bindings/module.cu:344-365).  A thin C++ layer
// that turns tensors and capsules into raw pointers and calls the C-ABI of
// libtcc_swtcf.so on torch's current HIP stream; all compute is in the HIP
// kernels.
//
// Both call forms are exported as pybind11 overloads:
//  * the compiled form (module.cu:100-108, 192-197): explicit device_id and a
//    caller-provided denseC capsule (from space_malloc); the result is a
//    tensor view of denseC with no deleter, like torch::from_blob there;
//  * the form the training scripts call (train/tcgnn_conv_release.py:116-130):
//    no device_id/denseC, a `data` tensor after each bitmap tensor, and the
//    output allocated here and kept until freeMatC() (:324).
// The reference kernels force every stored value to 1.0
// (spmm_kernel.cu:96-102); by default the `data` tensors are therefore not
// read, so results equal the reference's.  set_use_values(True) makes the
// kernels use them (value of bit i of block b = data[tcOffset[b] + rank]).
//
// forward_tensorcore (both forms) packs x into exact TF32 rows first when
// the BCSR gathers each row at least 16 times (tcc_spmm_cnic_forward_ws,
// the buffer from torch's caching allocator on the current stream).  It also
// keeps per-graph plans (tcc_hybrid_from_bcsr: dense degree-ordered tiles on
// MFMA plus the gather of the rest), found again by a device hash of the
// BCSR arrays (tcc_hash_arrays) and their sizes, so that a graph rewritten
// in place is recognised as new:
//  * by default (automatic), for a graph of at least kAutoMinBlocks blocks
//    and 64 blocks per row window on average (the skewed graphs where the
//    plan pays): one plan, built by the second call that finds the same
//    arrays, so a single call on a graph pays only the hash;
//  * after set_graph_plans(n > 0): up to n plans for any graph, built by the
//    first call; set_graph_plans(0) turns plans off, set_graph_plans(-1)
//    restores the automatic default.
// The environment variable TCC_SPMM_CNIC_PLANS=0 turns the automatic plans
// off from the first call.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "tcc_spmm_cnic.h"
#include "tcc_swtcf.h"

namespace py = pybind11;

namespace {

std::vector<torch::Tensor> g_outputs;  // Python-caller form outputs, released by freeMatC()
std::vector<void*> g_spaces;           // space_malloc buffers, released by finalize()
bool g_use_values = false;
std::uint32_t g_unit_blocks = 0;       // blocks per unit of work (0 = automatic)

// Per-graph plans, most recently used last (set_graph_plans); entries not
// yet built are graphs seen once in the automatic mode.  These globals, like
// the settings above, are guarded by the GIL: no function of the module
// releases it.
struct Plan {
    int device;
    std::uint32_t rows, cols, blocks, windows;
    bool values;
    std::uint64_t h0, h1;
    bool built;
    tcc_hybrid H;
};
std::vector<Plan> g_plans;
enum class PlanMode { Auto, Explicit, Off };
PlanMode g_plan_mode = PlanMode::Auto;
bool g_plan_env_read = false;
std::size_t g_max_plans = 1;
constexpr std::uint32_t kAutoMinBlocks = 1u << 16;
constexpr std::uint32_t kAutoMinBlocksPerWindow = 64;

void check(int rc) {
    if (rc != 0) {
        throw std::runtime_error(std::string("spmm_cnic: ") + tcc_last_error());
    }
}

void* stream_of(int device) {
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device)).stream());
}

const std::uint32_t* u32_ptr(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda() && t.is_contiguous(), name, " must be a contiguous device tensor");
    TORCH_CHECK(t.scalar_type() == torch::kInt32 || t.scalar_type() == torch::kUInt32, name,
                " must be int32/uint32");
    return reinterpret_cast<const std::uint32_t*>(t.data_ptr());
}

const std::uint64_t* u64_ptr(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda() && t.is_contiguous(), name, " must be a contiguous device tensor");
    TORCH_CHECK(t.element_size() == 8, name, " must hold 64-bit bitmaps");
    return reinterpret_cast<const std::uint64_t*>(t.data_ptr());
}

const float* values_ptr(const torch::Tensor* data) {
    if (!g_use_values || data == nullptr || !data->defined() || data->numel() == 0) return nullptr;
    TORCH_CHECK(data->is_cuda() && data->is_contiguous() && data->scalar_type() == torch::kFloat32,
                "data must be a contiguous float32 device tensor");
    return data->data_ptr<float>();
}

tcc_bcsr make_bcsr(std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz, std::uint32_t blocks,
                   std::uint32_t windows, const torch::Tensor& rwo, const torch::Tensor& tco,
                   const torch::Tensor& a2b, const torch::Tensor& bits, const torch::Tensor* data) {
    tcc_bcsr b{};
    b.num_rows = rows;
    b.num_cols = cols;
    b.nnz = nnz;
    b.num_TCBlocks = blocks;
    b.num_rowWindows = windows;
    b.rowWindowOffset = u32_ptr(rwo, "bcsr_rowWindowOffset");
    b.tcOffset = u32_ptr(tco, "bcsr_tcOffset");
    b.sparseA2B = u32_ptr(a2b, "bcsr_sparseA2B");
    b.tcLocalBit = u64_ptr(bits, "bcsr_tcLocalBit");
    b.data = values_ptr(data);
    b.unitBlocks = g_unit_blocks;
    return b;
}

tcc_bcsc make_bcsc(std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz, std::uint32_t blocks,
                   std::uint32_t windows, const torch::Tensor& cwo, const torch::Tensor& tco,
                   const torch::Tensor& a2c, const torch::Tensor& bits, const torch::Tensor* data) {
    tcc_bcsc b{};
    b.num_rows = rows;
    b.num_cols = cols;
    b.nnz = nnz;
    b.num_TCBlocks = blocks;
    b.num_colWindows = windows;
    b.colWindowOffset = u32_ptr(cwo, "bcsc_colWindowOffset");
    b.tcOffset = u32_ptr(tco, "bcsc_tcOffset");
    b.sparseA2C = u32_ptr(a2c, "bcsc_sparseA2C");
    b.tcLocalBit = u64_ptr(bits, "bcsc_tcLocalBit");
    b.data = values_ptr(data);
    b.unitBlocks = g_unit_blocks;
    return b;
}

// (num_rowWindows + 1) * 8 * F floats: spmm_launcher.cu:241-244
std::int64_t denseC_elems(std::uint32_t windows, std::int32_t F) {
    return (static_cast<std::int64_t>(windows) + 1) * 8 * F;
}

torch::Tensor view_of(float* p, std::uint32_t rows, std::int32_t F, int device) {
    return torch::from_blob(p, {static_cast<std::int64_t>(rows) * F},
                            torch::TensorOptions().dtype(torch::kFloat32).device(torch::kCUDA, device));
}

int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) throw std::runtime_error("spmm_cnic: hipGetDevice failed");
    return d;
}

// One error word per device for the feature lookups of this module's
// products (tcc_feature_source.device_error), allocated by initialize() or
// at the first product on the device; read and cleared by feature_error().
std::uint32_t* g_error_word[64] = {};

std::uint32_t* error_word(int device) {
    TORCH_CHECK(device >= 0 && device < 64, "spmm_cnic: device id out of range");
    if (g_error_word[device] == nullptr) {
        void* p = nullptr;
        if (hipMalloc(&p, sizeof(std::uint32_t)) != hipSuccess || hipMemset(p, 0, sizeof(std::uint32_t)) != hipSuccess)
            throw std::runtime_error("spmm_cnic: cannot allocate the feature error word");
        g_error_word[device] = static_cast<std::uint32_t*>(p);
    }
    return g_error_word[device];
}

tcc_feature_source feature_source(const torch::Tensor& id_map, py::capsule cpu_ptr,
                                  const torch::Tensor& cache_search_map, py::capsule gpu_ptr,
                                  std::int32_t gpu_node_capacity) {
    TORCH_CHECK(id_map.is_cuda() && id_map.scalar_type() == torch::kInt32 && id_map.is_contiguous(),
                "id_map must be a contiguous int32 device tensor");
    TORCH_CHECK(cache_search_map.is_cuda() && cache_search_map.scalar_type() == torch::kInt32 &&
                    cache_search_map.is_contiguous(),
                "cache_search_map must be a contiguous int32 device tensor");
    TORCH_CHECK(gpu_node_capacity > 0, "gpu_node_capacity must be positive");
    tcc_feature_source s{};
    s.id_map = id_map.data_ptr<std::int32_t>();
    s.cache_search_map = cache_search_map.data_ptr<std::int32_t>();
    s.gpu_feature_cache = static_cast<const float* const*>(gpu_ptr.get_pointer());
    s.gpu_node_capacity = gpu_node_capacity;
    // The host feature rows are read zero-copy: translate the pinned host
    // pointer to its device alias (mapped pinned memory only).
    void* host = cpu_ptr.get_pointer();
    void* dev = nullptr;
    if (host != nullptr && hipHostGetDevicePointer(&dev, host, 0) != hipSuccess) {
        throw std::runtime_error("spmm_cnic: cpu_feature_cache_ptr is not mapped pinned host memory");
    }
    s.cpu_features = static_cast<const float*>(dev);
    // cpu_float_feature_len is accepted and ignored, as the reference's
    // kernels ignore it (module.cu:27,75 never pass it on): its producer is
    // outside the reference, so its unit (floats or rows) is unknown, and a
    // bound taken in the wrong unit would refuse valid rows.  Host rows are
    // therefore not bounds-checked in this form.
    s.cpu_feature_len = 0;
    s.gpu_feature_cache_count = 1;  // one GPU: the clique's pointer table has a single entry
    s.device_error = error_word(current_device());
    return s;
}

// ---------------------------------------------------------------- the non-mixed forward

torch::Tensor device_bytes(std::size_t n, int device) {
    return torch::empty({static_cast<std::int64_t>(n)},
                        torch::TensorOptions().dtype(torch::kUInt8).device(torch::kCUDA, device));
}

void* aligned16(const torch::Tensor& t) {
    return reinterpret_cast<void*>((reinterpret_cast<std::uintptr_t>(t.data_ptr()) + 15) & ~std::uintptr_t(15));
}

void drop_plan(Plan& p) {
    // hipFree waits for the work in flight that may still read the arrays
    if (p.built && tcc_hybrid_release(&p.H) != 0)
        throw std::runtime_error(std::string("spmm_cnic: ") + tcc_last_error());
    p.built = false;
}

void release_plans() {
    for (Plan& p : g_plans) drop_plan(p);
    g_plans.clear();
}

// At most g_max_plans built plans and 2 g_max_plans + 2 entries, the least
// recently used (front) dropped first.
void trim_plans() {
    for (;;) {
        std::size_t built = 0;
        for (const Plan& p : g_plans) built += p.built ? 1 : 0;
        if (built <= g_max_plans) break;
        for (Plan& p : g_plans)
            if (p.built) {
                drop_plan(p);
                break;
            }
    }
    while (g_plans.size() > 2 * g_max_plans + 2) {
        drop_plan(g_plans.front());
        g_plans.erase(g_plans.begin());
    }
}

void set_graph_plans(std::int64_t n) {
    TORCH_CHECK(n >= -1, "set_graph_plans: a count of plans (0 = none, -1 = automatic)");
    g_plan_env_read = true;
    if (n < 0) {
        g_plan_mode = PlanMode::Auto;
        g_max_plans = 1;
    } else {
        g_plan_mode = n == 0 ? PlanMode::Off : PlanMode::Explicit;
        g_max_plans = static_cast<std::size_t>(n);
    }
    if (g_max_plans == 0) {
        release_plans();
        return;
    }
    trim_plans();
}

std::int64_t graph_plans() {
    std::int64_t n = 0;
    for (const Plan& p : g_plans) n += p.built ? 1 : 0;
    return n;
}

// The plan of A's graph on `device`, or nullptr when the default path
// should run: found by the hash of its arrays and its sizes; built by the
// first call in the explicit mode, by the second in the automatic one.
const tcc_hybrid* plan_for(const tcc_bcsr& A, int device, void* st) {
    if (!g_plan_env_read) {
        g_plan_env_read = true;
        if (const char* e = std::getenv("TCC_SPMM_CNIC_PLANS"))
            if (std::string(e) == "0") g_plan_mode = PlanMode::Off;
    }
    if (g_plan_mode == PlanMode::Off || g_max_plans == 0 || A.num_TCBlocks == 0 || A.phases > 1) return nullptr;
    if (g_plan_mode == PlanMode::Auto &&
        (A.num_TCBlocks < kAutoMinBlocks ||
         A.num_TCBlocks < static_cast<std::uint64_t>(kAutoMinBlocksPerWindow) * A.num_rowWindows))
        return nullptr;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(reinterpret_cast<hipStream_t>(st), &cap) != hipSuccess ||
        cap != hipStreamCaptureStatusNone)
        return nullptr;  // the hash is read back: not under graph capture
    const bool values = A.data != nullptr;
    const void* arrays[4] = {A.rowWindowOffset, A.sparseA2B, A.tcLocalBit, A.data};
    const std::uint64_t bytes[4] = {4ull * (A.num_rowWindows + 1ull), 32ull * A.num_TCBlocks, 8ull * A.num_TCBlocks,
                                    4ull * A.nnz};
    torch::Tensor h =
        torch::empty({TCC_HASH_WORDS}, torch::TensorOptions().dtype(torch::kInt64).device(torch::kCUDA, device));
    check(tcc_hash_arrays(arrays, bytes, values ? 4 : 3, reinterpret_cast<std::uint64_t*>(h.data_ptr()), st));
    torch::Tensor hh = torch::empty({TCC_HASH_WORDS}, torch::TensorOptions().dtype(torch::kInt64).pinned_memory(true));
    hh.copy_(h, /*non_blocking=*/true);
    if (hipStreamSynchronize(reinterpret_cast<hipStream_t>(st)) != hipSuccess)  // waits for the hash
        throw std::runtime_error("spmm_cnic: hipStreamSynchronize failed while reading the graph hash");
    const std::uint64_t* hw = reinterpret_cast<const std::uint64_t*>(hh.data_ptr());
    std::uint64_t h0 = 0, h1 = 0;
    for (unsigned k = 0; k < TCC_HASH_WORDS / 2; ++k) {
        h0 += hw[2 * k];
        h1 += hw[2 * k + 1];
    }
    for (std::size_t i = 0; i < g_plans.size(); ++i) {
        Plan& p = g_plans[i];
        if (p.device == device && p.rows == A.num_rows && p.cols == A.num_cols && p.blocks == A.num_TCBlocks &&
            p.windows == A.num_rowWindows && p.values == values && p.h0 == h0 && p.h1 == h1) {
            std::rotate(g_plans.begin() + static_cast<std::ptrdiff_t>(i), g_plans.begin() + static_cast<std::ptrdiff_t>(i) + 1,
                        g_plans.end());
            Plan& q = g_plans.back();
            if (!q.built) {
                // the automatic plan is an optimisation: if it cannot be
                // built (device memory), the default path runs
                if (tcc_hybrid_from_bcsr(&A, values ? 1 : 0, 0, 0, &q.H, st) != 0) {
                    if (g_plan_mode == PlanMode::Explicit) check(1);
                    g_plans.pop_back();
                    (void)hipGetLastError();
                    return nullptr;
                }
                q.built = true;
                trim_plans();
            }
            return &g_plans.back().H;
        }
    }
    Plan p{device, A.num_rows, A.num_cols, A.num_TCBlocks, A.num_rowWindows, values, h0, h1, false, tcc_hybrid{}};
    if (g_plan_mode == PlanMode::Explicit) {
        check(tcc_hybrid_from_bcsr(&A, values ? 1 : 0, 0, 0, &p.H, st));
        p.built = true;
    }
    g_plans.push_back(p);
    trim_plans();
    return g_plans.back().built ? &g_plans.back().H : nullptr;
}

// denseC[(r_win+1)*8*F] = A x + B x (launch_spmm_kernel, spmm_launcher.cu:203-271)
void forward(const tcc_bcsr& A, const tcc_bcsc& B, const torch::Tensor& x, float* C, std::int32_t F, int device) {
    TORCH_CHECK(x.is_cuda() && x.is_contiguous() && x.scalar_type() == torch::kFloat32, "x must be fp32 on device");
    void* st = stream_of(device);
    const float* X = x.data_ptr<float>();
    if (const tcc_hybrid* plan = plan_for(A, device, st)) {
        const tcc_hybrid& H = *plan;
        const std::size_t need = tcc_hybrid_workspace_bytes(&H, static_cast<std::uint32_t>(F));
        torch::Tensor ws = device_bytes(need + 16, device);
        check(tcc_hybrid_spmm(&H, X, C, static_cast<std::uint32_t>(F), 0, aligned16(ws), need, st));
        // rows past the plan's 8-row windows (the reference's extra window and any more) are zero
        const std::int64_t done = static_cast<std::int64_t>(H.rest.num_rowWindows / std::max(1u, H.rest.phases)) * 8 * F;
        const std::int64_t all = denseC_elems(A.num_rowWindows, F);
        if (all > done) view_of(C, static_cast<std::uint32_t>(all / F), F, device).narrow(0, done, all - done).zero_();
        check(tcc_bcsc_spmm(&B, X, C, static_cast<std::uint32_t>(F), st));
        return;
    }
    const std::size_t need = tcc_spmm_cnic_forward_workspace_bytes(&A, static_cast<std::uint32_t>(F));
    torch::Tensor ws;
    if (need) ws = device_bytes(need, device);
    check(tcc_spmm_cnic_forward_ws(&A, &B, X, C, static_cast<std::uint32_t>(F), need ? ws.data_ptr() : nullptr, need,
                                   st));
}

// ---------------------------------------------------------------- compiled form

torch::Tensor fwd_mixed_bound(std::uint32_t r_rows, std::uint32_t r_cols, std::uint32_t r_nnz, std::uint32_t r_blk,
                              std::uint32_t r_win, torch::Tensor r_rwo, torch::Tensor r_tco, torch::Tensor r_a2b,
                              torch::Tensor r_bits, std::uint32_t c_rows, std::uint32_t c_cols, std::uint32_t c_nnz,
                              std::uint32_t c_blk, std::uint32_t c_win, torch::Tensor c_cwo, torch::Tensor c_tco,
                              torch::Tensor c_a2c, torch::Tensor c_bits, std::int64_t cpu_len, std::int32_t cap,
                              std::int32_t F, torch::Tensor id_map, py::capsule cpu_ptr, torch::Tensor csm,
                              py::capsule gpu_ptr, torch::Tensor x, std::int32_t device_id, py::capsule denseC) {
    // module.cu:100-190 (the compiled variant computes with x; an empty x
    // selects the hot/cold feature source instead)
    tcc_bcsr A = make_bcsr(r_rows, r_cols, r_nnz, r_blk, r_win, r_rwo, r_tco, r_a2b, r_bits, nullptr);
    tcc_bcsc B = make_bcsc(c_rows, c_cols, c_nnz, c_blk, c_win, c_cwo, c_tco, c_a2c, c_bits, nullptr);
    float* C = static_cast<float*>(denseC.get_pointer());
    if (x.defined() && x.numel() > 0) {
        forward(A, B, x, C, F, device_id);
    } else {
        const tcc_feature_source s = feature_source(id_map, cpu_ptr, csm, gpu_ptr, cap);
        check(tcc_spmm_cnic_forward_mixed(&A, &B, &s, C, F, stream_of(device_id)));
    }
    return view_of(C, r_rows, F, current_device());
}

torch::Tensor fwd_mixed_bound_nox(std::uint32_t r_rows, std::uint32_t r_cols, std::uint32_t r_nnz, std::uint32_t r_blk,
                                  std::uint32_t r_win, torch::Tensor r_rwo, torch::Tensor r_tco, torch::Tensor r_a2b,
                                  torch::Tensor r_bits, std::uint32_t c_rows, std::uint32_t c_cols,
                                  std::uint32_t c_nnz, std::uint32_t c_blk, std::uint32_t c_win, torch::Tensor c_cwo,
                                  torch::Tensor c_tco, torch::Tensor c_a2c, torch::Tensor c_bits, std::int64_t cpu_len,
                                  std::int32_t cap, std::int32_t F, torch::Tensor id_map, py::capsule cpu_ptr,
                                  torch::Tensor csm, py::capsule gpu_ptr, std::int32_t device_id,
                                  py::capsule denseC) {
    // the use_mixed_memory_access variant (module.cu:21-97)
    return fwd_mixed_bound(r_rows, r_cols, r_nnz, r_blk, r_win, r_rwo, r_tco, r_a2b, r_bits, c_rows, c_cols, c_nnz,
                           c_blk, c_win, c_cwo, c_tco, c_a2c, c_bits, cpu_len, cap, F, id_map, cpu_ptr, csm, gpu_ptr,
                           torch::Tensor(), device_id, denseC);
}

torch::Tensor fwd_bound(std::uint32_t r_rows, std::uint32_t r_cols, std::uint32_t r_nnz, std::uint32_t r_blk,
                        std::uint32_t r_win, torch::Tensor r_rwo, torch::Tensor r_tco, torch::Tensor r_a2b,
                        torch::Tensor r_bits, std::uint32_t c_rows, std::uint32_t c_cols, std::uint32_t c_nnz,
                        std::uint32_t c_blk, std::uint32_t c_win, torch::Tensor c_cwo, torch::Tensor c_tco,
                        torch::Tensor c_a2c, torch::Tensor c_bits, std::int32_t F, torch::Tensor x,
                        std::int32_t device_id, py::capsule denseC) {
    // module.cu:192-273
    tcc_bcsr A = make_bcsr(r_rows, r_cols, r_nnz, r_blk, r_win, r_rwo, r_tco, r_a2b, r_bits, nullptr);
    tcc_bcsc B = make_bcsc(c_rows, c_cols, c_nnz, c_blk, c_win, c_cwo, c_tco, c_a2c, c_bits, nullptr);
    float* C = static_cast<float*>(denseC.get_pointer());
    forward(A, B, x, C, F, device_id);
    return view_of(C, r_rows, F, current_device());
}

// ---------------------------------------------------------------- Python-caller form

torch::Tensor alloc_output(std::uint32_t windows, std::int32_t F) {
    TORCH_CHECK(F >= 1, "feature_dim must be positive");
    const int dev = current_device();
    auto out = torch::empty({denseC_elems(windows, F)},
                            torch::TensorOptions().dtype(torch::kFloat32).device(torch::kCUDA, dev));
    g_outputs.push_back(out);
    return out;
}

torch::Tensor fwd_mixed_py(std::uint32_t r_rows, std::uint32_t r_cols, std::uint32_t r_nnz, std::uint32_t r_blk,
                           std::uint32_t r_win, torch::Tensor r_rwo, torch::Tensor r_tco, torch::Tensor r_a2b,
                           torch::Tensor r_bits, torch::Tensor r_data, std::uint32_t c_rows, std::uint32_t c_cols,
                           std::uint32_t c_nnz, std::uint32_t c_blk, std::uint32_t c_win, torch::Tensor c_cwo,
                           torch::Tensor c_tco, torch::Tensor c_a2c, torch::Tensor c_bits, torch::Tensor c_data,
                           std::int64_t cpu_len, std::int32_t cap, std::int32_t F, torch::Tensor id_map,
                           py::capsule cpu_ptr, torch::Tensor csm, py::capsule gpu_ptr) {
    // train/tcgnn_conv_release.py:116-122
    tcc_bcsr A = make_bcsr(r_rows, r_cols, r_nnz, r_blk, r_win, r_rwo, r_tco, r_a2b, r_bits, &r_data);
    tcc_bcsc B = make_bcsc(c_rows, c_cols, c_nnz, c_blk, c_win, c_cwo, c_tco, c_a2c, c_bits, &c_data);
    const tcc_feature_source s = feature_source(id_map, cpu_ptr, csm, gpu_ptr, cap);
    torch::Tensor out = alloc_output(r_win, F);
    void* st = stream_of(current_device());
    check(tcc_spmm_cnic_forward_mixed(&A, &B, &s, out.data_ptr<float>(), F, st));
    return out.narrow(0, 0, static_cast<std::int64_t>(r_rows) * F);
}

torch::Tensor fwd_py(std::uint32_t r_rows, std::uint32_t r_cols, std::uint32_t r_nnz, std::uint32_t r_blk,
                     std::uint32_t r_win, torch::Tensor r_rwo, torch::Tensor r_tco, torch::Tensor r_a2b,
                     torch::Tensor r_bits, torch::Tensor r_data, std::uint32_t c_rows, std::uint32_t c_cols,
                     std::uint32_t c_nnz, std::uint32_t c_blk, std::uint32_t c_win, torch::Tensor c_cwo,
                     torch::Tensor c_tco, torch::Tensor c_a2c, torch::Tensor c_bits, torch::Tensor c_data,
                     std::int32_t F, torch::Tensor x) {
    // train/tcgnn_conv_release.py:124-130
    tcc_bcsr A = make_bcsr(r_rows, r_cols, r_nnz, r_blk, r_win, r_rwo, r_tco, r_a2b, r_bits, &r_data);
    tcc_bcsc B = make_bcsc(c_rows, c_cols, c_nnz, c_blk, c_win, c_cwo, c_tco, c_a2c, c_bits, &c_data);
    torch::Tensor out = alloc_output(r_win, F);
    forward(A, B, x, out.data_ptr<float>(), F, current_device());
    return out.narrow(0, 0, static_cast<std::int64_t>(r_rows) * F);
}

// ---------------------------------------------------------------- lifecycle

void initialize(int device_id) {
    // module.cu:299-304; work is ordered on torch's current stream instead of
    // two private streams, so the returned tensors are safe to use at once.
    if (hipSetDevice(device_id) != hipSuccess) throw std::runtime_error("spmm_cnic: hipSetDevice failed");
    (void)error_word(device_id);
}

// No reference counterpart: TCC_DEVERR_FEATURE_INDEX (7) if a first-layer
// product on the device looked up a feature row outside its table (read as
// zeros) since the last call, else 0.  Synchronises the device and clears
// the word.
std::uint32_t feature_error(int device_id) {
    std::uint32_t* w = error_word(device_id);
    std::uint32_t v = 0;
    if (hipSetDevice(device_id) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(&v, w, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess || hipMemset(w, 0, sizeof(v)) != hipSuccess)
        throw std::runtime_error("spmm_cnic: cannot read the feature error word");
    return v;
}

std::vector<py::capsule> space_malloc(int device_id, std::uint32_t denseC_size) {
    // module.cu:306-327: two zeroed fp32 buffers of denseC_size elements
    if (hipSetDevice(device_id) != hipSuccess) throw std::runtime_error("spmm_cnic: hipSetDevice failed");
    std::vector<py::capsule> out;
    for (const char* name : {"denseC", "denseC_2"}) {
        void* p = nullptr;
        const std::size_t bytes = static_cast<std::size_t>(denseC_size) * sizeof(float);
        if (hipMalloc(&p, bytes) != hipSuccess || hipMemset(p, 0, bytes) != hipSuccess) {
            throw std::runtime_error("spmm_cnic: space_malloc failed");
        }
        g_spaces.push_back(p);
        out.emplace_back(p, name);
    }
    return out;
}

void finalize(int device_id) {
    // module.cu:329-341
    if (hipSetDevice(device_id) != hipSuccess) throw std::runtime_error("spmm_cnic: hipSetDevice failed");
    if (hipDeviceSynchronize() != hipSuccess) throw std::runtime_error("spmm_cnic: hipDeviceSynchronize failed");
    for (void* p : g_spaces) (void)hipFree(p);
    g_spaces.clear();
    g_outputs.clear();
    release_plans();
}

void freeMatC() {
    g_outputs.clear();
}

void set_unit_blocks(std::uint32_t blocks) { g_unit_blocks = blocks; }

void set_use_values(bool on) { g_use_values = on; }

void read_cpu_feature_cache(py::capsule p, std::int32_t len) {
    const float* f = static_cast<const float*>(p.get_pointer());
    std::printf("h_cpu_feature_cache: { ");
    for (std::int32_t i = 0; i < len; ++i) std::printf("%f, ", f[i]);
    std::printf("}\n");
}

void read_gpu0_feature_cache(py::capsule p) {
    float h[100];
    if (hipMemcpy(h, p.get_pointer(), sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) {
        throw std::runtime_error("spmm_cnic: hipMemcpy failed");
    }
    std::printf("gpu feature: { ");
    for (float v : h) std::printf("%f, ", v);
    std::printf("}\n");
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "spmm_cnic for ROCm / MI355X (block-sparse TF32-numerics SpMM over libtcc_swtcf)";
    m.def("forward_tensorcore_mixed", &fwd_mixed_py, "first-layer SpMM, Python-caller form (allocates the output)");
    m.def("forward_tensorcore_mixed", &fwd_mixed_bound, "first-layer SpMM, compiled form with x, device_id, denseC");
    m.def("forward_tensorcore_mixed", &fwd_mixed_bound_nox, "first-layer SpMM, mixed-memory compiled form");
    m.def("forward_tensorcore", &fwd_py, "SpMM, Python-caller form (allocates the output)");
    m.def("forward_tensorcore", &fwd_bound, "SpMM, compiled form with device_id and denseC");
    m.def("read_cpu_feature_cache", &read_cpu_feature_cache, "print host feature rows");
    m.def("read_gpu0_feature_cache", &read_gpu0_feature_cache, "print the first 100 floats of a device cache");
    m.def("initialize", &initialize, "select the device");
    m.def("space_malloc", &space_malloc, "two zeroed denseC buffers (capsules)");
    m.def("finalize", &finalize, "free space_malloc buffers and outputs");
    m.def("freeMatC", &freeMatC, "release the outputs of the Python-caller form");
    m.def("feature_error", &feature_error,
          "7 (TCC_DEVERR_FEATURE_INDEX) if a feature lookup fell outside its table since the last call, else 0");
    m.def("set_use_values", &set_use_values, "read the per-block data values (default: all entries 1.0)");
    m.def("set_unit_blocks", &set_unit_blocks,
          "blocks each wave of work walks (default 0 = chosen from the block count)");
    m.def("set_graph_plans", &set_graph_plans,
          "per-graph plans (dense tiles on MFMA + gather), found by a hash of the BCSR arrays: n > 0 keeps up to n, "
          "built by the first call on a graph; 0 turns them off; -1 restores the default (one plan, for large "
          "skewed graphs, built by the second call that finds the same arrays)");
    m.def("release_plans", &release_plans, "release every per-graph plan");
    m.def("graph_plans", &graph_plans, "the number of per-graph plans held");
}
