// Python binding of the W4A16 AWQ entry point for torch tensors (host code
// only; the kernels are behind the C ABI of libawq_w4a16.so,
// include/awq_w4a16.h).
//
// awq_gemm_forward(x, qweight, qzeros, scales, group_size) replaces the
// reference's entry point of the same name (kernels/awq_gemm.py:237-284) on
// the eager path: operand checks, the [M, K] flattening
// (kernels/awq_gemm.py:244-246), the fp16 output allocation, the plan, the
// split-K workspace and the current stream are all handled here, so that an
// eager call costs one Python -> C++ transition and one kernel launch (the
// reference engine makes 112 of these calls per token and never replays a
// graph, inference/engine.py:114-139).  The checks and their messages are
// the Python mirror's (kernels/awq_gemm.py in this package): ValueError for
// a bad operand, RuntimeError for a failed launch.
//
// Workspace registry: one list of zero-filled float32 buffers per device,
// grown on demand and never shrunk; earlier buffers stay referenced so that
// graphs captured with them keep valid memory.  Counters and fixed-point
// slots are zero between calls (every call leaves them zero), as the C ABI
// requires.  Growing while the stream is being captured is refused.
#include <torch/extension.h>

#include <ATen/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <unordered_map>
#include <vector>

#include "../../include/awq_w4a16.h"

namespace {

constexpr int64_t kWorkspaceAlign = 1 << 20;
constexpr size_t kPlanCacheMax = 4096;

struct PlanKey {
    int64_t M, N, K;
    int32_t group_size, path;
    int dev;
    bool operator==(const PlanKey& o) const {
        return M == o.M && N == o.N && K == o.K && group_size == o.group_size && path == o.path && dev == o.dev;
    }
};
struct PlanKeyHash {
    size_t operator()(const PlanKey& k) const {
        uint64_t h = (uint64_t)k.M * 0x9E3779B97F4A7C15ull;
        h ^= (uint64_t)k.N + 0x7F4A7C159E3779B9ull + (h << 6) + (h >> 2);
        h ^= (uint64_t)k.K + 0x2545F4914F6CDD1Dull + (h << 6) + (h >> 2);
        h ^= (uint64_t)(k.group_size * 131 + k.path * 7 + k.dev) + (h << 6) + (h >> 2);
        return (size_t)h;
    }
};

// Called with the Python GIL held (pybind11's default), so the two maps need
// no lock of their own.
std::unordered_map<PlanKey, awq_w4a16_plan, PlanKeyHash> g_plans;
std::unordered_map<int, std::vector<at::Tensor>> g_workspaces;

void check_status(int st, const char* where) {
    TORCH_CHECK(st == AWQ_OK, where, ": status ", st, ": ", awq_w4a16_error_string(st));
}

// The plan for a shape on a device (the planner sizes grids by the device's
// compute units, so the device must be current when it plans).
const awq_w4a16_plan& plan_for(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t path, int dev) {
    const PlanKey key{M, N, K, group_size, path, dev};
    auto it = g_plans.find(key);
    if (it != g_plans.end()) return it->second;
    awq_w4a16_plan p;
    check_status(awq_w4a16_plan_for(M, N, K, group_size, path, &p), "awq_w4a16_plan_for");
    if (g_plans.size() >= kPlanCacheMax) g_plans.clear();
    return g_plans.emplace(key, p).first->second;
}

// The device's largest workspace buffer, grown to at least `bytes`.
at::Tensor& workspace_for(const at::Device& device, uint64_t bytes, hipStream_t stream) {
    auto& bufs = g_workspaces[device.index()];
    if (!bufs.empty() && (uint64_t)bufs.back().numel() * 4u >= bytes) return bufs.back();
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    TORCH_CHECK(hipStreamIsCapturing(stream, &cap) == hipSuccess, "hipStreamIsCapturing failed");
    TORCH_CHECK(cap == hipStreamCaptureStatusNone, "awq_gemm workspace must grow to ", bytes,
                " bytes during graph capture; run the largest shape once eagerly before capturing");
    const int64_t size = ((int64_t)bytes + kWorkspaceAlign - 1) / kWorkspaceAlign * kWorkspaceAlign;
    bufs.push_back(at::zeros({size / 4}, at::TensorOptions().dtype(at::kFloat).device(device)));
    return bufs.back();
}

// `t` when its data starts on a 16-byte boundary, else a copy (the kernels use
// 16-byte vector accesses; the reference's Triton path takes any view).
at::Tensor aligned16(const at::Tensor& t) {
    return (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) == 0 ? t : t.clone();
}

at::Tensor awq_gemm_forward(const at::Tensor& x, const at::Tensor& qweight, const at::Tensor& qzeros,
                            const at::Tensor& scales, int64_t group_size) {
    TORCH_CHECK_VALUE(x.scalar_type() == at::kHalf, "x must be float16, got ", x.scalar_type());
    TORCH_CHECK_VALUE(qweight.scalar_type() == at::kInt && qzeros.scalar_type() == at::kInt,
                      "qweight/qzeros must be int32, got ", qweight.scalar_type(), "/", qzeros.scalar_type());
    TORCH_CHECK_VALUE(scales.scalar_type() == at::kHalf, "scales must be float16, got ", scales.scalar_type());
    TORCH_CHECK_VALUE(group_size == 128, "group_size ", group_size, " is not served (only 128)");
    TORCH_CHECK_VALUE(qweight.dim() == 2 && qzeros.dim() == 2 && scales.dim() == 2 && x.dim() >= 1,
                      "qweight, qzeros and scales must be 2-D and x at least 1-D");
    const int64_t K = x.size(-1);
    const int64_t N = scales.size(1);
    TORCH_CHECK_VALUE(N > 0 && N % 8 == 0, "N = scales.shape[1] = ", N, " must be a positive multiple of 8");
    TORCH_CHECK_VALUE(K > 0 && K % group_size == 0, "K = ", K, " must be a positive multiple of group_size ",
                      group_size);
    TORCH_CHECK_VALUE(qweight.size(0) == K && qweight.size(1) == N / 8, "qweight shape ", qweight.sizes(),
                      " != (K, N/8) = (", K, ", ", N / 8, ")");
    TORCH_CHECK_VALUE(qzeros.size(0) == K / group_size && qzeros.size(1) == N / 8, "qzeros shape ",
                      qzeros.sizes(), " != (K/G, N/8) = (", K / group_size, ", ", N / 8, ")");
    TORCH_CHECK_VALUE(scales.size(0) == K / group_size, "scales shape ", scales.sizes(), " != (K/G, N) = (",
                      K / group_size, ", ", N, ")");
    const at::Device device = x.device();
    TORCH_CHECK_VALUE(device.is_cuda(), "operands must be on a ROCm device, got ", device);
    TORCH_CHECK_VALUE(qweight.device() == device && qzeros.device() == device && scales.device() == device,
                      "all operands must be on ", device);

    const at::Tensor x2 = aligned16((x.dim() == 2 ? x : x.reshape({-1, K})).contiguous());
    const at::Tensor qw = qweight.contiguous();
    const at::Tensor qz = qzeros.contiguous();
    const at::Tensor sc = aligned16(scales.contiguous());
    const int64_t M = x2.size(0);
    std::vector<int64_t> out_shape(x.sizes().begin(), x.sizes().end() - 1);
    out_shape.push_back(N);
    at::Tensor out = at::empty({M, N}, x.options());
    if (M == 0) return out.view(out_shape);

    const at::DeviceGuard guard(device);
    const int dev = device.index();
    const awq_w4a16_plan& p = plan_for(M, N, K, (int32_t)group_size, AWQ_PATH_AUTO, dev);
    hipStream_t stream = c10::hip::getCurrentHIPStream(dev).stream();
    void* ws = nullptr;
    size_t ws_bytes = 0;
    if (p.workspace_bytes > 0) {
        at::Tensor& w = workspace_for(device, p.workspace_bytes, stream);
        ws = w.data_ptr();
        ws_bytes = (size_t)w.numel() * 4u;
    }
    const int st = awq_w4a16_gemm_planned(x2.data_ptr(), qw.data_ptr<int32_t>(), qz.data_ptr<int32_t>(),
                                          sc.data_ptr(), out.data_ptr(), M, N, K, (int32_t)group_size, ws,
                                          ws_bytes, &p, stream);
    check_status(st, "awq_w4a16_gemm_planned");
    return out.view(out_shape);
}

// The registry's buffer for `device_index` holding at least `nbytes` (grown
// if needed, refused during capture), for the Python entry points that pass
// a workspace through the C ABI themselves.
at::Tensor workspace(int64_t device_index, int64_t nbytes) {
    const at::Device device(at::kCUDA, (c10::DeviceIndex)device_index);
    const at::DeviceGuard guard(device);
    hipStream_t stream = c10::hip::getCurrentHIPStream((c10::DeviceIndex)device_index).stream();
    return workspace_for(device, (uint64_t)nbytes, stream);
}

// Every buffer the registry holds for `device_index`, oldest first.
std::vector<at::Tensor> workspace_buffers(int64_t device_index) {
    auto it = g_workspaces.find((int)device_index);
    return it == g_workspaces.end() ? std::vector<at::Tensor>{} : it->second;
}

}  // namespace

PYBIND11_MODULE(_awq_torch, m) {
    m.doc() = "torch binding of the W4A16 AWQ GEMM C ABI (eager entry point, plan cache, workspace registry)";
    m.def("awq_gemm_forward", &awq_gemm_forward, "x @ dequant(qweight, qzeros, scales), fp16 (AUTO plan)",
          py::arg("x"), py::arg("qweight"), py::arg("qzeros"), py::arg("scales"), py::arg("group_size") = 128);
    m.def("workspace", &workspace, "the device's workspace buffer, at least nbytes", py::arg("device_index"),
          py::arg("nbytes"));
    m.def("workspace_buffers", &workspace_buffers, "every workspace buffer of a device", py::arg("device_index"));
    m.def("abi_version", [] { return awq_w4a16_abi_version(); });
}
