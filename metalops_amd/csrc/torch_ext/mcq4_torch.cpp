// PyTorch-ROCm extension over the C ABI: the binding a metalcore maintainer
// adds in place of the Metal one.  It mirrors matmul_ggml_q4_0_metal
// (native/core_mps.mm:5917-5975, registered as "matmul_ggml_q4_0" at :6938):
// fp16 X [M, K] and uint8 W_blocks [K/32, N, 18] on the GPU, contiguous copies
// made by the callee, Y [M, N] fp16 allocated by the callee, errors as
// RuntimeError (TORCH_CHECK), work enqueued on the current stream without a
// synchronisation.  The split-K workspace is kept per (device, stream),
// zero-filled once (every call leaves its counters zero).
#include <string>
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>
#include <c10/core/DeviceGuard.h>

#include <map>
#include <mutex>
#include <utility>

#include "mcq4.h"

namespace {

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, torch::Tensor> g_ws;

torch::Tensor workspace(const torch::Tensor &like, hipStream_t stream, size_t need) {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto &buf = g_ws[{like.get_device(), stream}];
    if (!buf.defined() || (size_t)buf.numel() < need)
        buf = torch::zeros({(int64_t)std::max<size_t>(need, 1 << 20)}, like.options().dtype(torch::kUInt8));
    return buf;
}

}  // namespace

torch::Tensor matmul_ggml_q4_0(torch::Tensor X, torch::Tensor W_blocks) {
    TORCH_CHECK(X.is_cuda(), "X must be on a ROCm GPU");
    TORCH_CHECK(W_blocks.is_cuda() && W_blocks.get_device() == X.get_device(),
                "W_blocks must be on X's GPU");
    TORCH_CHECK(X.scalar_type() == torch::kHalf, "X must be float16");
    TORCH_CHECK(W_blocks.scalar_type() == torch::kUInt8, "W_blocks must be uint8");
    TORCH_CHECK(X.dim() == 2 && W_blocks.dim() == 3, "X must be [M, K] and W_blocks [K/32, N, 18]");
    TORCH_CHECK(W_blocks.size(2) == 18, "W_blocks last dim must be 18 (block_q4_0 size)");
    auto x = X.contiguous();
    auto w = W_blocks.contiguous();
    const int64_t M = x.size(0), K = w.size(0) * 32, N = w.size(1);
    TORCH_CHECK(x.size(1) == K, "X K dimension must match W K dimension");
    if (reinterpret_cast<uintptr_t>(x.data_ptr()) % 16) x = x.clone();   // storage offsets
    if (reinterpret_cast<uintptr_t>(w.data_ptr()) % 2) w = w.clone();
    auto Y = torch::empty({M, N}, x.options());
    if (M == 0 || N == 0) return Y;
    if (K == 0) return Y.zero_();
    const c10::DeviceGuard guard(x.device());   // generic: torch labels ROCm devices "cuda"
    hipStream_t stream = c10::hip::getCurrentHIPStream(x.get_device()).stream();
    const size_t need = mcq4_matmul_workspace_bytes(M, K, N);
    torch::Tensor ws;
    if (need) ws = workspace(x, stream, need);
    const int st = mcq4_matmul_q4_0_f16(x.data_ptr(), K, w.data_ptr<uint8_t>(), Y.data_ptr(), N, M, K, N,
                                        need ? ws.data_ptr() : nullptr, need ? (size_t)ws.numel() : 0,
                                        stream);
    if (st != MCQ4_OK) {
        // A call that failed after some split-K workgroups drew tickets would leave
        // the per-stream workspace's counter area non-zero for the next call: zero
        // it again (a fill kernel on the same stream) before reporting the error.
        const std::string msg = mcq4_last_error();
        if (need) (void)mcq4_reset_workspace(ws.data_ptr(), (size_t)ws.numel(), stream);
        TORCH_CHECK(false, "matmul_ggml_q4_0: ", mcq4_status_string(st), ": ", msg);
    }
    return Y;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("matmul_ggml_q4_0", &matmul_ggml_q4_0, "GGML block_q4_0 matmul (gfx950 HIP kernels)");
}
