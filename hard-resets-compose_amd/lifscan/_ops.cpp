// C++ autograd function of lif_tuned's recomputing pair (triton_lif.py:654-687 LIFTuned, with the
// forward storing the chunk entry states instead of U and the adjoint replaying each chunk from
// them): the same two C-ABI entry points the Python layer calls (lsh_lif_scan_exact_fwd_starts,
// lsh_lif_scan_fused_bwd_starts), called from C++ so that a layer call costs one Python -> C++
// crossing instead of an autograd Function in Python plus ctypes calls.  The entry points'
// addresses are handed over once from the library the Python package has loaded (no link-time
// dependency, one copy of the library in the process).
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <string>

namespace {

using FwdStarts = int (*)(const float*, const float*, float*, float*, int64_t, int64_t, float, float,
                          float, int, void*, size_t, void*);
using BwdStarts = int (*)(const float*, const float*, const float*, float*, double*, int64_t,
                          int64_t, float, float, float, float, int, void*);
using StatusString = const char* (*)(int);

FwdStarts g_fwd = nullptr;
BwdStarts g_bwd = nullptr;
StatusString g_status = nullptr;

void set_entry_points(int64_t fwd, int64_t bwd, int64_t status) {
  g_fwd = reinterpret_cast<FwdStarts>(fwd);
  g_bwd = reinterpret_cast<BwdStarts>(bwd);
  g_status = reinterpret_cast<StatusString>(status);
}

void check(int rc, const char* what) {
  if (rc == 0) return;
  const std::string msg = std::string(what) + ": " + (g_status ? g_status(rc) : "error") +
                          " (status " + std::to_string(rc) + ")";
  // argument errors are ValueError on the Python side, as the ctypes path raises them
  if (rc == -1 || rc == -2 || rc == -3) TORCH_CHECK_VALUE(false, msg);
  TORCH_CHECK(false, msg);
}

void* stream_of(const torch::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

struct LIFTunedRC : public torch::autograd::Function<LIFTunedRC> {
  // I [T, N] fp32 (any layout), u0 [N] fp32 contiguous, hdr: the counters header of the
  // starts-only forward (its bounded hand-off waits count give-ups there), C the chunk length.
  static torch::Tensor forward(AutogradContext* ctx, const torch::Tensor& I_in,
                               const torch::Tensor& u0, double beta, double theta, double u_r,
                               double alpha, const torch::Tensor& hdr, int64_t C) {
    TORCH_CHECK(g_fwd && g_bwd, "lifscan ops: entry points not set");
    TORCH_CHECK_VALUE(I_in.dim() == 2 && I_in.is_cuda() && I_in.scalar_type() == torch::kFloat32,
                      "I must be a float32 [T, N] GPU tensor");
    const torch::Tensor I = I_in.contiguous();
    const int64_t T = I.size(0), N = I.size(1);
    TORCH_CHECK_VALUE(u0.dim() == 1 && u0.size(0) == N && u0.is_contiguous() &&
                          u0.scalar_type() == torch::kFloat32 && u0.device() == I.device(),
                      "u0 must be a float32 [N] tensor on I's device");
    TORCH_CHECK_VALUE(C > 0 && T % C == 0, "T must be a multiple of the chunk length");
    auto S = torch::empty_like(I);
    auto ST = torch::empty({T / C, N}, I.options());
    check(g_fwd(I.data_ptr<float>(), u0.data_ptr<float>(), ST.data_ptr<float>(), S.data_ptr<float>(),
                T, N, (float)beta, (float)theta, (float)u_r, (int)C, hdr.data_ptr(),
                (size_t)hdr.numel(), stream_of(I)),
          "lsh_lif_scan_exact_fwd_starts");
    ctx->save_for_backward({I, ST});
    ctx->saved_data["beta"] = beta;
    ctx->saved_data["theta"] = theta;
    ctx->saved_data["u_r"] = u_r;
    ctx->saved_data["alpha"] = alpha;
    ctx->saved_data["C"] = C;
    return S;
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const torch::Tensor& I = saved[0];
    const torch::Tensor& ST = saved[1];
    const double beta = ctx->saved_data["beta"].toDouble();
    const double theta = ctx->saved_data["theta"].toDouble();
    const double u_r = ctx->saved_data["u_r"].toDouble();
    const double alpha = ctx->saved_data["alpha"].toDouble();
    const int64_t C = ctx->saved_data["C"].toInt();
    const torch::Tensor gS = grads[0].contiguous();
    const int64_t T = I.size(0), N = I.size(1);
    auto Lam = torch::empty_like(I);
    check(g_bwd(I.data_ptr<float>(), ST.data_ptr<float>(), gS.data_ptr<float>(),
                Lam.data_ptr<float>(), nullptr, T, N, (float)beta, (float)theta, (float)u_r,
                (float)alpha, (int)C, stream_of(I)),
          "lsh_lif_scan_fused_bwd_starts");
    torch::Tensor du0;
    if (ctx->needs_input_grad(1)) du0 = Lam[0] * (float)beta;  // dL/du0 = beta * Lam[0]
    return {Lam, du0, torch::Tensor(), torch::Tensor(), torch::Tensor(), torch::Tensor(),
            torch::Tensor(), torch::Tensor()};
  }
};

torch::Tensor lif_tuned_rc(const torch::Tensor& I, const torch::Tensor& u0, double beta,
                           double theta, double u_r, double alpha, const torch::Tensor& hdr,
                           int64_t C) {
  return LIFTunedRC::apply(I, u0, beta, theta, u_r, alpha, hdr, C);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "C++ autograd function of lif_tuned's recomputing pair over the lifscan C ABI";
  m.def("set_entry_points", &set_entry_points, "addresses of the two C-ABI entry points and of "
        "lsh_status_string");
  m.def("lif_tuned_rc", &lif_tuned_rc, "lif_tuned forward (S) with the recomputing adjoint");
}
