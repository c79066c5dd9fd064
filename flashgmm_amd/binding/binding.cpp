// pybind11 module `flash_gmm_native` over this package's two C ABIs: the
// compiled counterpart of the reference's binding (flash_gmm/csrc/binding.cpp),
// for callers that want a torch extension rather than the ctypes module
// flashgmm_amd/flash_gmm_native.py.  Same names, arguments, defaults, return
// order and TORCH_CHECK messages (binding.cpp:35-109); dispatch on X's
// device: ROCm tensors -> libflashgmm.so (HIP kernels for gfx950, torch's
// current stream, a workspace from torch's caching allocator), CPU tensors ->
// libflashgmm_cpu.so (C++/OpenMP host path, torch's intra-op thread count).
// Unlike the reference, flash_e_step runs on the GPU too.
// Built by flashgmm_amd/binding/setup.py.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include "flashgmm.h"
#include "flashgmm_cpu.h"

namespace {

using torch::Tensor;

void* stream_of(const Tensor& X) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(X.get_device()).stream());
}

void check_gpu(int rc) { TORCH_CHECK(rc == FGMM_OK, "flashgmm_amd: ", fgmm_last_error()); }
void check_cpu(int rc) {
  TORCH_CHECK(rc == FGMM_OK, "flashgmm_amd (host): ", fgmm_cpu_last_error());
}

// Shape and device checks shared by the entry points that take parameters.
void check_params(const Tensor& X, const Tensor& mu, const Tensor& var, const Tensor& lp) {
  TORCH_CHECK(X.dim() == 2, "X must be 2D");
  TORCH_CHECK(X.size(0) >= 1 && X.size(1) >= 1 && X.size(1) <= 256,
              "X must be [N, d] with N >= 1 and 1 <= d <= 256");
  const int64_t K = mu.size(0), d = X.size(1);
  TORCH_CHECK(mu.dim() == 2 && mu.size(1) == d && K >= 1, "mu must be [K, d]");
  TORCH_CHECK(var.sizes() == mu.sizes(), "var must be [K, d]");
  TORCH_CHECK(lp.dim() == 1 && lp.size(0) == K, "log_pi must be [K]");
  for (const Tensor* t : {&mu, &var, &lp}) {
    TORCH_CHECK(t->scalar_type() == torch::kFloat32, "parameters must be float32");
    TORCH_CHECK(t->device() == X.device(), "parameters must be on X's device");
  }
  TORCH_CHECK(X.is_cuda() || X.is_cpu(), "tensors must be on a ROCm device or the CPU");
}

Tensor workspace(const Tensor& X, size_t bytes) {
  TORCH_CHECK(bytes > 0, "flashgmm_amd: ", fgmm_last_error());
  return torch::empty({(int64_t)bytes}, X.options().dtype(torch::kUInt8));
}

int threads() { return std::max(1, at::get_num_threads()); }

std::vector<Tensor> e_step(Tensor X, Tensor mu, Tensor var, Tensor log_pi, bool standard) {
  check_params(X, mu, var, log_pi);
  X = X.contiguous(); mu = mu.contiguous(); var = var.contiguous(); log_pi = log_pi.contiguous();
  const int64_t N = X.size(0), d = X.size(1), K = mu.size(0);
  auto gamma = torch::empty({N, K}, X.options());
  auto ln = torch::empty({N}, X.options());
  if (X.is_cpu()) {
    check_cpu(fgmm_cpu_e_step(X.data_ptr<float>(), mu.data_ptr<float>(), var.data_ptr<float>(),
                              log_pi.data_ptr<float>(), N, K, d, threads(),
                              gamma.data_ptr<float>(), ln.data_ptr<float>()));
    return {gamma, ln};
  }
  const size_t wsb = standard ? fgmm_standard_e_step_workspace_bytes(N, K, d, FGMM_VARIANT_AUTO)
                              : fgmm_workspace_bytes(N, K, d, FGMM_VARIANT_AUTO);
  auto ws = workspace(X, wsb);
  auto fn = standard ? fgmm_standard_e_step : fgmm_flash_e_step;
  check_gpu(fn(X.data_ptr<float>(), mu.data_ptr<float>(), var.data_ptr<float>(),
               log_pi.data_ptr<float>(), N, K, d, FGMM_VARIANT_AUTO, gamma.data_ptr<float>(),
               ln.data_ptr<float>(), ws.data_ptr(), wsb, stream_of(X)));
  return {gamma, ln};
}

std::vector<Tensor> standard_e_step(Tensor X, Tensor mu, Tensor var, Tensor log_pi) {
  TORCH_CHECK(X.dtype() == torch::kFloat32, "X must be float32");
  TORCH_CHECK(X.dim() == 2, "X must be 2D");
  return e_step(X, mu, var, log_pi, true);
}

std::vector<Tensor> flash_e_step(Tensor X, Tensor mu, Tensor var, Tensor log_pi, int BK) {
  TORCH_CHECK(X.dtype() == torch::kFloat32, "X must be float32");
  TORCH_CHECK(BK >= 1, "BK must be >= 1");
  return e_step(X, mu, var, log_pi, false);
}

std::vector<Tensor> flash_em_fused(Tensor X, Tensor mu, Tensor var, Tensor log_pi, int BN,
                                   int BK) {
  TORCH_CHECK(X.dtype() == torch::kFloat32, "X must be float32");
  TORCH_CHECK(BN >= 1 && BK >= 1, "BN and BK must be >= 1");
  check_params(X, mu, var, log_pi);
  X = X.contiguous(); mu = mu.contiguous(); var = var.contiguous(); log_pi = log_pi.contiguous();
  const int64_t N = X.size(0), d = X.size(1), K = mu.size(0);
  auto opts = X.options();
  auto new_mu = torch::empty({K, d}, opts), new_var = torch::empty({K, d}, opts);
  auto new_lp = torch::empty({K}, opts), ln = torch::empty({N}, opts);
  if (X.is_cpu()) {
    check_cpu(fgmm_cpu_em_fused(X.data_ptr<float>(), mu.data_ptr<float>(),
                                var.data_ptr<float>(), log_pi.data_ptr<float>(), N, K, d,
                                threads(), new_mu.data_ptr<float>(), new_var.data_ptr<float>(),
                                new_lp.data_ptr<float>(), ln.data_ptr<float>()));
    return {new_mu, new_var, new_lp, ln};
  }
  const size_t wsb = fgmm_em_fused_workspace_bytes(N, K, d, FGMM_VARIANT_AUTO);
  auto ws = workspace(X, wsb);
  check_gpu(fgmm_em_fused(X.data_ptr<float>(), mu.data_ptr<float>(), var.data_ptr<float>(),
                          log_pi.data_ptr<float>(), N, K, d, FGMM_VARIANT_AUTO,
                          new_mu.data_ptr<float>(), new_var.data_ptr<float>(),
                          new_lp.data_ptr<float>(), ln.data_ptr<float>(), ws.data_ptr(), wsb,
                          stream_of(X)));
  return {new_mu, new_var, new_lp, ln};
}

std::vector<Tensor> standard_m_step(Tensor X, Tensor gamma) {
  TORCH_CHECK(X.dtype() == torch::kFloat32, "X must be float32");
  TORCH_CHECK(X.dim() == 2 && gamma.dim() == 2 && gamma.size(0) == X.size(0),
              "gamma must be [N, K] for X [N, d]");
  TORCH_CHECK(gamma.scalar_type() == torch::kFloat32 && gamma.device() == X.device(),
              "gamma must be float32 on X's device");
  X = X.contiguous(); gamma = gamma.contiguous();
  const int64_t N = X.size(0), d = X.size(1), K = gamma.size(1);
  auto opts = X.options();
  auto mu = torch::empty({K, d}, opts), var = torch::empty({K, d}, opts);
  auto lp = torch::empty({K}, opts);
  if (X.is_cpu()) {
    check_cpu(fgmm_cpu_standard_m_step(X.data_ptr<float>(), gamma.data_ptr<float>(), N, K, d,
                                       threads(), mu.data_ptr<float>(), var.data_ptr<float>(),
                                       lp.data_ptr<float>()));
    return {mu, var, lp};
  }
  const size_t wsb = fgmm_standard_m_step_workspace_bytes(N, K, d);
  auto ws = workspace(X, wsb);
  check_gpu(fgmm_standard_m_step(X.data_ptr<float>(), gamma.data_ptr<float>(), N, K, d,
                                 mu.data_ptr<float>(), var.data_ptr<float>(),
                                 lp.data_ptr<float>(), ws.data_ptr(), wsb, stream_of(X)));
  return {mu, var, lp};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Flash-GMM on MI355X: HIP kernels (ROCm tensors) and a C++/OpenMP host path";
  m.def("standard_e_step", &standard_e_step, "Standard E-step (materialises gamma)",
        py::arg("X"), py::arg("mu"), py::arg("var"), py::arg("log_pi"));
  m.def("flash_e_step", &flash_e_step, "Flash E-step returning gamma", py::arg("X"),
        py::arg("mu"), py::arg("var"), py::arg("log_pi"), py::arg("BK") = 4);
  m.def("flash_em_fused", &flash_em_fused, "Fused EM iteration, no N x K array",
        py::arg("X"), py::arg("mu"), py::arg("var"), py::arg("log_pi"), py::arg("BN") = 64,
        py::arg("BK") = 8);
  m.def("standard_m_step", &standard_m_step, "Standard M-step from gamma", py::arg("X"),
        py::arg("gamma"));
}
