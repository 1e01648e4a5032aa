// PyTorch-ROCm binding of the gfx950 self-attention library (include/rk_sdpa.h).
//
// The python_extension artifact that sdpa dispatch entries name (module rk_sdpa_gfx950).  Its
// entrypoint keeps the calling convention the reference's runtime uses for native winners
// (src/radeon_kernels/providers/native.py:25 calls entrypoint(*native_arguments, **launch), and
// src/radeon_kernels/ops/sdpa/api.py:98 builds native_arguments = (query, key, value, is_causal,
// scale)): it validates, allocates the output from the caching allocator on the current HIP stream,
// launches asynchronously and returns the new tensor.  No host synchronisation, no device-to-host
// reads: safe under HIP graph capture.
//
// The kernels (sdpa_gfx950.hip) are linked into this module, so it depends on no other file of the
// pack and the digest a dispatch entry pins for it covers the kernels it runs.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <cmath>
#include <string>

#include "rk_sdpa.h"

namespace {

void check_data(const at::Tensor& t, const char* name) {
  TORCH_CHECK_VALUE(t.is_cuda(), name, " must be a ROCm tensor");
  TORCH_CHECK_VALUE(t.dim() == 4, name, " must be rank 4");
  TORCH_CHECK_VALUE(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK_TYPE(t.scalar_type() == at::kHalf || t.scalar_type() == at::kBFloat16, name, " must use FP16 or BF16");
}

at::Tensor forward(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value, bool is_causal,
                   double scale) {
  check_data(query, "query");
  check_data(key, "key");
  check_data(value, "value");
  const auto device = query.device();
  TORCH_CHECK_VALUE(key.device() == device && value.device() == device, "all tensors must be on the query device");
  TORCH_CHECK_TYPE(key.scalar_type() == query.scalar_type() && value.scalar_type() == query.scalar_type(),
                   "query, key and value dtypes must match");
  TORCH_CHECK_VALUE(key.sizes() == value.sizes(), "key and value shapes must match");
  TORCH_CHECK_VALUE(key.size(0) == query.size(0) && key.size(2) == query.size(2) && key.size(3) == query.size(3),
                    "key and value must share batch, sequence and head_dim with the query");
  TORCH_CHECK_VALUE(std::isfinite(scale) && scale > 0.0, "scale must be positive and finite");
  TORCH_CHECK_VALUE(!query.requires_grad() && !key.requires_grad() && !value.requires_grad(),
                    "sdpa is inference-only");
  c10::DeviceGuard guard(device);
  at::Tensor output = at::empty_like(query);
  const hipStream_t stream = c10::hip::getCurrentHIPStream(device.index()).stream();
  const int status = rk_sdpa_forward(query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(),
                                     query.size(0), query.size(1), key.size(1), query.size(2), query.size(3),
                                     is_causal ? 1 : 0, static_cast<float>(scale),
                                     query.scalar_type() == at::kBFloat16 ? RK_SDPA_DTYPE_BF16 : RK_SDPA_DTYPE_FP16,
                                     stream);
  if (status == RK_SDPA_ERR_INVALID_ARGUMENT || status == RK_SDPA_ERR_UNSUPPORTED) {
    TORCH_CHECK_VALUE(false, "rk_sdpa_gfx950: ", rk_sdpa_last_error());
  }
  TORCH_CHECK(status == RK_SDPA_OK, "rk_sdpa_gfx950: ", rk_sdpa_last_error());
  return output;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, module) {
  module.doc() = "gfx950 flash-attention forward (S^T and O^T on v_mfma_f32_32x32x16)";
  module.def("forward", &forward, "scaled dot-product self-attention, optional causal mask and GQA",
             py::arg("query"), py::arg("key"), py::arg("value"), py::arg("is_causal"), py::arg("scale"));
  module.def("version", []() { return std::string(rk_sdpa_version()); });
}
