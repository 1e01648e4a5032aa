// PyTorch-ROCm binding of the gfx950 paged KV-cache library (include/rk_kv_cache.h).
//
// The python_extension artifacts that kv_cache_append and kv_cache_copy dispatch entries name (one
// module per operator, rk_kv_append_gfx950 and rk_kv_copy_gfx950, both built from this file).  Its
// entrypoints keep the calling convention of the reference bindings
// (benchmarks/kv_cache/native_kv_cache.hip:259-298, invoked by src/radeon_kernels/providers/native.py:25
// as append(key, value, key_cache, value_cache, slot_mapping) and copy(key_cache, value_cache,
// block_mapping)): they validate, write the caches in place on the current HIP stream and return
// them.  No host synchronisation, no device-to-host reads: safe under HIP graph capture.
//
// The kernels (kv_cache_gfx950.hip) are linked into this module, so it depends on no other file of
// the pack and the digest a dispatch entry pins for it covers the kernels it runs.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <string>
#include <vector>

#include "rk_kv_cache.h"

namespace {

void check_data(const at::Tensor& t, const char* name, int64_t rank) {
  TORCH_CHECK_VALUE(t.is_cuda(), name, " must be a ROCm tensor");
  TORCH_CHECK_VALUE(t.dim() == rank, name, " must be rank ", rank);
  TORCH_CHECK_VALUE(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK_TYPE(t.scalar_type() == at::kHalf || t.scalar_type() == at::kBFloat16, name,
                   " must use FP16 or BF16");
}

std::vector<at::Tensor> append(const at::Tensor& key, const at::Tensor& value, at::Tensor key_cache,
                               at::Tensor value_cache, const at::Tensor& slot_mapping) {
  check_data(key, "key", 3);
  check_data(value, "value", 3);
  check_data(key_cache, "key_cache", 4);
  check_data(value_cache, "value_cache", 4);
  TORCH_CHECK_VALUE(slot_mapping.is_cuda() && slot_mapping.dim() == 1 && slot_mapping.is_contiguous(),
                    "slot_mapping must be a contiguous rank-1 ROCm tensor");
  TORCH_CHECK_TYPE(slot_mapping.scalar_type() == at::kInt || slot_mapping.scalar_type() == at::kLong,
                   "slot_mapping must use INT32 or INT64");
  const auto device = key.device();
  TORCH_CHECK_VALUE(value.device() == device && key_cache.device() == device &&
                        value_cache.device() == device && slot_mapping.device() == device,
                    "all tensors must be on the key device");
  TORCH_CHECK_TYPE(value.scalar_type() == key.scalar_type() &&
                       key_cache.scalar_type() == key.scalar_type() &&
                       value_cache.scalar_type() == key.scalar_type(),
                   "key, value and cache dtypes must match");
  TORCH_CHECK_VALUE(key.sizes() == value.sizes(), "key and value shapes must match");
  TORCH_CHECK_VALUE(key_cache.sizes() == value_cache.sizes(), "cache shapes must match");
  TORCH_CHECK_VALUE(key.size(0) == slot_mapping.size(0), "slot_mapping must match tokens");
  TORCH_CHECK_VALUE(key.size(1) == key_cache.size(2) && key.size(2) == key_cache.size(3),
                    "key/value shape must match cache heads and head dimension");
  c10::DeviceGuard guard(device);
  const hipStream_t stream = c10::hip::getCurrentHIPStream(device.index()).stream();
  const int status = rk_kv_cache_append(
      key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
      slot_mapping.data_ptr(), key.size(0), key.size(1), key.size(2), key_cache.size(0),
      key_cache.size(1), key.scalar_type() == at::kBFloat16 ? RK_KV_DTYPE_BF16 : RK_KV_DTYPE_FP16,
      slot_mapping.scalar_type() == at::kLong ? RK_KV_INDEX_INT64 : RK_KV_INDEX_INT32, stream);
  if (status == RK_KV_ERR_INVALID_ARGUMENT || status == RK_KV_ERR_UNSUPPORTED) {
    TORCH_CHECK_VALUE(false, "rk_kv: ", rk_kv_last_error());
  }
  TORCH_CHECK(status == RK_KV_OK, "rk_kv: ", rk_kv_last_error());
  return {key_cache, value_cache};
}

std::vector<at::Tensor> copy(at::Tensor key_cache, at::Tensor value_cache, const at::Tensor& block_mapping) {
  check_data(key_cache, "key_cache", 4);
  check_data(value_cache, "value_cache", 4);
  TORCH_CHECK_VALUE(block_mapping.is_cuda() && block_mapping.dim() == 2 && block_mapping.is_contiguous(),
                    "block_mapping must be a contiguous rank-2 ROCm tensor");
  TORCH_CHECK_TYPE(block_mapping.scalar_type() == at::kInt || block_mapping.scalar_type() == at::kLong,
                   "block_mapping must use INT32 or INT64");
  const auto device = key_cache.device();
  TORCH_CHECK_VALUE(value_cache.device() == device && block_mapping.device() == device,
                    "all tensors must be on the key_cache device");
  TORCH_CHECK_TYPE(value_cache.scalar_type() == key_cache.scalar_type(), "cache dtypes must match");
  TORCH_CHECK_VALUE(key_cache.sizes() == value_cache.sizes(), "cache shapes must match");
  TORCH_CHECK_VALUE(block_mapping.size(1) == 2, "block_mapping must have shape [pairs, 2]");
  c10::DeviceGuard guard(device);
  const hipStream_t stream = c10::hip::getCurrentHIPStream(device.index()).stream();
  const int status = rk_kv_cache_copy(
      key_cache.data_ptr(), value_cache.data_ptr(), block_mapping.data_ptr(), block_mapping.size(0),
      key_cache.size(0), key_cache.size(1), key_cache.size(2), key_cache.size(3),
      key_cache.scalar_type() == at::kBFloat16 ? RK_KV_DTYPE_BF16 : RK_KV_DTYPE_FP16,
      block_mapping.scalar_type() == at::kLong ? RK_KV_INDEX_INT64 : RK_KV_INDEX_INT32, stream);
  if (status == RK_KV_ERR_INVALID_ARGUMENT || status == RK_KV_ERR_UNSUPPORTED) {
    TORCH_CHECK_VALUE(false, "rk_kv: ", rk_kv_last_error());
  }
  TORCH_CHECK(status == RK_KV_OK, "rk_kv: ", rk_kv_last_error());
  return {key_cache, value_cache};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, module) {
  module.doc() = "gfx950 paged KV-cache append (row gather/scatter) and block copy";
  module.def("append", &append, "append token K/V rows to their paged-cache slots", py::arg("key"),
             py::arg("value"), py::arg("key_cache"), py::arg("value_cache"), py::arg("slot_mapping"));
  module.def("copy", &copy, "copy whole cache blocks (source, destination pairs)", py::arg("key_cache"),
             py::arg("value_cache"), py::arg("block_mapping"));
  module.def("version", []() { return std::string(rk_kv_version()); });
}
