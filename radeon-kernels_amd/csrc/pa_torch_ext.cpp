// PyTorch-ROCm binding of the gfx950 paged-attention decode library (include/rk_paged_attention.h).
//
// This is the python_extension artifact that dispatch entries name.  Its entrypoints keep the
// calling convention of the reference bindings (benchmarks/paged_attention/native_paged_attention.hip:244-283,
// invoked by src/radeon_kernels/providers/native.py:25 as entrypoint(q, k, v, bt, cl, scale, **launch)):
// they validate, allocate the output (and the split-K workspace) from the caching allocator on the
// current HIP stream, launch asynchronously and return the new tensor.  No host synchronisation,
// no device-to-host reads: safe under HIP graph capture.
//
// The launch parameter `merge` picks how split-K partition records are merged:
//   "reduce"  the two-launch form (rk_pa_decode): partition kernel, then the reduce kernel;
//   "fused"   the single-launch form (rk_pa_decode_fused): the partition kernel's last workgroup per
//             (sequence, head slot) merges; it saves the reduce launch but every workgroup then
//             waits for its records' write-through and one counter round trip before it exits;
//   "auto"    fused: 8-9% faster on 256-workgroup grids, where the saved launch dominates, and 1%
//             faster on the 128-sequence ragged workload's 8192 work items, which run on the
//             work-queue schedule (the grid schedule there was 0.5% slower fused than reduce).
// The fused form's arrival counters live in one zero-initialised buffer per (device, stream),
// created on first use and kept for the life of the process; every completed call leaves it zero
// for the next call on that stream.  Calls made while the stream is being captured into a graph
// always use the two-launch form, which needs no state that outlives the call.
//
// The launch parameter `grow_partitions` (default false) sets RK_PA_PARTITION_GROW: partition_tokens
// is then the smallest partition size, and on the work-queue schedule the kernel doubles it while
// its square stays within 1440 times the context tokens per workgroup, from the live context lengths.
//
// decode_append_mfma (no reference counterpart) is one serving step in the decode's launch: it
// stores each sequence's new token (position context_length - 1) into the caches in place and
// returns the decode of the updated context, bit-identical to kv_cache_append then decode_mfma.
//
// The kernels (pa_decode_gfx950.hip) are linked into this module, so it depends on no other file
// of the pack and the digest a dispatch entry pins for it covers the kernels it runs.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "rk_paged_attention.h"

namespace {

void check_data(const at::Tensor& t, const char* name, int64_t rank) {
  TORCH_CHECK_VALUE(t.is_cuda(), name, " must be a ROCm tensor");
  TORCH_CHECK_VALUE(t.dim() == rank, name, " must be rank ", rank);
  TORCH_CHECK_VALUE(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK_TYPE(t.scalar_type() == at::kHalf || t.scalar_type() == at::kBFloat16, name,
                   " must use FP16 or BF16");
}

void check_index(const at::Tensor& t, const char* name, int64_t rank) {
  TORCH_CHECK_VALUE(t.is_cuda(), name, " must be a ROCm tensor");
  TORCH_CHECK_VALUE(t.dim() == rank, name, " must be rank ", rank);
  TORCH_CHECK_VALUE(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK_TYPE(t.scalar_type() == at::kInt || t.scalar_type() == at::kLong, name,
                   " must use INT32 or INT64");
}

void raise_status(int status) {
  const std::string message = rk_pa_last_error();
  if (status == RK_ERR_INVALID_ARGUMENT || status == RK_ERR_UNSUPPORTED) {
    TORCH_CHECK_VALUE(false, "rk_pa_gfx950: ", message);
  }
  TORCH_CHECK(false, "rk_pa_gfx950: ", message);
}

// Zeroed arrival counters for fused launches on `stream`, at least `words` long.  A buffer is only
// ever used on the stream it is keyed by, so calls on one stream (stream-ordered) never overlap on
// it.  Growing allocates a fresh zeroed buffer on that stream; the old one returns to the caching
// allocator in stream order.
uint32_t* stream_counters(const at::Tensor& like, hipStream_t stream, size_t words) {
  constexpr int64_t kMinWords = 1 << 16;
  static std::mutex mutex;
  static auto* buffers = new std::map<std::pair<int, hipStream_t>, at::Tensor>();  // never freed
  std::lock_guard<std::mutex> lock(mutex);
  at::Tensor& buffer = (*buffers)[{like.device().index(), stream}];
  if (!buffer.defined() || static_cast<size_t>(buffer.numel()) < words) {
    const int64_t n = std::max<int64_t>(kMinWords, static_cast<int64_t>(words));
    buffer = at::zeros({n}, like.options().dtype(at::kInt));
  }
  return reinterpret_cast<uint32_t*>(buffer.data_ptr<int32_t>());
}

bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  TORCH_CHECK(hipStreamIsCapturing(stream, &status) == hipSuccess, "rk_pa_gfx950: hipStreamIsCapturing failed");
  return status != hipStreamCaptureStatusNone;
}

bool fused_merge_requested(const std::string& merge) {
  if (merge == "fused") return true;
  if (merge == "reduce") return false;
  TORCH_CHECK_VALUE(merge == "auto", "rk_pa_gfx950: merge must be \"auto\", \"fused\" or \"reduce\" (got \"",
                    merge, "\")");
  return true;
}

// new_key / new_value: undefined for a plain decode; for append-and-decode the [batch, kv_heads,
// head_dim] rows of each sequence's new token (rk_pa_decode_append).
at::Tensor decode(const at::Tensor& query, const at::Tensor& key_cache,
                  const at::Tensor& value_cache, const at::Tensor& block_tables,
                  const at::Tensor& context_lengths, double scale, int64_t partition_tokens,
                  const std::string& merge, int variant, const at::Tensor& new_key = at::Tensor(),
                  const at::Tensor& new_value = at::Tensor()) {
  check_data(query, "query", 3);
  check_data(key_cache, "key_cache", 4);
  check_data(value_cache, "value_cache", 4);
  check_index(block_tables, "block_tables", 2);
  check_index(context_lengths, "context_lengths", 1);
  const auto device = query.device();
  TORCH_CHECK_VALUE(key_cache.device() == device && value_cache.device() == device &&
                        block_tables.device() == device && context_lengths.device() == device,
                    "all tensors must be on the query device");
  TORCH_CHECK_TYPE(key_cache.scalar_type() == query.scalar_type() &&
                       value_cache.scalar_type() == query.scalar_type(),
                   "query and cache dtypes must match");
  TORCH_CHECK_TYPE(block_tables.scalar_type() == context_lengths.scalar_type(),
                   "index dtypes must match");
  TORCH_CHECK_VALUE(key_cache.sizes() == value_cache.sizes(), "K/V cache shapes must match");
  TORCH_CHECK_VALUE(block_tables.size(0) == query.size(0), "block table batch must match query");
  TORCH_CHECK_VALUE(context_lengths.size(0) == query.size(0),
                    "context length batch must match query");
  TORCH_CHECK_VALUE(query.size(2) == key_cache.size(3),
                    "query and cache head dimensions must match");
  TORCH_CHECK_VALUE(std::isfinite(scale) && scale > 0.0, "scale must be positive and finite");
  TORCH_CHECK_VALUE(!query.requires_grad() && !key_cache.requires_grad() &&
                        !value_cache.requires_grad(),
                    "paged attention decode is inference-only");

  const bool append = new_key.defined();
  if (append) {
    check_data(new_key, "new_key", 3);
    check_data(new_value, "new_value", 3);
    TORCH_CHECK_VALUE(new_key.device() == device && new_value.device() == device,
                      "all tensors must be on the query device");
    TORCH_CHECK_TYPE(new_key.scalar_type() == query.scalar_type() &&
                         new_value.scalar_type() == query.scalar_type(),
                     "new_key, new_value and query dtypes must match");
    TORCH_CHECK_VALUE(new_key.sizes() == new_value.sizes() && new_key.size(0) == query.size(0) &&
                          new_key.size(1) == key_cache.size(2) && new_key.size(2) == key_cache.size(3),
                      "new_key and new_value must have shape [batch, kv_heads, head_dim]");
  }
  const int64_t batch = query.size(0);
  const int64_t query_heads = query.size(1);
  const int64_t head_dim = query.size(2);
  const int64_t num_blocks = key_cache.size(0);
  const int64_t block_size = key_cache.size(1);
  const int64_t kv_heads = key_cache.size(2);
  const int64_t max_blocks = block_tables.size(1);
  const int dtype = query.scalar_type() == at::kBFloat16 ? RK_DTYPE_BF16 : RK_DTYPE_FP16;
  const int index_dtype = block_tables.scalar_type() == at::kLong ? RK_INDEX_INT64 : RK_INDEX_INT32;

  size_t workspace_bytes = 0;
  int status = rk_pa_decode_workspace_bytes(batch, query_heads, head_dim, block_size, max_blocks,
                                            partition_tokens, &workspace_bytes);
  if (status != RK_OK) raise_status(status);

  at::DeviceGuard guard(device);
  at::Tensor output = at::empty_like(query);
  at::Tensor workspace;
  void* workspace_ptr = nullptr;
  if (workspace_bytes > 0) {
    workspace = at::empty({static_cast<int64_t>(workspace_bytes)}, query.options().dtype(at::kByte));
    workspace_ptr = workspace.data_ptr();
  }
  hipStream_t stream = c10::hip::getCurrentHIPStream(device.index()).stream();
  size_t words = 0;
  status = rk_pa_decode_counter_words(batch, query_heads, kv_heads, &words);
  if (status != RK_OK) raise_status(status);
  const bool fused = fused_merge_requested(merge);
  if (append) {
    uint32_t* counters = fused && workspace_bytes > 0 && !capturing(stream) ? stream_counters(query, stream, words)
                                                                            : nullptr;
    status = rk_pa_decode_append(query.data_ptr(), new_key.data_ptr(), new_value.data_ptr(),
                                 key_cache.data_ptr(), value_cache.data_ptr(), block_tables.data_ptr(),
                                 context_lengths.data_ptr(), output.data_ptr(), workspace_ptr,
                                 workspace_bytes, counters, counters != nullptr ? words : 0, batch,
                                 query_heads, kv_heads, head_dim, num_blocks, block_size, max_blocks,
                                 static_cast<float>(scale), dtype, index_dtype, partition_tokens, variant,
                                 stream);
  } else if (fused && workspace_bytes > 0 && !capturing(stream)) {
    uint32_t* counters = stream_counters(query, stream, words);
    status = rk_pa_decode_fused(query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                                block_tables.data_ptr(), context_lengths.data_ptr(), output.data_ptr(),
                                workspace_ptr, workspace_bytes, counters, words, batch, query_heads,
                                kv_heads, head_dim, num_blocks, block_size, max_blocks,
                                static_cast<float>(scale), dtype, index_dtype, partition_tokens, variant,
                                stream);
  } else {
    status = rk_pa_decode(query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                          block_tables.data_ptr(), context_lengths.data_ptr(), output.data_ptr(),
                          workspace_ptr, workspace_bytes, batch, query_heads, kv_heads, head_dim,
                          num_blocks, block_size, max_blocks, static_cast<float>(scale), dtype,
                          index_dtype, partition_tokens, variant, stream);
  }
  if (status != RK_OK) raise_status(status);
  return output;
}

int grow_bits(bool grow_partitions) { return grow_partitions ? RK_PA_PARTITION_GROW : 0; }

at::Tensor decode_mfma(const at::Tensor& query, const at::Tensor& key_cache,
                       const at::Tensor& value_cache, const at::Tensor& block_tables,
                       const at::Tensor& context_lengths, double scale, int64_t partition_tokens,
                       const std::string& merge, bool grow_partitions) {
  return decode(query, key_cache, value_cache, block_tables, context_lengths, scale,
                partition_tokens, merge, RK_PA_VARIANT_MFMA | grow_bits(grow_partitions));
}

at::Tensor decode_valu(const at::Tensor& query, const at::Tensor& key_cache,
                       const at::Tensor& value_cache, const at::Tensor& block_tables,
                       const at::Tensor& context_lengths, double scale, int64_t partition_tokens,
                       const std::string& merge, bool grow_partitions) {
  return decode(query, key_cache, value_cache, block_tables, context_lengths, scale,
                partition_tokens, merge, RK_PA_VARIANT_VALU | grow_bits(grow_partitions));
}

at::Tensor decode_mfma_qk(const at::Tensor& query, const at::Tensor& key_cache,
                          const at::Tensor& value_cache, const at::Tensor& block_tables,
                          const at::Tensor& context_lengths, double scale, int64_t partition_tokens,
                          const std::string& merge, bool grow_partitions) {
  return decode(query, key_cache, value_cache, block_tables, context_lengths, scale,
                partition_tokens, merge, RK_PA_VARIANT_MFMA_QK | grow_bits(grow_partitions));
}

// Append-and-decode: writes each sequence's new token into the caches (in place) and returns the
// decode of the updated context, as kv_cache_append followed by decode_mfma would.
at::Tensor decode_append_mfma(const at::Tensor& query, const at::Tensor& new_key,
                              const at::Tensor& new_value, const at::Tensor& key_cache,
                              const at::Tensor& value_cache, const at::Tensor& block_tables,
                              const at::Tensor& context_lengths, double scale, int64_t partition_tokens,
                              const std::string& merge, bool grow_partitions) {
  return decode(query, key_cache, value_cache, block_tables, context_lengths, scale, partition_tokens,
                merge, RK_PA_VARIANT_MFMA | grow_bits(grow_partitions), new_key, new_value);
}

}  // namespace

PYBIND11_MODULE(rk_pa_gfx950, module) {
  module.doc() = "gfx950 split-K paged-attention decode (QK^T and PV on MFMA or on fp32 FMAs)";
  module.def("decode_mfma", &decode_mfma, "paged decode, QK^T and PV on MFMA", py::arg("query"),
             py::arg("key_cache"), py::arg("value_cache"), py::arg("block_tables"),
             py::arg("context_lengths"), py::arg("scale"), py::kw_only(),
             py::arg("partition_tokens") = 512, py::arg("merge") = "auto",
             py::arg("grow_partitions") = false);
  module.def("decode_append_mfma", &decode_append_mfma,
             "append each sequence's new token to the paged caches, then paged decode (one launch)",
             py::arg("query"), py::arg("new_key"), py::arg("new_value"), py::arg("key_cache"),
             py::arg("value_cache"), py::arg("block_tables"), py::arg("context_lengths"), py::arg("scale"),
             py::kw_only(), py::arg("partition_tokens") = 512, py::arg("merge") = "auto",
             py::arg("grow_partitions") = false);
  module.def("decode_mfma_qk", &decode_mfma_qk, "paged decode, QK^T on MFMA, PV on fp32 FMAs", py::arg("query"),
             py::arg("key_cache"), py::arg("value_cache"), py::arg("block_tables"),
             py::arg("context_lengths"), py::arg("scale"), py::kw_only(),
             py::arg("partition_tokens") = 512, py::arg("merge") = "auto",
             py::arg("grow_partitions") = false);
  module.def("decode_valu", &decode_valu, "paged decode, QK^T on fp32 FMAs", py::arg("query"),
             py::arg("key_cache"), py::arg("value_cache"), py::arg("block_tables"),
             py::arg("context_lengths"), py::arg("scale"), py::kw_only(),
             py::arg("partition_tokens") = 512, py::arg("merge") = "auto",
             py::arg("grow_partitions") = false);
  module.def("version", []() { return std::string(rk_pa_version()); });
}
