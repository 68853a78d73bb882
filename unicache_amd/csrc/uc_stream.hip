// Streaming decode: one launch appends the new token(s) of a decode step to
// the residual windows of many packed segments in place, and moves each
// window past a flush the caller has just packed, by editing the device item
// table that the decode kernels read.  The host keeps no per-step table
// rebuild and copies nothing to the device.
//
// Workgroup e handles entry e: it reads its item's fields, copies the rows in
// 16-byte units (and the logical ids), then -- after a barrier, so every
// thread has read the old fields -- thread 0 writes the new lengths and
// residual pointers with ordinary vector stores.  Later kernels on the stream
// see them (kernel boundaries order global memory).
#include "uc_common.h"

namespace uc {
namespace {

constexpr int kAppendThreads = 256;
constexpr int kMaxAppendEntries = 128;

struct AppendEntry {
  int64_t item, advance;
  int64_t *ids;
};

struct AppendArgs {
  uc_kivi_item *items;
  const uint8_t *key, *value;
  const int64_t *ids;
  int64_t n, row_bytes;
  AppendEntry e[kMaxAppendEntries];
};

__global__ __launch_bounds__(kAppendThreads) void residual_append_kernel(AppendArgs a) {
  const int e = blockIdx.x, tid = threadIdx.x;
  const AppendEntry en = a.e[e];
  uc_kivi_item *it = a.items + en.item;
  const int64_t tq = it->quantized_tokens + en.advance;
  const int64_t tr = it->residual_tokens - en.advance;
  uint8_t *rk = static_cast<uint8_t *>(const_cast<void *>(it->residual_key)) + en.advance * a.row_bytes;
  uint8_t *rv = static_cast<uint8_t *>(const_cast<void *>(it->residual_value)) + en.advance * a.row_bytes;
  const int64_t units = a.n * a.row_bytes / 16;
  const uint4 *sk = reinterpret_cast<const uint4 *>(a.key + e * a.n * a.row_bytes);
  const uint4 *sv = reinterpret_cast<const uint4 *>(a.value + e * a.n * a.row_bytes);
  uint4 *dk = reinterpret_cast<uint4 *>(rk + tr * a.row_bytes);
  uint4 *dv = reinterpret_cast<uint4 *>(rv + tr * a.row_bytes);
  for (int64_t i = tid; i < units; i += kAppendThreads) {
    dk[i] = sk[i];
    dv[i] = sv[i];
  }
  if (a.ids != nullptr && en.ids != nullptr)
    for (int64_t i = tid; i < a.n; i += kAppendThreads) en.ids[tq + tr + i] = a.ids[e * a.n + i];
  __syncthreads();  // the old fields are read by every thread before they change
  if (tid == 0) {
    it->quantized_tokens = tq;
    it->residual_tokens = tr + a.n;
    it->residual_key = rk;
    it->residual_value = rv;
  }
}

}  // namespace
}  // namespace uc

using namespace uc;

extern "C" int uc_kivi_residual_append(uc_kivi_item *items_device, const uc_append_entry *entries_host,
                                       int n_entries, const void *key, const void *value, const int64_t *ids,
                                       int64_t n_tokens, int64_t heads_kv, int64_t head_dim, int dtype,
                                       uc_stream_t stream) {
  clear_error();
  UC_REQUIRE(n_entries >= 0 && n_entries <= kMaxAppendEntries, "uc_kivi_residual_append: 0..%d entries (got %d)",
             kMaxAppendEntries, n_entries);
  if (n_entries == 0) return UC_OK;
  UC_REQUIRE(items_device != nullptr && entries_host != nullptr, "uc_kivi_residual_append: NULL table or entries");
  UC_REQUIRE(n_tokens >= 0 && heads_kv > 0 && head_dim > 0, "uc_kivi_residual_append: bad shape");
  UC_REQUIRE(dtype == UC_BF16 || dtype == UC_FP16, "uc_kivi_residual_append: residual rows must be bf16 or fp16");
  const int64_t row_bytes = heads_kv * head_dim * 2;
  UC_REQUIRE(row_bytes % 16 == 0, "uc_kivi_residual_append: a row (heads_kv * head_dim * 2 bytes) must be a "
             "multiple of 16 bytes");
  UC_REQUIRE(n_tokens == 0 || (key != nullptr && value != nullptr &&
                               ((reinterpret_cast<uintptr_t>(key) | reinterpret_cast<uintptr_t>(value)) & 15) == 0),
             "uc_kivi_residual_append: key/value must be 16-byte aligned");
  AppendArgs a{};
  a.items = items_device;
  a.key = static_cast<const uint8_t *>(key);
  a.value = static_cast<const uint8_t *>(value);
  a.ids = ids;
  a.n = n_tokens;
  a.row_bytes = row_bytes;
  for (int i = 0; i < n_entries; ++i) {
    const uc_append_entry &en = entries_host[i];
    UC_REQUIRE(en.item >= 0 && en.advance >= 0, "uc_kivi_residual_append: negative item or advance");
    for (int j = 0; j < i; ++j)
      UC_REQUIRE(entries_host[j].item != en.item, "uc_kivi_residual_append: item %lld listed twice",
                 (long long)en.item);
    a.e[i] = AppendEntry{en.item, en.advance, en.ids};
  }
  hipLaunchKernelGGL(residual_append_kernel, dim3(n_entries), dim3(kAppendThreads), 0, as_stream(stream), a);
  return check_launch("uc_kivi_residual_append");
}
