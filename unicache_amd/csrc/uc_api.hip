// Error state, version and workspace sizing of the C ABI.
#include "uc_common.h"
#include "uc_decode.h"

namespace uc {

int64_t h2o_mfma_workspace_bytes(int64_t heads_q, int64_t query_len, int64_t tokens);

namespace {
thread_local std::string g_last_error;
}

void set_error(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
    return UC_ERUNTIME;
  }
  clear_error();
  return UC_OK;
}

}  // namespace uc

extern "C" int uc_abi_version(void) { return UC_ABI_VERSION; }

extern "C" const char *uc_last_error(void) { return uc::g_last_error.c_str(); }

extern "C" int64_t uc_workspace_bytes(int op, int64_t n_items, int64_t heads_q, int64_t query_len,
                                      int64_t head_dim, int64_t max_tokens) {
  if (n_items < 0 || heads_q < 0 || query_len < 0 || head_dim < 0 || max_tokens < 0) return -1;
  switch (op) {
    case UC_OP_KIVI_AV: {
      int64_t splits = uc::av_num_splits(heads_q, query_len, max_tokens);
      // per (item, query head, query row, split): D partial outputs + (max, sum);
      // dense MFMA path: V transposed, [KV heads <= query heads][D][tokens rounded up to 64] 16-bit
      const int64_t partials = n_items * heads_q * query_len * splits * (head_dim + 2) * int64_t(sizeof(float));
      // (taken only with >= 64 query rows per KV head, so only when heads_q * query_len >= 64)
      const int64_t staged = heads_q * query_len >= 64
                                 ? n_items * heads_q * head_dim * uc::ceil_div(max_tokens, int64_t(64)) * 64 * 2
                                 : 0;
      return partials > staged ? partials : staged;
    }
    case UC_OP_H2O_SCORES: {
      // generic path: per (query head, row) the softmax max and sum; MFMA path:
      // per (query row block, KV head) a partial score for every key
      const int64_t stats = heads_q * query_len * 2 * int64_t(sizeof(float));
      const int64_t partial = uc::h2o_mfma_workspace_bytes(heads_q, query_len, max_tokens);
      return stats > partial ? stats : partial;
    }
    default:
      return -1;
  }
}

extern "C" int64_t uc_kivi_decode_workspace_bytes(int64_t n_items, int bits, int group_size, int64_t heads_q,
                                                  int64_t heads_kv, int64_t head_dim, int64_t query_len,
                                                  int64_t max_quantized_tokens, int64_t max_residual_tokens) {
  if (n_items < 0 || heads_q <= 0 || heads_kv <= 0 || head_dim <= 0 || query_len <= 0 ||
      max_quantized_tokens < 0 || max_residual_tokens < 0)
    return -1;
  const int64_t rows = (heads_q / heads_kv) * query_len;
  if (uc::decode_mfma_supported(bits, group_size, head_dim, rows)) {
    const int64_t splits = uc::decode_mfma_num_splits(bits, uc::kDecodeMfmaNst, max_quantized_tokens,
                                                      max_residual_tokens);
    return uc::decode_mfma_workspace_bytes(n_items, heads_kv, splits);
  }
  const int64_t splits = uc::ceil_div(max_quantized_tokens, uc::kDecodeSplitTokens) +
                         uc::ceil_div(max_residual_tokens, uc::kDecodeSplitTokens);
  return n_items * heads_q * query_len * splits * (head_dim + 2) * int64_t(sizeof(float));
}
