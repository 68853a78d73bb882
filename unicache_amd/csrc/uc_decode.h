// Split-K geometry shared by the decode kernels and uc_workspace_bytes.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/unicache_hip.h"

namespace uc {

// Tokens handled by one split-K workgroup of the decode kernels.
constexpr int64_t kDecodeSplitTokens = 512;

// Upper bound of split count for an item of `max_tokens` = Tq + Tr keys:
// ceil(Tq/S) + ceil(Tr/S) <= ceil((Tq+Tr)/S) + 1.
inline int64_t decode_num_splits(int64_t max_tokens) {
  return (max_tokens + kDecodeSplitTokens - 1) / kDecodeSplitTokens + 1;
}

// uc_kivi_av (probabilities given): calls with few query rows (decode-like,
// heads_q * query_len <= 64) split every 64 keys so a short segment still
// spreads over the CUs; longer calls keep kDecodeSplitTokens.
inline int64_t av_split_tokens(int64_t heads_q, int64_t query_len) {
  return heads_q * query_len <= 64 ? 64 : kDecodeSplitTokens;
}
inline int64_t av_num_splits(int64_t heads_q, int64_t query_len, int64_t max_tokens) {
  const int64_t s = av_split_tokens(heads_q, query_len);
  return (max_tokens + s - 1) / s + 1;
}

// attention_parts over the kernel-native 2/4-bit layout (uc_parts.hip).
bool parts_fast_supported(int bits, int group, int64_t head_dim, int stats_dtype, int res_dtype, int64_t r_st,
                          int64_t r_sh, const void *residual, int64_t residual_tokens);
int launch_parts_qk(const void *query, int q_dtype, int64_t Lq, int64_t Hq, const void *kc, const void *ks,
                    const void *km, int sd, int64_t Tq, int64_t cap, int bits, int G, const void *rk, int rd,
                    int64_t Tr, int64_t r_st, int64_t r_sh, int64_t Hkv, float sm_scale, float *logits,
                    hipStream_t stream);
int launch_parts_av(const void *probs, int p_dtype, int64_t p_sh, int64_t p_si, int64_t p_st, int64_t Lq, int64_t Hq,
                    const void *vc, const void *vs, const void *vm, int sd, int64_t Tq, int64_t cap, int bits, int G,
                    const void *rv, int rd, int64_t Tr, int64_t r_st, int64_t r_sh, int64_t Hkv, void *out, int od,
                    void *workspace, int64_t split_tokens, hipStream_t stream);

// MFMA decode (uc_decode_mfma.hip): head_dim 128, 2/4-bit codes.
#ifndef UC_DECODE_MFMA_NST
#define UC_DECODE_MFMA_NST 8
#endif
constexpr int64_t kDecodeMfmaNst = UC_DECODE_MFMA_NST;  // super-tiles per packed split
bool decode_mfma_supported(int bits, int group, int64_t head_dim, int64_t rows);
int64_t decode_mfma_split_tokens(int bits, int64_t nst);
int64_t decode_mfma_num_splits(int bits, int64_t nst, int64_t max_tq, int64_t max_tr);
int64_t decode_mfma_res_split_tokens(int64_t max_tr);
int64_t decode_mfma_workspace_bytes(int64_t n_items, int64_t heads_kv, int64_t splits);
int launch_decode_mfma(const uc_kivi_item *items_dev, const uc_kivi_item *single, int64_t n_items, int bits,
                       int group_size, int64_t Hq, int64_t Hkv, int64_t Lq, int q_dtype, int res_dtype,
                       int out_dtype, float sm_scale, int64_t max_tq, int64_t max_tr, int64_t nst, int64_t segs,
                       void *workspace, int64_t workspace_bytes, hipStream_t stream);

}  // namespace uc
