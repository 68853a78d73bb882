// Split-K geometry shared by the decode kernels and uc_workspace_bytes.
#pragma once
#include <stdint.h>

namespace uc {

// Tokens handled by one split-K workgroup of the decode kernels.
constexpr int64_t kDecodeSplitTokens = 512;

// Upper bound of split count for an item of `max_tokens` = Tq + Tr keys:
// ceil(Tq/S) + ceil(Tr/S) <= ceil((Tq+Tr)/S) + 1.
inline int64_t decode_num_splits(int64_t max_tokens) {
  return (max_tokens + kDecodeSplitTokens - 1) / kDecodeSplitTokens + 1;
}

}  // namespace uc
