// Log-sum-exp merge of normalised attention summaries over disjoint key
// segments (adapters/bagel.py:57-72).
#include "uc_common.h"

namespace uc {
namespace {

constexpr int kMaxSegments = 16;

struct MergeArgs {
  const void *outs[kMaxSegments];
  const float *lses[kMaxSegments];
  int n;
  int64_t Lq, Hq, D;
  void *out;
  float *out_lse;
};

// One workgroup per (query head, query row).  Follows torch.logsumexp: the
// max is taken over segments and replaced by 0 when infinite, then
// lse = log(sum exp(l_s - m)) + m; the output accumulates
// out_s * exp(l_s - lse) in segment order starting from zero.
template <int OD>
__global__ __launch_bounds__(128) void lse_merge_kernel(MergeArgs a) {
  const int64_t hq = blockIdx.x / a.Lq, i = blockIdx.x % a.Lq;
  float l[kMaxSegments];
  float m = -__builtin_huge_valf();
  for (int s = 0; s < a.n; ++s) {
    l[s] = a.lses[s][hq * a.Lq + i];
    m = fmaxf(m, l[s]);
  }
  if (fabsf(m) == __builtin_huge_valf()) m = 0.0f;
  float sum = 0.0f;
  for (int s = 0; s < a.n; ++s) sum = add_rn(sum, expf(sub_rn(l[s], m)));
  const float total = add_rn(logf(sum), m);
  float w[kMaxSegments];
  for (int s = 0; s < a.n; ++s) w[s] = expf(sub_rn(l[s], total));
  for (int64_t d = threadIdx.x; d < a.D; d += blockDim.x) {
    const int64_t off = (i * a.Hq + hq) * a.D + d;
    float o = 0.0f;
    for (int s = 0; s < a.n; ++s) o = add_rn(o, mul_rn(load_as_f32<OD>(a.outs[s], off), w[s]));
    store_from_f32<OD>(a.out, off, o);
  }
  if (threadIdx.x == 0 && a.out_lse != nullptr) a.out_lse[hq * a.Lq + i] = total;
}

// Segment weights of one (query head, row): the lse and w of lse_merge_kernel.
__device__ __forceinline__ float merge_weights(const MergeArgs &a, int64_t li, float (&w)[kMaxSegments]) {
  float l[kMaxSegments];
  float m = -__builtin_huge_valf();
  for (int s = 0; s < a.n; ++s) {
    l[s] = a.lses[s][li];
    m = fmaxf(m, l[s]);
  }
  if (fabsf(m) == __builtin_huge_valf()) m = 0.0f;
  float sum = 0.0f;
  for (int s = 0; s < a.n; ++s) sum = add_rn(sum, expf(sub_rn(l[s], m)));
  const float total = add_rn(logf(sum), m);
  for (int s = 0; s < a.n; ++s) w[s] = expf(sub_rn(l[s], total));
  return total;
}

// Rows as whole 16-byte chunks (8 half or 4 float channels per thread, chunks
// of a row on neighbouring lanes); every thread of a row recomputes its
// weights.  The same arithmetic per element as lse_merge_kernel.
template <int OD>
__global__ __launch_bounds__(256) void lse_merge_vec_kernel(MergeArgs a) {
  constexpr int CH = OD == UC_FP32 ? 4 : 8;
  const int64_t chunks = a.D / CH;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= a.Lq * a.Hq * chunks) return;
  // row = i * Hq + hq (memory order of out); 32-bit divisions: the launch
  // keeps the index below 2^31
  const uint32_t i32 = static_cast<uint32_t>(idx), c32 = static_cast<uint32_t>(chunks);
  const uint32_t hq32 = static_cast<uint32_t>(a.Hq), r32 = i32 / c32, q32 = r32 / hq32;
  const int64_t c = i32 - r32 * c32, row = r32;
  const int64_t i = q32, hq = r32 - q32 * hq32;
  float w[kMaxSegments];
  const float total = merge_weights(a, hq * a.Lq + i, w);
  const int64_t off = row * a.D + c * CH;
  float o[CH];
#pragma unroll
  for (int e = 0; e < CH; ++e) o[e] = 0.0f;
  for (int s = 0; s < a.n; ++s) {
    const uint4 raw = *reinterpret_cast<const uint4 *>(static_cast<const char *>(a.outs[s]) +
                                                      off * (OD == UC_FP32 ? 4 : 2));
    const uint32_t r4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int e = 0; e < CH; ++e) {
      float x;
      if constexpr (OD == UC_FP32) x = __uint_as_float(r4[e]);
      else x = half_bits_to_f32<OD>(r4[e / 2] >> (16 * (e % 2)));
      o[e] = add_rn(o[e], mul_rn(x, w[s]));
    }
  }
  uint32_t r4[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (OD == UC_FP32) {
      r4[q] = __float_as_uint(o[q]);
    } else {
      const uint32_t lo = OD == UC_BF16 ? f32_to_bf16_bits(o[2 * q]) : f32_to_f16_bits(o[2 * q]);
      const uint32_t hi = OD == UC_BF16 ? f32_to_bf16_bits(o[2 * q + 1]) : f32_to_f16_bits(o[2 * q + 1]);
      r4[q] = lo | (hi << 16);
    }
  }
  *reinterpret_cast<uint4 *>(static_cast<char *>(a.out) + off * (OD == UC_FP32 ? 4 : 2)) =
      make_uint4(r4[0], r4[1], r4[2], r4[3]);
  if (c == 0 && a.out_lse != nullptr) a.out_lse[hq * a.Lq + i] = total;
}

}  // namespace
}  // namespace uc

using namespace uc;

extern "C" int uc_lse_merge(const void *const *outs, const float *const *lses, int n_segments, int out_dtype,
                            int64_t query_len, int64_t heads_q, int64_t head_dim, void *out, float *out_lse,
                            uc_stream_t stream) {
  UC_REQUIRE(n_segments >= 1, "At least one attention summary is required");
  UC_REQUIRE(n_segments <= kMaxSegments, "uc_lse_merge: at most %d segments", kMaxSegments);
  UC_REQUIRE(valid_dtype(out_dtype), "uc_lse_merge: unknown dtype code");
  UC_REQUIRE(outs != nullptr && lses != nullptr && out != nullptr, "uc_lse_merge: NULL pointer");
  UC_REQUIRE(query_len >= 0 && heads_q >= 0 && head_dim >= 0, "uc_lse_merge: bad shape");
  if (query_len == 0 || heads_q == 0) return UC_OK;
  MergeArgs a{};
  for (int s = 0; s < n_segments; ++s) {
    UC_REQUIRE(outs[s] != nullptr && lses[s] != nullptr, "uc_lse_merge: NULL segment pointer");
    a.outs[s] = outs[s];
    a.lses[s] = lses[s];
  }
  a.n = n_segments; a.Lq = query_len; a.Hq = heads_q; a.D = head_dim; a.out = out; a.out_lse = out_lse;
  hipStream_t s = as_stream(stream);
  const int ch = out_dtype == UC_FP32 ? 4 : 8;
  bool vec = head_dim % ch == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  for (int i = 0; i < n_segments; ++i) vec = vec && (reinterpret_cast<uintptr_t>(outs[i]) & 15) == 0;
  if (vec) {
    const int64_t n = query_len * heads_q * (head_dim / ch);
    UC_REQUIRE(n < (int64_t(1) << 31), "uc_lse_merge: too many elements for one call");
    UC_DISPATCH_DTYPE(out_dtype, OD, [&] {
      hipLaunchKernelGGL((lse_merge_vec_kernel<OD>), dim3(ceil_div(n, int64_t(256))), dim3(256), 0, s, a);
    });
    return check_launch("uc_lse_merge");
  }
  UC_DISPATCH_DTYPE(out_dtype, OD, [&] {
    hipLaunchKernelGGL((lse_merge_kernel<OD>), dim3(heads_q * query_len), dim3(128), 0, s, a);
  });
  return check_launch("uc_lse_merge");
}
