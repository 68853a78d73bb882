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
  UC_DISPATCH_DTYPE(out_dtype, OD, [&] {
    hipLaunchKernelGGL((lse_merge_kernel<OD>), dim3(heads_q * query_len), dim3(128), 0, s, a);
  });
  return check_launch("uc_lse_merge");
}
