// H2O attention-mass scores on MFMA (head_dim 128, bf16/fp16 Q and K):
//   P = bf16(softmax_t(sm_scale * q . k_t)) per query head and row
//   scores[h, t] (+)= sum over the group's query heads and rows of P
// (operators/physical.py:62-65 applied to the bf16 probabilities of
// adapters/bagel.py:1213-1243), without materialising P.
//
// The rows of one KV head (group * Lq of them) are cut into blocks of 256
// (4 waves x 64 rows, held in registers as MFMA fragments) and the keys into
// chunks of whole 64-key tiles, staged through double-buffered LDS:
//   h2o_stats_kernel   (row block, key chunk): S^T = K Q^T, running max and
//                      sum per row over the chunk -> (max, sum) per chunk;
//   h2o_scores_kernel  (row block, key chunk): merges the chunks' (max, sum)
//                      in order, S = Q K^T, p = bf16(2^(s*scale - max - log2 sum)),
//                      per-key sums of p over the block's rows -> one partial
//                      per (row block, key); the row sum runs on the matrix
//                      cores as ones(16x32) . P, exact in fp32 for bf16 inputs;
//   h2o_reduce_kernel  adds the row blocks' partials in order.
// Every sum has a fixed order, so the scores are deterministic.
#include "uc_common.h"
#include "uc_mfma.h"

namespace uc {
namespace {

using namespace mf;

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f8 __attribute__((ext_vector_type(8)));

// Q and K enter the matrix cores in their own dtype: products are exact and
// accumulate in fp32, and bf16 keeps its range.
template <int DT>
struct HsOp;
template <>
struct HsOp<UC_BF16> {
  using V = bf8;
  static __device__ __forceinline__ f4 mma(V a, V b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};
template <>
struct HsOp<UC_FP16> {
  using V = h8;
  static __device__ __forceinline__ f4 mma(V a, V b, f4 c) { return mfma32(a, b, c); }
};

constexpr int kHsWaves = 4;
constexpr int kHsThreads = kHsWaves * kWave;
constexpr int kHsQB = 4;  // 16-row blocks per wave
constexpr int kHsRowsPerWave = 16 * kHsQB;
constexpr int kHsRows = kHsWaves * kHsRowsPerWave;
constexpr int kHsTile = 64;
constexpr int kHsPad = kD + 8;
constexpr int64_t kHsMinChunk = 256;
constexpr int64_t kHsTargetBlocks = 1024;

struct HsParams {
  const uint16_t *q;
  int64_t q_si, q_sh;  // element strides of query rows (i) and heads
  const uint16_t *k;
  int64_t k_st, k_sh;  // element strides of key tokens and heads
  int64_t Lq, Hq, Hkv, group, rows, T;
  int64_t row_blocks, chunks, chunk;
  float scale_log2;
  float2 *ml;          // [Hkv][row_blocks][chunks][kHsRows]: (max * log2 e units, sum)
  float *partial;      // [row_blocks][Hkv][T]
};

struct HsShared {
  uint16_t kt[2][kHsTile][kHsPad];
  float col[2][kHsWaves][kHsTile];
};

// 64 B of one key row per thread: key t0 + tid/4, channels 32*(tid%4) + [0, 32).
__device__ __forceinline__ void load_keys(uint4 (&r)[4], const HsParams &p, int64_t h, int64_t t0) {
  const int tid = threadIdx.x, tok = tid / 4, cq = tid % 4;
  const int64_t t = t0 + tok;
#pragma unroll
  for (int q = 0; q < 4; ++q) r[q] = make_uint4(0, 0, 0, 0);
  if (t < p.T) {
    const uint4 *src = reinterpret_cast<const uint4 *>(p.k + t * p.k_st + h * p.k_sh + 32 * cq);
#pragma unroll
    for (int q = 0; q < 4; ++q) r[q] = src[q];
  }
}

__device__ __forceinline__ void store_keys(uint16_t (*kt)[kHsPad], const uint4 (&r)[4]) {
  const int tid = threadIdx.x, tok = tid / 4, cq = tid % 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4 *>(&kt[tok][32 * cq + 8 * q]) = r[q];
}

template <int DT>
__device__ __forceinline__ typename HsOp<DT>::V key_frag(const uint16_t (*kt)[kHsPad], int row, int col) {
  return __builtin_bit_cast(typename HsOp<DT>::V, *reinterpret_cast<const uint4 *>(&kt[row][col]));
}

// Query fragments of the wave's 64 rows: lane (n, k) holds row 16*qb + n,
// channels 32*kb + 8k + [0, 8).  They are the B operand of K Q^T and the A
// operand of Q K^T alike.  Rows past the end are zero.
template <int DT>
__device__ __forceinline__ void load_queries(typename HsOp<DT>::V (&qf)[kHsQB][4], const HsParams &p, int64_t h,
                                             int64_t row0) {
  const int lane = threadIdx.x & 63, r = lane & 15, kap = lane >> 4;
#pragma unroll
  for (int qb = 0; qb < kHsQB; ++qb) {
    const int64_t row = row0 + 16 * qb + r;
    const bool ok = row < p.rows;
    const int64_t g = ok ? row / p.Lq : 0, i = ok ? row % p.Lq : 0;
    const uint16_t *q16 = p.q + i * p.q_si + (h * p.group + g) * p.q_sh + 8 * kap;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      qf[qb][kb] = __builtin_bit_cast(typename HsOp<DT>::V, ok ? *reinterpret_cast<const uint4 *>(q16 + 32 * kb)
                                                                : make_uint4(0, 0, 0, 0));
  }
}

template <int DT>
__global__ __launch_bounds__(kHsThreads) __attribute__((amdgpu_waves_per_eu(2))) void h2o_stats_kernel(HsParams p) {
  __shared__ __align__(16) HsShared sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const int64_t rb = blockIdx.x, c = blockIdx.y, h = blockIdx.z;
  const int64_t t_begin = c * p.chunk, t_end = min(p.T, t_begin + p.chunk);
  const int n_tiles = static_cast<int>((t_end - t_begin + kHsTile - 1) / kHsTile);

  typename HsOp<DT>::V qf[kHsQB][4];
  load_queries<DT>(qf, p, h, rb * kHsRows + wave * kHsRowsPerWave);

  float m[kHsQB], l[kHsQB];
#pragma unroll
  for (int qb = 0; qb < kHsQB; ++qb) m[qb] = kNegInf, l[qb] = 0.0f;

  uint4 kr[4];
  load_keys(kr, p, h, t_begin);
  store_keys(sh.kt[0], kr);
  __syncthreads();
  for (int i = 0; i < n_tiles; ++i) {
    const int64_t t0 = t_begin + int64_t(i) * kHsTile;
    if (i + 1 < n_tiles) load_keys(kr, p, h, t0 + kHsTile);
    const uint16_t(*kt)[kHsPad] = sh.kt[i & 1];
    f4 acc[4][kHsQB];  // lane (n, k): keys 16*tb + 4k + v of row 16*qb + n
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int qb = 0; qb < kHsQB; ++qb) acc[tb][qb] = f4{0, 0, 0, 0};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const auto a = key_frag<DT>(kt, 16 * tb + r, 32 * kb + 8 * kap);
#pragma unroll
        for (int qb = 0; qb < kHsQB; ++qb) acc[tb][qb] = HsOp<DT>::mma(a, qf[qb][kb], acc[tb][qb]);
      }
    const int valid = static_cast<int>(min<int64_t>(kHsTile, t_end - t0));
    if (valid < kHsTile) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (16 * tb + 4 * kap + v >= valid)
#pragma unroll
            for (int qb = 0; qb < kHsQB; ++qb) acc[tb][qb][v] = kNegInf;
    }
#pragma unroll
    for (int qb = 0; qb < kHsQB; ++qb) {
      float mx = kNegInf;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int v = 0; v < 4; ++v) mx = fmaxf(mx, acc[tb][qb][v]);
      const float m_new = fmaxf(m[qb], max_over_slices(mx) * p.scale_log2);
      float sum = 0.0f;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int v = 0; v < 4; ++v) sum += fast_exp2(__builtin_fmaf(acc[tb][qb][v], p.scale_log2, -m_new));
      l[qb] = l[qb] * fast_exp2(m[qb] - m_new) + sum;
      m[qb] = m_new;
    }
    if (i + 1 < n_tiles) store_keys(sh.kt[(i + 1) & 1], kr);
    __syncthreads();
  }

  float2 *out = p.ml + ((h * p.row_blocks + rb) * p.chunks + c) * kHsRows + wave * kHsRowsPerWave;
#pragma unroll
  for (int qb = 0; qb < kHsQB; ++qb) {
    const float lt = sum_over_slices(l[qb]);
    if (kap == 0) out[16 * qb + r] = make_float2(m[qb], lt);
  }
}

template <int DT>
__global__ __launch_bounds__(kHsThreads) __attribute__((amdgpu_waves_per_eu(2))) void h2o_scores_kernel(HsParams p) {
  __shared__ __align__(16) HsShared sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const int64_t rb = blockIdx.x, c = blockIdx.y, h = blockIdx.z;
  const int64_t t_begin = c * p.chunk, t_end = min(p.T, t_begin + p.chunk);
  const int n_tiles = static_cast<int>((t_end - t_begin + kHsTile - 1) / kHsTile);
  const int64_t row0 = rb * kHsRows + wave * kHsRowsPerWave;

  uint4 kr[4];
  load_keys(kr, p, h, t_begin);
  typename HsOp<DT>::V qf[kHsQB][4];
  load_queries<DT>(qf, p, h, row0);

  // lane j merges the chunks of row row0 + j: p = 2^(s*scale - bias),
  // bias = max + log2(sum); rows past the end get +inf (p = 0)
  float bias;
  {
    const float2 *src = p.ml + (h * p.row_blocks + rb) * p.chunks * kHsRows + wave * kHsRowsPerWave + lane;
    float mt = kNegInf;
    for (int64_t s = 0; s < p.chunks; ++s) mt = fmaxf(mt, src[s * kHsRows].x);
    float lt = 0.0f;
    for (int64_t s = 0; s < p.chunks; ++s) {
      const float2 ml = src[s * kHsRows];
      lt += ml.y * fast_exp2(ml.x - mt);
    }
    bias = row0 + lane < p.rows ? mt + __log2f(lt) : __builtin_inff();
  }
  float nb[kHsQB][4];  // -bias of rows 16*qb + 4k + v, the rows lane (n, k) sees in Q K^T
#pragma unroll
  for (int qb = 0; qb < kHsQB; ++qb)
#pragma unroll
    for (int v = 0; v < 4; ++v) nb[qb][v] = -__shfl(bias, 16 * qb + 4 * kap + v, kWave);

  bf8 ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = static_cast<__bf16>(1.0f);

  store_keys(sh.kt[0], kr);
  __syncthreads();
  float *out = p.partial + (rb * p.Hkv + h) * p.T;
  for (int i = 0; i < n_tiles; ++i) {
    const int64_t t0 = t_begin + int64_t(i) * kHsTile;
    if (i + 1 < n_tiles) load_keys(kr, p, h, t0 + kHsTile);
    const uint16_t(*kt)[kHsPad] = sh.kt[i & 1];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      typename HsOp<DT>::V kf[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) kf[kb] = key_frag<DT>(kt, 16 * tb + r, 32 * kb + 8 * kap);
      f8 e[2];
#pragma unroll
      for (int qb = 0; qb < kHsQB; ++qb) {
        f4 s = f4{0, 0, 0, 0};  // lane (n, k): rows 16*qb + 4k + v, key 16*tb + n
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) s = HsOp<DT>::mma(qf[qb][kb], kf[kb], s);
#pragma unroll
        for (int v = 0; v < 4; ++v)
          e[qb >> 1][4 * (qb & 1) + v] = fast_exp2(__builtin_fmaf(s[v], p.scale_log2, nb[qb][v]));
      }
      // column sums over the 64 rows: two k-slices of 32 rows each
      f4 cs = f4{0, 0, 0, 0};
      cs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, __builtin_convertvector(e[0], bf8), cs, 0, 0, 0);
      cs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, __builtin_convertvector(e[1], bf8), cs, 0, 0, 0);
      if (kap == 0) sh.col[i & 1][wave][16 * tb + r] = cs[0];
    }
    if (i > 0 && tid < kHsTile) {  // previous tile: its sums were completed before the last barrier
      const float *cp = &sh.col[(i - 1) & 1][0][tid];
      const int64_t t = t0 - kHsTile + tid;
      if (t < t_end) out[t] = ((cp[0] + cp[kHsTile]) + cp[2 * kHsTile]) + cp[3 * kHsTile];
    }
    if (i + 1 < n_tiles) store_keys(sh.kt[(i + 1) & 1], kr);
    __syncthreads();
  }
  if (tid < kHsTile) {
    const float *cp = &sh.col[(n_tiles - 1) & 1][0][tid];
    const int64_t t = t_begin + int64_t(n_tiles - 1) * kHsTile + tid;
    if (t < t_end) out[t] = ((cp[0] + cp[kHsTile]) + cp[2 * kHsTile]) + cp[3 * kHsTile];
  }
}

// scores[h, t] (+)= sum over row blocks, in order, of the partials.
__global__ __launch_bounds__(256) void h2o_reduce_kernel(const float *partial, int64_t row_blocks, int64_t Hkv,
                                                         int64_t T, float *scores, int accumulate) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= Hkv * T) return;
  const int64_t h = idx / T, t = idx % T;
  float s = 0.0f;
  for (int64_t rb = 0; rb < row_blocks; ++rb) s += partial[(rb * Hkv + h) * T + t];
  scores[idx] = accumulate ? scores[idx] + s : s;
}

struct HsShape {
  int64_t row_blocks, chunks, chunk;
};

HsShape h2o_shape(int64_t heads_q, int64_t heads_kv, int64_t query_len, int64_t tokens) {
  HsShape s{};
  s.row_blocks = ceil_div((heads_q / heads_kv) * query_len, int64_t(kHsRows));
  const int64_t blocks = s.row_blocks * heads_kv;
  const int64_t want = ceil_div(kHsTargetBlocks, blocks);
  s.chunk = ceil_div(ceil_div(tokens, want), int64_t(kHsTile)) * kHsTile;
  if (s.chunk < kHsMinChunk) s.chunk = kHsMinChunk;
  s.chunks = ceil_div(tokens, s.chunk);
  return s;
}

// Row-block count bound that does not depend on heads_kv:
// heads_kv * ceil(group * Lq / 256) <= ceil(heads_q * Lq / 256) + heads_q.
int64_t row_block_bound(int64_t heads_q, int64_t query_len) {
  return ceil_div(heads_q * query_len, int64_t(kHsRows)) + heads_q;
}

}  // namespace

bool h2o_mfma_supported(int dtype, int64_t head_dim, const void *q, int64_t q_si, int64_t q_sh, int64_t q_sd,
                        const void *k, int64_t k_st, int64_t k_sh, int64_t k_sd) {
  const bool aligned = (reinterpret_cast<uintptr_t>(q) & 15) == 0 && (reinterpret_cast<uintptr_t>(k) & 15) == 0 &&
                       q_si % 8 == 0 && q_sh % 8 == 0 && k_st % 8 == 0 && k_sh % 8 == 0;
  return (dtype == UC_BF16 || dtype == UC_FP16) && head_dim == kD && q_sd == 1 && k_sd == 1 && aligned;
}

// Stats first ((max, sum) per row block, chunk and row: at most
// (row blocks + target blocks) * 256 rows of 8 bytes, since chunks exceed 1
// only while row blocks * chunks stays near the target), then the partials.
int64_t h2o_mfma_workspace_bytes(int64_t heads_q, int64_t query_len, int64_t tokens) {
  const int64_t rbb = row_block_bound(heads_q, query_len);
  return (rbb + kHsTargetBlocks) * kHsRows * int64_t(sizeof(float2)) + rbb * tokens * int64_t(sizeof(float));
}

int launch_h2o_mfma(int dtype, const void *q, int64_t q_si, int64_t q_sh, const void *k, int64_t k_st, int64_t k_sh,
                    int64_t Lq, int64_t Hq, int64_t T, int64_t Hkv, float sm_scale, int accumulate, float *scores,
                    void *workspace, hipStream_t stream) {
  const HsShape shape = h2o_shape(Hq, Hkv, Lq, T);
  const int64_t rbb = row_block_bound(Hq, Lq);
  UC_REQUIRE(shape.row_blocks * Hkv <= rbb && shape.row_blocks * Hkv * shape.chunks <= rbb + kHsTargetBlocks,
             "uc_h2o_scores: internal workspace bound violated");
  UC_REQUIRE(shape.row_blocks <= 65535 && shape.chunks <= 65535 && Hkv <= 65535, "uc_h2o_scores: grid too large");
  HsParams p{};
  p.q = static_cast<const uint16_t *>(q);
  p.q_si = q_si; p.q_sh = q_sh;
  p.k = static_cast<const uint16_t *>(k);
  p.k_st = k_st; p.k_sh = k_sh;
  p.Lq = Lq; p.Hq = Hq; p.Hkv = Hkv; p.group = Hq / Hkv; p.rows = p.group * Lq; p.T = T;
  p.row_blocks = shape.row_blocks; p.chunks = shape.chunks; p.chunk = shape.chunk;
  p.scale_log2 = sm_scale * kLog2e;
  p.ml = static_cast<float2 *>(workspace);
  p.partial = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                        (rbb + kHsTargetBlocks) * kHsRows * int64_t(sizeof(float2)));
  const dim3 grid(static_cast<unsigned>(p.row_blocks), static_cast<unsigned>(p.chunks), static_cast<unsigned>(Hkv));
  if (dtype == UC_FP16)
    hipLaunchKernelGGL((h2o_stats_kernel<UC_FP16>), grid, dim3(kHsThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((h2o_stats_kernel<UC_BF16>), grid, dim3(kHsThreads), 0, stream, p);
  int rc = check_launch("uc_h2o_scores (MFMA stats)");
  if (rc != UC_OK) return rc;
  if (dtype == UC_FP16)
    hipLaunchKernelGGL((h2o_scores_kernel<UC_FP16>), grid, dim3(kHsThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((h2o_scores_kernel<UC_BF16>), grid, dim3(kHsThreads), 0, stream, p);
  rc = check_launch("uc_h2o_scores (MFMA scores)");
  if (rc != UC_OK) return rc;
  hipLaunchKernelGGL(h2o_reduce_kernel, dim3(static_cast<unsigned>(ceil_div(Hkv * T, int64_t(256)))), dim3(256), 0,
                     stream, p.partial, p.row_blocks, Hkv, T, scores, accumulate);
  return check_launch("uc_h2o_scores (MFMA reduce)");
}

}  // namespace uc
