// H2O attention-mass scores on MFMA (head_dim 128, bf16/fp16 Q and K):
//   P = bf16(softmax_t(sm_scale * q . k_t)) per query head and row
//   scores[h, t] (+)= sum over the group's query heads and rows of P
// (operators/physical.py:62-65 applied to the bf16 probabilities of
// adapters/bagel.py:1213-1243), without materialising P.
//
// The rows of one KV head (group * Lq of them) are cut into blocks of 256
// (4 waves x 64 rows, held in registers as MFMA fragments) and the keys into
// chunks of whole 64-key tiles.  Tiles stream into a ring of LDS slots by
// direct buffer-to-LDS loads issued kHsStages - 1 tiles ahead:
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

#include <type_traits>

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
constexpr int64_t kHsMinChunk = 256;
constexpr int64_t kHsTargetBlocks = 768;  // one round: 3 workgroups (51 KB LDS) x 256 CUs

struct HsParams {
  const uint16_t *q;
  int64_t q_si, q_sh;  // element strides of query rows (i) and heads
  const uint16_t *k;
  int64_t k_st, k_sh;  // element strides of key tokens and heads
  int64_t Lq, Hq, Hkv, group, rows, T;
  int64_t row_blocks, chunks, chunk;
  int64_t items, per_xcd;  // work items (KV head, row block, chunk) and items per XCD
  float scale_log2;
  float2 *ml;          // [Hkv][row_blocks][chunks][kHsRows]: (max * log2 e units, sum)
  float *partial;      // [row_blocks][Hkv][T]
  const float *lse;    // optional [Hq][Lq] natural-log normaliser given by the caller
  float *logits;       // qk_logits_kernel: [Hq][Lq][T] = scale * q . k
  float scale;
};

// Workgroups are dealt to the 8 XCDs round-robin by launch index.  Work item
// w = (h * row_blocks + rb) * chunks + c goes to launch index
// 8 * (w % per_xcd) + w / per_xcd, so each XCD walks one contiguous run of
// items: one or two KV heads' keys and a few query row blocks at a time,
// which its own L2 holds.
constexpr int kXcds = 8;

struct HsItem {
  int64_t h, rb, c;
  bool valid;
};

// 32-bit arithmetic: the launch keeps the grid and every item count below 2^31
// (64-bit divisions cost the scalar unit a few hundred instructions each).
__device__ __forceinline__ HsItem hs_item(const HsParams &p) {
  const uint32_t id = blockIdx.x;
  const uint32_t chunks = static_cast<uint32_t>(p.chunks), row_blocks = static_cast<uint32_t>(p.row_blocks);
  const uint32_t w = (id % kXcds) * static_cast<uint32_t>(p.per_xcd) + id / kXcds;
  HsItem it;
  it.valid = w < static_cast<uint32_t>(p.items);
  const uint32_t q = w / chunks;
  it.c = w - q * chunks;
  it.rb = q % row_blocks;
  it.h = q / row_blocks;
  return it;
}

constexpr int kHsStages = 3;

// Key tile slot: row t (256 B of one key) holds its 16-byte chunk c at
// position c ^ (t & 15), so the 16 rows one MFMA fragment read touches sit in
// 16 different bank groups.
struct HsShared {
  uint4 kt[kHsStages][kHsTile * 16];
  float col[2][kHsWaves][kHsTile];
};

// The key rows [t_begin, t_end) of one KV head, streamed a tile at a time.
// Rows past t_end fall outside the buffer resource and read as zero.
struct KeyStream {
  Rsrc rs;
  uint32_t row_bytes;
  int n_tiles;

  __device__ KeyStream(const HsParams &p, int64_t h, int64_t t_begin, int64_t t_end) {
    row_bytes = static_cast<uint32_t>(p.k_st * 2);
    rs = make_rsrc(p.k + h * p.k_sh + t_begin * p.k_st, (t_end - t_begin - 1) * p.k_st * 2 + kD * 2);
    n_tiles = static_cast<int>((t_end - t_begin + kHsTile - 1) / kHsTile);
  }

  // every thread: 4 loads of 16 B; wave w fills rows 16w .. 16w + 15 of the slot
  __device__ __forceinline__ void issue(HsShared &sh, int tile) const {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint4 *slot = sh.kt[tile % kHsStages];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 16 * wave + 4 * j + (lane >> 4);
      const uint32_t off = static_cast<uint32_t>(tile * kHsTile + row) * row_bytes + 16u * ((lane & 15) ^ (row & 15));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void *)(slot + (16 * wave + 4 * j) * 16), 16, off, 0,
          0, 0);
    }
  }

  __device__ __forceinline__ void prologue(HsShared &sh) const {
    for (int t = 0; t < kHsStages - 1 && t < n_tiles; ++t) issue(sh, t);
  }

  // Tile i is in LDS for the whole workgroup; then the slot freed by tile i - 1
  // is refilled with tile i + kHsStages - 1.
  __device__ __forceinline__ void acquire(HsShared &sh, int i) const {
    const int ahead = min(n_tiles - 1, i + kHsStages - 2) - i;  // later tiles this thread still loads
    static_assert(kHsStages <= 4, "vmcnt cases below");
    if (ahead >= 2)
      __builtin_amdgcn_s_waitcnt(kWaitVm8);
    else if (ahead == 1)
      __builtin_amdgcn_s_waitcnt(kWaitVm4);
    else
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (i + kHsStages - 1 < n_tiles) issue(sh, i + kHsStages - 1);
  }

  // s_waitcnt immediates (gfx9 layout): vmcnt <= N, expcnt and lgkmcnt not waited on
  static constexpr int kWaitVm0 = 0x0F70, kWaitVm4 = 0x0F74, kWaitVm8 = 0x0F78;
};

template <int DT>
__device__ __forceinline__ typename HsOp<DT>::V key_frag(const uint4 *slot, int row, int chunk) {
  return __builtin_bit_cast(typename HsOp<DT>::V, slot[row * 16 + (chunk ^ (row & 15))]);
}

// Query fragments of the wave's 64 rows: lane (n, k) holds row 16*qb + n,
// channels 32*kb + 8k + [0, 8).  They are the B operand of K Q^T and the A
// operand of Q K^T alike.  Rows past the end load the last row again; their
// statistics are never used and their probabilities are zeroed.
template <int DT>
__device__ __forceinline__ void load_queries(typename HsOp<DT>::V (&qf)[kHsQB][4], const HsParams &p, int64_t h,
                                             int64_t row0) {
  const int lane = threadIdx.x & 63, r = lane & 15, kap = lane >> 4;
#pragma unroll
  for (int qb = 0; qb < kHsQB; ++qb) {
    const int64_t row = min(row0 + 16 * qb + r, p.rows - 1);  // rows past the end repeat the last one
    const uint32_t row32 = static_cast<uint32_t>(row), lq = static_cast<uint32_t>(p.Lq);
    const int64_t g = row32 / lq, i = row32 % lq;
    const uint16_t *q16 = p.q + i * p.q_si + (h * p.group + g) * p.q_sh + 8 * kap;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      qf[qb][kb] = __builtin_bit_cast(typename HsOp<DT>::V, *reinterpret_cast<const uint4 *>(q16 + 32 * kb));
  }
}

// Exponentials are taken against a per-row reference that is raised only
// when a logit exceeds it by more than kHsSlack (log2 units): terms stay below
// 2^kHsSlack, and the common 16-key block needs no rescale and no wait for the
// rest of the tile.
constexpr float kHsSlack = 8.0f;

template <int DT>
__global__ __launch_bounds__(kHsThreads) __attribute__((amdgpu_waves_per_eu(3))) void h2o_stats_kernel(HsParams p) {
  __shared__ __align__(16) HsShared sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const HsItem it = hs_item(p);
  if (!it.valid) return;
  const int64_t rb = it.rb, c = it.c, h = it.h;
  const int64_t t_begin = c * p.chunk, t_end = min(p.T, t_begin + p.chunk);

  typename HsOp<DT>::V qf[kHsQB][4];
  load_queries<DT>(qf, p, h, rb * kHsRows + wave * kHsRowsPerWave);
  const KeyStream ks(p, h, t_begin, t_end);
  ks.prologue(sh);

  // m: reference of row 16*qb + n (equal in the four k-slices), thr: the raw
  // logit above which it must move; l: this lane's share of the row sum
  float m[kHsQB], thr[kHsQB], l[kHsQB];
#pragma unroll
  for (int qb = 0; qb < kHsQB; ++qb) m[qb] = kNegInf, thr[qb] = kNegInf, l[qb] = 0.0f;

  for (int i = 0; i < ks.n_tiles; ++i) {
    ks.acquire(sh, i);
    const int64_t t0 = t_begin + int64_t(i) * kHsTile;
    const uint4 *kt = sh.kt[i % kHsStages];
    const int valid = static_cast<int>(min<int64_t>(kHsTile, t_end - t0));
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      f4 acc[kHsQB];  // lane (n, k): keys 16*tb + 4k + v of row 16*qb + n
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const auto a = key_frag<DT>(kt, 16 * tb + r, 4 * kb + kap);
#pragma unroll
        for (int qb = 0; qb < kHsQB; ++qb) acc[qb] = HsOp<DT>::mma(a, qf[qb][kb], kb ? acc[qb] : f4{0, 0, 0, 0});
      }
      if (valid < kHsTile) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (16 * tb + 4 * kap + v >= valid)
#pragma unroll
            for (int qb = 0; qb < kHsQB; ++qb) acc[qb][v] = kNegInf;
      }
      float bm[kHsQB];
      bool raise = false;
#pragma unroll
      for (int qb = 0; qb < kHsQB; ++qb) {
        bm[qb] = fmaxf(fmaxf(acc[qb][0], acc[qb][1]), fmaxf(acc[qb][2], acc[qb][3]));
        raise |= bm[qb] > thr[qb];
      }
      if (__any(raise)) {
#pragma unroll
        for (int qb = 0; qb < kHsQB; ++qb) {
          const float m_new = fmaxf(m[qb], max_over_slices(bm[qb]) * p.scale_log2);
          l[qb] *= fast_exp2(m[qb] - m_new);
          m[qb] = m_new;
          thr[qb] = (m_new + kHsSlack) / p.scale_log2;
        }
      }
#pragma unroll
      for (int qb = 0; qb < kHsQB; ++qb)
#pragma unroll
        for (int v = 0; v < 4; ++v) l[qb] += fast_exp2(__builtin_fmaf(acc[qb][v], p.scale_log2, -m[qb]));
    }
  }

  float2 *out = p.ml + ((h * p.row_blocks + rb) * p.chunks + c) * kHsRows + wave * kHsRowsPerWave;
#pragma unroll
  for (int qb = 0; qb < kHsQB; ++qb) {
    const float lt = sum_over_slices(l[qb]);
    if (kap == 0) out[16 * qb + r] = make_float2(m[qb], lt);
  }
}

template <int DT>
__global__ __launch_bounds__(kHsThreads) __attribute__((amdgpu_waves_per_eu(3))) void h2o_scores_kernel(HsParams p) {
  __shared__ __align__(16) HsShared sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const HsItem it = hs_item(p);
  if (!it.valid) return;
  const int64_t rb = it.rb, c = it.c, h = it.h;
  const int64_t t_begin = c * p.chunk, t_end = min(p.T, t_begin + p.chunk);
  const int64_t row0 = rb * kHsRows + wave * kHsRowsPerWave;
  // the first key tiles are requested before the query rows and the
  // normaliser, so the three latencies overlap (the normaliser is used before
  // the first tile, and a use waits for every load issued before it)
  const KeyStream ks(p, h, t_begin, t_end);
  ks.prologue(sh);

  typename HsOp<DT>::V qf[kHsQB][4];
  load_queries<DT>(qf, p, h, row0);

  // lane j merges the chunks of row row0 + j: p = 2^(s*scale - bias),
  // bias = max + log2(sum); rows past the end get +inf (p = 0)
  float bias;
  if (p.lse != nullptr) {  // probabilities against the caller's normaliser
    const int64_t row = row0 + lane;
    const uint32_t rc = row < p.rows ? static_cast<uint32_t>(row) : 0u, lq = static_cast<uint32_t>(p.Lq);
    const uint32_t g = rc / lq, i = rc - g * lq;
    const float l = p.lse[(h * p.group + g) * p.Lq + i];  // row rc exists: loaded unconditionally
    bias = row < p.rows ? l * kLog2e : __builtin_inff();
  } else {
    const float2 *src = p.ml + (h * p.row_blocks + rb) * p.chunks * kHsRows + wave * kHsRowsPerWave + lane;
    float mt = kNegInf, lt = 0.0f;
    for (int64_t s0 = 0; s0 < p.chunks; s0 += 8) {  // eight loads in flight, merged in chunk order
      float2 ml[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) ml[j] = s0 + j < p.chunks ? src[(s0 + j) * kHsRows] : make_float2(kNegInf, 0.0f);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float m_new = fmaxf(mt, ml[j].x);
        if (m_new != kNegInf) lt = lt * fast_exp2(mt - m_new) + ml[j].y * fast_exp2(ml[j].x - m_new);
        mt = m_new;
      }
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

  float *out = p.partial + (rb * p.Hkv + h) * p.T;
  for (int i = 0; i < ks.n_tiles; ++i) {
    ks.acquire(sh, i);
    const int64_t t0 = t_begin + int64_t(i) * kHsTile;
    if (i > 0 && tid < kHsTile) {  // previous tile: its sums were completed before the barrier
      const float *cp = &sh.col[(i - 1) & 1][0][tid];
      const int64_t t = t0 - kHsTile + tid;
      if (t < t_end) out[t] = ((cp[0] + cp[kHsTile]) + cp[2 * kHsTile]) + cp[3 * kHsTile];
    }
    const uint4 *kt = sh.kt[i % kHsStages];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      typename HsOp<DT>::V kf[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) kf[kb] = key_frag<DT>(kt, 16 * tb + r, 4 * kb + kap);
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
  }
  __syncthreads();
  if (tid < kHsTile) {
    const float *cp = &sh.col[(ks.n_tiles - 1) & 1][0][tid];
    const int64_t t = t_begin + int64_t(ks.n_tiles - 1) * kHsTile + tid;
    if (t < t_end) out[t] = ((cp[0] + cp[kHsTile]) + cp[2 * kHsTile]) + cp[3 * kHsTile];
  }
}

// Logits of dense keys, fp32 [Hq][Lq][T] = scale * q . k (physical.py:20-39).
// The tiles are computed as S^T = K Q^T, so lane (n, k) holds four
// consecutive keys 16 tb + 4k .. + 3 of row 16 qb + n and writes them with one
// 16-byte store: a store instruction covers 16 rows x 64 contiguous bytes.
template <int DT>
__global__ __launch_bounds__(kHsThreads) __attribute__((amdgpu_waves_per_eu(3))) void qk_logits_kernel(HsParams p) {
  __shared__ __align__(16) HsShared sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const HsItem it = hs_item(p);
  if (!it.valid) return;
  const int64_t rb = it.rb, c = it.c, h = it.h;
  const int64_t t_begin = c * p.chunk, t_end = min(p.T, t_begin + p.chunk);
  const int64_t row0 = rb * kHsRows + wave * kHsRowsPerWave;
  // 16-byte stores need rows that start on 16 bytes (uniform)
  const bool vec = (p.T & 3) == 0 && (reinterpret_cast<uintptr_t>(p.logits) & 15) == 0;

  // the first key tiles are requested before the query rows, so the two
  // latencies overlap
  const KeyStream ks(p, h, t_begin, t_end);
  ks.prologue(sh);
  typename HsOp<DT>::V qf[kHsQB][4];
  load_queries<DT>(qf, p, h, row0);
  // start of the logits row of row 16*qb + n, the row lane (n, k) holds in
  // S^T; -1 past the last row (rows < 2^31: 32-bit division)
  int64_t ro[kHsQB];
#pragma unroll
  for (int qb = 0; qb < kHsQB; ++qb) {
    const int64_t row = row0 + 16 * qb + r;
    const uint32_t lq = static_cast<uint32_t>(p.Lq), g = static_cast<uint32_t>(row) / lq;
    const uint32_t i = static_cast<uint32_t>(row) - g * lq;
    ro[qb] = row < p.rows ? ((h * p.group + g) * p.Lq + i) * p.T : -1;
  }
  for (int i = 0; i < ks.n_tiles; ++i) {
    ks.acquire(sh, i);
    const int64_t t0 = t_begin + int64_t(i) * kHsTile;
    const uint4 *kt = sh.kt[i % kHsStages];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      typename HsOp<DT>::V kf[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) kf[kb] = key_frag<DT>(kt, 16 * tb + r, 4 * kb + kap);
      const int64_t t = t0 + 16 * tb + 4 * kap;  // first of this lane's four keys
#pragma unroll
      for (int qb = 0; qb < kHsQB; ++qb) {
        f4 s = f4{0, 0, 0, 0};  // lane (n, k): keys 16*tb + 4k + v of row 16*qb + n
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) s = HsOp<DT>::mma(kf[kb], qf[qb][kb], s);
        if (ro[qb] < 0) continue;
        float *dst = p.logits + ro[qb] + t;
        if (vec && t + 4 <= t_end) {
          *reinterpret_cast<f4 *>(dst) = s * p.scale;
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (t + v < t_end) dst[v] = s[v] * p.scale;
        }
      }
    }
  }
}

// ------------------------------------------------------------ dense P.V --
// out[hq, i, :] = P[hq, i, :] . V[:, h, :] with P cast to the value dtype
// first (physical.py:42-63), fp32 accumulation.  pv_stage_kernel writes V
// transposed, [Hkv][128][Tp] (Tp = T rounded up to 64, zero tail); in
// pv_mfma_kernel a workgroup owns 64 query rows of one KV head in three key
// parts of 4 waves (a 16-row block per wave); each part streams the 64-key
// tiles of its third of V^T through its own LDS ring and reads the P^T
// fragments straight from global memory:
//   O^T[16 channels x 16 rows] += V^T[16 x 32 keys] . P^T[32 keys x 16 rows],
// and the other parts' sums are added to the first's through LDS at the end.
// Three parts put 12 waves of loads in flight per CU for the ~224 workgroups
// of a config-3 layer (one per CU).
constexpr int kPvWaves = 4;                          // waves per key part: 16 rows each
constexpr int kPvParts = 3;                         // key parts of a workgroup
constexpr int kPvPartThreads = kPvWaves * kWave;
constexpr int kPvThreads = kPvParts * kPvPartThreads;
constexpr int kPvRows = 16 * kPvWaves;
constexpr int kPvTile = 64;
constexpr int kPvStages = 3;

template <int VD>
struct PvOp;
template <>
struct PvOp<UC_BF16> {
  using V = bf8;
  static __device__ __forceinline__ f4 mma(V a, V b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
  static __device__ __forceinline__ uint16_t bits(float x) { return f32_to_bf16_bits(x); }
};
template <>
struct PvOp<UC_FP16> {
  using V = h8;
  static __device__ __forceinline__ f4 mma(V a, V b, f4 c) { return mfma32(a, b, c); }
  static __device__ __forceinline__ uint16_t bits(float x) { return f32_to_f16_bits(x); }
};

// One 64-key tile of V for one KV head, transposed through LDS.
__global__ __launch_bounds__(256) void pv_stage_kernel(const uint16_t *v, int64_t v_st, int64_t v_sh, int64_t T,
                                                       int64_t Tp, uint16_t *vt) {
  __shared__ uint16_t tile[kPvTile][kD + 8];
  const int tid = threadIdx.x;
  const int64_t h = blockIdx.y, t0 = int64_t(blockIdx.x) * kPvTile;
#pragma unroll
  for (int j = 0; j < 4; ++j) {  // 64 keys x 16 chunks of 8 channels
    const int c = j * 256 + tid, key = c / 16, c8 = c % 16;
    const uint4 x = t0 + key < T ? *reinterpret_cast<const uint4 *>(v + (t0 + key) * v_st + h * v_sh + 8 * c8)
                                 : make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4 *>(&tile[key][8 * c8]) = x;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {  // 128 channels x 8 chunks of 8 keys
    const int c = j * 256 + tid, ch = c / 8, k8 = c % 8;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = tile[8 * k8 + 2 * e][ch] | (uint32_t(tile[8 * k8 + 2 * e + 1][ch]) << 16);
    *reinterpret_cast<uint4 *>(vt + (h * kD + ch) * Tp + t0 + 8 * k8) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

struct PvParams {
  const void *p;
  int64_t p_sh, p_si;  // element strides of query heads and rows (keys are unit stride)
  const uint16_t *vt;  // [Hkv][128][Tp]
  int64_t T, Tp, Lq, Hq, Hkv, group, rows;
  int64_t row_blocks, items, per_xcd;
  void *out;  // [Hq][Lq][128], value dtype
};

// V^T slot: channel row c (128 B = 8 chunks of 8 keys) keeps chunk q at
// position q ^ (c & 7), so the 16 rows of a fragment read hit 8 bank groups twice.
struct PvShared {
  uint4 vt[kPvParts][kPvStages][kD * 8];
};

// Raw P bytes of one lane's eight keys: one 16-byte load for 16-bit P, two for fp32.
template <int PD>
struct PRaw {
  static constexpr int N = PD == UC_FP32 ? 2 : 1;
  uint4 x[N];
};

// P^T fragment in the value dtype (the cast of physical.py:59); keys at or past
// T are zero.
template <int PD, int VD>
__device__ __forceinline__ typename PvOp<VD>::V p_frag(const PRaw<PD> &raw, int64_t t, int64_t T) {
  uint32_t w[4];
  if constexpr (PD == VD) {
    w[0] = raw.x[0].x, w[1] = raw.x[0].y, w[2] = raw.x[0].z, w[3] = raw.x[0].w;
    if (t + 8 > T) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (t + 2 * e >= T) w[e] &= 0xffff0000u;
        if (t + 2 * e + 1 >= T) w[e] &= 0x0000ffffu;
      }
    }
  } else {
    float x[8];
    if constexpr (PD == UC_FP32) {
      const uint32_t u[8] = {raw.x[0].x, raw.x[0].y, raw.x[0].z, raw.x[0].w,
                             raw.x[1].x, raw.x[1].y, raw.x[1].z, raw.x[1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = __uint_as_float(u[e]);
    } else {
      const uint32_t u[4] = {raw.x[0].x, raw.x[0].y, raw.x[0].z, raw.x[0].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = half_bits_to_f32<PD>(u[e / 2] >> (16 * (e % 2)));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (t + e >= T) x[e] = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = uint32_t(PvOp<VD>::bits(x[2 * e])) | (uint32_t(PvOp<VD>::bits(x[2 * e + 1])) << 16);
  }
  return __builtin_bit_cast(typename PvOp<VD>::V, make_uint4(w[0], w[1], w[2], w[3]));
}

// s_waitcnt immediate (gfx9 layout): vmcnt <= n, expcnt and lgkmcnt not waited on
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

template <int PD, int VD>
__global__ __launch_bounds__(kPvThreads) void pv_mfma_kernel(PvParams p) {
  __shared__ __align__(16) PvShared sh;
  constexpr int kAhead = kPvStages - 1;            // tiles in flight
  constexpr int kEl = PD == UC_FP32 ? 4 : 2;       // bytes per probability
  constexpr int kOps = 2 * PRaw<PD>::N + 4;        // memory ops per tile and thread: P halves + V^T slots
  const int tid = threadIdx.x, lane = tid & 63;
  const int part = __builtin_amdgcn_readfirstlane(tid / kPvPartThreads);
  const int ptid = tid % kPvPartThreads;
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) % kPvWaves);  // scalar: the P resource stays in SGPRs
  const int r = lane & 15, kap = lane >> 4;
  const int64_t id = blockIdx.x, w = (id % kXcds) * p.per_xcd + id / kXcds;
  if (w >= p.items) return;  // uniform: the whole workgroup leaves
  const int64_t h = w / p.row_blocks, rb = w % p.row_blocks;
  // the wave's 16 rows are consecutive rows of P (contiguous [query head][row]):
  // a buffer resource over them reads zero past the last row
  const int64_t row0w = rb * kPvRows + wave * 16;
  const int64_t nrows = max<int64_t>(0, min<int64_t>(16, p.rows - row0w));
  const Rsrc rp = make_rsrc(static_cast<const char *>(p.p) + (h * p.group * p.Lq + row0w) * p.p_si * kEl,
                            nrows * p.p_si * kEl);
  const uint32_t p_lane = static_cast<uint32_t>((r * p.p_si + 8 * kap) * kEl);
  const Rsrc rs = make_rsrc(p.vt + h * kD * p.Tp, kD * p.Tp * 2);
  // part k takes tiles [k n_part, (k + 1) n_part); every part runs n_part steps
  // (the barriers are shared), the last ones idling when the count falls short
  const int n_tiles = static_cast<int>(p.Tp / kPvTile);
  const int n_part = (n_tiles + kPvParts - 1) / kPvParts;
  const int first = part * n_part, mine = max(0, min(n_part, n_tiles - first));

  auto load_p = [&](PRaw<PD> (&dst)[2], int i) {
    const int tile = first + i;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int j = 0; j < PRaw<PD>::N; ++j)
        dst[ks].x[j] = bload128(rp, p_lane + static_cast<uint32_t>((tile * kPvTile + 32 * ks) * kEl + 16 * j));
  };
  auto issue_vt = [&](int i) {
    const int64_t tile = first + i;
    uint4 *slot = sh.vt[part][i % kPvStages];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int s4 = q * kPvPartThreads + ptid, ch = s4 / 8, pos = s4 % 8, chunk = pos ^ (ch & 7);
      const uint32_t off = static_cast<uint32_t>((ch * p.Tp + tile * kPvTile) * 2 + chunk * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void *)(slot + q * kPvPartThreads + wave * kWave), 16, off, 0, 0,
          0);
    }
  };

  PRaw<PD> pb[kAhead][2];  // P of the tiles in flight, oldest first
#pragma unroll
  for (int t = 0; t < kAhead; ++t) {
    if (t < mine) {
      load_p(pb[t], t);
      issue_vt(t);
    }
  }
  f4 o[8];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) o[cb] = f4{0, 0, 0, 0};
  for (int it = 0; it < n_part; ++it) {
    // tile it has landed once at most (later tiles issued) x kOps ops remain
    const int later = max(0, min(mine - 1, it + kAhead - 1) - it);
    if (later >= 2)
      wait_vm<2 * kOps>();
    else if (later == 1)
      wait_vm<kOps>();
    else
      wait_vm<0>();
    __syncthreads();
    PRaw<PD> nb[2];
    const bool more = it + kAhead < mine;  // the slot it refills was last read in tile it - 1
    if (more) {
      load_p(nb, it + kAhead);
      issue_vt(it + kAhead);
    }
    if (it < mine) {  // uniform per part
      const int64_t t0 = int64_t(first + it) * kPvTile;
      const uint4 *vt = sh.vt[part][it % kPvStages];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const auto b = p_frag<PD, VD>(pb[0][ks], t0 + 32 * ks + 8 * kap, p.T);
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
          const int ch = 16 * cb + r, q = 4 * ks + kap;
          o[cb] = PvOp<VD>::mma(__builtin_bit_cast(typename PvOp<VD>::V, vt[ch * 8 + (q ^ (ch & 7))]), b, o[cb]);
        }
      }
    }
#pragma unroll
    for (int t = 0; t + 1 < kAhead; ++t) pb[t][0] = pb[t + 1][0], pb[t][1] = pb[t + 1][1];
    if (more) pb[kAhead - 1][0] = nb[0], pb[kAhead - 1][1] = nb[1];
  }
  __syncthreads();  // the rings are free: parts 1.. hand their sums to part 0 through LDS
  constexpr int kRedPad = kD + 4;  // fp32 row pad: the 16 rows of one store hit distinct banks
  static_assert(sizeof(float) * kPvRows * kRedPad <= sizeof(sh.vt[1]), "the reduction rows fit a part's ring");
  if (part > 0) {
    float *red = reinterpret_cast<float *>(&sh.vt[part][0][0]);  // [64 rows][132]
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) *reinterpret_cast<f4 *>(&red[(wave * 16 + r) * kRedPad + 16 * cb + 4 * kap]) = o[cb];
  }
  __syncthreads();
  uint16_t *ob = reinterpret_cast<uint16_t *>(&sh.vt[0][0][0]);  // [64 rows][136]
  constexpr int kRowPad = kD + 8;
  static_assert(sizeof(uint16_t) * kPvRows * kRowPad <= sizeof(sh.vt[0]), "output staging fits part 0's ring");
  if (part == 0) {
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      f4 s = o[cb];
#pragma unroll
      for (int k = 1; k < kPvParts; ++k)
        s += *reinterpret_cast<const f4 *>(reinterpret_cast<const float *>(&sh.vt[k][0][0]) +
                                           (wave * 16 + r) * kRedPad + 16 * cb + 4 * kap);
#pragma unroll
      for (int v = 0; v < 4; ++v) ob[(wave * 16 + r) * kRowPad + 16 * cb + 4 * kap + v] = PvOp<VD>::bits(s[v]);
    }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < (kPvRows * (kD / 8) + kPvThreads - 1) / kPvThreads; ++q) {  // 16-byte chunks of whole rows
    const int c = q * kPvThreads + tid, rr = c / (kD / 8), c8 = c % (kD / 8);
    const int64_t orow = rb * kPvRows + rr;
    if (c >= kPvRows * (kD / 8) || orow >= p.rows) continue;
    const int64_t og = orow / p.Lq, oi = orow % p.Lq;
    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(p.out) + ((h * p.group + og) * p.Lq + oi) * kD + 8 * c8) =
        *reinterpret_cast<const uint4 *>(&ob[rr * kRowPad + 8 * c8]);
  }
}

// scores[h, t] (+)= sum over row blocks, in order, of the partials.
__global__ __launch_bounds__(64) void h2o_reduce_kernel(const float *partial, int64_t row_blocks, int64_t Hkv,
                                                        int64_t T, float *scores, int accumulate) {
  const int64_t idx = int64_t(blockIdx.x) * 64 + threadIdx.x;
  if (idx >= Hkv * T) return;
  const float *src = partial + idx;  // (rb * Hkv + h) * T + t = rb * Hkv * T + idx
  const int64_t stride = Hkv * T;
  float s = 0.0f;
  for (int64_t rb0 = 0; rb0 < row_blocks; rb0 += 16) {  // 16 loads in flight: config 3's 14 row blocks in one round
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = rb0 + j < row_blocks ? src[(rb0 + j) * stride] : 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s += v[j];
  }
  scores[idx] = accumulate ? scores[idx] + s : s;
}

struct HsShape {
  int64_t row_blocks, chunks, chunk;
};

HsShape h2o_shape(int64_t heads_q, int64_t heads_kv, int64_t query_len, int64_t tokens) {
  HsShape s{};
  s.row_blocks = ceil_div((heads_q / heads_kv) * query_len, int64_t(kHsRows));
  const int64_t blocks = s.row_blocks * heads_kv;
  // at most one round of workgroups: a second, mostly empty round would cost
  // as much as the first
  const int64_t want = blocks < kHsTargetBlocks ? kHsTargetBlocks / blocks : 1;
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

// 16-byte aligned rows of 128 contiguous channels, keys at least a row apart,
// and 32-bit byte offsets within a key chunk.
bool h2o_mfma_supported(int dtype, int64_t head_dim, const void *q, int64_t q_si, int64_t q_sh, int64_t q_sd,
                        const void *k, int64_t k_st, int64_t k_sh, int64_t k_sd, int64_t query_len, int64_t heads_q,
                        int64_t tokens, int64_t heads_kv) {
  const bool aligned = (reinterpret_cast<uintptr_t>(q) & 15) == 0 && (reinterpret_cast<uintptr_t>(k) & 15) == 0 &&
                       q_si % 8 == 0 && q_sh % 8 == 0 && k_st % 8 == 0 && k_sh % 8 == 0;
  if (!((dtype == UC_BF16 || dtype == UC_FP16) && head_dim == kD && q_sd == 1 && k_sd == 1 && aligned && k_st >= kD))
    return false;
  const HsShape shape = h2o_shape(heads_q, heads_kv, query_len, tokens);
  return (shape.chunk + kHsTile) * k_st * 2 < (int64_t(1) << 32) && heads_q / heads_kv * query_len < (int64_t(1) << 31);
}

// Stats first ((max, sum) per row block, chunk and row: at most
// (row blocks + target blocks) * 256 rows of 8 bytes, since chunks exceed 1
// only while row blocks * chunks stays near the target), then the partials.
int64_t h2o_mfma_workspace_bytes(int64_t heads_q, int64_t query_len, int64_t tokens) {
  const int64_t rbb = row_block_bound(heads_q, query_len);
  return (rbb + kHsTargetBlocks) * kHsRows * int64_t(sizeof(float2)) + rbb * tokens * int64_t(sizeof(float));
}

int launch_qk_logits_mfma(int dtype, const void *q, int64_t q_si, int64_t q_sh, const void *k, int64_t k_st,
                          int64_t k_sh, int64_t Lq, int64_t Hq, int64_t T, int64_t Hkv, float scale, float *logits,
                          hipStream_t stream) {
  const HsShape shape = h2o_shape(Hq, Hkv, Lq, T);
  UC_REQUIRE(shape.row_blocks * shape.chunks * Hkv < (int64_t(1) << 31), "uc_kivi_qk: grid too large");
  HsParams p{};
  p.q = static_cast<const uint16_t *>(q);
  p.q_si = q_si; p.q_sh = q_sh;
  p.k = static_cast<const uint16_t *>(k);
  p.k_st = k_st; p.k_sh = k_sh;
  p.Lq = Lq; p.Hq = Hq; p.Hkv = Hkv; p.group = Hq / Hkv; p.rows = p.group * Lq; p.T = T;
  p.row_blocks = shape.row_blocks; p.chunks = shape.chunks; p.chunk = shape.chunk;
  p.logits = logits;
  p.scale = scale;
  p.items = p.row_blocks * p.chunks * Hkv;
  p.per_xcd = ceil_div(p.items, int64_t(kXcds));
  const dim3 grid(static_cast<unsigned>(p.per_xcd * kXcds));
  if (dtype == UC_FP16)
    hipLaunchKernelGGL((qk_logits_kernel<UC_FP16>), grid, dim3(kHsThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((qk_logits_kernel<UC_BF16>), grid, dim3(kHsThreads), 0, stream, p);
  return check_launch("uc_kivi_qk (MFMA logits)");
}

// Dense P.V on MFMA: 16-bit values with unit channel stride and 8-element
// aligned token/head strides; probabilities with unit key stride whose rows
// of consecutive query heads follow each other ([Hq][Lq][>= T]).
bool pv_mfma_supported(int p_dtype, const void *probs, int64_t p_sh, int64_t p_si, int64_t p_st, int v_dtype,
                       const void *v, int64_t v_st, int64_t v_sh, int64_t head_dim, int64_t Lq, int64_t rows,
                       int64_t T) {
  const bool aligned = (reinterpret_cast<uintptr_t>(probs) & 15) == 0 && (reinterpret_cast<uintptr_t>(v) & 15) == 0 &&
                       p_sh % 8 == 0 && p_si % 8 == 0 && v_st % 8 == 0 && v_sh % 8 == 0;
  const int64_t el = p_dtype == UC_FP32 ? 4 : 2;
  return (v_dtype == UC_BF16 || v_dtype == UC_FP16) && head_dim == kD && p_st == 1 && aligned && rows >= kPvRows &&
         kD * ceil_div(T, int64_t(kPvTile)) * kPvTile * 2 < (int64_t(1) << 31) && p_si >= T && p_sh == Lq * p_si &&
         16 * p_si * el < (int64_t(1) << 31);
}

int launch_pv_mfma(int p_dtype, const void *probs, int64_t p_sh, int64_t p_si, int v_dtype, const void *v,
                   int64_t v_st, int64_t v_sh, int64_t Lq, int64_t Hq, int64_t T, int64_t Hkv, void *out,
                   void *workspace, hipStream_t stream) {
  PvParams p{};
  p.p = probs; p.p_sh = p_sh; p.p_si = p_si;
  p.vt = static_cast<const uint16_t *>(workspace);
  p.T = T; p.Tp = ceil_div(T, int64_t(kPvTile)) * kPvTile;
  p.Lq = Lq; p.Hq = Hq; p.Hkv = Hkv; p.group = Hq / Hkv; p.rows = p.group * Lq;
  p.row_blocks = ceil_div(p.rows, int64_t(kPvRows));
  p.items = p.row_blocks * Hkv;
  p.per_xcd = ceil_div(p.items, int64_t(kXcds));
  p.out = out;
  UC_REQUIRE(p.per_xcd * kXcds < (int64_t(1) << 31), "uc_kivi_av: grid too large");
  hipLaunchKernelGGL(pv_stage_kernel, dim3(static_cast<unsigned>(p.Tp / kPvTile), static_cast<unsigned>(Hkv)),
                     dim3(256), 0, stream, static_cast<const uint16_t *>(v), v_st, v_sh, T, p.Tp,
                     static_cast<uint16_t *>(workspace));
  int rc = check_launch("uc_kivi_av (V staging)");
  if (rc != UC_OK) return rc;
  const dim3 grid(static_cast<unsigned>(p.per_xcd * kXcds));
  auto go = [&](auto pd_tag) {
    constexpr int PD = decltype(pd_tag)::value;
    if (v_dtype == UC_FP16)
      hipLaunchKernelGGL((pv_mfma_kernel<PD, UC_FP16>), grid, dim3(kPvThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((pv_mfma_kernel<PD, UC_BF16>), grid, dim3(kPvThreads), 0, stream, p);
  };
  if (p_dtype == UC_BF16) go(std::integral_constant<int, UC_BF16>{});
  else if (p_dtype == UC_FP16) go(std::integral_constant<int, UC_FP16>{});
  else go(std::integral_constant<int, UC_FP32>{});
  return check_launch("uc_kivi_av (MFMA)");
}

int launch_h2o_mfma(int dtype, const void *q, int64_t q_si, int64_t q_sh, const void *k, int64_t k_st, int64_t k_sh,
                    int64_t Lq, int64_t Hq, int64_t T, int64_t Hkv, float sm_scale, const float *lse, int accumulate,
                    float *scores, void *workspace, hipStream_t stream) {
  const HsShape shape = h2o_shape(Hq, Hkv, Lq, T);
  const int64_t rbb = row_block_bound(Hq, Lq);
  UC_REQUIRE(shape.row_blocks * Hkv <= rbb && shape.row_blocks * Hkv * shape.chunks <= rbb + kHsTargetBlocks,
             "uc_h2o_scores: internal workspace bound violated");
  UC_REQUIRE(shape.row_blocks * shape.chunks * Hkv < (int64_t(1) << 31), "uc_h2o_scores: grid too large");
  HsParams p{};
  p.q = static_cast<const uint16_t *>(q);
  p.q_si = q_si; p.q_sh = q_sh;
  p.k = static_cast<const uint16_t *>(k);
  p.k_st = k_st; p.k_sh = k_sh;
  p.Lq = Lq; p.Hq = Hq; p.Hkv = Hkv; p.group = Hq / Hkv; p.rows = p.group * Lq; p.T = T;
  p.row_blocks = shape.row_blocks; p.chunks = shape.chunks; p.chunk = shape.chunk;
  p.scale_log2 = sm_scale * kLog2e;
  p.lse = lse;
  p.ml = static_cast<float2 *>(workspace);
  p.partial = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                        (rbb + kHsTargetBlocks) * kHsRows * int64_t(sizeof(float2)));
  p.items = p.row_blocks * p.chunks * Hkv;
  p.per_xcd = ceil_div(p.items, int64_t(kXcds));
  const dim3 grid(static_cast<unsigned>(p.per_xcd * kXcds));
  int rc;
  if (lse == nullptr) {
    if (dtype == UC_FP16)
      hipLaunchKernelGGL((h2o_stats_kernel<UC_FP16>), grid, dim3(kHsThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((h2o_stats_kernel<UC_BF16>), grid, dim3(kHsThreads), 0, stream, p);
    rc = check_launch("uc_h2o_scores (MFMA stats)");
    if (rc != UC_OK) return rc;
  }
  if (dtype == UC_FP16)
    hipLaunchKernelGGL((h2o_scores_kernel<UC_FP16>), grid, dim3(kHsThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((h2o_scores_kernel<UC_BF16>), grid, dim3(kHsThreads), 0, stream, p);
  rc = check_launch("uc_h2o_scores (MFMA scores)");
  if (rc != UC_OK) return rc;
  hipLaunchKernelGGL(h2o_reduce_kernel, dim3(static_cast<unsigned>(ceil_div(Hkv * T, int64_t(64)))), dim3(64), 0,
                     stream, p.partial, p.row_blocks, Hkv, T, scores, accumulate);
  return check_launch("uc_h2o_scores (MFMA reduce)");
}

}  // namespace uc
