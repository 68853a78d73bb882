// H2O attention-mass accumulation, deterministic top-k selection and the GQA
// compaction gather (operators/physical.py:51-101; physical.py:493-654).
#include "uc_common.h"
#include "uc_mfma.h"

namespace uc {

bool h2o_mfma_supported(int dtype, int64_t head_dim, const void *q, int64_t q_si, int64_t q_sh, int64_t q_sd,
                        const void *k, int64_t k_st, int64_t k_sh, int64_t k_sd, int64_t query_len, int64_t heads_q,
                        int64_t tokens, int64_t heads_kv);
int64_t h2o_mfma_workspace_bytes(int64_t heads_q, int64_t query_len, int64_t tokens);
int launch_h2o_mfma(int dtype, const void *q, int64_t q_si, int64_t q_sh, const void *k, int64_t k_st, int64_t k_sh,
                    int64_t Lq, int64_t Hq, int64_t T, int64_t Hkv, float sm_scale, const float *lse, int accumulate,
                    float *scores, void *workspace, hipStream_t stream);

namespace {

// stats[row] = (lse, 1): the generic score pass then yields exp(x - lse).
__global__ void lse_stats_kernel(const float *lse, int64_t n, float *stats) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) {
    stats[2 * i] = lse[i];
    stats[2 * i + 1] = 1.0f;
  }
}

// Zero fill (used instead of a memset node so the call can be graph-captured).
__global__ void zero_kernel(float *p, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

constexpr float kNegInf = -__builtin_huge_valf();
constexpr int kRows = 16;
constexpr int kTile = 64;
constexpr int kThreads = 256;
constexpr int kMaxD = 256;

// ----------------------------------------------------------------- scores --
struct ScoreArgs {
  const void *q;
  int64_t q_si, q_sh, q_sd;
  const void *k;
  int64_t k_st, k_sh, k_sd;
  int64_t Lq, Hq, T, Hkv, D, group, rows;
  float scale;  // sm_scale
  float *stats; // [Hq, Lq, 2]: row max and sum of exp(x - max)
  float *scores;
  int accumulate;
};

struct ScoreShared {
  float q[kRows][kMaxD];
  float red[4][kRows][kTile];
  float col[4][kTile];
};

template <int DT>
__device__ void load_rows(ScoreShared &s, const ScoreArgs &a, int64_t h, int64_t row0) {
  for (int64_t idx = threadIdx.x; idx < kRows * a.D; idx += kThreads) {
    const int64_t r = idx / a.D, d = idx % a.D;
    float v = 0.0f;
    if (row0 + r < a.rows) {
      const int64_t g = (row0 + r) / a.Lq, i = (row0 + r) % a.Lq;
      v = load_as_f32<DT>(a.q, i * a.q_si + (h * a.group + g) * a.q_sh + d * a.q_sd);
    }
    s.q[r][d] = v;
  }
}

// red[wave][r][lane] = partial q_r . k_t over the wave's quarter of channels
template <int DT>
__device__ void logits_tile(ScoreShared &s, const ScoreArgs &a, int64_t h, int64_t t) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  float acc[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) acc[r] = 0.0f;
  if (t < a.T) {
    const int64_t dq = (a.D + 3) / 4, d0 = wave * dq, d1 = min(a.D, d0 + dq);
    for (int64_t d = d0; d < d1; ++d) {
      const float k = load_as_f32<DT>(a.k, t * a.k_st + h * a.k_sh + d * a.k_sd);
#pragma unroll
      for (int r = 0; r < kRows; ++r) acc[r] = fmaf(s.q[r][d], k, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) s.red[wave][r][lane] = acc[r];
}

// Pass 1: per (KV head, 16-row chunk), the softmax max and denominator of each
// query row over all T keys.
template <int DT>
__global__ __launch_bounds__(kThreads) void score_stats_kernel(ScoreArgs a) {
  __shared__ ScoreShared s;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t h = blockIdx.y, row0 = int64_t(blockIdx.x) * kRows;
  load_rows<DT>(s, a, h, row0);
  __syncthreads();
  float m[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m[j] = kNegInf;
    l[j] = 0.0f;
  }
  for (int64_t t0 = 0; t0 < a.T; t0 += kTile) {
    const int64_t t = t0 + lane;
    logits_tile<DT>(s, a, h, t);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = wave + 4 * j;
      float x = kNegInf;
      if (t < a.T) x = (s.red[0][r][lane] + s.red[1][r][lane] + s.red[2][r][lane] + s.red[3][r][lane]) * a.scale;
      const float mn = fmaxf(m[j], wave_max(x));
      const float e = (x == kNegInf) ? 0.0f : expf(x - mn);
      l[j] = l[j] * ((m[j] == kNegInf) ? 0.0f : expf(m[j] - mn)) + wave_sum(e);
      m[j] = mn;
    }
    __syncthreads();
  }
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t rr = row0 + wave + 4 * j;
      if (rr >= a.rows) continue;
      const int64_t g = rr / a.Lq, i = rr % a.Lq, hq = h * a.group + g;
      a.stats[(hq * a.Lq + i) * 2 + 0] = m[j];
      a.stats[(hq * a.Lq + i) * 2 + 1] = l[j];
    }
  }
}

// Pass 2: per (KV head, 64-key tile), recompute the logits of every query row
// of the head, form p = bf16(exp(x - max) / sum) and sum p over rows in a
// fixed order (deterministic).
template <int DT>
__global__ __launch_bounds__(kThreads) void score_colsum_kernel(ScoreArgs a) {
  __shared__ ScoreShared s;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t h = blockIdx.y, t0 = int64_t(blockIdx.x) * kTile, t = t0 + lane;
  float col = 0.0f;
  for (int64_t row0 = 0; row0 < a.rows; row0 += kRows) {
    load_rows<DT>(s, a, h, row0);
    __syncthreads();
    logits_tile<DT>(s, a, h, t);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = wave + 4 * j;
      const int64_t rr = row0 + r;
      if (rr >= a.rows || t >= a.T) continue;
      const int64_t g = rr / a.Lq, i = rr % a.Lq, hq = h * a.group + g;
      const float mx = a.stats[(hq * a.Lq + i) * 2 + 0];
      const float sum = a.stats[(hq * a.Lq + i) * 2 + 1];
      const float x = (s.red[0][r][lane] + s.red[1][r][lane] + s.red[2][r][lane] + s.red[3][r][lane]) * a.scale;
      const float pr = expf(x - mx) * (1.0f / sum);
      col += bf16_bits_to_f32(f32_to_bf16_bits(pr));
    }
    __syncthreads();
  }
  s.col[wave][lane] = col;
  __syncthreads();
  if (wave == 0 && t < a.T) {
    const float total = s.col[0][lane] + s.col[1][lane] + s.col[2][lane] + s.col[3][lane];
    float *dst = a.scores + h * a.T + t;
    *dst = a.accumulate ? *dst + total : total;
  }
}

// ------------------------------------------------------------------ colsum --
struct ColsumArgs {
  const void *p;
  int64_t p_sh, p_si, p_st;
  int64_t Hq, Lq, T, Hkv, group;
  int accumulate;
  float *out;
};

// out[h, t] (+)= sum over (g, i) of probs[h*group+g, i, t]: the query sum of
// each query head first, then the sum over the group (physical.py:607-609).
template <int PD>
__global__ __launch_bounds__(256) void colsum_kernel(ColsumArgs a) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= a.Hkv * a.T) return;
  const int64_t h = idx / a.T, t = idx % a.T;
  float total = 0.0f;
  for (int64_t g = 0; g < a.group; ++g) {
    float s = 0.0f;
    const int64_t base = (h * a.group + g) * a.p_sh + t * a.p_st;
    for (int64_t i = 0; i < a.Lq; ++i) s += load_as_f32<PD>(a.p, base + i * a.p_si);
    total += s;
  }
  a.out[idx] = a.accumulate ? a.out[idx] + total : total;
}

// Unit token stride: one workgroup per (KV head, 64 tokens), lane = token;
// wave w sums the rows of query heads w, w + 8, ... in row order, 64 loads
// in flight, and wave 0 adds the heads in order -- the same additions
// as colsum_kernel, so the same result.
constexpr int kCsWaves = 8;
constexpr int kCsMaxGroup = 64;
constexpr int kCsBatch = 64;  // loads in flight per wave: a CU's 7-8 waves keep ~60 KB moving

template <int PD>
__global__ __launch_bounds__(kCsWaves * kWave) void colsum_rows_kernel(ColsumArgs a) {
  __shared__ float part[kCsMaxGroup][kWave];
  constexpr int kEl = PD == UC_FP32 ? 4 : 2;
  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform (scalar) so the buffer resources below stay in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t tiles = (a.T + kWave - 1) / kWave;
  const int64_t h = blockIdx.x / tiles, t = (blockIdx.x % tiles) * kWave + lane;
  const int64_t tc = t < a.T ? t : a.T - 1;  // lanes past the end read the last column and store nothing
  const uint32_t voff = static_cast<uint32_t>(tc * kEl);
  for (int64_t g = wave; g < a.group; g += kCsWaves) {
    // the query head's rows through one buffer resource: the row offset is the
    // same for every lane, so it rides in the scalar offset
    const mf::Rsrc rs = mf::make_rsrc(static_cast<const char *>(a.p) + (h * a.group + g) * a.p_sh * kEl,
                                      a.Lq * a.p_si * kEl);
    const uint32_t row_bytes = static_cast<uint32_t>(a.p_si * kEl);
    float s = 0.0f;
    for (int64_t i0 = 0; i0 < a.Lq; i0 += kCsBatch) {
      float v[kCsBatch];
#pragma unroll
      for (int j = 0; j < kCsBatch; ++j) {
        const uint32_t soff = static_cast<uint32_t>(i0 + j) * row_bytes;  // rows past Lq read zero
        if constexpr (PD == UC_FP32)
          v[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0));
        else
          v[j] = half_bits_to_f32<PD>(__builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff, 0));
      }
#pragma unroll
      for (int j = 0; j < kCsBatch; ++j) s += v[j];  // + 0 past the last row: s starts at +0, so it is never -0
    }
    part[g][lane] = s;
  }
  __syncthreads();
  if (wave == 0 && t < a.T) {
    float total = 0.0f;
    for (int64_t g = 0; g < a.group; ++g) total += part[g][lane];
    float *dst = a.out + h * a.T + t;
    *dst = a.accumulate ? *dst + total : total;
  }
}

// ------------------------------------------------------------------ select --
constexpr int kSelThreads = 1024;

// Order-preserving map of fp32 to uint32 (larger float -> larger key); NaN is
// canonicalised to the largest key, matching torch.topk's NaN-is-largest.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct SelectArgs {
  const float *scores;
  int64_t s_sh, s_st;
  int64_t T, heavy_k, recent;
  int64_t *indices;
};

// One workgroup per KV head.  A four-pass 8-bit radix select finds the key of
// the heavy_k-th largest score; tokens strictly above it are all kept and
// equal ones are taken in ascending index order until heavy_k are chosen.
// An ordered block scan writes the kept indices in ascending order.
// Each pass counts into per-wave histograms (scores of a head share their top
// bytes, so one shared histogram would serialise on a few bins), sums them per
// bin, and wave 0 finds the bin holding the threshold with a suffix scan over
// its lanes (4 bins each).  With REGS, the head's candidates (at most
// kSelThreads * kSelRegs) are read once into registers and every pass and the
// scan run on them; otherwise each pass reads the scores again.
constexpr int kSelWaves = kSelThreads / kWave;
constexpr int kSelRegs = 8;

template <bool REGS>
__global__ __launch_bounds__(kSelThreads) void h2o_select_kernel(SelectArgs a) {
  __shared__ uint32_t whist[kSelWaves][256];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t sh_prefix, sh_need;
  __shared__ uint32_t wave_tot[2][kSelWaves];
  const int64_t h = blockIdx.x;
  const int64_t hist_end = a.T - a.recent;
  const float *sc = a.scores + h * a.s_sh;
  int64_t *out = a.indices + h * (a.heavy_k + a.recent);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;

  if (a.heavy_k > 0) {
    // candidate keys of this thread (REGS): token r * kSelThreads + tid
    uint32_t keys[REGS ? kSelRegs : 1];
    if constexpr (REGS) {
      // every load issued before any is used; tokens past the history read token 0
      float v[kSelRegs];
#pragma unroll
      for (int r = 0; r < kSelRegs; ++r) {
        const int64_t t = int64_t(r) * kSelThreads + tid;
        v[r] = sc[(t < hist_end ? t : 0) * a.s_st];
      }
#pragma unroll
      for (int r = 0; r < kSelRegs; ++r) keys[r] = int64_t(r) * kSelThreads + tid < hist_end ? order_key(v[r]) : 0u;
    }
    uint32_t prefix = 0, mask = 0;
    uint32_t need = static_cast<uint32_t>(a.heavy_k);
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      for (int i = tid; i < kSelWaves * 256; i += kSelThreads) (&whist[0][0])[i] = 0;
      __syncthreads();
      if constexpr (REGS) {
#pragma unroll
        for (int r = 0; r < kSelRegs; ++r) {
          const int64_t t = int64_t(r) * kSelThreads + tid;
          if (t < hist_end && (keys[r] & mask) == prefix) atomicAdd(&whist[wave][(keys[r] >> shift) & 255u], 1u);
        }
      } else {
        for (int64_t t = tid; t < hist_end; t += kSelThreads) {
          const uint32_t key = order_key(sc[t * a.s_st]);
          if ((key & mask) == prefix) atomicAdd(&whist[wave][(key >> shift) & 255u], 1u);
        }
      }
      __syncthreads();
      if (tid < 256) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < kSelWaves; ++w) c += whist[w][tid];
        hist[tid] = c;
      }
      __syncthreads();
      if (wave == 0) {
        // lane l owns bins 4l .. 4l + 3; above = count in bins above lane l's
        const uint32_t b0 = hist[4 * lane], b1 = hist[4 * lane + 1], b2 = hist[4 * lane + 2], b3 = hist[4 * lane + 3];
        const uint32_t mine = b0 + b1 + b2 + b3;
        uint32_t incl = mine;  // suffix sum over lanes >= l
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
          const uint32_t v = __shfl_down(incl, o, kWave);
          if (lane + o < kWave) incl += v;
        }
        const uint32_t above = incl - mine;
        // the threshold bin is in the lane whose range crosses `need` (the
        // lowest bin, 0, takes whatever is left)
        const bool here = above < need && (incl >= need || lane == 0);
        if (here) {
          uint32_t acc = above;
          int b = 4 * lane + 3;
          const uint32_t bins[4] = {b0, b1, b2, b3};
#pragma unroll
          for (int j = 3; j > 0; --j) {
            if (acc + bins[j] >= need) break;
            acc += bins[j];
            --b;
          }
          sh_prefix = prefix | (uint32_t(b) << shift);
          sh_need = need - acc;
        }
      }
      __syncthreads();
      prefix = sh_prefix;
      need = sh_need;
      mask |= 255u << shift;
      __syncthreads();
    }
    // prefix is the threshold key; `need` tokens equal to it are kept.
    uint32_t base_sel = 0, base_eq = 0;
    for (int64_t c0 = 0; c0 < hist_end; c0 += kSelThreads) {
      const int64_t t = c0 + tid;
      uint32_t key = 0;
      if constexpr (REGS) {
        // chunk c0 / kSelThreads of the register keys (uniform index)
#pragma unroll
        for (int r = 0; r < kSelRegs; ++r)
          if (c0 == int64_t(r) * kSelThreads) key = keys[r];
      } else if (t < hist_end) {
        key = order_key(sc[t * a.s_st]);
      }
      const bool eq = t < hist_end && key == prefix;
      const bool gt = t < hist_end && key > prefix;
      // exclusive scan of eq, then of selection
      const uint64_t eq_ball = __ballot(eq);
      const uint32_t eq_before_lane = __popcll(eq_ball & ((1ull << lane) - 1ull));
      if (lane == 0) wave_tot[0][wave] = __popcll(eq_ball);
      __syncthreads();
      uint32_t eq_before = base_eq + eq_before_lane;
      for (int w = 0; w < wave; ++w) eq_before += wave_tot[0][w];
      const bool sel = gt || (eq && eq_before < need);
      const uint64_t sel_ball = __ballot(sel);
      const uint32_t sel_before_lane = __popcll(sel_ball & ((1ull << lane) - 1ull));
      if (lane == 0) wave_tot[1][wave] = __popcll(sel_ball);
      __syncthreads();
      uint32_t sel_before = base_sel + sel_before_lane;
      for (int w = 0; w < wave; ++w) sel_before += wave_tot[1][w];
      if (sel) out[sel_before] = t;
      uint32_t tot_eq = 0, tot_sel = 0;
      for (int w = 0; w < kSelWaves; ++w) {
        tot_eq += wave_tot[0][w];
        tot_sel += wave_tot[1][w];
      }
      base_eq += tot_eq;
      base_sel += tot_sel;
      __syncthreads();
    }
  }
  for (int64_t j = tid; j < a.recent; j += kSelThreads) out[a.heavy_k + j] = hist_end + j;
}

// ------------------------------------------------------------------ gather --
struct GatherArgs {
  const void *key, *value;
  int64_t k_st, k_sh, k_sd;
  int64_t Hkv, D, R;
  const int64_t *idx;
  const int64_t *ids;
  int64_t ids_sh, ids_st;
  const float *scores;
  int64_t s_sh, s_st;
  void *okey, *ovalue;
  int64_t *oids;
  float *oscores;
};

template <typename E>
__global__ __launch_bounds__(256) void gqa_gather_kernel(GatherArgs a) {
  // one thread per output element of [Hkv, R, D]
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= a.Hkv * a.R * a.D) return;
  const int64_t d = idx % a.D, j = (idx / a.D) % a.R, h = idx / (a.D * a.R);
  const int64_t r = a.idx[h * a.R + j];
  const int64_t src = r * a.k_st + h * a.k_sh + d * a.k_sd;
  static_cast<E *>(a.okey)[idx] = static_cast<const E *>(a.key)[src];
  static_cast<E *>(a.ovalue)[idx] = static_cast<const E *>(a.value)[src];
  if (d == 0) {
    if (a.oids) a.oids[h * a.R + j] = a.ids[h * a.ids_sh + r * a.ids_st];
    if (a.oscores) a.oscores[h * a.R + j] = a.scores[h * a.s_sh + r * a.s_st];
  }
}


// --------------------------------------- select + gather of several segments --
// One launch for up to kSgMaxSegs H2O segments (uc_h2o_segment each).  A
// workgroup serves (segment, KV head, part): it selects the head's kept tokens
// itself -- the parts of a head repeat the selection, which costs far less
// than a second launch -- and gathers its part of the kept rows.
//
// Selection.  The heavy_k-th largest order key th is found bit pair by bit
// pair from the top: with th's higher bits fixed, the block counts the keys
// >= th | 1 << b, th | 2 << b and th | 3 << b (counted per wave by ballots,
// summed over the 16 waves by one 64-bit LDS add each, one barrier per pair)
// and keeps the largest candidate that still has heavy_k keys at or above it.  Keys above th are all kept; keys equal to th are kept
// in ascending token order until heavy_k are chosen (torch.topk's tie rule as
// the reference applies it, physical.py:516-527).  A token's place in the
// ascending output is (#kept-above before it) + min(#equal before it, need):
// one block scan of per-(chunk, wave) counts gives both prefixes.  The recent
// window follows (physical.py:528-531).
constexpr int kSgMaxSegs = 8;
constexpr int kSgThreads = 1024;
constexpr int kSgWaves = kSgThreads / kWave;
constexpr int kSgRegs = 8;                          // keys per thread: history <= 8192 tokens
constexpr int kSgMaxKeep = kSgThreads * kSgRegs;    // kept rows held in LDS

struct SgArgs {
  uc_h2o_segment seg[kSgMaxSegs];
  int wg_begin[kSgMaxSegs + 1];  // first workgroup of each segment
  int parts[kSgMaxSegs];         // workgroups per KV head
  int64_t Hkv, D;
};

__global__ __launch_bounds__(kSgThreads) void h2o_select_gather_kernel(SgArgs a) {
  __shared__ unsigned long long cnt[3];  // block counts of one bit pair, 21 bits each
  __shared__ uint32_t tab[2][kSgRegs * kSgWaves];  // gt / eq counts per (chunk, wave), then prefixes
  __shared__ uint32_t totals[2];
  __shared__ int32_t keep[kSgMaxKeep];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  int si = 0;
  while (si + 1 < kSgMaxSegs && int(blockIdx.x) >= a.wg_begin[si + 1]) ++si;
  const uc_h2o_segment &g = a.seg[si];
  const int local = int(blockIdx.x) - a.wg_begin[si];
  const int64_t h = local / a.parts[si];
  const int part = local % a.parts[si];
  const int64_t hist_end = g.tokens - g.recent, R = g.heavy_k + g.recent;
  const uint32_t heavy = uint32_t(g.heavy_k);
  const float *sc = g.scores + h * g.s_sh;

  if (heavy > 0) {
    // every load issued before any is used (a load under the token test would
    // be waited for one at a time); tokens past the history read token 0
    float v[kSgRegs];
#pragma unroll
    for (int r = 0; r < kSgRegs; ++r) {
      const int64_t t = int64_t(r) * kSgThreads + tid;
      v[r] = sc[(t < hist_end ? t : 0) * g.s_st];
    }
    uint32_t keys[kSgRegs];
#pragma unroll
    for (int r = 0; r < kSgRegs; ++r)  // order keys of real scores are never 0
      keys[r] = int64_t(r) * kSgThreads + tid < hist_end ? order_key(v[r]) : 0u;
    if (tid == 0) cnt[0] = 0;
    __syncthreads();
    uint32_t th = 0;
    for (int it = 0; it < 16; ++it) {
      const int b = 30 - 2 * it;
      const uint32_t c1 = th | (1u << b), c2 = th | (2u << b), c3 = th | (3u << b);
      // wave counts by ballots (keys of invalid tokens are 0, below every
      // candidate): at most 512 per wave, 8192 per block
      uint32_t n1 = 0, n2 = 0, n3 = 0;
#pragma unroll
      for (int r = 0; r < kSgRegs; ++r) {
        n1 += __popcll(__ballot(keys[r] >= c1));
        n2 += __popcll(__ballot(keys[r] >= c2));
        n3 += __popcll(__ballot(keys[r] >= c3));
      }
      // one 64-bit LDS add per wave sums the three counts over the block.
      // Slots rotate over three words: slot it % 3 was cleared in round
      // it - 1, and slot (it + 1) % 3 was last read in round it - 2, before
      // every wave reached the previous barrier.
      if (lane == 0) {
        if (wave == 0) cnt[(it + 1) % 3] = 0;
        atomicAdd(&cnt[it % 3], (unsigned long long)n1 | (unsigned long long)n2 << 21 |
                                    (unsigned long long)n3 << 42);
      }
      __syncthreads();
      const unsigned long long sum = cnt[it % 3];
      const uint32_t s1 = uint32_t(sum) & 0x1fffffu, s2 = uint32_t(sum >> 21) & 0x1fffffu, s3 = uint32_t(sum >> 42);
      th = s3 >= heavy ? c3 : s2 >= heavy ? c2 : s1 >= heavy ? c1 : th;
    }
    // per (chunk, wave) counts of keys above / equal to th
    uint64_t gt_ball[kSgRegs], eq_ball[kSgRegs];
#pragma unroll
    for (int r = 0; r < kSgRegs; ++r) {
      const bool ok = int64_t(r) * kSgThreads + tid < hist_end;
      gt_ball[r] = __ballot(ok && keys[r] > th);
      eq_ball[r] = __ballot(ok && keys[r] == th);
      if (lane == 0) {
        tab[0][r * kSgWaves + wave] = __popcll(gt_ball[r]);
        tab[1][r * kSgWaves + wave] = __popcll(eq_ball[r]);
      }
    }
    __syncthreads();
    if (wave == 0) {  // exclusive scans of the 128 (chunk, wave) counts, chunk-major
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint32_t x0 = tab[k][2 * lane], x1 = tab[k][2 * lane + 1];
        uint32_t incl = x0 + x1;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
          const uint32_t y = __shfl_up(incl, o, kWave);
          if (lane >= o) incl += y;
        }
        const uint32_t excl = incl - x0 - x1;
        tab[k][2 * lane] = excl;
        tab[k][2 * lane + 1] = excl + x0;
        if (lane == kWave - 1) totals[k] = incl;
      }
    }
    __syncthreads();
    const uint32_t need = heavy - totals[0];  // equal keys to keep, lowest tokens first
    const uint64_t below = (uint64_t(1) << lane) - 1u;
#pragma unroll
    for (int r = 0; r < kSgRegs; ++r) {
      const bool gt = (gt_ball[r] >> lane) & 1u, eq = (eq_ball[r] >> lane) & 1u;
      if (!gt && !eq) continue;
      const uint32_t gb = tab[0][r * kSgWaves + wave] + __popcll(gt_ball[r] & below);
      const uint32_t eb = tab[1][r * kSgWaves + wave] + __popcll(eq_ball[r] & below);
      if (gt || eb < need) keep[gb + (eb < need ? eb : need)] = r * kSgThreads + tid;
    }
  }
  for (int64_t k = tid; k < g.recent; k += kSgThreads) keep[g.heavy_k + k] = int32_t(hist_end + k);
  __syncthreads();

  // gather this part's rows: 16-byte chunks of the K and V rows
  const int64_t per = (R + a.parts[si] - 1) / a.parts[si];
  const int64_t j0 = part * per, j1 = j0 + per < R ? j0 + per : R;
  const int chunks = int(a.D / 8);  // 16-byte chunks per 16-bit row
  const int rows_per = kSgThreads / chunks;
  const int c = tid % chunks;
  for (int64_t j = j0 + tid / chunks; j < j1; j += rows_per) {
    const int64_t r = keep[j];
    const int64_t src = r * g.k_st + h * g.k_sh + int64_t(c) * 8, dst = (h * R + j) * a.D + int64_t(c) * 8;
    const uint4 kv = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g.key) + src);
    const uint4 vv = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(g.value) + src);
    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(g.out_key) + dst) = kv;
    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(g.out_value) + dst) = vv;
  }
  for (int64_t j = j0 + tid; j < j1; j += kSgThreads) {
    const int64_t r = keep[j];
    g.indices[h * R + j] = r;
    if (g.out_ids) g.out_ids[h * R + j] = g.ids[h * g.ids_sh + r * g.ids_st];
    if (g.out_scores) g.out_scores[h * R + j] = sc[r * g.s_st];
  }
}

}  // namespace
}  // namespace uc

using namespace uc;

namespace uc {
namespace {

int h2o_scores_impl(const void *query, int64_t q_si, int64_t q_sh, int64_t q_sd, const void *key, int64_t k_st,
                    int64_t k_sh, int64_t k_sd, int dtype, int64_t query_len, int64_t heads_q, int64_t tokens,
                    int64_t heads_kv, int64_t head_dim, float sm_scale, const float *lse, int accumulate,
                    float *scores, void *workspace, uc_stream_t stream) {
  UC_REQUIRE(valid_dtype(dtype), "uc_h2o_scores: unknown dtype code");
  UC_REQUIRE(heads_q > 0 && heads_kv > 0 && heads_q % heads_kv == 0,
             "BAGEL query heads must be divisible by KV heads");
  UC_REQUIRE(head_dim > 0 && head_dim <= kMaxD, "uc_h2o_scores: head_dim must be <= %d", kMaxD);
  UC_REQUIRE(query_len >= 0 && tokens >= 0, "uc_h2o_scores: bad shape");
  UC_REQUIRE(workspace != nullptr || query_len == 0, "uc_h2o_scores: workspace is NULL");
  hipStream_t s = as_stream(stream);
  if (tokens == 0) return UC_OK;
  if (query_len == 0) {
    if (!accumulate) {
      hipLaunchKernelGGL(zero_kernel, dim3(static_cast<unsigned>(ceil_div(heads_kv * tokens, int64_t(256)))),
                         dim3(256), 0, s, scores, heads_kv * tokens);
      return check_launch("uc_h2o_scores (zero)");
    }
    return UC_OK;
  }
  if (h2o_mfma_supported(dtype, head_dim, query, q_si, q_sh, q_sd, key, k_st, k_sh, k_sd, query_len, heads_q, tokens,
                         heads_kv))
    return launch_h2o_mfma(dtype, query, q_si, q_sh, key, k_st, k_sh, query_len, heads_q, tokens, heads_kv, sm_scale,
                           lse, accumulate, scores, workspace, s);
  ScoreArgs a{};
  a.q = query; a.q_si = q_si; a.q_sh = q_sh; a.q_sd = q_sd;
  a.k = key; a.k_st = k_st; a.k_sh = k_sh; a.k_sd = k_sd;
  a.Lq = query_len; a.Hq = heads_q; a.T = tokens; a.Hkv = heads_kv; a.D = head_dim;
  a.group = heads_q / heads_kv; a.rows = a.group * query_len; a.scale = sm_scale;
  a.stats = static_cast<float *>(workspace); a.scores = scores; a.accumulate = accumulate;
  if (lse != nullptr)
    hipLaunchKernelGGL(lse_stats_kernel, dim3(static_cast<unsigned>(ceil_div(heads_q * query_len, int64_t(256)))),
                       dim3(256), 0, s, lse, heads_q * query_len, a.stats);
  UC_DISPATCH_DTYPE(dtype, DT, [&] {
    if (lse == nullptr)
      hipLaunchKernelGGL((score_stats_kernel<DT>), dim3(ceil_div(a.rows, kRows), heads_kv), dim3(kThreads), 0, s, a);
    hipLaunchKernelGGL((score_colsum_kernel<DT>), dim3(ceil_div(tokens, kTile), heads_kv), dim3(kThreads), 0, s, a);
  });
  return check_launch("uc_h2o_scores");
}

}  // namespace
}  // namespace uc

extern "C" int uc_h2o_scores(const void *query, int64_t q_si, int64_t q_sh, int64_t q_sd,
                             const void *key, int64_t k_st, int64_t k_sh, int64_t k_sd, int dtype,
                             int64_t query_len, int64_t heads_q, int64_t tokens, int64_t heads_kv,
                             int64_t head_dim, float sm_scale, int accumulate,
                             float *scores, void *workspace, uc_stream_t stream) {
  return uc::h2o_scores_impl(query, q_si, q_sh, q_sd, key, k_st, k_sh, k_sd, dtype, query_len, heads_q, tokens,
                             heads_kv, head_dim, sm_scale, nullptr, accumulate, scores, workspace, stream);
}

extern "C" int uc_h2o_scores_lse(const void *query, int64_t q_si, int64_t q_sh, int64_t q_sd,
                                 const void *key, int64_t k_st, int64_t k_sh, int64_t k_sd, int dtype,
                                 int64_t query_len, int64_t heads_q, int64_t tokens, int64_t heads_kv,
                                 int64_t head_dim, float sm_scale, const float *lse, int accumulate,
                                 float *scores, void *workspace, uc_stream_t stream) {
  UC_REQUIRE(lse != nullptr || query_len == 0, "uc_h2o_scores_lse: lse is NULL");
  return uc::h2o_scores_impl(query, q_si, q_sh, q_sd, key, k_st, k_sh, k_sd, dtype, query_len, heads_q, tokens,
                             heads_kv, head_dim, sm_scale, lse, accumulate, scores, workspace, stream);
}

extern "C" int uc_h2o_colsum(const void *probs, int p_dtype, int64_t p_sh, int64_t p_si, int64_t p_st,
                             int64_t heads_q, int64_t query_len, int64_t tokens, int64_t heads_kv,
                             int accumulate, float *out, uc_stream_t stream) {
  UC_REQUIRE(valid_dtype(p_dtype), "uc_h2o_colsum: unknown dtype code");
  UC_REQUIRE(heads_q > 0 && heads_kv > 0 && heads_q % heads_kv == 0,
             "Query heads must be divisible by KV heads for GQA H2O");
  UC_REQUIRE(query_len >= 0 && tokens >= 0, "uc_h2o_colsum: bad shape");
  if (tokens == 0) return UC_OK;
  ColsumArgs a{};
  a.p = probs; a.p_sh = p_sh; a.p_si = p_si; a.p_st = p_st;
  a.Hq = heads_q; a.Lq = query_len; a.T = tokens; a.Hkv = heads_kv; a.group = heads_q / heads_kv;
  a.accumulate = accumulate; a.out = out;
  hipStream_t s = as_stream(stream);
  const int64_t el = p_dtype == UC_FP32 ? 4 : 2;
  if (p_st == 1 && a.group <= kCsMaxGroup && p_si * el * (query_len + kCsBatch) < (int64_t(1) << 31)) {
    const int64_t blocks = heads_kv * ceil_div(tokens, int64_t(kWave));
    UC_DISPATCH_DTYPE(p_dtype, PD, [&] {
      hipLaunchKernelGGL((colsum_rows_kernel<PD>), dim3(blocks), dim3(kCsWaves * kWave), 0, s, a);
    });
    return check_launch("uc_h2o_colsum");
  }
  UC_DISPATCH_DTYPE(p_dtype, PD, [&] {
    hipLaunchKernelGGL((colsum_kernel<PD>), dim3(ceil_div(heads_kv * tokens, 256)), dim3(256), 0, s, a);
  });
  return check_launch("uc_h2o_colsum");
}

extern "C" int uc_h2o_select(const float *scores, int64_t s_sh, int64_t s_st, int64_t heads_kv, int64_t tokens,
                             int64_t heavy_k, int64_t recent, int64_t *indices, uc_stream_t stream) {
  UC_REQUIRE(heads_kv >= 0 && tokens >= 0 && heavy_k >= 0 && recent >= 0, "uc_h2o_select: negative size");
  UC_REQUIRE(recent <= tokens && heavy_k <= tokens - recent,
             "uc_h2o_select: heavy_k + recent exceeds the token count");
  UC_REQUIRE(tokens < (int64_t(1) << 31), "uc_h2o_select: too many tokens");
  if (heads_kv == 0 || heavy_k + recent == 0) return UC_OK;
  SelectArgs a{};
  a.scores = scores; a.s_sh = s_sh; a.s_st = s_st; a.T = tokens; a.heavy_k = heavy_k; a.recent = recent;
  a.indices = indices;
  if (tokens - recent <= int64_t(kSelThreads) * kSelRegs)
    hipLaunchKernelGGL(h2o_select_kernel<true>, dim3(heads_kv), dim3(kSelThreads), 0, as_stream(stream), a);
  else
    hipLaunchKernelGGL(h2o_select_kernel<false>, dim3(heads_kv), dim3(kSelThreads), 0, as_stream(stream), a);
  return check_launch("uc_h2o_select");
}

extern "C" int uc_gqa_gather(const void *key, const void *value, int64_t k_st, int64_t k_sh, int64_t k_sd,
                             int dtype, int64_t heads_kv, int64_t head_dim,
                             const int64_t *indices, int64_t retained,
                             const int64_t *ids, int64_t ids_sh, int64_t ids_st,
                             const float *scores, int64_t s_sh, int64_t s_st,
                             void *out_key, void *out_value, int64_t *out_ids, float *out_scores,
                             uc_stream_t stream) {
  UC_REQUIRE(valid_dtype(dtype), "uc_gqa_gather: unknown dtype code");
  UC_REQUIRE(heads_kv >= 0 && head_dim > 0 && retained >= 0, "uc_gqa_gather: bad shape");
  UC_REQUIRE((ids == nullptr) == (out_ids == nullptr), "uc_gqa_gather: ids and out_ids go together");
  UC_REQUIRE((scores == nullptr) == (out_scores == nullptr), "uc_gqa_gather: scores and out_scores go together");
  if (heads_kv == 0 || retained == 0) return UC_OK;
  GatherArgs a{};
  a.key = key; a.value = value; a.k_st = k_st; a.k_sh = k_sh; a.k_sd = k_sd;
  a.Hkv = heads_kv; a.D = head_dim; a.R = retained; a.idx = indices;
  a.ids = ids; a.ids_sh = ids_sh; a.ids_st = ids_st; a.scores = scores; a.s_sh = s_sh; a.s_st = s_st;
  a.okey = out_key; a.ovalue = out_value; a.oids = out_ids; a.oscores = out_scores;
  const int64_t blocks = ceil_div(heads_kv * retained * head_dim, 256);
  hipStream_t s = as_stream(stream);
  if (dtype == UC_FP32)
    hipLaunchKernelGGL((gqa_gather_kernel<float>), dim3(blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((gqa_gather_kernel<uint16_t>), dim3(blocks), dim3(256), 0, s, a);
  return check_launch("uc_gqa_gather");
}

extern "C" int uc_h2o_select_gather(const void *key, const void *value, int64_t k_st, int64_t k_sh, int64_t k_sd,
                                    int dtype, int64_t heads_kv, int64_t tokens, int64_t head_dim,
                                    const float *scores, int64_t s_sh, int64_t s_st, int64_t heavy_k,
                                    int64_t recent, const int64_t *ids, int64_t ids_sh, int64_t ids_st,
                                    int64_t *indices, void *out_key, void *out_value, int64_t *out_ids,
                                    float *out_scores, uc_stream_t stream) {
  UC_REQUIRE(scores != nullptr && indices != nullptr, "uc_h2o_select_gather: scores and indices are required");
  int rc = uc_h2o_select(scores, s_sh, s_st, heads_kv, tokens, heavy_k, recent, indices, stream);
  if (rc != UC_OK) return rc;
  return uc_gqa_gather(key, value, k_st, k_sh, k_sd, dtype, heads_kv, head_dim, indices, heavy_k + recent, ids,
                       ids_sh, ids_st, scores, s_sh, s_st, out_key, out_value, out_ids, out_scores, stream);
}

extern "C" int uc_h2o_select_gather_segments(const uc_h2o_segment *segments, int n_segments, int dtype,
                                             int64_t heads_kv, int64_t head_dim, uc_stream_t stream) {
  UC_REQUIRE(valid_dtype(dtype), "uc_h2o_select_gather_segments: unknown dtype code");
  UC_REQUIRE(n_segments >= 0 && (n_segments == 0 || segments != nullptr),
             "uc_h2o_select_gather_segments: segments is NULL");
  UC_REQUIRE(heads_kv > 0 && head_dim > 0, "uc_h2o_select_gather_segments: bad shape");
  SgArgs a{};
  a.Hkv = heads_kv;
  a.D = head_dim;
  int n = 0, wg = 0;
  const int64_t el = dtype == UC_FP32 ? 4 : 2;
  for (int i = 0; i < n_segments; ++i) {
    const uc_h2o_segment &g = segments[i];
    UC_REQUIRE(g.scores != nullptr && g.indices != nullptr && g.key != nullptr && g.value != nullptr,
               "uc_h2o_select_gather_segments: segment %d lacks scores, indices, key or value", i);
    UC_REQUIRE((g.ids == nullptr) == (g.out_ids == nullptr),
               "uc_h2o_select_gather_segments: ids and out_ids go together (segment %d)", i);
    UC_REQUIRE(g.tokens >= 0 && g.heavy_k >= 0 && g.recent >= 0 && g.recent <= g.tokens &&
                   g.heavy_k <= g.tokens - g.recent,
               "uc_h2o_select_gather_segments: heavy_k + recent exceeds the token count (segment %d)", i);
    const int64_t R = g.heavy_k + g.recent;
    if (R == 0) continue;
    // one launch takes 16-bit rows read as 16-byte chunks and a history of at
    // most kSgMaxKeep tokens; other segments run as uc_h2o_select_gather
    const bool fits = el == 2 && head_dim % 8 == 0 && g.k_sd == 1 && g.k_st % 8 == 0 && g.k_sh % 8 == 0 &&
                      (reinterpret_cast<uintptr_t>(g.key) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(g.value) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(g.out_key) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(g.out_value) & 15) == 0 && g.tokens <= kSgMaxKeep &&
                      n < kSgMaxSegs;
    if (!fits) {
      const int rc = uc_h2o_select_gather(g.key, g.value, g.k_st, g.k_sh, g.k_sd, dtype, heads_kv, g.tokens, head_dim,
                                          g.scores, g.s_sh, g.s_st, g.heavy_k, g.recent, g.ids, g.ids_sh, g.ids_st,
                                          g.indices, g.out_key, g.out_value, g.out_ids, g.out_scores, stream);
      if (rc != UC_OK) return rc;
      continue;
    }
    a.seg[n] = g;
    a.parts[n] = int(R > 16 * 128 ? 16 : (R + 127) / 128);
    a.wg_begin[n] = wg;
    wg += int(heads_kv) * a.parts[n];
    ++n;
  }
  if (n == 0) return UC_OK;
  for (int i = n; i <= kSgMaxSegs; ++i) a.wg_begin[i] = wg;
  hipLaunchKernelGGL(h2o_select_gather_kernel, dim3(wg), dim3(kSgThreads), 0, as_stream(stream), a);
  return check_launch("uc_h2o_select_gather_segments");
}
