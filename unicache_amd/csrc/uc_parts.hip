// attention_parts over the kernel-native 2/4-bit layout (head_dim 128): the
// scaled logits [Hq, Lq, Tq + Tr] of the packed prefix and the residual
// (storage/kivi_cuda.py:238-287) and the P.V product of given probabilities
// (kivi_cuda.py:289-327), for up to 16 query rows per KV head at a time.
//
// parts_qk_kernel: one workgroup per (64-token tile, KV head, 16-row chunk).
//   The tile's key words, its groups' scales and minima (as fp32) and the
//   chunk's query rows (fp32, channel-major) are staged in LDS once; lane t
//   then forms key channel d of token t as code * scale + minimum in fp32 (the
//   dequantisation of physical.py:190-201) and wave w accumulates every live
//   row over channels 32w .. 32w + 31; the four quarters meet in LDS.  Residual
//   tokens of the tile are read from LDS-staged 16-bit rows.  Logits leave as
//   whole 64-token runs per row.
// parts_av_kernel: one workgroup per (token split, KV head, chunk of 8 or 16
//   rows); thread (row r, 8-channel slice, token phase) accumulates
//   P[r, t] * value(t, channels) in fp32 over the split, 64 tokens at a time: the chunk's probabilities, value
//   words and value statistics are staged in LDS first.  Partials
//   [Hq, Lq, split, D] are summed in split order by parts_av_reduce_kernel,
//   which writes the output dtype.
#include "uc_common.h"
#include "uc_decode.h"

namespace uc {
namespace {

constexpr int kPD = 128;       // head_dim
constexpr int kPRows = 16;     // query rows per workgroup
constexpr int kPTile = 64;     // tokens per QK workgroup
constexpr int kPThreads = 256;

struct PartsArgs {
  // token-major storage of `cap` tokens per head (uc_kivi_pack's layout)
  const uint32_t *kc, *vc;
  const void *ks, *km, *vs, *vm;
  int sd;  // stats dtype (fp16 / bf16)
  int64_t cap, Tq, Tr, T;
  int64_t Hq, Hkv, Lq, group, rows;
  int G;
  const void *rk, *rv;  // residual rows, channel stride 1
  int rd;
  int64_t r_st, r_sh;
  // QK
  const void *q;
  int qd;
  float sm_scale;
  float *logits;  // [Hq, Lq, T]
  // AV
  const void *p;
  int pd;
  int64_t p_sh, p_si, p_st;
  int64_t split, splits;
  float *partial;  // [Hq, Lq, splits, D]
  void *out;       // [Hq, Lq, D]
  int od;
};

__device__ __forceinline__ float stat_f32(const void *p, int64_t i, int sd) {
  const uint16_t b = static_cast<const uint16_t *>(p)[i];
  return sd == UC_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Query head and row of chunk row r (r = g * Lq + i of KV head h).
__device__ __forceinline__ void row_of(const PartsArgs &a, int64_t h, int64_t rr, int64_t &hq, int64_t &i) {
  const int64_t g = rr / a.Lq;
  i = rr - g * a.Lq;
  hq = h * a.group + g;
}

template <int BITS>
__global__ __launch_bounds__(kPThreads) void parts_qk_kernel(PartsArgs a) {
  constexpr int kPer = 32 / BITS, kWordRows = kPTile / kPer;
  __shared__ float qs[kPD][kPRows];          // query chunk, channel-major
  __shared__ float ss[4][kPD], ms[4][kPD];   // the tile's groups (at most 4: G >= 16)
  __shared__ uint32_t kw[kWordRows][kPD];    // the tile's key words
  __shared__ uint16_t rk[kPTile][kPD + 8];   // the tile's residual rows (16-bit)
  __shared__ float red[4][kPRows][kPTile];   // per-wave partial logits
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = int64_t(blockIdx.x) * kPTile, h = blockIdx.y, r0 = int64_t(blockIdx.z) * kPRows;

  // staging: each thread issues all of its loads before any LDS store (fixed
  // trip counts, unrolled), so the loads' latencies overlap
  {
    constexpr int kN = kPRows * kPD / kPThreads;
    float v[kN];
#pragma unroll
    for (int k = 0; k < kN; ++k) {
      const int idx = tid + k * kPThreads, r = idx / kPD, d = idx % kPD;
      v[k] = 0.0f;
      if (r0 + r < a.rows) {
        int64_t hq, i;
        row_of(a, h, r0 + r, hq, i);
        v[k] = load_dyn(a.q, (i * a.Hq + hq) * kPD + d, a.qd);
      }
    }
#pragma unroll
    for (int k = 0; k < kN; ++k) {
      const int idx = tid + k * kPThreads;
      qs[idx % kPD][idx / kPD] = v[k];
    }
  }
  if (t0 < a.Tq) {
    const int64_t w0 = t0 / kPer, kwh = a.cap / kPer;  // word rows per head
    constexpr int kN = kWordRows * kPD / kPThreads;
    uint32_t w[kN];
#pragma unroll
    for (int k = 0; k < kN; ++k) {
      const int idx = tid + k * kPThreads, j = idx / kPD, d = idx % kPD;
      w[k] = (w0 + j) * kPer < a.Tq ? a.kc[(h * kwh + w0 + j) * kPD + d] : 0u;
    }
    const int64_t g0 = t0 / a.G, gh = a.cap / a.G;
    const int ng = a.G >= kPTile ? 1 : kPTile / a.G;
    float sv[2], mv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = tid + k * kPThreads, j = idx / kPD, d = idx % kPD;
      const bool in = j < ng && (g0 + j) * a.G < a.Tq;
      const int64_t o = (h * gh + g0 + j) * kPD + d;
      sv[k] = in ? stat_f32(a.ks, o, a.sd) : 0.0f;
      mv[k] = in ? stat_f32(a.km, o, a.sd) : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kN; ++k) {
      const int idx = tid + k * kPThreads;
      kw[idx / kPD][idx % kPD] = w[k];
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = tid + k * kPThreads;
      if (idx / kPD < ng) {
        ss[idx / kPD][idx % kPD] = sv[k];
        ms[idx / kPD][idx % kPD] = mv[k];
      }
    }
  }
  if (t0 + kPTile > a.Tq && a.Tr > 0) {
    constexpr int kN = kPTile * (kPD / 8) / kPThreads;
    uint4 v[kN];
#pragma unroll
    for (int k = 0; k < kN; ++k) {
      const int idx = tid + k * kPThreads, tt = idx / (kPD / 8), c8 = idx % (kPD / 8);
      const int64_t t = t0 + tt;
      v[k] = make_uint4(0, 0, 0, 0);
      if (t >= a.Tq && t < a.T)
        v[k] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.rk) + (t - a.Tq) * a.r_st +
                                                h * a.r_sh + 8 * c8);
    }
#pragma unroll
    for (int k = 0; k < kN; ++k) {
      const int idx = tid + k * kPThreads;
      *reinterpret_cast<uint4 *>(&rk[idx / (kPD / 8)][8 * (idx % (kPD / 8))]) = v[k];
    }
  }
  __syncthreads();

  // lane = token, wave = quarter of the channels; all the chunk's rows
  const int64_t t = t0 + lane;
  const int nr4 = static_cast<int>(min<int64_t>(kPRows, a.rows - r0) + 3) / 4;  // live row quads
  float acc[kPRows];
#pragma unroll
  for (int r = 0; r < kPRows; ++r) acc[r] = 0.0f;
  const int d0 = 32 * wave;
  if (t < a.Tq) {
    const int wr = lane / kPer, sh = (lane % kPer) * BITS;
    const int gi = a.G >= kPTile ? 0 : lane / a.G;  // group of token t among the tile's groups
#pragma unroll 2
    for (int d = d0; d < d0 + 32; ++d) {
      const float k = fmaf(float((kw[wr][d] >> sh) & ((1u << BITS) - 1u)), ss[gi][d], ms[gi][d]);
#pragma unroll
      for (int r4 = 0; r4 < kPRows / 4; ++r4) {
        if (r4 < nr4) {  // uniform
          const float4 q4 = *reinterpret_cast<const float4 *>(&qs[d][4 * r4]);
          acc[4 * r4] = fmaf(q4.x, k, acc[4 * r4]);
          acc[4 * r4 + 1] = fmaf(q4.y, k, acc[4 * r4 + 1]);
          acc[4 * r4 + 2] = fmaf(q4.z, k, acc[4 * r4 + 2]);
          acc[4 * r4 + 3] = fmaf(q4.w, k, acc[4 * r4 + 3]);
        }
      }
    }
  } else if (t < a.T) {
#pragma unroll 2
    for (int d = d0; d < d0 + 32; ++d) {
      const float k = a.rd == UC_BF16 ? bf16_bits_to_f32(rk[lane][d]) : f16_bits_to_f32(rk[lane][d]);
#pragma unroll
      for (int r4 = 0; r4 < kPRows / 4; ++r4) {
        if (r4 < nr4) {
          const float4 q4 = *reinterpret_cast<const float4 *>(&qs[d][4 * r4]);
          acc[4 * r4] = fmaf(q4.x, k, acc[4 * r4]);
          acc[4 * r4 + 1] = fmaf(q4.y, k, acc[4 * r4 + 1]);
          acc[4 * r4 + 2] = fmaf(q4.z, k, acc[4 * r4 + 2]);
          acc[4 * r4 + 3] = fmaf(q4.w, k, acc[4 * r4 + 3]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kPRows; ++r) red[wave][r][lane] = acc[r];
  __syncthreads();
  // thread (row quad of 4, token): the four quarters added in channel order
  const int tt = tid & 63;
  const int64_t tok = t0 + tt;
  if (tok >= a.T) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * (tid >> 6) + j;
    const int64_t rr = r0 + r;
    if (rr >= a.rows) break;
    int64_t hq, i;
    row_of(a, h, rr, hq, i);
    const float x = ((red[0][r][tt] + red[1][r][tt]) + red[2][r][tt]) + red[3][r][tt];
    a.logits[(hq * a.Lq + i) * a.T + tok] = x * a.sm_scale;
  }
}

// RW query rows per workgroup (8 or 16): thread (8-channel slice, row, token
// phase), the kPThreads / (16 RW) phases taking every phase-th token of a
// chunk; the phases' sums meet in LDS at the end.
template <int BITS, int RW>
__global__ __launch_bounds__(kPThreads) void parts_av_kernel(PartsArgs a) {
  constexpr int kVW = kPD * BITS / 32;        // value words per token
  constexpr int kPh = kPThreads / (16 * RW);  // token phases
  __shared__ float ps[RW][kPTile + 4];        // probabilities of a 64-token chunk
  __shared__ uint32_t vw[kPTile][kVW + 1];    // its value words
  __shared__ float vsc[kPTile][8], vmn[kPTile][8];  // its value scales and minima (G >= 16: <= 8 groups)
  __shared__ float4 mg[kPh > 1 ? kPh - 1 : 1][RW][16][2];  // phases 1.. for the final sum
  const int tid = threadIdx.x, c8 = tid & 15, r = (tid >> 4) % RW, ph = tid / (16 * RW);
  const int64_t s = blockIdx.x, h = blockIdx.y, r0 = int64_t(blockIdx.z) * RW;
  const int64_t t_begin = s * a.split, t_end = min(a.T, t_begin + a.split);
  const int gpt = kPD / a.G;      // value groups per token
  const int gi = (8 * c8) / a.G;  // this thread's 8 channels lie in one group
  const int64_t vsh = a.cap * gpt;
  const bool live = r0 + r < a.rows;

  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t c0 = t_begin; c0 < t_end; c0 += kPTile) {
    const int n = static_cast<int>(min<int64_t>(kPTile, t_end - c0));
    const int np = static_cast<int>(max<int64_t>(0, min<int64_t>(n, a.Tq - c0)));  // packed tokens of the chunk
    // staging: all loads of a thread first (fixed trip counts), then the stores
    constexpr int kNP = RW * kPTile / kPThreads, kNW = kPTile * kVW / kPThreads;
    float pv[kNP];
    uint32_t wv[kNW];
    float sv[2], mv[2];
#pragma unroll
    for (int k = 0; k < kNP; ++k) {
      const int idx = tid + k * kPThreads, rr = idx / kPTile, tt = idx % kPTile;
      pv[k] = 0.0f;
      if (r0 + rr < a.rows && tt < n) {
        int64_t hq, i;
        row_of(a, h, r0 + rr, hq, i);
        pv[k] = load_dyn(a.p, hq * a.p_sh + i * a.p_si + (c0 + tt) * a.p_st, a.pd);
      }
    }
#pragma unroll
    for (int k = 0; k < kNW; ++k) {
      const int idx = tid + k * kPThreads, tt = idx / kVW, w = idx % kVW;
      wv[k] = tt < np ? a.vc[(h * a.cap + c0 + tt) * kVW + w] : 0u;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = tid + k * kPThreads, tt = idx / gpt, g = idx % gpt;
      const int64_t o = h * vsh + (c0 + tt) * gpt + g;
      sv[k] = idx < kPTile * gpt && tt < np ? stat_f32(a.vs, o, a.sd) : 0.0f;
      mv[k] = idx < kPTile * gpt && tt < np ? stat_f32(a.vm, o, a.sd) : 0.0f;
    }
    __syncthreads();  // the previous chunk is consumed
#pragma unroll
    for (int k = 0; k < kNP; ++k) {
      const int idx = tid + k * kPThreads;
      ps[idx / kPTile][idx % kPTile] = pv[k];
    }
#pragma unroll
    for (int k = 0; k < kNW; ++k) {
      const int idx = tid + k * kPThreads;
      vw[idx / kVW][idx % kVW] = wv[k];
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = tid + k * kPThreads;
      if (idx < kPTile * gpt) {
        vsc[idx / gpt][idx % gpt] = sv[k];
        vmn[idx / gpt][idx % gpt] = mv[k];
      }
    }
    __syncthreads();
    if (!live) continue;
    // packed tokens: this thread's channels are bits [8 * c8 * BITS, + 8 * BITS) of the words
    const int wi = (8 * c8 * BITS) / 32, sh = (8 * c8 * BITS) % 32;
    for (int tt = ph; tt < np; tt += kPh) {
      const uint32_t bits = vw[tt][wi] >> sh;
      const float sc = vsc[tt][gi], mn = vmn[tt][gi], p = ps[r][tt];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = fmaf(float((bits >> (j * BITS)) & ((1u << BITS) - 1u)), sc, mn);
        acc[j] = fmaf(p, v, acc[j]);
      }
    }
    for (int tt = np + ((ph - np) % kPh + kPh) % kPh; tt < n; tt += kPh) {
      const int64_t t = c0 + tt;
      const uint4 raw = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.rv) + (t - a.Tq) * a.r_st +
                                                         h * a.r_sh + 8 * c8);
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
      const float p = ps[r][tt];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = w[j] & 0xffffu, hi = w[j] >> 16;
        const float v0 = a.rd == UC_BF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(static_cast<uint16_t>(lo));
        const float v1 = a.rd == UC_BF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(static_cast<uint16_t>(hi));
        acc[2 * j] = fmaf(p, v0, acc[2 * j]);
        acc[2 * j + 1] = fmaf(p, v1, acc[2 * j + 1]);
      }
    }
  }
  if constexpr (kPh > 1) {
    __syncthreads();
    if (ph > 0) {
      mg[ph - 1][r][c8][0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      mg[ph - 1][r][c8][1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
    __syncthreads();
    if (ph > 0) return;
#pragma unroll
    for (int k = 0; k < kPh - 1; ++k) {
      const float4 lo = mg[k][r][c8][0], hi = mg[k][r][c8][1];
      acc[0] += lo.x; acc[1] += lo.y; acc[2] += lo.z; acc[3] += lo.w;
      acc[4] += hi.x; acc[5] += hi.y; acc[6] += hi.z; acc[7] += hi.w;
    }
  }
  if (!live) return;
  int64_t hq, i;
  row_of(a, h, r0 + r, hq, i);
  float *dst = a.partial + ((hq * a.Lq + i) * a.splits + s) * kPD + 8 * c8;
  *reinterpret_cast<float4 *>(dst) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  *reinterpret_cast<float4 *>(dst + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

// out[hq, i, d] = sum over splits, in order, of the partials.
__global__ __launch_bounds__(kPD) void parts_av_reduce_kernel(PartsArgs a) {
  const int64_t row = blockIdx.x;  // hq * Lq + i
  const int d = threadIdx.x;
  const float *src = a.partial + row * a.splits * kPD + d;
  float s = 0.0f;
  for (int64_t k0 = 0; k0 < a.splits; k0 += 8) {  // eight loads in flight, added in split order
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = k0 + j < a.splits ? src[(k0 + j) * kPD] : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[j];
  }
  store_dyn(a.out, row * kPD + d, s, a.od);
}

}  // namespace

bool parts_fast_supported(int bits, int group, int64_t head_dim, int stats_dtype, int res_dtype, int64_t r_st,
                          int64_t r_sh, const void *residual, int64_t residual_tokens) {
  const bool half_res = res_dtype == UC_BF16 || res_dtype == UC_FP16;
  return (bits == 2 || bits == 4) && group >= 16 && group <= 128 && head_dim == kPD &&
         (stats_dtype == UC_FP16 || stats_dtype == UC_BF16) &&
         (residual_tokens == 0 || (half_res && r_st % 8 == 0 && r_sh % 8 == 0 &&
                                   reinterpret_cast<uintptr_t>(residual) % 16 == 0));
}

int launch_parts_qk(const void *query, int q_dtype, int64_t Lq, int64_t Hq, const void *kc, const void *ks,
                    const void *km, int sd, int64_t Tq, int64_t cap, int bits, int G, const void *rk, int rd,
                    int64_t Tr, int64_t r_st, int64_t r_sh, int64_t Hkv, float sm_scale, float *logits,
                    hipStream_t stream) {
  PartsArgs a{};
  a.kc = static_cast<const uint32_t *>(kc); a.ks = ks; a.km = km; a.sd = sd;
  a.cap = cap > 0 ? cap : Tq; a.Tq = Tq; a.Tr = Tr; a.T = Tq + Tr;
  a.Hq = Hq; a.Hkv = Hkv; a.Lq = Lq; a.group = Hq / Hkv; a.rows = a.group * Lq; a.G = G;
  a.rk = rk; a.rd = rd; a.r_st = r_st; a.r_sh = r_sh;
  a.q = query; a.qd = q_dtype; a.sm_scale = sm_scale; a.logits = logits;
  const dim3 grid(static_cast<unsigned>(ceil_div(a.T, int64_t(kPTile))), static_cast<unsigned>(Hkv),
                  static_cast<unsigned>(ceil_div(a.rows, int64_t(kPRows))));
  if (bits == 2)
    hipLaunchKernelGGL(parts_qk_kernel<2>, grid, dim3(kPThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(parts_qk_kernel<4>, grid, dim3(kPThreads), 0, stream, a);
  return check_launch("uc_kivi_qk");
}

int launch_parts_av(const void *probs, int p_dtype, int64_t p_sh, int64_t p_si, int64_t p_st, int64_t Lq, int64_t Hq,
                    const void *vc, const void *vs, const void *vm, int sd, int64_t Tq, int64_t cap, int bits, int G,
                    const void *rv, int rd, int64_t Tr, int64_t r_st, int64_t r_sh, int64_t Hkv, void *out, int od,
                    void *workspace, int64_t split_tokens, hipStream_t stream) {
  PartsArgs a{};
  a.vc = static_cast<const uint32_t *>(vc); a.vs = vs; a.vm = vm; a.sd = sd;
  a.cap = cap > 0 ? cap : Tq; a.Tq = Tq; a.Tr = Tr; a.T = Tq + Tr;
  a.Hq = Hq; a.Hkv = Hkv; a.Lq = Lq; a.group = Hq / Hkv; a.rows = a.group * Lq; a.G = G;
  a.rv = rv; a.rd = rd; a.r_st = r_st; a.r_sh = r_sh;
  a.p = probs; a.pd = p_dtype; a.p_sh = p_sh; a.p_si = p_si; a.p_st = p_st;
  a.split = split_tokens; a.splits = ceil_div(a.T, split_tokens);
  a.partial = static_cast<float *>(workspace); a.out = out; a.od = od;
  UC_REQUIRE(split_tokens > 0, "uc_kivi_av: split of %lld tokens", (long long)split_tokens);
  const int rw = a.rows <= 8 ? 8 : 16;  // rows per workgroup: two token phases below 9 rows
  const dim3 grid(static_cast<unsigned>(a.splits), static_cast<unsigned>(Hkv),
                  static_cast<unsigned>(ceil_div(a.rows, int64_t(rw))));
  if (rw == 8) {
    if (bits == 2) hipLaunchKernelGGL((parts_av_kernel<2, 8>), grid, dim3(kPThreads), 0, stream, a);
    else hipLaunchKernelGGL((parts_av_kernel<4, 8>), grid, dim3(kPThreads), 0, stream, a);
  } else {
    if (bits == 2) hipLaunchKernelGGL((parts_av_kernel<2, 16>), grid, dim3(kPThreads), 0, stream, a);
    else hipLaunchKernelGGL((parts_av_kernel<4, 16>), grid, dim3(kPThreads), 0, stream, a);
  }
  int rc = check_launch("uc_kivi_av");
  if (rc != UC_OK) return rc;
  hipLaunchKernelGGL(parts_av_reduce_kernel, dim3(static_cast<unsigned>(Hq * Lq)), dim3(kPD), 0, stream, a);
  return check_launch("uc_kivi_av (reduce)");
}

}  // namespace uc
