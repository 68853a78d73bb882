// Packed-KIVI attention for short queries: fused split-K decode with an LSE
// combine, and the separate QK / AV products behind attention_parts().
//
// Geometry: one workgroup owns (item, KV head, token split).  The
// group*query_len <= 16 query rows that share a KV head live in LDS, so
// every packed word and scale is read from HBM once per (item, KV head).
#include <mutex>

#include "uc_common.h"
#include "uc_decode.h"

namespace uc {

bool h2o_mfma_supported(int dtype, int64_t head_dim, const void *q, int64_t q_si, int64_t q_sh, int64_t q_sd,
                        const void *k, int64_t k_st, int64_t k_sh, int64_t k_sd, int64_t query_len, int64_t heads_q,
                        int64_t tokens, int64_t heads_kv);
int launch_qk_logits_mfma(int dtype, const void *q, int64_t q_si, int64_t q_sh, const void *k, int64_t k_st,
                          int64_t k_sh, int64_t Lq, int64_t Hq, int64_t T, int64_t Hkv, float scale, float *logits,
                          hipStream_t stream);
bool pv_mfma_supported(int p_dtype, const void *probs, int64_t p_sh, int64_t p_si, int64_t p_st, int v_dtype,
                       const void *v, int64_t v_st, int64_t v_sh, int64_t head_dim, int64_t Lq, int64_t rows,
                       int64_t T);
int launch_pv_mfma(int p_dtype, const void *probs, int64_t p_sh, int64_t p_si, int v_dtype, const void *v,
                   int64_t v_st, int64_t v_sh, int64_t Lq, int64_t Hq, int64_t T, int64_t Hkv, void *out,
                   void *workspace, hipStream_t stream);

namespace {

constexpr int kRows = 16;     // query rows per workgroup
constexpr int kTile = 64;     // tokens per inner tile
constexpr int kThreads = 256; // 4 waves
constexpr int kMaxD = 256;    // largest head_dim handled
constexpr float kNegInf = -__builtin_huge_valf();

// Strided view of one packed segment plus its dense residual
// ([Tr, Hkv, D] contiguous).  Offsets follow uc_kivi_pack's stride contract.
struct PackedView {
  const void *kcode, *kscale, *kmin, *vcode, *vscale, *vmin;
  int64_t kc_sh, kc_sd, kc_sw, ks_sh, ks_sd, ks_sg;
  int64_t vc_sh, vc_st, vc_sw, vs_sh, vs_st, vs_sg;
  const void *rkey, *rval;
  int64_t Tq, Tr, Hkv, D;
  int lg;      // log2(group_size)
  int sd, rd;  // stats and residual dtype codes
  int64_t r_st, r_sh;  // residual strides (token, head); channel stride 1
};

__host__ __device__ inline int log2i(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

// Strides of the 2/4-bit packed tensors in the ABI's token-major layout with
// capacity `cap` tokens per head.
__host__ __device__ inline void set_packed_strides(PackedView &v, int64_t cap, int bits, int group, int64_t D) {
  const int64_t kw = cap * bits / 32, vw = D * bits / 32;
  v.kc_sh = kw * D; v.kc_sd = 1; v.kc_sw = D;
  v.ks_sh = (cap / group) * D; v.ks_sd = 1; v.ks_sg = D;
  v.vc_sh = cap * vw; v.vc_st = vw; v.vc_sw = 1;
  v.vs_sh = cap * (D / group); v.vs_st = D / group; v.vs_sg = 1;
}

__host__ __device__ inline int64_t item_capacity(const uc_kivi_item &it) {
  return it.packed_capacity > 0 ? it.packed_capacity : it.quantized_tokens;
}

__host__ __device__ inline PackedView native_view(const uc_kivi_item &it, int bits, int group,
                                                  int64_t Hkv, int64_t D, int rd) {
  PackedView v{};
  v.lg = log2i(group);
  v.sd = UC_FP16;
  v.rd = rd;
  const int64_t Tq = it.quantized_tokens;
  v.kcode = it.key_code; v.kscale = it.key_scale; v.kmin = it.key_min;
  v.vcode = it.value_code; v.vscale = it.value_scale; v.vmin = it.value_min;
  set_packed_strides(v, item_capacity(it), bits, group, D);
  v.rkey = it.residual_key; v.rval = it.residual_value;
  v.Tq = Tq; v.Tr = it.residual_tokens; v.Hkv = Hkv; v.D = D;
  residual_strides(it, Hkv, D, v.r_st, v.r_sh);
  return v;
}

// Dequantised key element (fp32 code*scale+min) or residual key element.
template <int BITS>
__device__ __forceinline__ float key_at(const PackedView &v, int64_t h, int64_t t, int64_t d) {
  if (t < v.Tq) {
    constexpr int kPerWord = BITS == 8 ? 1 : 32 / BITS;
    const uint32_t c = read_code<BITS>(v.kcode, h * v.kc_sh + d * v.kc_sd + (t / kPerWord) * v.kc_sw,
                                       t % kPerWord);
    const int64_t so = h * v.ks_sh + d * v.ks_sd + (t >> v.lg) * v.ks_sg;
    return fmaf(float(c), load_dyn(v.kscale, so, v.sd), load_dyn(v.kmin, so, v.sd));
  }
  return load_dyn(v.rkey, (t - v.Tq) * v.r_st + h * v.r_sh + d, v.rd);
}

template <int BITS>
__device__ __forceinline__ float value_at(const PackedView &v, int64_t h, int64_t t, int64_t d) {
  if (t < v.Tq) {
    constexpr int kPerWord = BITS == 8 ? 1 : 32 / BITS;
    const uint32_t c = read_code<BITS>(v.vcode, h * v.vc_sh + t * v.vc_st + (d / kPerWord) * v.vc_sw,
                                       d % kPerWord);
    const int64_t so = h * v.vs_sh + t * v.vs_st + (d >> v.lg) * v.vs_sg;
    return fmaf(float(c), load_dyn(v.vscale, so, v.sd), load_dyn(v.vmin, so, v.sd));
  }
  return load_dyn(v.rval, (t - v.Tq) * v.r_st + h * v.r_sh + d, v.rd);
}

struct SharedTile {
  float q[kRows][kMaxD];           // query rows of this KV head (fp32)
  float red[4][kRows][kTile];      // per-wave QK partials; reused for the final reduction
  float p[kRows][kTile];           // probabilities of the current tile
  float alpha[kRows];              // rescale factor of the running output
};

// Load query rows r = g*Lq + i (g < group) of KV head h into LDS.
__device__ void load_query_rows(SharedTile &s, const void *query, int qd, int64_t h, int64_t row0, int64_t rows,
                                int64_t group, int64_t Lq, int64_t Hq, int64_t D) {
  for (int64_t idx = threadIdx.x; idx < kRows * D; idx += kThreads) {
    const int64_t r = idx / D, d = idx % D;
    float val = 0.0f;
    if (row0 + r < rows) {
      const int64_t g = (row0 + r) / Lq, i = (row0 + r) % Lq;
      val = load_dyn(query, (i * Hq + h * group + g) * D + d, qd);
    }
    s.q[r][d] = val;
  }
}

// red[wave][r][lane] = partial <q_r, k_t> over the wave's quarter of channels.
template <int BITS>
__device__ void qk_tile(SharedTile &s, const PackedView &v, int64_t h, int64_t t, bool valid) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  float acc[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) acc[r] = 0.0f;
  if (valid) {
    const int64_t dq = (v.D + 3) / 4;
    const int64_t d0 = wave * dq, d1 = min(v.D, d0 + dq);
    for (int64_t d = d0; d < d1; ++d) {
      const float k = key_at<BITS>(v, h, t, d);
#pragma unroll
      for (int r = 0; r < kRows; ++r) acc[r] = fmaf(s.q[r][d], k, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) s.red[wave][r][lane] = acc[r];
}

struct DecodeParams {
  int64_t Hq, Hkv, D, Lq, group, rows;
  int64_t splits_packed, splits_total;
  int64_t split_tokens;  // keys per split
  float scale_log2;  // sm_scale * log2(e)
  float *ws_o;       // [items, Hq, Lq, splits, D]
  float *ws_ml;      // [items, Hq, Lq, splits, 2]
  // AV mode (probabilities supplied instead of a softmax)
  const void *probs;
  int64_t p_sh, p_si, p_st;
  int bits, group_size;
  int qd, pd, rd;  // query, probability and residual dtype codes
};

// Partial attention (or P.V when AV) of one (item, KV head, split).
template <int BITS, bool AV, bool TABLE>
__global__ __launch_bounds__(kThreads) void decode_partial_kernel(const uc_kivi_item *items,
                                                                   uc_kivi_item single, PackedView single_view,
                                                                   DecodeParams p) {
  __shared__ SharedTile s;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t item = AV ? 0 : blockIdx.z;
  const int64_t row0 = AV ? int64_t(blockIdx.z) * kRows : 0;
  const uc_kivi_item it = TABLE ? items[item] : single;
  const int64_t h = blockIdx.y, split = blockIdx.x;
  const PackedView v = TABLE ? native_view(it, BITS, 1 << single_view.lg, p.Hkv, p.D, p.rd) : single_view;
  const int64_t D = p.D;
  const int64_t nrows = min<int64_t>(kRows, p.rows - row0);
  if (nrows <= 0) return;

  int64_t t_begin, t_end;
  if (split < p.splits_packed) {
    t_begin = split * p.split_tokens;
    t_end = min(v.Tq, t_begin + p.split_tokens);
  } else {
    t_begin = v.Tq + (split - p.splits_packed) * p.split_tokens;
    t_end = min(v.Tq + v.Tr, t_begin + p.split_tokens);
  }

  if (!AV) load_query_rows(s, it.query, p.qd, h, row0, p.rows, p.group, p.Lq, p.Hq, D);
  for (int idx = threadIdx.x; idx < kRows * kTile; idx += kThreads) (&s.p[0][0])[idx] = 0.0f;
  __syncthreads();

  constexpr int kCpt = kMaxD / kWave;  // channels per thread in the AV phase
  float acc_o[kRows][kCpt];
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int c = 0; c < kCpt; ++c) acc_o[r][c] = 0.0f;
  float m_run[4], l_run[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m_run[j] = kNegInf;
    l_run[j] = 0.0f;
  }

  for (int64_t t0 = t_begin; t0 < t_end; t0 += kTile) {
    if constexpr (!AV) {
      const int64_t t = t0 + lane;
      qk_tile<BITS>(s, v, h, t, t < t_end);
      __syncthreads();
      // wave w owns rows w, w+4, w+8, w+12: online softmax in base 2
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = wave + 4 * j;
        if (r >= nrows) continue;
        float x = kNegInf;
        if (t < t_end) x = (s.red[0][r][lane] + s.red[1][r][lane] + s.red[2][r][lane] + s.red[3][r][lane]) * p.scale_log2;
        const float m_new = fmaxf(m_run[j], wave_max(x));
        const float pr = (x == kNegInf) ? 0.0f : exp2f(x - m_new);
        const float alpha = (m_run[j] == kNegInf) ? 0.0f : exp2f(m_run[j] - m_new);
        l_run[j] = l_run[j] * alpha + wave_sum(pr);
        m_run[j] = m_new;
        s.p[r][lane] = pr;
        if (lane == 0) s.alpha[r] = alpha;
      }
    } else {
      for (int idx = threadIdx.x; idx < kRows * kTile; idx += kThreads) {
        const int r = idx / kTile, tt = idx % kTile;
        float pr = 0.0f;
        if (r < nrows && t0 + tt < t_end) {
          const int64_t rr = row0 + r, g = rr / p.Lq, i = rr % p.Lq;
          pr = load_dyn(p.probs, (h * p.group + g) * p.p_sh + i * p.p_si + (t0 + tt) * p.p_st, p.pd);
        }
        s.p[r][tt] = pr;
      }
    }
    __syncthreads();
    // P.V: wave w owns tokens [16w, 16w+16) of the tile, lane owns channels lane + 64c
    if constexpr (!AV) {
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const float a = r < nrows ? s.alpha[r] : 0.0f;
#pragma unroll
        for (int c = 0; c < kCpt; ++c) acc_o[r][c] *= a;
      }
    }
    for (int k = 0; k < kTile / 4; ++k) {
      const int tt = wave * (kTile / 4) + k;
      const int64_t t = t0 + tt;
      if (t >= t_end) break;
#pragma unroll
      for (int c = 0; c < kCpt; ++c) {
        const int64_t d = lane + kWave * c;
        if (d >= D) continue;
        const float val = value_at<BITS>(v, h, t, d);
#pragma unroll
        for (int r = 0; r < kRows; ++r) acc_o[r][c] = fmaf(s.p[r][tt], val, acc_o[r][c]);
      }
    }
    __syncthreads();
  }

  // reduce the four waves' partial outputs through LDS ([kRows][kMaxD] view of red)
  float *fin = &s.red[0][0][0];
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int c = 0; c < kCpt; ++c) {
          const int64_t d = lane + kWave * c;
          if (d < D) fin[r * kMaxD + d] = (w == 0 ? 0.0f : fin[r * kMaxD + d]) + acc_o[r][c];
        }
    }
    __syncthreads();
  }
  for (int64_t idx = threadIdx.x; idx < nrows * D; idx += kThreads) {
    const int64_t r = idx / D, d = idx % D;
    const int64_t rr = row0 + r, g = rr / p.Lq, i = rr % p.Lq, hq = h * p.group + g;
    const int64_t slot = ((item * p.Hq + hq) * p.Lq + i) * p.splits_total + split;
    p.ws_o[slot * D + d] = fin[r * kMaxD + d];
  }
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = wave + 4 * j;
      if (r >= nrows) continue;
      const int64_t rr = row0 + r, g = rr / p.Lq, i = rr % p.Lq, hq = h * p.group + g;
      const int64_t slot = ((item * p.Hq + hq) * p.Lq + i) * p.splits_total + split;
      p.ws_ml[slot * 2 + 0] = AV ? 0.0f : m_run[j];
      p.ws_ml[slot * 2 + 1] = AV ? 1.0f : l_run[j];
    }
  }
}

struct CombineParams {
  int64_t Hq, Lq, D, splits;
  int64_t o_si, o_sh;  // output strides of query row i and query head hq
  const float *ws_o, *ws_ml;
  int normalize;       // 0: plain sum of partial outputs (AV mode)
  int od;              // output dtype code
};

// Merge the split partials of one (item, query head, query row):
// M = max m_s, L = sum l_s 2^(m_s-M), out = sum o_s 2^(m_s-M) / L.
template <bool TABLE>
__global__ __launch_bounds__(128) void decode_combine_kernel(const uc_kivi_item *items, uc_kivi_item single,
                                                              CombineParams p) {
  const int64_t item = blockIdx.y;
  const uc_kivi_item it = TABLE ? items[item] : single;
  const int64_t hq = blockIdx.x / p.Lq, i = blockIdx.x % p.Lq;
  const int64_t base = ((item * p.Hq + hq) * p.Lq + i) * p.splits;
  float M = kNegInf;
  for (int64_t sidx = 0; sidx < p.splits; ++sidx) M = fmaxf(M, p.ws_ml[(base + sidx) * 2]);
  float L = 0.0f;
  for (int64_t sidx = 0; sidx < p.splits; ++sidx) {
    const float m = p.ws_ml[(base + sidx) * 2], l = p.ws_ml[(base + sidx) * 2 + 1];
    if (l > 0.0f && m != kNegInf) L += l * exp2f(m - M);
  }
  const float inv = (p.normalize && L > 0.0f) ? 1.0f / L : 1.0f;
  for (int64_t d = threadIdx.x; d < p.D; d += blockDim.x) {
    float o = 0.0f;
    for (int64_t sidx = 0; sidx < p.splits; ++sidx) {
      const float m = p.ws_ml[(base + sidx) * 2], l = p.ws_ml[(base + sidx) * 2 + 1];
      if (!p.normalize) {
        o += p.ws_o[(base + sidx) * p.D + d];
      } else if (l > 0.0f && m != kNegInf) {
        o = fmaf(p.ws_o[(base + sidx) * p.D + d], exp2f(m - M), o);
      }
    }
    store_dyn(it.out, i * p.o_si + hq * p.o_sh + d, o * inv, p.od);
  }
  if (threadIdx.x == 0 && p.normalize && it.lse != nullptr) {
    it.lse[hq * p.Lq + i] = L > 0.0f ? (M + log2f(L)) * kLn2 : kNegInf;
  }
}

// Scaled logits of a (token tile, KV head, 16-row chunk).
struct QKParams {
  int64_t Hq, Lq, group, rows, total;
  float sm_scale;
  const void *query;
  int qd;
  float *logits;  // [Hq, Lq, total]
};

template <int BITS>
__global__ __launch_bounds__(kThreads) void qk_kernel(PackedView v, QKParams p) {
  __shared__ SharedTile s;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t h = blockIdx.y, row0 = int64_t(blockIdx.z) * kRows;
  const int64_t t0 = int64_t(blockIdx.x) * kTile;
  load_query_rows(s, p.query, p.qd, h, row0, p.rows, p.group, p.Lq, p.Hq, v.D);
  __syncthreads();
  const int64_t t = t0 + lane;
  qk_tile<BITS>(s, v, h, t, t < p.total);
  __syncthreads();
  if (t >= p.total) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = wave + 4 * j;
    const int64_t rr = row0 + r;
    if (rr >= p.rows) continue;
    const float x = (s.red[0][r][lane] + s.red[1][r][lane] + s.red[2][r][lane] + s.red[3][r][lane]) * p.sm_scale;
    const int64_t g = rr / p.Lq, i = rr % p.Lq;
    p.logits[((h * p.group + g) * p.Lq + i) * p.total + t] = x;
  }
}

// Strides of the packed tensors for the QK/AV entry points: kernel-native
// layout for 2/4-bit, UniCache's uint8 layout for 8-bit (physical.py:66-68).
PackedView parts_view(const void *kc, const void *ks, const void *km, const void *vc, const void *vs,
                             const void *vm, int64_t Tq, int64_t cap, int bits, int group, const void *rk,
                             const void *rv, int64_t Tr, int64_t r_st, int64_t r_sh, int64_t Hkv, int64_t D, int sd,
                             int rd) {
  PackedView v{};
  v.r_st = r_st;
  v.r_sh = r_sh;
  v.lg = log2i(group);
  v.sd = sd;
  v.rd = rd;
  v.kcode = kc; v.kscale = ks; v.kmin = km; v.vcode = vc; v.vscale = vs; v.vmin = vm;
  v.rkey = rk; v.rval = rv; v.Tq = Tq; v.Tr = Tr; v.Hkv = Hkv; v.D = D;
  if (bits == 8) {
    v.kc_sh = D; v.kc_sd = 1; v.kc_sw = Hkv * D;
    v.ks_sh = D; v.ks_sd = 1; v.ks_sg = Hkv * D;
    v.vc_sh = D; v.vc_st = Hkv * D; v.vc_sw = 1;
    v.vs_sh = D / group; v.vs_st = Hkv * (D / group); v.vs_sg = 1;
  } else {
    set_packed_strides(v, cap > 0 ? cap : Tq, bits, group, D);
  }
  return v;
}

bool ok_bits_group(int bits, int group) {
  return (bits == 2 || bits == 4 || bits == 8) &&
         (group == 16 || group == 32 || group == 64 || group == 128);
}

int decode_common(const uc_kivi_item *items_dev, const uc_kivi_item *single, int64_t n_items, int bits,
                  int group_size, int64_t Hq, int64_t Hkv, int64_t D, int64_t Lq, int q_dtype,
                  int res_dtype, int out_dtype, float sm_scale, int64_t max_tq, int64_t max_tr,
                  void *workspace, int64_t workspace_bytes, hipStream_t stream, const char *name,
                  int64_t segs = 1) {
  UC_REQUIRE(bits == 2 || bits == 4, "%s: packed decode supports 2 or 4 bit codes", name);
  UC_REQUIRE(group_size == 16 || group_size == 32 || group_size == 64 || group_size == 128,
             "%s: group_size must be 16, 32, 64 or 128", name);
  UC_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "Query heads must be divisible by KIVI KV heads");
  UC_REQUIRE(D > 0 && D <= kMaxD && D % group_size == 0, "%s: head_dim must divide by group_size and be <= %d",
             name, kMaxD);
  UC_REQUIRE(Lq > 0 && (Hq / Hkv) * Lq <= kRows, "%s: (query heads per KV head) * query_len must be <= %d",
             name, kRows);
  UC_REQUIRE(half_dtype(q_dtype) && half_dtype(res_dtype) && valid_dtype(out_dtype),
             "%s: query/residual must be bf16 or fp16", name);
  UC_REQUIRE(max_tq % group_size == 0, "%s: quantized tokens must be a multiple of group_size", name);
  UC_REQUIRE(single == nullptr || single->packed_capacity == 0 ||
                 (single->packed_capacity >= single->quantized_tokens && single->packed_capacity % group_size == 0),
             "%s: packed_capacity must be 0 or a multiple of group_size >= quantized_tokens", name);
  if (n_items == 0) return UC_OK;
  UC_REQUIRE(segs == 1 || decode_mfma_supported(bits, group_size, D, (Hq / Hkv) * Lq),
             "%s: segment groups need head_dim 128, group 32/64/128 and at most 16 query rows per KV head", name);
  if (decode_mfma_supported(bits, group_size, D, (Hq / Hkv) * Lq)) {
    // the MFMA kernel reads query rows 16 bytes at a time (batched items: the
    // caller's contract in the header)
    UC_REQUIRE(single == nullptr || (reinterpret_cast<uintptr_t>(single->query) & 15) == 0,
               "%s: query must be 16-byte aligned", name);
    return launch_decode_mfma(items_dev, single, n_items, bits, group_size, Hq, Hkv, Lq, q_dtype, res_dtype,
                              out_dtype, sm_scale, max_tq, max_tr, kDecodeMfmaNst, segs, workspace,
                              workspace_bytes, stream);
  }
  const int64_t sp_packed = ceil_div(max_tq, kDecodeSplitTokens);
  const int64_t sp_res = ceil_div(max_tr, kDecodeSplitTokens);
  const int64_t splits = sp_packed + sp_res;
  UC_REQUIRE(splits > 0, "%s: empty segment", name);
  const int64_t need = n_items * Hq * Lq * splits * (D + 2) * int64_t(sizeof(float));
  UC_REQUIRE(workspace != nullptr && workspace_bytes >= need, "%s: workspace too small (%lld < %lld bytes)", name,
             (long long)workspace_bytes, (long long)need);
  DecodeParams p{};
  p.Hq = Hq; p.Hkv = Hkv; p.D = D; p.Lq = Lq; p.group = Hq / Hkv; p.rows = p.group * Lq;
  p.splits_packed = sp_packed; p.splits_total = splits; p.split_tokens = kDecodeSplitTokens;
  p.scale_log2 = sm_scale * kLog2e;
  p.ws_o = static_cast<float *>(workspace);
  p.ws_ml = p.ws_o + n_items * Hq * Lq * splits * D;
  p.bits = bits; p.group_size = group_size;
  p.qd = q_dtype; p.rd = res_dtype; p.pd = UC_FP32;
  const bool table = items_dev != nullptr;
  const uc_kivi_item one = single ? *single : uc_kivi_item{};
  const PackedView one_view = native_view(one, bits, group_size, Hkv, D, res_dtype);
  dim3 grid(splits, Hkv, n_items);
  if (bits == 2) {
    if (table)
      hipLaunchKernelGGL((decode_partial_kernel<2, false, true>), grid, dim3(kThreads), 0, stream, items_dev, one, one_view, p);
    else
      hipLaunchKernelGGL((decode_partial_kernel<2, false, false>), grid, dim3(kThreads), 0, stream, items_dev, one, one_view, p);
  } else {
    if (table)
      hipLaunchKernelGGL((decode_partial_kernel<4, false, true>), grid, dim3(kThreads), 0, stream, items_dev, one, one_view, p);
    else
      hipLaunchKernelGGL((decode_partial_kernel<4, false, false>), grid, dim3(kThreads), 0, stream, items_dev, one, one_view, p);
  }
  int rc = check_launch(name);
  if (rc != UC_OK) return rc;
  CombineParams c{};
  c.Hq = Hq; c.Lq = Lq; c.D = D; c.splits = splits;
  c.o_si = Hq * D; c.o_sh = D;
  c.ws_o = p.ws_o; c.ws_ml = p.ws_ml; c.normalize = 1;
  dim3 cgrid(Hq * Lq, n_items);
  c.od = out_dtype;
  if (table)
    hipLaunchKernelGGL((decode_combine_kernel<true>), cgrid, dim3(128), 0, stream, items_dev, one, c);
  else
    hipLaunchKernelGGL((decode_combine_kernel<false>), cgrid, dim3(128), 0, stream, items_dev, one, c);
  return check_launch(name);
}

}  // namespace
}  // namespace uc

using namespace uc;

extern "C" int uc_kivi_attn_decode(const uc_kivi_item *item_host, int bits, int group_size,
                                   int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t query_len,
                                   int q_dtype, int res_dtype, int out_dtype, float sm_scale,
                                   void *workspace, int64_t workspace_bytes, uc_stream_t stream) {
  UC_REQUIRE(item_host != nullptr, "uc_kivi_attn_decode: item is NULL");
  UC_REQUIRE(item_host->quantized_tokens >= 0 && item_host->residual_tokens >= 0,
             "uc_kivi_attn_decode: negative token count");
  return decode_common(nullptr, item_host, 1, bits, group_size, heads_q, heads_kv, head_dim, query_len, q_dtype,
                       res_dtype, out_dtype, sm_scale, item_host->quantized_tokens, item_host->residual_tokens,
                       workspace, workspace_bytes, as_stream(stream), "uc_kivi_attn_decode");
}

extern "C" int uc_kivi_attn_decode_batch(const uc_kivi_item *items_device, int64_t n_items, int bits,
                                         int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                                         int64_t query_len, int q_dtype, int res_dtype, int out_dtype,
                                         float sm_scale, int64_t max_quantized_tokens, int64_t max_residual_tokens,
                                         void *workspace, int64_t workspace_bytes, uc_stream_t stream) {
  UC_REQUIRE(n_items >= 0 && (n_items == 0 || items_device != nullptr), "uc_kivi_attn_decode_batch: bad item table");
  UC_REQUIRE(max_quantized_tokens >= 0 && max_residual_tokens >= 0, "uc_kivi_attn_decode_batch: negative tokens");
  return decode_common(items_device, nullptr, n_items, bits, group_size, heads_q, heads_kv, head_dim, query_len,
                       q_dtype, res_dtype, out_dtype, sm_scale, max_quantized_tokens, max_residual_tokens,
                       workspace, workspace_bytes, as_stream(stream), "uc_kivi_attn_decode_batch");
}

extern "C" int uc_kivi_attn_decode_segments(const uc_kivi_item *items_device, int64_t n_items,
                                            int64_t segments_per_query, int bits, int group_size, int64_t heads_q,
                                            int64_t heads_kv, int64_t head_dim, int64_t query_len, int q_dtype,
                                            int res_dtype, int out_dtype, float sm_scale,
                                            int64_t max_quantized_tokens, int64_t max_residual_tokens,
                                            void *workspace, int64_t workspace_bytes, uc_stream_t stream) {
  UC_REQUIRE(n_items >= 0 && (n_items == 0 || items_device != nullptr),
             "uc_kivi_attn_decode_segments: bad item table");
  UC_REQUIRE(segments_per_query >= 1 && n_items % segments_per_query == 0,
             "uc_kivi_attn_decode_segments: %lld items do not form groups of %lld", (long long)n_items,
             (long long)segments_per_query);
  UC_REQUIRE(max_quantized_tokens >= 0 && max_residual_tokens >= 0,
             "uc_kivi_attn_decode_segments: negative tokens");
  return decode_common(items_device, nullptr, n_items, bits, group_size, heads_q, heads_kv, head_dim, query_len,
                       q_dtype, res_dtype, out_dtype, sm_scale, max_quantized_tokens, max_residual_tokens,
                       workspace, workspace_bytes, as_stream(stream), "uc_kivi_attn_decode_segments",
                       segments_per_query);
}

extern "C" int uc_kivi_attn_decode_segments_host(const uc_kivi_item *items_host, int64_t n_items, int bits,
                                                 int group_size, int64_t heads_q, int64_t heads_kv,
                                                 int64_t head_dim, int64_t query_len, int q_dtype, int res_dtype,
                                                 int out_dtype, float sm_scale, void *workspace,
                                                 int64_t workspace_bytes, uc_stream_t stream) {
  clear_error();
  constexpr int64_t kMaxHostItems = 8;
  UC_REQUIRE(items_host != nullptr && n_items >= 1 && n_items <= kMaxHostItems,
             "uc_kivi_attn_decode_segments_host: 1..%lld items", (long long)kMaxHostItems);
  UC_REQUIRE(heads_kv > 0 && head_dim > 0, "uc_kivi_attn_decode_segments_host: bad head shape");
  uc_kivi_item items[kMaxHostItems];
  int64_t max_tq = 0, max_tr = 0;
  for (int64_t i = 0; i < n_items; ++i) {
    uc_kivi_item it = items_host[i];
    // one query group: every segment reads the first item's query; its out / lse get the result
    it.query = items_host[0].query;
    it.out = items_host[0].out;
    it.lse = items_host[0].lse;
    UC_REQUIRE(it.quantized_tokens >= 0 && it.residual_tokens >= 0 && it.quantized_tokens % group_size == 0,
               "uc_kivi_attn_decode_segments_host: item %lld: bad token counts", (long long)i);
    UC_REQUIRE(it.quantized_tokens == 0 ||
                   (it.key_code && it.key_scale && it.key_min && it.value_code && it.value_scale && it.value_min &&
                    (it.packed_capacity == 0 ||
                     (it.packed_capacity >= it.quantized_tokens && it.packed_capacity % group_size == 0))),
               "uc_kivi_attn_decode_segments_host: item %lld: packed tensors or capacity", (long long)i);
    if (it.residual_tokens) {
      int64_t ts, hs;
      residual_strides(it, heads_kv, head_dim, ts, hs);
      UC_REQUIRE(it.residual_key && it.residual_value &&
                     ((reinterpret_cast<uintptr_t>(it.residual_key) | reinterpret_cast<uintptr_t>(it.residual_value)) &
                      15) == 0 && ts > 0 && hs >= 0 && ts % 8 == 0 && hs % 8 == 0,
                 "uc_kivi_attn_decode_segments_host: item %lld: residual rows must be 16-byte aligned with strides "
                 "in multiples of 8 elements", (long long)i);
      UC_REQUIRE(((it.residual_tokens - 1) * ts + (heads_kv - 1) * hs + head_dim) * 2 < (int64_t(1) << 31),
                 "uc_kivi_attn_decode_segments_host: item %lld: residual rows span 2 GiB or more", (long long)i);
    }
    max_tq = max(max_tq, it.quantized_tokens);
    max_tr = max(max_tr, it.residual_tokens);
    items[i] = it;
  }
  return decode_common(nullptr, items, n_items, bits, group_size, heads_q, heads_kv, head_dim, query_len, q_dtype,
                       res_dtype, out_dtype, sm_scale, max_tq, max_tr, workspace, workspace_bytes, as_stream(stream),
                       "uc_kivi_attn_decode_segments_host", n_items);
}

extern "C" int uc_kivi_qk(const void *query, int q_dtype, int64_t query_len, int64_t heads_q,
                          const void *key_code, const void *key_scale, const void *key_min, int stats_dtype,
                          int64_t quantized_tokens, int64_t packed_capacity, int bits, int group_size,
                          const void *residual_key, int res_dtype, int64_t residual_tokens,
                          int64_t r_st, int64_t r_sh,
                          int64_t heads_kv, int64_t head_dim, float sm_scale,
                          float *logits, uc_stream_t stream) {
  UC_REQUIRE(ok_bits_group(bits, group_size), "uc_kivi_qk: unsupported bits/group_size");
  UC_REQUIRE(valid_dtype(q_dtype) && valid_dtype(res_dtype) && valid_dtype(stats_dtype),
             "uc_kivi_qk: unknown dtype code");
  UC_REQUIRE(heads_q > 0 && heads_kv > 0 && heads_q % heads_kv == 0, "Query heads must be divisible by KIVI KV heads");
  UC_REQUIRE(head_dim > 0 && head_dim <= kMaxD, "uc_kivi_qk: head_dim must be <= %d", kMaxD);
  UC_REQUIRE(quantized_tokens % group_size == 0 && residual_tokens >= 0, "uc_kivi_qk: bad token counts");
  UC_REQUIRE(packed_capacity == 0 || (packed_capacity >= quantized_tokens && packed_capacity % group_size == 0),
             "uc_kivi_qk: packed_capacity must be 0 or a multiple of group_size >= quantized_tokens");
  const int64_t total = quantized_tokens + residual_tokens;
  if (total == 0 || query_len == 0) return UC_OK;
  // dense keys and at least one wave of query rows per KV head: MFMA tiles
  const int64_t rows = heads_q / heads_kv * query_len;
  if (quantized_tokens == 0 && q_dtype == res_dtype && rows >= kWave &&
      h2o_mfma_supported(q_dtype, head_dim, query, heads_q * head_dim, head_dim, 1, residual_key, r_st, r_sh, 1,
                         query_len, heads_q, residual_tokens, heads_kv))
    return launch_qk_logits_mfma(q_dtype, query, heads_q * head_dim, head_dim, residual_key, r_st, r_sh, query_len,
                                 heads_q, residual_tokens, heads_kv, sm_scale, logits, as_stream(stream));
  if (parts_fast_supported(bits, group_size, head_dim, stats_dtype, res_dtype, r_st, r_sh, residual_key,
                           residual_tokens))
    return launch_parts_qk(query, q_dtype, query_len, heads_q, key_code, key_scale, key_min, stats_dtype,
                           quantized_tokens, packed_capacity, bits, group_size, residual_key, res_dtype,
                           residual_tokens, r_st, r_sh, heads_kv, sm_scale, logits, as_stream(stream));
  PackedView v = parts_view(key_code, key_scale, key_min, nullptr, nullptr, nullptr, quantized_tokens,
                            packed_capacity, bits, group_size, residual_key, nullptr, residual_tokens, r_st, r_sh,
                            heads_kv, head_dim, stats_dtype, res_dtype);
  QKParams p{};
  p.Hq = heads_q; p.Lq = query_len; p.group = heads_q / heads_kv; p.rows = p.group * query_len;
  p.total = total; p.sm_scale = sm_scale; p.query = query; p.qd = q_dtype; p.logits = logits;
  dim3 grid(ceil_div(total, kTile), heads_kv, ceil_div(p.rows, kRows));
  hipStream_t s = as_stream(stream);
  if (bits == 2)
    hipLaunchKernelGGL((qk_kernel<2>), grid, dim3(kThreads), 0, s, v, p);
  else if (bits == 4)
    hipLaunchKernelGGL((qk_kernel<4>), grid, dim3(kThreads), 0, s, v, p);
  else
    hipLaunchKernelGGL((qk_kernel<8>), grid, dim3(kThreads), 0, s, v, p);
  return check_launch("uc_kivi_qk");
}

extern "C" int uc_kivi_av(const void *probs, int p_dtype, int64_t p_sh, int64_t p_si, int64_t p_st,
                          int64_t query_len, int64_t heads_q,
                          const void *value_code, const void *value_scale, const void *value_min, int stats_dtype,
                          int64_t quantized_tokens, int64_t packed_capacity, int bits, int group_size,
                          const void *residual_value, int res_dtype, int64_t residual_tokens,
                          int64_t r_st, int64_t r_sh,
                          int64_t heads_kv, int64_t head_dim,
                          void *out, int out_dtype, void *workspace, uc_stream_t stream) {
  UC_REQUIRE(ok_bits_group(bits, group_size), "uc_kivi_av: unsupported bits/group_size");
  UC_REQUIRE(valid_dtype(p_dtype) && valid_dtype(res_dtype) && valid_dtype(stats_dtype) && valid_dtype(out_dtype),
             "uc_kivi_av: unknown dtype code");
  UC_REQUIRE(heads_q > 0 && heads_kv > 0 && heads_q % heads_kv == 0, "Query heads must be divisible by KIVI KV heads");
  UC_REQUIRE(head_dim > 0 && head_dim <= kMaxD, "uc_kivi_av: head_dim must be <= %d", kMaxD);
  UC_REQUIRE(quantized_tokens % group_size == 0 && residual_tokens >= 0, "uc_kivi_av: bad token counts");
  UC_REQUIRE(packed_capacity == 0 || (packed_capacity >= quantized_tokens && packed_capacity % group_size == 0),
             "uc_kivi_av: packed_capacity must be 0 or a multiple of group_size >= quantized_tokens");
  if (query_len == 0) return UC_OK;
  const int64_t total = quantized_tokens + residual_tokens;
  hipStream_t s = as_stream(stream);
  const int64_t split_tokens = av_split_tokens(heads_q, query_len);
  const int64_t sp_packed = ceil_div(quantized_tokens, split_tokens);
  const int64_t sp_res = ceil_div(residual_tokens, split_tokens);
  const int64_t splits = sp_packed + sp_res;
  if (splits == 0) {
    // no keys: the product is zero
    const int64_t bytes = heads_q * query_len * head_dim * (out_dtype == UC_FP32 ? 4 : 2);
    UC_REQUIRE_RT(hipMemsetAsync(out, 0, bytes, s) == hipSuccess, "uc_kivi_av: memset failed");
    return UC_OK;
  }
  UC_REQUIRE(workspace != nullptr, "uc_kivi_av: workspace is NULL");
  // dense values and at least one workgroup of query rows per KV head: MFMA
  // tiles with V staged transposed in the workspace
  if (quantized_tokens == 0 && out_dtype == res_dtype &&
      pv_mfma_supported(p_dtype, probs, p_sh, p_si, p_st, res_dtype, residual_value, r_st, r_sh, head_dim, query_len,
                        heads_q / heads_kv * query_len, total))
    return launch_pv_mfma(p_dtype, probs, p_sh, p_si, res_dtype, residual_value, r_st, r_sh, query_len, heads_q, total,
                          heads_kv, out, workspace, s);
  if (parts_fast_supported(bits, group_size, head_dim, stats_dtype, res_dtype, r_st, r_sh, residual_value,
                           residual_tokens))
    return launch_parts_av(probs, p_dtype, p_sh, p_si, p_st, query_len, heads_q, value_code, value_scale, value_min,
                           stats_dtype, quantized_tokens, packed_capacity, bits, group_size, residual_value, res_dtype,
                           residual_tokens, r_st, r_sh, heads_kv, out, out_dtype, workspace, split_tokens, s);
  (void)total;
  uc_kivi_item it{};
  it.value_code = value_code; it.value_scale = value_scale; it.value_min = value_min;
  it.residual_value = residual_value; it.out = out;
  it.quantized_tokens = quantized_tokens; it.residual_tokens = residual_tokens;
  it.packed_capacity = packed_capacity;
  DecodeParams p{};
  p.Hq = heads_q; p.Hkv = heads_kv; p.D = head_dim; p.Lq = query_len; p.group = heads_q / heads_kv;
  p.rows = p.group * query_len; p.splits_packed = sp_packed; p.splits_total = splits;
  p.split_tokens = split_tokens;
  p.ws_o = static_cast<float *>(workspace);
  p.ws_ml = p.ws_o + heads_q * query_len * splits * head_dim;
  p.probs = probs; p.p_sh = p_sh; p.p_si = p_si; p.p_st = p_st;
  p.bits = bits; p.group_size = group_size;
  p.qd = UC_BF16; p.pd = p_dtype; p.rd = res_dtype;
  dim3 grid(splits, heads_kv, ceil_div(p.rows, kRows));
  const PackedView v = parts_view(nullptr, nullptr, nullptr, value_code, value_scale, value_min, quantized_tokens,
                                  packed_capacity, bits, group_size, nullptr, residual_value, residual_tokens, r_st,
                                  r_sh, heads_kv, head_dim, stats_dtype, res_dtype);
  if (bits == 2)
    hipLaunchKernelGGL((decode_partial_kernel<2, true, false>), grid, dim3(kThreads), 0, s, nullptr, it, v, p);
  else if (bits == 4)
    hipLaunchKernelGGL((decode_partial_kernel<4, true, false>), grid, dim3(kThreads), 0, s, nullptr, it, v, p);
  else
    hipLaunchKernelGGL((decode_partial_kernel<8, true, false>), grid, dim3(kThreads), 0, s, nullptr, it, v, p);
  int rc = check_launch("uc_kivi_av");
  if (rc != UC_OK) return rc;
  CombineParams c{};
  c.Hq = heads_q; c.Lq = query_len; c.D = head_dim; c.splits = splits;
  c.o_si = head_dim; c.o_sh = query_len * head_dim;
  c.ws_o = p.ws_o; c.ws_ml = p.ws_ml; c.normalize = 0;
  dim3 cgrid(heads_q * query_len, 1);
  c.od = out_dtype;
  hipLaunchKernelGGL((decode_combine_kernel<false>), cgrid, dim3(128), 0, s, nullptr, it, c);
  return check_launch("uc_kivi_av");
}

// ------------------------------------------------- allocation-free decode --
// Split partials of uc_kivi_attn_decode_static live in this file-scope array
// (one copy per GPU, held until the process ends).  Host code never passes
// `scratch` itself to a kernel: its name is a host-side stand-in.  The device
// address comes from hipGetSymbolAddress, once per device, on that device's
// first call.
static constexpr int64_t kDecodeScratchBytes = int64_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

namespace {
constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchMaxDevices];

// Device address of `scratch` on the calling thread's current device.
int scratch_address(void **out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  UC_REQUIRE_RT(err == hipSuccess, "uc_kivi_attn_decode_static: hipGetDevice failed: %s", hipGetErrorString(err));
  UC_REQUIRE_RT(dev >= 0 && dev < kScratchMaxDevices, "uc_kivi_attn_decode_static: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    UC_REQUIRE_RT(err == hipSuccess && p != nullptr,
                  "uc_kivi_attn_decode_static: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(err));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return UC_OK;
}
}  // namespace

extern "C" int64_t uc_kivi_decode_scratch_bytes(void) { return kDecodeScratchBytes; }

extern "C" int uc_kivi_attn_decode_static(const uc_kivi_item *item_host, int bits, int group_size,
                                          int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t query_len,
                                          int q_dtype, int res_dtype, int out_dtype, float sm_scale,
                                          uc_stream_t stream) {
  UC_REQUIRE(item_host != nullptr, "uc_kivi_attn_decode_static: item is NULL");
  UC_REQUIRE(item_host->quantized_tokens >= 0 && item_host->residual_tokens >= 0,
             "uc_kivi_attn_decode_static: negative token count");
  const int64_t need = uc_kivi_decode_workspace_bytes(1, bits, group_size, heads_q, heads_kv, head_dim, query_len,
                                                      item_host->quantized_tokens, item_host->residual_tokens);
  UC_REQUIRE(need >= 0, "uc_kivi_attn_decode_static: bad arguments");
  UC_REQUIRE(need <= kDecodeScratchBytes,
             "uc_kivi_attn_decode_static: the call needs %lld bytes of split scratch, more than the library's "
             "fixed %lld (use uc_kivi_attn_decode with a workspace)",
             (long long)need, (long long)kDecodeScratchBytes);
  void *ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != UC_OK) return rc;
  return decode_common(nullptr, item_host, 1, bits, group_size, heads_q, heads_kv, head_dim, query_len, q_dtype,
                       res_dtype, out_dtype, sm_scale, item_host->quantized_tokens, item_host->residual_tokens, ws,
                       kDecodeScratchBytes, as_stream(stream), "uc_kivi_attn_decode_static");
}
