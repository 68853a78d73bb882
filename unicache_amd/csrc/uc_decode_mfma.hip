// MFMA split-K decode over KIVI-packed KV (head_dim 128, 2/4-bit codes).
//
// One workgroup (2 waves) owns (item, KV head, split of S packed tokens) or
// a residual split.  The <= 16 query rows of a KV head (query heads x query
// length) form the N = 16 columns of every MFMA, so each packed byte is read
// from HBM once per (item, KV head).
//
// Keys (QK^T on v_mfma_f32_16x16x32_f16).  A key word holds TPW = 32/bits
// tokens of one channel.  MFMA rows are 16 consecutive words at one token
// position p, so each lane keeps its row's words for 32 channels in
// registers and reuses them for all TPW positions.  A code is turned into
// fp16 by OR-ing its bits into the mantissa of 1024 (0x6400), subtracting
// 1024 exactly and one packed FMA with the fp16 scale/min:
// k = fp16(code*scale + min).  The query (fp16) is the constant B operand.
//
// Values (P.V on v_mfma_f32_16x16x16f16).  A value word holds TPW channels of
// one token, but the B operand wants token pairs per register.  Codes of a
// word are spread into an A fragment (rows = 16 tokens, k = 16 channels) and
// transposed by an MFMA with a constant selection matrix whose accumulator is
// seeded with minus the mantissa offset, so it returns the exact codes in the
// B layout.  The per-token value scale rides in the A operand (P * scale);
// the per-token value minimum is folded back with one more MFMA (P x min)
// whose column g holds sum_t P*min of value group g.
//
// Each split writes a normalised fp16 partial with its (max, sum); a second
// kernel merges the splits with a log-sum-exp combine.
#include "uc_common.h"
#include "uc_decode.h"
#include "uc_mfma.h"


namespace uc {
namespace {

using namespace mf;

constexpr int kWaves = 2;
constexpr int kThreads = kWaves * kWave;
constexpr int kResWaveTokens = 128;  // residual tokens per wave per residual split

template <int BITS, int G>
struct DecShared {
  using Gm = Geo<BITS>;
  static constexpr int T = kWaves * Gm::ST;  // tokens staged per iteration
  static constexpr int KG = T / G;           // key groups per iteration
  static constexpr int NGD = kD / G;         // value groups per token
  static constexpr int JW = T / Gm::TPW;     // key words per channel per iteration
  static constexpr int KPAD = kD + 8;        // padded key-stat row (spreads LDS banks)
  _Float16 ks[KG][KPAD], km[KG][KPAD];                  // key stats [group][channel]
  _Float16 vs[NGD][Gm::TPW][JW], vm[NGD][Gm::TPW][JW];  // value stats [group][position][word]
  uint32_t kw[kWaves][4][4][16][8];                     // key words [block][k-slice][row][channel]
  uint32_t vw[kWaves][Gm::TPW][16][Gm::VW];             // value words [position][row][word]
};

struct MfmaParams {
  int64_t Hq, Hkv, Lq, group, rows;
  int64_t splits_packed, splits_total, nst;  // nst: super-tiles per wave per packed split
  float scale_log2;
  _Float16 *ws_o;  // [items * Hkv * splits][16][128] normalised partial outputs
  float *ws_ml;    // [items * Hkv * splits][16][2] (max in log2 units, sum)
  int qd, rd, od;
};

// Online-softmax state of one wave: lane holds (max, sum) of query row lane%16.
struct WaveState {
  f4 o[8];     // unnormalised output: lane (k = lane/16, n = lane%16) -> rows 4k+v, channel 16*blk + n
  f4 cmin;     // sum_t P*min, column n = value group
  float m, l;
};

// Base-2 softmax of a tile of logits (acc[p][v] = row 4k+v of the C layout,
// column = query row), folded into the running state; returns with acc holding
// the probabilities and the output rescaled.
template <int NP>
__device__ __forceinline__ void softmax_tile(f4 (&acc)[NP], const bool (&valid)[4], float scale_log2, WaveState &st,
                                             int lane) {
  float mx = kNegInf;
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float x = valid[v] ? acc[pp][v] * scale_log2 : kNegInf;
      acc[pp][v] = x;
      mx = fmaxf(mx, x);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
  mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
  const float m_new = fmaxf(st.m, mx);
  const float m_ref = m_new == kNegInf ? 0.0f : m_new;  // keeps -inf - m_ref at -inf (exp 0), never NaN
  float sum = 0.0f;
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float e = fast_exp2(acc[pp][v] - m_ref);
      acc[pp][v] = e;
      sum += e;
    }
  sum += __shfl_xor(sum, 16, kWave);
  sum += __shfl_xor(sum, 32, kWave);
  const float alpha = fast_exp2(st.m - m_ref);
  st.l = st.l * alpha + sum;
  st.m = m_new;
  // rescale the output rows 4k+v by the alpha of query row 4k+v
  const int k = lane >> 4;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float a = __shfl(alpha, 4 * k + v, kWave);
#pragma unroll
    for (int b = 0; b < 8; ++b) st.o[b][v] *= a;
    st.cmin[v] *= a;
  }
}

// Selection matrix of the value transposition: B[k][n] = 1/scale(k) when the
// channel spread into k-slot k is channel n of the 16-channel block.
template <int BITS>
__device__ __forceinline__ h4 transpose_selector(int lane) {
  const int n = lane & 15, kap = lane >> 4;
  h4 b;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    int ch;
    float inv;
    if constexpr (BITS == 2) {
      const int a = 2 * kap;
      const int chans[4] = {a, a + 8, a + 1, a + 9};
      ch = chans[v];
      inv = v < 2 ? 1.0f : 0.25f;
    } else {
      const int base = 8 * (kap >> 1), sub = kap & 1;
      const int chans[4] = {base + 2 * sub, base + 2 * sub + 4, base + 2 * sub + 1, base + 2 * sub + 5};
      ch = chans[v];
      inv = v < 2 ? 1.0f : 0.0625f;
    }
    b[v] = to_h(ch == n ? inv : 0.0f);
  }
  return b;
}

// Identity selection (k-slot k -> column k) for dense residual rows.
__device__ __forceinline__ h4 identity_selector(int lane) {
  const int n = lane & 15, kap = lane >> 4;
  h4 b;
#pragma unroll
  for (int v = 0; v < 4; ++v) b[v] = to_h(4 * kap + v == n ? 1.0f : 0.0f);
  return b;
}

// Codes of 16-channel block `blk` of one token, spread into the lane's four
// k-slots as fp16 (1024 + code * scale) for the transposition MFMA.
template <int BITS>
__device__ __forceinline__ h4 spread_value_codes(uint32_t word, int kap) {
  uint32_t y, m0, m1;
  if constexpr (BITS == 2) {
    y = word >> (4 * kap);
    m0 = 0x00030003u;
    m1 = 0x000C000Cu;
  } else {
    y = word >> (8 * (kap & 1));
    m0 = 0x000F000Fu;
    m1 = 0x00F000F0u;
  }
  const h2 a = as_h2(and_or(y, m0, 0x64006400u));
  const h2 b = as_h2(and_or(y, m1, 0x64006400u));
  return h4{a[0], a[1], b[0], b[1]};
}

// ------------------------------------------------------------ packed path --
// Query rows of the KV head staged once per workgroup as fp16 [row][channel]
// (padded rows); lane (n, k-slice) reads its B fragment of block kb from here.
constexpr int kQPad = kD + 8;

template <int QD>
__device__ __forceinline__ void stage_queries_t(_Float16 (*sq)[kQPad], const void *query, int64_t h,
                                                const MfmaParams &p) {
  // 16 rows x 128 channels; thread t converts 16 consecutive channels of row t/8
  const int n = threadIdx.x / 8, d0 = (threadIdx.x % 8) * 16;
  uint4 raw[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
  if (n < p.rows) {
    const int64_t g = n / p.Lq, i = n % p.Lq;
    const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(query) +
                                                       (i * p.Hq + h * p.group + g) * kD + d0);
    raw[0] = src[0];
    raw[1] = src[1];
  }
  *reinterpret_cast<h8 *>(&sq[n][d0]) = halves_to_h8<QD>(raw[0]);
  *reinterpret_cast<h8 *>(&sq[n][d0 + 8]) = halves_to_h8<QD>(raw[1]);
}

// Query rows of the KV head staged once per workgroup as fp16 [row][channel];
// fp32 queries take the element-wise path.
__device__ __forceinline__ void stage_queries(_Float16 (*sq)[kQPad], const void *query, int64_t h,
                                              const MfmaParams &p) {
  static_assert(kThreads == 16 * 8, "one thread per 16 channels of a query row");
  if (p.qd == UC_BF16) {
    stage_queries_t<UC_BF16>(sq, query, h, p);
  } else if (p.qd == UC_FP16) {
    stage_queries_t<UC_FP16>(sq, query, h, p);
  } else {
    for (int idx = threadIdx.x; idx < 16 * kD; idx += kThreads) {
      const int n = idx / kD, d = idx % kD;
      float v = 0.0f;
      if (n < p.rows) {
        const int64_t g = n / p.Lq, i = n % p.Lq;
        v = static_cast<const float *>(query)[(i * p.Hq + h * p.group + g) * kD + d];
      }
      sq[n][d] = to_h(v);
    }
  }
}

__device__ __forceinline__ h8 query_frag(const _Float16 (*sq)[kQPad], int kb, int lane) {
  return *reinterpret_cast<const h8 *>(&sq[lane & 15][32 * kb + 8 * (lane >> 4)]);
}

// Everything one iteration (T tokens of one KV head) reads from HBM, held in
// registers so the next iteration's loads overlap this iteration's MFMAs.
template <int BITS, int G>
struct Prefetch {
  using Gm = Geo<BITS>;
  using Sh = DecShared<BITS, G>;
  static constexpr int NKS = Sh::KG * kD / kThreads;        // key stats per thread (per stat)
  static constexpr int NVS = Sh::T * Sh::NGD / 8;           // 16-byte chunks of value stats
  static constexpr int VS4 = (NVS + kThreads - 1) / kThreads;
  static constexpr int NVW = Gm::ST * Gm::VW / 4 / kWave;   // 16-byte chunks of value words per lane
  uint32_t ks[NKS], km[NKS];
  uint4 vs[VS4], vm[VS4];
  uint4 vw[NVW];
  uint32_t kw[4][8];
};

template <int BITS, int G>
struct PackedRegion {
  Rsrc kcode, kscale, kmin, vcode, vscale, vmin;
  uint32_t nkw, nkg;  // key words / key groups per channel row
};

// Issue the loads of the iteration starting at token t0 (multiple of T).
template <int BITS, int G>
__device__ __forceinline__ void issue_loads(Prefetch<BITS, G> &pf, const PackedRegion<BITS, G> &rg, uint32_t t0) {
  using Gm = Geo<BITS>;
  using Sh = DecShared<BITS, G>;
  using Pf = Prefetch<BITS, G>;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  // key stats [D][nkg]: consecutive lanes read consecutive groups of one channel
  const uint32_t kg0 = t0 / G;
#pragma unroll
  for (int q = 0; q < Pf::NKS; ++q) {
    const int e = q * kThreads + tid, c = e / Sh::KG, j = e % Sh::KG;
    const uint32_t off = (c * rg.nkg + kg0 + j) * 2u;
    pf.ks[q] = bload16(rg.kscale, off);
    pf.km[q] = bload16(rg.kmin, off);
  }
  // value stats [Tq][NGD]
#pragma unroll
  for (int q = 0; q < Pf::VS4; ++q) {
    const int i = q * kThreads + tid;
    const uint32_t off = (t0 * Sh::NGD + 8 * (i < Pf::NVS ? i : 0)) * 2u;
    pf.vs[q] = bload128(rg.vscale, off);
    pf.vm[q] = bload128(rg.vmin, off);
  }
  // value words [Tq][VW] of this wave's super-tile
  const uint32_t tw0 = t0 + wave * Gm::ST;
#pragma unroll
  for (int q = 0; q < Pf::NVW; ++q) pf.vw[q] = bload128(rg.vcode, (tw0 * Gm::VW + 4 * (q * kWave + lane)) * 4u);
  // key words [D][nkw]: lane (row r, k-slice kap) reads word J of 32 channels
  const uint32_t J = t0 / Gm::TPW + wave * 16 + r;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int c = 0; c < 8; ++c) pf.kw[kb][c] = bload32(rg.kcode, ((32 * kb + 8 * kap + c) * rg.nkw + J) * 4u);
}

// Move a landed prefetch into the LDS layouts the MFMA loops read.
template <int BITS, int G>
__device__ __forceinline__ void stage_lds(DecShared<BITS, G> &sh, const Prefetch<BITS, G> &pf) {
  using Gm = Geo<BITS>;
  using Sh = DecShared<BITS, G>;
  using Pf = Prefetch<BITS, G>;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
#pragma unroll
  for (int q = 0; q < Pf::NKS; ++q) {
    const int e = q * kThreads + tid, c = e / Sh::KG, j = e % Sh::KG;
    sh.ks[j][c] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(pf.ks[q]));
    sh.km[j][c] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(pf.km[q]));
  }
#pragma unroll
  for (int q = 0; q < Pf::VS4; ++q) {
    if (q * kThreads + tid >= Pf::NVS) break;
    const int e0 = 8 * (q * kThreads + tid);
    const uint32_t sw[4] = {pf.vs[q].x, pf.vs[q].y, pf.vs[q].z, pf.vs[q].w};
    const uint32_t mw[4] = {pf.vm[q].x, pf.vm[q].y, pf.vm[q].z, pf.vm[q].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tl = (e0 + e) / Sh::NGD, gd = (e0 + e) % Sh::NGD;
      sh.vs[gd][tl % Gm::TPW][tl / Gm::TPW] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(sw[e / 2] >> (16 * (e % 2))));
      sh.vm[gd][tl % Gm::TPW][tl / Gm::TPW] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(mw[e / 2] >> (16 * (e % 2))));
    }
  }
#pragma unroll
  for (int q = 0; q < Pf::NVW; ++q) {
    const int i = q * kWave + lane;
    const int tok = (4 * i) / Gm::VW, word = (4 * i) % Gm::VW;  // token within the super-tile
    *reinterpret_cast<uint4 *>(&sh.vw[wave][tok % Gm::TPW][tok / Gm::TPW][word]) = pf.vw[q];
  }
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    uint4 *dst = reinterpret_cast<uint4 *>(&sh.kw[wave][kb][kap][r][0]);
    dst[0] = make_uint4(pf.kw[kb][0], pf.kw[kb][1], pf.kw[kb][2], pf.kw[kb][3]);
    dst[1] = make_uint4(pf.kw[kb][4], pf.kw[kb][5], pf.kw[kb][6], pf.kw[kb][7]);
  }
}

// Logits, softmax and P.V of one staged iteration (this wave's super-tile).
template <int BITS, int G>
__device__ __forceinline__ void compute_tile(const DecShared<BITS, G> &sh, const _Float16 (*sq)[kQPad],
                                             uint32_t t0, uint32_t nkw, float scale_log2, WaveState &st) {
  using Gm = Geo<BITS>;
  using Sh = DecShared<BITS, G>;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const h4 sel = transpose_selector<BITS>(lane);
  // the transposition returns code + 1024/scale; seeding its accumulator with
  // minus that offset (per column) makes it return the code itself
  const float off = (r & 1) ? (BITS == 2 ? 256.0f : 64.0f) : 1024.0f;
  const f4 neg_off = f4{-off, -off, -off, -off};
  constexpr int NP = Gm::TPW / 2;  // positions per half word
  const int gl = ((wave * 16 + r) * Gm::TPW) / G;  // key group of this lane's row
  bool valid[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) valid[v] = (t0 / Gm::TPW + wave * 16 + 4 * kap + v) < nkw;
#pragma unroll 1
  for (int half = 0; half < 2; ++half) {
    // ---- keys: logits for 16 word rows x NP positions x 16 query rows
    f4 acc[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) acc[q] = f4{0, 0, 0, 0};
    const uint32_t sel_half = half ? 0x07060302u : 0x05040100u;
#pragma unroll 1
    for (int kb = 0; kb < 4; ++kb) {
      const uint4 *kp = reinterpret_cast<const uint4 *>(&sh.kw[wave][kb][kap][r][0]);
      const uint4 w0 = kp[0], w1 = kp[1];
      const uint32_t kw[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      const h8 s8 = *reinterpret_cast<const h8 *>(&sh.ks[gl][32 * kb + 8 * kap]);
      const h8 m8 = *reinterpret_cast<const h8 *>(&sh.km[gl][32 * kb + 8 * kap]);
      const h8 qfrag = query_frag(sq, kb, lane);
      uint32_t y[4];
      h2 sp[4], mp[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        y[u] = __builtin_amdgcn_perm(kw[2 * u + 1], kw[2 * u], sel_half);
        sp[u] = h2{s8[2 * u], s8[2 * u + 1]};
        mp[u] = h2{m8[2 * u], m8[2 * u + 1]};
      }
#pragma unroll
      for (int pq = 0; pq < NP; ++pq) {
        const bool direct = pq <= Gm::PMAX;
        const int pe = direct ? pq : pq - (Gm::PMAX + 1);
        const _Float16 inv = to_h(1.0f / float(1u << (BITS * pe)));
        h8 a;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t src = direct ? y[u] : (y[u] >> Gm::SH);
          const h2 x = code_pair<BITS>(src, pe);
          const h2 k = __builtin_elementwise_fma(x, sp[u] * h2{inv, inv}, mp[u]);
          a[2 * u] = k[0];
          a[2 * u + 1] = k[1];
        }
        acc[pq] = mfma32(a, qfrag, acc[pq]);
      }
    }
    softmax_tile<NP>(acc, valid, scale_log2, st, lane);

    // ---- values of these positions
    const int jw = wave * 16 + 4 * kap;
#pragma unroll
    for (int pq = 0; pq < NP; ++pq) {
      const int pp = half * NP + pq;
      const h4 ap = cvt4(acc[pq]);  // A: rows = query rows, k = word rows 4k..4k+3 at position pp
      h4 as[Sh::NGD];
#pragma unroll
      for (int gd = 0; gd < Sh::NGD; ++gd) as[gd] = ap * *reinterpret_cast<const h4 *>(&sh.vs[gd][pp][jw]);
      const h4 bm = r < Sh::NGD ? *reinterpret_cast<const h4 *>(&sh.vm[r < Sh::NGD ? r : 0][pp][jw])
                                : h4{to_h(0.0f), to_h(0.0f), to_h(0.0f), to_h(0.0f)};
      st.cmin = mfma16(ap, bm, st.cmin);
      // the word holding channel block blk for this lane's k-slice: 2-bit rows
      // keep 16 channels per word, 4-bit rows 8 (even/odd word by k-slice pair)
      uint32_t words[8];
      if constexpr (BITS == 2) {
        const uint4 *row = reinterpret_cast<const uint4 *>(&sh.vw[wave][pp][r][0]);
        const uint4 a = row[0], b = row[1];
        words[0] = a.x; words[1] = a.y; words[2] = a.z; words[3] = a.w;
        words[4] = b.x; words[5] = b.y; words[6] = b.z; words[7] = b.w;
      } else {
        const uint32_t *row = &sh.vw[wave][pp][r][kap >> 1];
#pragma unroll
        for (int blk = 0; blk < 8; ++blk) words[blk] = row[2 * blk];
      }
      // all eight transpositions first, so their latency overlaps
      f4 ct[8];
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) ct[blk] = mfma16(spread_value_codes<BITS>(words[blk], kap), sel, neg_off);
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) st.o[blk] = mfma16(as[(16 * blk) / G], cvt4(ct[blk]), st.o[blk]);
    }
  }
}

template <int BITS, int G>
__device__ __forceinline__ void packed_split(DecShared<BITS, G> &sh, const _Float16 (*sq)[kQPad],
                                             const uc_kivi_item &it, int64_t h, int64_t t_split,
                                             const MfmaParams &p, WaveState &st) {
  using Gm = Geo<BITS>;
  using Sh = DecShared<BITS, G>;
  const int lane = threadIdx.x & 63;
  const int64_t Tq = it.quantized_tokens;
  PackedRegion<BITS, G> rg;
  rg.nkw = static_cast<uint32_t>(Tq / Gm::TPW);
  rg.nkg = static_cast<uint32_t>(Tq / G);
  const int64_t kcode_bytes = int64_t(kD) * rg.nkw * 4, kstat_bytes = int64_t(kD) * rg.nkg * 2;
  const int64_t vcode_bytes = Tq * Gm::VW * 4, vstat_bytes = Tq * Sh::NGD * 2;
  rg.kcode = make_rsrc(static_cast<const char *>(it.key_code) + h * kcode_bytes, kcode_bytes);
  rg.kscale = make_rsrc(static_cast<const char *>(it.key_scale) + h * kstat_bytes, kstat_bytes);
  rg.kmin = make_rsrc(static_cast<const char *>(it.key_min) + h * kstat_bytes, kstat_bytes);
  rg.vcode = make_rsrc(static_cast<const char *>(it.value_code) + h * vcode_bytes, vcode_bytes);
  rg.vscale = make_rsrc(static_cast<const char *>(it.value_scale) + h * vstat_bytes, vstat_bytes);
  rg.vmin = make_rsrc(static_cast<const char *>(it.value_min) + h * vstat_bytes, vstat_bytes);
  const int64_t left = Tq - t_split;
  const int n_it = static_cast<int>(min<int64_t>(p.nst, (left + Sh::T - 1) / Sh::T));
  Prefetch<BITS, G> pf;
  issue_loads<BITS, G>(pf, rg, static_cast<uint32_t>(t_split));
  for (int i = 0; i < n_it; ++i) {
    const uint32_t t0 = static_cast<uint32_t>(t_split + int64_t(i) * Sh::T);
    __syncthreads();  // every wave is done reading the previous iteration from LDS
    stage_lds<BITS, G>(sh, pf);
    __syncthreads();
    if (i + 1 < n_it) issue_loads<BITS, G>(pf, rg, t0 + Sh::T);  // lands while this iteration computes
    compute_tile<BITS, G>(sh, sq, t0, rg.nkw, p.scale_log2, st);
  }
  // fold the value minima back in: sum_t P*min of group gd sits in column gd
#pragma unroll
  for (int blk = 0; blk < 8; ++blk) {
    const int gd = (16 * blk) / G;
#pragma unroll
    for (int v = 0; v < 4; ++v) st.o[blk][v] += __shfl(st.cmin[v], (lane & 48) | gd, kWave);
  }
}

// --------------------------------------------------------- residual path --
// Dense residual tokens [tw, tw + kResWaveTokens) of this wave ([Tr, Hkv, 128]
// contiguous, bf16 or fp16), converted to fp16 for the same MFMAs; rows past
// Tr read as zero through the buffer range check and are masked.
template <int RD>
__device__ __forceinline__ h8 load8_h(Rsrc r, uint32_t off) {
  const uint4 raw = bload128(r, off);
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  h8 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[2 * j] = to_h(half_bits_to_f32<RD>(w[j]));
    out[2 * j + 1] = to_h(half_bits_to_f32<RD>(w[j] >> 16));
  }
  return out;
}

template <int RD>
__device__ __forceinline__ h4 load4_h(Rsrc r, uint32_t off) {
  const uint2 raw = bload64(r, off);
  return h4{to_h(half_bits_to_f32<RD>(raw.x)), to_h(half_bits_to_f32<RD>(raw.x >> 16)),
            to_h(half_bits_to_f32<RD>(raw.y)), to_h(half_bits_to_f32<RD>(raw.y >> 16))};
}

template <int RD>
__device__ __forceinline__ void residual_split(const _Float16 (*sq)[kQPad], const uc_kivi_item &it, int64_t h,
                                               int64_t tr0, const MfmaParams &p, WaveState &st) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const int64_t Tr = it.residual_tokens;
  const int64_t bytes = Tr * p.Hkv * kD * 2;
  const Rsrc rk = make_rsrc(it.residual_key, bytes), rv = make_rsrc(it.residual_value, bytes);
  const int64_t tw = tr0 + wave * kResWaveTokens;
  constexpr int kBlocks = kResWaveTokens / 16;
  const h4 ident = identity_selector(lane);
  f4 acc[kBlocks];
#pragma unroll
  for (int b = 0; b < kBlocks; ++b) {
    acc[b] = f4{0, 0, 0, 0};
    const uint32_t base = static_cast<uint32_t>(((tw + 16 * b + r) * p.Hkv + h) * kD * 2);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      acc[b] = mfma32(load8_h<RD>(rk, base + (32 * kb + 8 * kap) * 2), query_frag(sq, kb, lane), acc[b]);
  }
  float mx = kNegInf;
#pragma unroll
  for (int b = 0; b < kBlocks; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const bool ok = tw + 16 * b + 4 * kap + v < Tr;
      const float x = ok ? acc[b][v] * p.scale_log2 : kNegInf;
      acc[b][v] = x;
      mx = fmaxf(mx, x);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
  mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
  float sum = 0.0f;
#pragma unroll
  for (int b = 0; b < kBlocks; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float e = acc[b][v] == kNegInf ? 0.0f : exp2f(acc[b][v] - mx);
      acc[b][v] = e;
      sum += e;
    }
  sum += __shfl_xor(sum, 16, kWave);
  sum += __shfl_xor(sum, 32, kWave);
  st.m = mx;
  st.l = sum;
#pragma unroll
  for (int b = 0; b < kBlocks; ++b) {
    const h4 ap = cvt4(acc[b]);
    const uint32_t base = static_cast<uint32_t>(((tw + 16 * b + r) * p.Hkv + h) * kD * 2);
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      const f4 ct = mfma16(load4_h<RD>(rv, base + (16 * blk + 4 * kap) * 2), ident, f4{0, 0, 0, 0});
      st.o[blk] = mfma16(ap, cvt4(ct), st.o[blk]);
    }
  }
}

// ------------------------------------------------------------------ kernel --
static_assert(kThreads == kD, "key-stat staging maps one thread per channel");

template <int BITS, int G, int RD, bool TABLE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void decode_mfma_kernel(
    const uc_kivi_item *items, uc_kivi_item single, MfmaParams p) {
  __shared__ DecShared<BITS, G> sh;
  __shared__ _Float16 sq[16][kQPad];
  __shared__ float mrg_ml[kWaves][16][2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t item = TABLE ? blockIdx.z : 0;
  const uc_kivi_item it = TABLE ? items[item] : single;
  const int64_t h = blockIdx.y, split = blockIdx.x;

  stage_queries(sq, it.query, h, p);
  WaveState st;
#pragma unroll
  for (int b = 0; b < 8; ++b) st.o[b] = f4{0, 0, 0, 0};
  st.cmin = f4{0, 0, 0, 0};
  st.m = kNegInf;
  st.l = 0.0f;
  __syncthreads();

  if (split < p.splits_packed) {
    const int64_t t_split = split * p.nst * DecShared<BITS, G>::T;
    if (t_split < it.quantized_tokens) packed_split<BITS, G>(sh, sq, it, h, t_split, p, st);
  } else {
    const int64_t tr0 = (split - p.splits_packed) * kWaves * kResWaveTokens;
    if (tr0 < it.residual_tokens) residual_split<RD>(sq, it, h, tr0, p, st);
  }

  // ---- merge the two waves: rows 4k+v of o need the (m, l) of query row 4k+v
  __syncthreads();
  if ((lane >> 4) == 0) {
    mrg_ml[wave][lane][0] = st.m;
    mrg_ml[wave][lane][1] = st.l;
  }
  __syncthreads();
  float *fin = reinterpret_cast<float *>(sh.vw);  // [16][128] partial of wave 1
  const int kap = lane >> 4, n = lane & 15;
  float scale[4], Lrow[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int row = 4 * kap + v;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mrg_ml[w][row][0]);
    float L = 0.0f, mine = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = mrg_ml[w][row][0];
      const float f = mw == kNegInf ? 0.0f : exp2f(mw - M);
      L += mrg_ml[w][row][1] * f;
      if (w == wave) mine = f;
    }
    scale[v] = mine;
    Lrow[v] = L;
  }
  if (wave == 1) {
#pragma unroll
    for (int blk = 0; blk < 8; ++blk)
#pragma unroll
      for (int v = 0; v < 4; ++v) fin[(4 * kap + v) * kD + 16 * blk + n] = st.o[blk][v] * scale[v];
  }
  __syncthreads();
  const int64_t slot = (item * p.Hkv + h) * p.splits_total + split;
  if (wave == 0) {
    _Float16 *po = p.ws_o + slot * 16 * kD;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = 4 * kap + v;
      const float inv = Lrow[v] > 0.0f ? 1.0f / Lrow[v] : 0.0f;
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) {
        const float o = st.o[blk][v] * scale[v] + fin[row * kD + 16 * blk + n];
        po[row * kD + 16 * blk + n] = to_h(o * inv);
      }
    }
    if (kap == 0) {
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mrg_ml[w][n][0]);
      float L = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float mw = mrg_ml[w][n][0];
        L += mw == kNegInf ? 0.0f : mrg_ml[w][n][1] * exp2f(mw - M);
      }
      p.ws_ml[(slot * 16 + n) * 2 + 0] = M;
      p.ws_ml[(slot * 16 + n) * 2 + 1] = L;
    }
  }
}

// Merge the split partials of one (item, KV head): per query row the split
// weights l_s 2^(m_s - M) / L, then the weighted sum of the fp16 partials.
template <bool TABLE>
__global__ __launch_bounds__(256) void decode_mfma_combine(const uc_kivi_item *items, uc_kivi_item single,
                                                            MfmaParams p) {
  constexpr int kMaxSplits = 64;
  __shared__ float wts[16][kMaxSplits];
  const int64_t item = TABLE ? blockIdx.y : 0;
  const uc_kivi_item it = TABLE ? items[item] : single;
  const int64_t h = blockIdx.x;
  const int64_t slot0 = (item * p.Hkv + h) * p.splits_total;
  const int tid = threadIdx.x;
  const int nsplit = int(p.splits_total);
  for (int s0 = 0; s0 < nsplit; s0 += kMaxSplits) {
    const int ns = min(kMaxSplits, nsplit - s0);
    __syncthreads();
    if (tid < p.rows) {
      float M = kNegInf;
      for (int s = 0; s < nsplit; ++s) M = fmaxf(M, p.ws_ml[((slot0 + s) * 16 + tid) * 2]);
      float L = 0.0f;
      for (int s = 0; s < nsplit; ++s) {
        const float m = p.ws_ml[((slot0 + s) * 16 + tid) * 2], l = p.ws_ml[((slot0 + s) * 16 + tid) * 2 + 1];
        if (l > 0.0f && m != kNegInf) L += l * exp2f(m - M);
      }
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      for (int s = 0; s < ns; ++s) {
        const float m = p.ws_ml[((slot0 + s0 + s) * 16 + tid) * 2], l = p.ws_ml[((slot0 + s0 + s) * 16 + tid) * 2 + 1];
        wts[tid][s] = (l > 0.0f && m != kNegInf) ? l * exp2f(m - M) * inv : 0.0f;
      }
      if (s0 == 0 && it.lse != nullptr) {
        const int64_t g = tid / p.Lq, i = tid % p.Lq;
        it.lse[(h * p.group + g) * p.Lq + i] = L > 0.0f ? (M + log2f(L)) * kLn2 : kNegInf;
      }
    }
    __syncthreads();
    // each thread: 8 channels of one row
    for (int idx = tid; idx < p.rows * (kD / 8); idx += blockDim.x) {
      const int row = idx / (kD / 8), c8 = (idx % (kD / 8)) * 8;
      float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (s0 > 0) {
        // later chunks accumulate onto the output written by the first chunk
        const int64_t g = row / p.Lq, i = row % p.Lq;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = load_dyn(it.out, (i * p.Hq + h * p.group + g) * kD + c8 + j, p.od);
      }
      for (int s = 0; s < ns; ++s) {
        const float w = wts[row][s];
        if (w == 0.0f) continue;
        const h8 v = *reinterpret_cast<const h8 *>(p.ws_o + ((slot0 + s0 + s) * 16 + row) * kD + c8);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = fmaf(float(v[j]), w, o[j]);
      }
      const int64_t g = row / p.Lq, i = row % p.Lq;
#pragma unroll
      for (int j = 0; j < 8; ++j) store_dyn(it.out, (i * p.Hq + h * p.group + g) * kD + c8 + j, o[j], p.od);
    }
  }
}

}  // namespace

// Packed tokens per split of the MFMA decode for `bits` (super-tiles per
// wave x waves x tokens per super-tile).
int64_t decode_mfma_split_tokens(int bits, int64_t nst) { return nst * kWaves * 16 * (32 / bits); }

int64_t decode_mfma_res_split_tokens() { return kWaves * kResWaveTokens; }

bool decode_mfma_supported(int bits, int group, int64_t D, int64_t rows) {
  return (bits == 2 || bits == 4) && (group == 32 || group == 64 || group == 128) && D == kD && rows <= 16;
}

int64_t decode_mfma_workspace_bytes(int64_t n_items, int64_t heads_kv, int64_t splits) {
  const int64_t slots = n_items * heads_kv * splits;
  return slots * 16 * kD * int64_t(sizeof(_Float16)) + slots * 16 * 2 * int64_t(sizeof(float));
}

template <int BITS, int G, int RD>
static void launch_typed(bool table, dim3 grid, hipStream_t stream, const uc_kivi_item *items_dev,
                         const uc_kivi_item &one, const MfmaParams &p) {
  if (table)
    hipLaunchKernelGGL((decode_mfma_kernel<BITS, G, RD, true>), grid, dim3(kThreads), 0, stream, items_dev, one, p);
  else
    hipLaunchKernelGGL((decode_mfma_kernel<BITS, G, RD, false>), grid, dim3(kThreads), 0, stream, items_dev, one, p);
}

template <int BITS, int G>
static void launch_group(bool table, int rd, dim3 grid, hipStream_t stream, const uc_kivi_item *items_dev,
                         const uc_kivi_item &one, const MfmaParams &p) {
  if (rd == UC_FP16)
    launch_typed<BITS, G, UC_FP16>(table, grid, stream, items_dev, one, p);
  else
    launch_typed<BITS, G, UC_BF16>(table, grid, stream, items_dev, one, p);
}

int launch_decode_mfma(const uc_kivi_item *items_dev, const uc_kivi_item *single, int64_t n_items, int bits,
                       int group_size, int64_t Hq, int64_t Hkv, int64_t Lq, int q_dtype, int res_dtype,
                       int out_dtype, float sm_scale, int64_t max_tq, int64_t max_tr, int64_t nst, void *workspace,
                       int64_t workspace_bytes, hipStream_t stream) {
  const int64_t s_tok = decode_mfma_split_tokens(bits, nst);
  const int64_t r_tok = decode_mfma_res_split_tokens();
  MfmaParams p{};
  p.Hq = Hq; p.Hkv = Hkv; p.Lq = Lq; p.group = Hq / Hkv; p.rows = p.group * Lq;
  p.splits_packed = ceil_div(max_tq, s_tok);
  p.splits_total = p.splits_packed + ceil_div(max_tr, r_tok);
  p.nst = nst;
  p.scale_log2 = sm_scale * kLog2e;
  p.qd = q_dtype; p.rd = res_dtype; p.od = out_dtype;
  if (p.splits_total == 0) return UC_OK;
  // buffer offsets are 32-bit: one KV head's packed rows and the whole residual must fit
  UC_REQUIRE(max_tq * (kD / 8) * 4 < (int64_t(1) << 31) && max_tr * Hkv * kD * 2 < (int64_t(1) << 31),
             "decode: segment too long for 32-bit buffer offsets (%lld packed, %lld residual tokens)",
             (long long)max_tq, (long long)max_tr);
  const int64_t need = decode_mfma_workspace_bytes(n_items, Hkv, p.splits_total);
  UC_REQUIRE(workspace != nullptr && workspace_bytes >= need, "decode: workspace too small (%lld < %lld bytes)",
             (long long)workspace_bytes, (long long)need);
  const int64_t slots = n_items * Hkv * p.splits_total;
  p.ws_o = static_cast<_Float16 *>(workspace);
  p.ws_ml = reinterpret_cast<float *>(static_cast<char *>(workspace) + slots * 16 * kD * sizeof(_Float16));
  const bool table = items_dev != nullptr;
  const uc_kivi_item one = single ? *single : uc_kivi_item{};
  const dim3 grid(p.splits_total, Hkv, n_items);
  if (bits == 2) {
    if (group_size == 32) launch_group<2, 32>(table, res_dtype, grid, stream, items_dev, one, p);
    else if (group_size == 64) launch_group<2, 64>(table, res_dtype, grid, stream, items_dev, one, p);
    else launch_group<2, 128>(table, res_dtype, grid, stream, items_dev, one, p);
  } else {
    if (group_size == 32) launch_group<4, 32>(table, res_dtype, grid, stream, items_dev, one, p);
    else if (group_size == 64) launch_group<4, 64>(table, res_dtype, grid, stream, items_dev, one, p);
    else launch_group<4, 128>(table, res_dtype, grid, stream, items_dev, one, p);
  }
  int rc = check_launch("decode (MFMA)");
  if (rc != UC_OK) return rc;
  if (table)
    hipLaunchKernelGGL((decode_mfma_combine<true>), dim3(Hkv, n_items), dim3(256), 0, stream, items_dev, one, p);
  else
    hipLaunchKernelGGL((decode_mfma_combine<false>), dim3(Hkv, n_items), dim3(256), 0, stream, items_dev, one, p);
  return check_launch("decode (MFMA combine)");
}

}  // namespace uc
