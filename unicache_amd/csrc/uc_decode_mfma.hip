// MFMA split-K decode over KIVI-packed KV (head_dim 128, 2/4-bit codes).
//
// One workgroup (2 waves) owns a packed split of one unit (item, KV head) --
// every S-th super-tile (16 key words of every channel) starting at the split
// index -- or a residual split.  The S splits of a unit run side by side on
// one XCD, so the 128-byte lines of the channel-major key streams are read
// from HBM about once although each split uses a part of them.  An iteration
// stages one super-tile and each wave takes half of its token positions.  The
// <= 16 query rows of a KV head (query heads x query length) form the N = 16
// columns of every MFMA.
//
// Keys (QK^T on v_mfma_f32_16x16x32_f16).  A key word holds TPW = 32/bits
// tokens of one channel.  MFMA rows are 16 consecutive words at one token
// position p, so each lane keeps its row's words for 32 channels in
// registers and reuses them for all positions of its half.  A code at bit
// offset BITS*e of a 16-bit half is turned into fp16 by OR-ing its bits into
// the mantissa of 2^(10 - BITS*e), whose mantissa unit is then exactly 1, and
// subtracting that power of two; one packed FMA with the fp16 scale/min gives
// k = fp16(code*scale + min).  The query (fp16) is the constant B operand.
//
// Values (O^T += V^T P^T on v_mfma_f32_16x16x32_f16).  A value word holds
// TPW channels of one token; the A operand wants token pairs of one channel
// per register.  A 32-channel block is split into its even and odd channels
// (MFMA row r = channel 32b + 2r + i), so the two channels of a lane share one
// byte: one v_perm gathers that byte of two tokens into the two 16-bit halves
// and one AND per channel leaves code << offset in each half -- an fp16
// denormal code * 2^(offset - 24), which the MFMA multiplies exactly; the
// power of two is undone per channel at the end.  The per-token value scale
// rides in the B operand (P * scale); the per-token value minimum is folded
// back with one more MFMA (min x P) whose rows all hold sum_t P*min of value
// group g.
//
// Each split writes a normalised fp16 partial with its (max, sum); a second
// kernel merges the splits with a log-sum-exp combine.
#include "uc_common.h"
#include "uc_decode.h"
#include "uc_mfma.h"


namespace uc {
namespace {

using namespace mf;

constexpr int kXcds = 8;  // XCDs of an MI355X; workgroup i of a launch runs on XCD i % 8
constexpr int kWaves = 2;
constexpr int kThreads = kWaves * kWave;
constexpr int kResWaveTokens = 128;  // residual tokens per wave per residual split

template <int BITS, int G>
struct DecShared {
  using Gm = Geo<BITS>;
  static constexpr int T = Gm::ST;           // tokens staged per iteration (one super-tile)
  static constexpr int KG = T / G;           // key groups per iteration
  static constexpr int NGD = kD / G;         // value groups per token
  static constexpr int JW = T / Gm::TPW;     // key words per channel per iteration
  static constexpr int KPAD = kD + 16;       // key-stat row of 72 dwords: the 8 groups one read touches start 8 banks apart
  _Float16 ks[KG][KPAD], km[KG][KPAD];                  // key stats [group][channel]
  // value stats [group][position / 2][word / 4][position % 2][word % 4]: the
  // 8 values one MFMA k-slice needs (words 4k..4k+3 at positions 2j, 2j+1) are
  // one 16-byte read
  _Float16 vs[NGD][Gm::TPW / 2][JW / 4][2][4], vm[NGD][Gm::TPW / 2][JW / 4][2][4];
  uint32_t kw[4][4][16][8];                             // key words [block][k-slice][row][channel]
  // value words [position][word][row], rows padded to 20 dwords: a lane reads
  // four rows of one word as 16 bytes, and staging writes hit distinct banks
  static constexpr int VROW = 20;
  uint32_t vw[Gm::TPW][Gm::VW][VROW];
};

struct MfmaParams {
  int64_t Hq, Hkv, Lq, group, rows;
  int64_t splits_packed, splits_total, nst;  // nst: super-tiles per packed split
  int64_t segs;                              // consecutive items that share one query and output
  int64_t units;                             // items x KV heads
  int64_t super_tokens;                      // tokens per super-tile (16 key words)
  int xcd_grouped;                           // splits of a unit on one XCD (see the kernel)
  float scale_log2;
  _Float16 *ws_o;  // [items * Hkv * splits][16][128] normalised partial outputs
  float *ws_ml;    // [items * Hkv * splits][16][2] (max in log2 units, sum)
  int qd, rd, od;
};

// Whether split `split` of an item with tq packed and tr residual tokens has
// work: residual splits come first, then packed splits of every S-th
// super-tile.  Splits without work write only (max, sum) = (-inf, 0), so a
// segment table whose items differ in length launches cheap empty splits.
__device__ __forceinline__ bool split_has_work(int64_t split, int64_t tq, int64_t tr, const MfmaParams &p) {
  const int64_t splits_res = p.splits_total - p.splits_packed;
  return split >= splits_res ? (split - splits_res) * p.super_tokens < tq : split * kWaves * kResWaveTokens < tr;
}

// Online-softmax state of one wave.  The output is accumulated transposed
// (O^T = V^T P^T): lane (n, k) owns query column n, so every rescale is
// lane-local.
struct WaveState {
  f4 o[8];     // lane (n = lane%16, k = lane/16): query n, channel out_channel(cb, k, v)
  f4 cmin[4];  // sum_t P*min of value group g (every row of the block holds it)
  float m;     // running max of query n (log2 units), equal across the k-slices
  float l;     // this lane's share of the running sum (reduced over the k-slices at the end)
};

// Base-2 softmax of a tile of logits (acc[p][v] = row 4k+v of the C layout,
// column = query), folded into the running state; returns with acc holding the
// probabilities and the output rescaled.
template <int NP>
__device__ __forceinline__ void softmax_tile(f4 (&acc)[NP], const bool (&valid)[4], bool full, float scale_log2,
                                             WaveState &st) {
  if (!full) {  // only the last iteration of a segment has rows past its end
#pragma unroll
    for (int pp = 0; pp < NP; ++pp)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (!valid[v]) acc[pp][v] = kNegInf;
  }
  float mx = kNegInf;
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int v = 0; v < 4; ++v) mx = fmaxf(mx, acc[pp][v]);
  mx = max_over_slices(mx);
  const float m_new = fmaxf(st.m, mx * scale_log2);
  const float m_ref = m_new == kNegInf ? 0.0f : m_new;  // keeps -inf - m_ref at -inf (exp 0), never NaN
  float sum = 0.0f;
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float e = fast_exp2(__builtin_fmaf(acc[pp][v], scale_log2, -m_ref));
      acc[pp][v] = e;
      sum += e;
    }
  const float alpha = fast_exp2(st.m - m_ref);
  st.l = st.l * alpha + sum;
  st.m = m_new;
  if (__any(alpha != 1.0f)) {
#pragma unroll
    for (int b = 0; b < 8; ++b) st.o[b] *= alpha;
#pragma unroll
    for (int g = 0; g < 4; ++g) st.cmin[g] *= alpha;
  }
}

// Output row v of accumulator cb in lane k-slice kap: channel
// 32 (cb / 2) + 8 kap + 2 v + cb % 2 -- MFMA cb holds the even (cb % 2 = 0) or
// odd channels of the 32-channel block cb / 2, so a lane's eight outputs of a
// block are the contiguous channels 32 (cb / 2) + 8 kap + [0, 8).
__device__ __forceinline__ constexpr int out_channel(int cb, int kap, int v) {
  return 32 * (cb >> 1) + 8 * kap + 2 * v + (cb & 1);
}

// Bit offset of channel c's code inside the byte that holds it.
template <int BITS>
__device__ __forceinline__ constexpr int value_shift(int c) {
  return BITS == 2 ? 2 * (c & 3) : 4 * (c & 1);
}

// Selection B operand that picks channel 2n + i of a 32-channel A fragment
// into column n: B[k][n] = (k == 2n + i).
__device__ __forceinline__ h8 channel_selector(int lane, int i) {
  const int n = lane & 15, kap = lane >> 4;
  h8 b;
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = to_h(8 * kap + j == 2 * n + i ? 1.0f : 0.0f);
  return b;
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
  static constexpr int NKD = (Sh::KG + 1) / 2 + 1;         // dwords of one key-stat row segment
  static constexpr int NVS = Sh::T * Sh::NGD / 8;           // 16-byte chunks of value stats
  static constexpr int VS4 = (NVS + kThreads - 1) / kThreads;
  static constexpr int NVW = Gm::ST * Gm::VW / 4 / kThreads;  // 16-byte chunks of value words per thread
  static constexpr int NKB = 4 / kWaves;                       // key-word blocks per thread
  uint32_t ks[NKD], km[NKD];  // thread = channel: KG halves from a 4-byte aligned start
  uint4 vs[VS4], vm[VS4];
  uint4 vw[NVW];
  uint32_t kw[NKB][8];
};

template <int BITS, int G>
struct PackedRegion {
  Rsrc kcode, kscale, kmin, vcode, vscale, vmin;
  uint32_t nkw, nkg;  // key words / key groups per channel row
};

// Which 16-byte chunk of value words load q of lane group a brings: the four
// groups of one load land on four different 16-dword bank windows of the
// [position][word][row] staging layout (block stride 20 dwords).
template <int BITS>
__device__ __forceinline__ void value_chunk(int q, int a, int &pos, int &quad) {
  if constexpr (BITS == 2) {  // 8 words = 2 quads per token, 16 positions: 8 loads
    pos = 2 * q + (a >> 1);
    quad = a & 1;
  } else {                    // 16 words = 4 quads per token, 8 positions: 8 loads
    pos = q;
    quad = a;
  }
}

// The first N dwords of d: consecutive dwords from byte offset `off` (4-byte
// aligned) in the fewest loads.
template <int N, int M>
__device__ __forceinline__ void load_dwords(uint32_t (&d)[M], Rsrc r, uint32_t off) {
  static_assert(N <= M, "load fits the array");
  int q = 0;
#pragma unroll
  for (; q + 4 <= N; q += 4) {
    const uint4 v = bload128(r, off + 4u * q);
    d[q] = v.x, d[q + 1] = v.y, d[q + 2] = v.z, d[q + 3] = v.w;
  }
  if constexpr (N % 4 >= 2) {
    const uint2 v = bload64(r, off + 4u * q);
    d[q] = v.x, d[q + 1] = v.y;
    q += 2;
  }
  if constexpr (N % 2 == 1) d[N - 1] = bload32(r, off + 4u * (N - 1));
}

// Issue the loads of the iteration starting at token t0 (multiple of T).
template <int BITS, int G>
__device__ __forceinline__ void issue_loads(Prefetch<BITS, G> &pf, const PackedRegion<BITS, G> &rg, uint32_t t0) {
  using Gm = Geo<BITS>;
  using Sh = DecShared<BITS, G>;
  using Pf = Prefetch<BITS, G>;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  // key stats [D][nkg]: thread = channel, its KG groups as dwords from the
  // 4-byte boundary at or below the first (realigned when staged)
  // (one 16-byte load per four dwords: each load of a wave touches 64 rows, so
  // fewer, wider loads mean fewer memory requests; when every row segment
  // starts on a dword -- even nkg and t0 / G -- the last dword is not needed)
  {
    const uint32_t d0 = (tid * rg.nkg + t0 / G) >> 1;
    if (((rg.nkg | (t0 / G)) & 1u) == 0u) {
      load_dwords<Pf::NKD - 1>(pf.ks, rg.kscale, d0 * 4u);
      load_dwords<Pf::NKD - 1>(pf.km, rg.kmin, d0 * 4u);
      pf.ks[Pf::NKD - 1] = pf.km[Pf::NKD - 1] = 0u;  // read by the realignment with shift 0
    } else {
      load_dwords<Pf::NKD>(pf.ks, rg.kscale, d0 * 4u);
      load_dwords<Pf::NKD>(pf.km, rg.kmin, d0 * 4u);
    }
  }
  // value stats [Tq][NGD]
#pragma unroll
  for (int q = 0; q < Pf::VS4; ++q) {
    const int i = q * kThreads + tid;
    const uint32_t off = (t0 * Sh::NGD + 8 * (i < Pf::NVS ? i : 0)) * 2u;
    pf.vs[q] = bload128(rg.vscale, off);
    pf.vm[q] = bload128(rg.vmin, off);
  }
  // value words [Tq][VW] of the super-tile, 16 bytes (4 words of one token)
  // per load: lane (row = lane%16, group a = lane/16) of wave w takes word-row
  // `row` at (position, word quad) = value_chunk(q * kWaves + w, a)
#pragma unroll
  for (int q = 0; q < Pf::NVW; ++q) {
    int pos, quad;
    value_chunk<BITS>(q * kWaves + wave, lane >> 4, pos, quad);
    const uint32_t tok = t0 + (lane & 15) * Gm::TPW + pos;
    pf.vw[q] = bload128(rg.vcode, (tok * Gm::VW + 4 * quad) * 4u);
  }
  // key words [D][nkw]: lane (row r, k-slice kap) of wave w reads word J of
  // the 16 channels 32 kb + 8 kap + [0, 8) of its blocks kb = NKB w + [0, NKB)
  const uint32_t J = t0 / Gm::TPW + r;
#pragma unroll
  for (int b = 0; b < Pf::NKB; ++b)
#pragma unroll
    for (int c = 0; c < 8; ++c)
      pf.kw[b][c] = bload32(rg.kcode, ((32 * (Pf::NKB * wave + b) + 8 * kap + c) * rg.nkw + J) * 4u);
}

// Move a landed prefetch into the LDS layouts the MFMA loops read.
template <int BITS, int G>
__device__ __forceinline__ void stage_lds(DecShared<BITS, G> &sh, const Prefetch<BITS, G> &pf, uint32_t t0,
                                          uint32_t nkg) {
  using Gm = Geo<BITS>;
  using Sh = DecShared<BITS, G>;
  using Pf = Prefetch<BITS, G>;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  {
    const uint32_t shift = ((tid * nkg + t0 / G) & 1u) * 16u;  // odd first element: start at the high half
#pragma unroll
    for (int q = 0; q < (Sh::KG + 1) / 2; ++q) {
      const uint32_t s2 = __builtin_amdgcn_alignbit(pf.ks[q + 1], pf.ks[q], shift);
      const uint32_t m2 = __builtin_amdgcn_alignbit(pf.km[q + 1], pf.km[q], shift);
      sh.ks[2 * q][tid] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(s2));
      sh.km[2 * q][tid] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(m2));
      if (2 * q + 1 < Sh::KG) {
        sh.ks[2 * q + 1][tid] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(s2 >> 16));
        sh.km[2 * q + 1][tid] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(m2 >> 16));
      }
    }
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
      const int pos = tl % Gm::TPW, row = tl / Gm::TPW;
      sh.vs[gd][pos / 2][row / 4][pos % 2][row % 4] =
          __builtin_bit_cast(_Float16, static_cast<uint16_t>(sw[e / 2] >> (16 * (e % 2))));
      sh.vm[gd][pos / 2][row / 4][pos % 2][row % 4] =
          __builtin_bit_cast(_Float16, static_cast<uint16_t>(mw[e / 2] >> (16 * (e % 2))));
    }
  }
#pragma unroll
  for (int q = 0; q < Pf::NVW; ++q) {
    int pos, quad;
    value_chunk<BITS>(q * kWaves + wave, lane >> 4, pos, quad);
    const uint32_t w4[4] = {pf.vw[q].x, pf.vw[q].y, pf.vw[q].z, pf.vw[q].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) sh.vw[pos][4 * quad + j][lane & 15] = w4[j];
  }
#pragma unroll
  for (int b = 0; b < Pf::NKB; ++b) {
    uint4 *dst = reinterpret_cast<uint4 *>(&sh.kw[Pf::NKB * wave + b][kap][r][0]);
    dst[0] = make_uint4(pf.kw[b][0], pf.kw[b][1], pf.kw[b][2], pf.kw[b][3]);
    dst[1] = make_uint4(pf.kw[b][4], pf.kw[b][5], pf.kw[b][6], pf.kw[b][7]);
  }
}

// Logits, softmax and P.V of this wave's half of the staged super-tile.
template <int BITS, int G>
__device__ __forceinline__ void compute_tile(const DecShared<BITS, G> &sh, const _Float16 (*sq)[kQPad],
                                             uint32_t t0, uint32_t nkw, float scale_log2, WaveState &st) {
  using Gm = Geo<BITS>;
  using Sh = DecShared<BITS, G>;
  const int tid = threadIdx.x, lane = tid & 63, half = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  constexpr int NP = Gm::TPW / 2;  // positions per half word
  const int gl = (r * Gm::TPW) / G;  // key group of this lane's row
  bool valid[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) valid[v] = (t0 / Gm::TPW + 4 * kap + v) < nkw;
  const bool full = t0 / Gm::TPW + 16 <= nkw;  // every word row of the iteration is a real token

  // ---- keys: logits for 16 word rows x NP positions x 16 query rows
  f4 acc[NP];
#pragma unroll
  for (int q = 0; q < NP; ++q) acc[q] = f4{0, 0, 0, 0};
  const uint32_t sel_half = half ? 0x07060302u : 0x05040100u;
  // field masks and per-offset fp16 powers of two, kept in registers so each
  // extraction is a single v_and_or_b32 (as literals the compiler splits it
  // in two); the empty asm only hides the constants from constant folding
  uint32_t kmask[Gm::PMAX + 1], magic[Gm::PMAX + 1];
#pragma unroll
  for (int e = 0; e <= Gm::PMAX; ++e) {
    kmask[e] = (Gm::MASK << (BITS * e)) | (Gm::MASK << (16 + BITS * e));
    const uint32_t m16 = uint32_t(25 - BITS * e) << 10;  // fp16 2^(10 - BITS*e)
    magic[e] = m16 | (m16 << 16);
    asm("" : "+v"(kmask[e]));
    asm("" : "+v"(magic[e]));
  }
#pragma unroll 1
  for (int kb = 0; kb < 4; ++kb) {
    const uint4 *kp = reinterpret_cast<const uint4 *>(&sh.kw[kb][kap][r][0]);
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
      h8 a;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t src = direct ? y[u] : (y[u] >> Gm::SH);
        const h2 x = as_h2(and_or(src, kmask[pe], magic[pe])) - as_h2(magic[pe]);
        const h2 k = __builtin_elementwise_fma(x, sp[u], mp[u]);
        a[2 * u] = k[0];
        a[2 * u + 1] = k[1];
      }
      acc[pq] = mfma32(a, qfrag, acc[pq]);
    }
  }
  softmax_tile<NP>(acc, valid, full, scale_log2, st);

  // ---- values of these positions, two at a time: O^T += V^T P^T on
  // v_mfma_f32_16x16x32_f16 with k = (word rows 4k..4k+3) x (positions pa, pb).
  // Row r of MFMA (b, i) is channel 32b + 2r + i: both channels of the lane
  // sit in byte vbyte of word vword(b) of every token (2-bit: a byte holds 4
  // channels, the lane takes two neighbours; 4-bit: a byte holds 2)
  const int vbyte = BITS == 2 ? (r >> 1) & 3 : r & 3;
  const int vword = BITS == 2 ? r >> 3 : r >> 2;  // word of the block
  constexpr int WPB = 32 / Gm::TPW;               // value words per 32-channel block
  const uint32_t vsel = uint32_t(vbyte) | (0x0cu << 8) | ((4u + vbyte) << 16) | (0x0cu << 24);  // [lo.b, 0, hi.b, 0]
  const int o0 = value_shift<BITS>(2 * r);
  uint32_t vmask[2] = {(Gm::MASK << o0) | (Gm::MASK << (16 + o0)), (Gm::MASK << (o0 + BITS)) | (Gm::MASK << (16 + o0 + BITS))};
#pragma unroll
  for (int j = 0; j < NP / 2; ++j) {
    const int pa = half * NP + 2 * j, pb = pa + 1;
    const h4 pa4 = cvt4(acc[2 * j]), pb4 = cvt4(acc[2 * j + 1]);
    const h8 p8 = h8{pa4[0], pa4[1], pa4[2], pa4[3], pb4[0], pb4[1], pb4[2], pb4[3]};
    h8 ps[Sh::NGD];  // P * value scale, per value group
#pragma unroll
    for (int g = 0; g < Sh::NGD; ++g) {
      const h8 s8 = *reinterpret_cast<const h8 *>(&sh.vs[g][pa / 2][kap][0][0]);
      const h8 m8 = *reinterpret_cast<const h8 *>(&sh.vm[g][pa / 2][kap][0][0]);
      ps[g] = p8 * s8;
      // every row of A = the value minima: each output row gets sum_t P*min
      st.cmin[g] = mfma32(m8, p8, st.cmin[g]);
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int wi = WPB * b + vword;
      const uint4 wa = *reinterpret_cast<const uint4 *>(&sh.vw[pa][wi][4 * kap]);
      const uint4 wb = *reinterpret_cast<const uint4 *>(&sh.vw[pb][wi][4 * kap]);
      const uint32_t y[4] = {__builtin_amdgcn_perm(wa.y, wa.x, vsel), __builtin_amdgcn_perm(wa.w, wa.z, vsel),
                             __builtin_amdgcn_perm(wb.y, wb.x, vsel), __builtin_amdgcn_perm(wb.w, wb.z, vsel)};
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint4 x = make_uint4(y[0] & vmask[i], y[1] & vmask[i], y[2] & vmask[i], y[3] & vmask[i]);
        st.o[2 * b + i] = mfma32(__builtin_bit_cast(h8, x), ps[(32 * b) / G], st.o[2 * b + i]);
      }
    }
  }
}

template <int BITS, int G>
__device__ __forceinline__ void packed_split(DecShared<BITS, G> &sh, const _Float16 (*sq)[kQPad],
                                             const uc_kivi_item &it, int64_t h, int64_t split,
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
  // super-tiles split, split + S, split + 2S, ... (S = packed splits): the S
  // splits of a unit run side by side on one XCD and read neighbouring parts
  // of the same 128-byte key-code and key-stat lines at about the same time
  const int64_t n_super = (Tq + Sh::T - 1) / Sh::T;
  const int64_t stride = p.splits_packed * Sh::T;
  const int n_it = static_cast<int>(min<int64_t>(p.nst, (n_super - split + p.splits_packed - 1) / p.splits_packed));
  Prefetch<BITS, G> pf;
  issue_loads<BITS, G>(pf, rg, static_cast<uint32_t>(split * Sh::T));
  for (int i = 0; i < n_it; ++i) {
    const uint32_t t0 = static_cast<uint32_t>((split + int64_t(i) * p.splits_packed) * Sh::T);
    __syncthreads();  // every wave is done reading the previous iteration from LDS
    stage_lds<BITS, G>(sh, pf, t0, rg.nkg);
    __syncthreads();
    if (i + 1 < n_it) issue_loads<BITS, G>(pf, rg, static_cast<uint32_t>(t0 + stride));  // lands during this iteration
    compute_tile<BITS, G>(sh, sq, t0, rg.nkw, p.scale_log2, st);
  }
  // undo the denormal code scaling 2^(e - 24) of each output channel (e
  // depends on the channel mod 4 / mod 2, i.e. on cb and v) and add the
  // value minima
#pragma unroll
  for (int cb = 0; cb < 8; ++cb)
#pragma unroll
    for (int v = 0; v < 4; ++v)
      st.o[cb][v] = st.o[cb][v] * (16777216.0f / float(1 << value_shift<BITS>(out_channel(cb, 0, v)))) +
                    st.cmin[(32 * (cb >> 1)) / G][v];
  (void)lane;
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
__device__ __forceinline__ void residual_split(const _Float16 (*sq)[kQPad], const uc_kivi_item &it, int64_t h,
                                               int64_t tr0, const MfmaParams &p, WaveState &st) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const int64_t Tr = it.residual_tokens;
  const int64_t bytes = Tr * p.Hkv * kD * 2;
  const Rsrc rk = make_rsrc(it.residual_key, bytes), rv = make_rsrc(it.residual_value, bytes);
  const int64_t tw = tr0 + wave * kResWaveTokens;
  constexpr int kBlocks = kResWaveTokens / 16;
  const h8 csel[2] = {channel_selector(lane, 0), channel_selector(lane, 1)};
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
      const float x = ok ? acc[b][v] : kNegInf;
      acc[b][v] = x;
      mx = fmaxf(mx, x);
    }
  const float m = max_over_slices(mx) * p.scale_log2;
  const float m_ref = m == kNegInf ? 0.0f : m;
  float sum = 0.0f;
#pragma unroll
  for (int b = 0; b < kBlocks; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float e = fast_exp2(__builtin_fmaf(acc[b][v], p.scale_log2, -m_ref));
      acc[b][v] = e;
      sum += e;
    }
  st.m = m;
  st.l = sum;
  // O^T += V^T P^T: the 8 channels x 16 tokens a lane loads from a residual
  // row block come out of a selection MFMA as 4 tokens of channel 32b + 2n + i
  // (the A layout of accumulator 2b + i, as in the packed path)
#pragma unroll
  for (int j = 0; j < kBlocks / 2; ++j) {
    const h4 pa4 = cvt4(acc[2 * j]), pb4 = cvt4(acc[2 * j + 1]);
    const h8 p8 = h8{pa4[0], pa4[1], pa4[2], pa4[3], pb4[0], pb4[1], pb4[2], pb4[3]};
    const uint32_t base0 = static_cast<uint32_t>(((tw + 32 * j + r) * p.Hkv + h) * kD * 2);
    const uint32_t base1 = static_cast<uint32_t>(((tw + 32 * j + 16 + r) * p.Hkv + h) * kD * 2);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const h8 v0 = load8_h<RD>(rv, base0 + (32 * b + 8 * kap) * 2);
      const h8 v1 = load8_h<RD>(rv, base1 + (32 * b + 8 * kap) * 2);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const h4 a0 = cvt4(mfma32(v0, csel[i], f4{0, 0, 0, 0})), a1 = cvt4(mfma32(v1, csel[i], f4{0, 0, 0, 0}));
        st.o[2 * b + i] = mfma32(h8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]}, p8, st.o[2 * b + i]);
      }
    }
  }
}

// ------------------------------------------------------------------ kernel --
static_assert(kThreads == kD, "key-stat staging maps one thread per channel");

template <int BITS, int G, int RD, bool TABLE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void decode_mfma_kernel(
    const uc_kivi_item *items, uc_kivi_item single, MfmaParams p) {
  __shared__ __align__(16) DecShared<BITS, G> sh;
  __shared__ _Float16 sq[16][kQPad];
  __shared__ float mrg_ml[kWaves][16][2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Workgroup i runs on XCD i % 8; with enough units its k = i / 8-th
  // workgroup there is split k % S of unit (item, KV head) u = 8 (k / S) + i % 8,
  // so the S splits of a unit are dispatched back to back on one XCD and share
  // its L2.  A launch of few units spreads each unit's splits over the XCDs.
  int64_t u, split;
  if (p.xcd_grouped) {
    const int64_t x = blockIdx.x % kXcds, k = blockIdx.x / kXcds;
    u = (k / p.splits_total) * kXcds + x;
    split = k % p.splits_total;
  } else {
    u = blockIdx.x / p.splits_total;
    split = blockIdx.x % p.splits_total;
  }
  if (u >= p.units) return;  // uniform: the whole workgroup leaves
  const int64_t item = TABLE ? u / p.Hkv : 0;
  const uc_kivi_item it = TABLE ? items[item] : single;
  const int64_t h = u % p.Hkv;
  if (!split_has_work(split, it.quantized_tokens, it.residual_tokens, p)) {  // uniform
    // only the statistics: (-inf, 0) gives the split weight 0 in the combine,
    // which then never reads its (unwritten) partial output
    if (tid < 16) {
      const int64_t slot = (item * p.Hkv + h) * p.splits_total + split;
      reinterpret_cast<float2 *>(p.ws_ml)[slot * 16 + tid] = make_float2(kNegInf, 0.0f);
    }
    return;
  }

  stage_queries(sq, it.query, h, p);
  WaveState st;
#pragma unroll
  for (int b = 0; b < 8; ++b) st.o[b] = f4{0, 0, 0, 0};
#pragma unroll
  for (int g = 0; g < 4; ++g) st.cmin[g] = f4{0, 0, 0, 0};
  st.m = kNegInf;
  st.l = 0.0f;
  __syncthreads();

  // residual splits first, so their short runs are spread over the launch
  // instead of forming its tail
  const int64_t splits_res = p.splits_total - p.splits_packed;
  if (split >= splits_res) {
    const int64_t sp = split - splits_res;
    if (sp * DecShared<BITS, G>::T < it.quantized_tokens) packed_split<BITS, G>(sh, sq, it, h, sp, p, st);
  } else {
    const int64_t tr0 = split * kWaves * kResWaveTokens;
    if (tr0 < it.residual_tokens) residual_split<RD>(sq, it, h, tr0, p, st);
  }

  // ---- merge the two waves; lane (n, k) holds query n, channels out_channel(cb, k, v)
  const int kap = lane >> 4, n = lane & 15;
  const float l_all = sum_over_slices(st.l);
  __syncthreads();
  if (kap == 0) {
    mrg_ml[wave][n][0] = st.m;
    mrg_ml[wave][n][1] = l_all;
  }
  __syncthreads();
  float M = kNegInf;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mrg_ml[w][n][0]);
  const float M_ref = M == kNegInf ? 0.0f : M;
  float L = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) L += mrg_ml[w][n][1] * fast_exp2(mrg_ml[w][n][0] - M_ref);
  const float mine = fast_exp2(st.m - M_ref);
  float *fin = reinterpret_cast<float *>(sh.vw);  // [16][128] partial of wave 1
  static_assert(sizeof(sh.vw) >= 16 * kD * sizeof(float), "wave merge fits the value-word staging");
  if (wave == 1) {
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
#pragma unroll
      for (int v = 0; v < 4; ++v) fin[n * kD + out_channel(cb, kap, v)] = st.o[cb][v] * mine;
  }
  __syncthreads();
  const int64_t slot = (item * p.Hkv + h) * p.splits_total + split;
  if (wave == 0) {
    _Float16 *po = p.ws_o + slot * 16 * kD;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {  // channels 32b + 8kap + [0, 8): accumulators 2b (even), 2b + 1 (odd)
      h8 o8;
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          o8[2 * v + i] = to_h((st.o[2 * b + i][v] * mine + fin[n * kD + out_channel(2 * b + i, kap, v)]) * inv);
      *reinterpret_cast<h8 *>(&po[n * kD + 32 * b + 8 * kap]) = o8;
    }
    if (kap == 0) {
      p.ws_ml[(slot * 16 + n) * 2 + 0] = M;
      p.ws_ml[(slot * 16 + n) * 2 + 1] = L;
    }
  }
}

// Merge the split partials of one (query, KV head) -- every split of the
// p.segs items that share the query -- for a quarter of the channels
// (blockIdx.z).  Thread (row = tid / 8, j = tid % 8) folds the (max, sum) of
// slots j, j + 8, ... into an online (M, L), the 8 threads of a row combine
// theirs with lane shuffles, and each then accumulates its 4 channels over all
// slots with weights l_s 2^(m_s - M) / L, eight slots' loads in flight.  No
// LDS and no barrier: the launch is a short chain of independent loads.  The
// output goes to the first item of the group.
constexpr int kCombineThreads = 128;
constexpr int kCombineParts = 4;  // channel quarters per (query, KV head)
constexpr int kCombineLanes = 8;  // threads per query row

__device__ __forceinline__ void ml_fold(float &M, float &L, float m, float l) {
  if (!(l > 0.0f) || m == kNegInf) return;
  if (m > M) {
    L = (L > 0.0f ? L * exp2f(M - m) : 0.0f) + l;
    M = m;
  } else {
    L += l * exp2f(m - M);
  }
}

template <bool TABLE>
__global__ __launch_bounds__(kCombineThreads) void decode_mfma_combine(const uc_kivi_item *items, uc_kivi_item single,
                                                                       MfmaParams p) {
  const int64_t first = TABLE ? blockIdx.y * p.segs : 0;
  const uc_kivi_item it = TABLE ? items[first] : single;
  const int64_t h = blockIdx.x;
  const int part = blockIdx.z;
  const int tid = threadIdx.x, row = tid / kCombineLanes, j = tid % kCombineLanes;
  const int nflat = int(p.segs * p.splits_total);
  static_assert(16 * kCombineLanes == kCombineThreads && kD / kCombineParts == 4 * kCombineLanes,
                "thread = (row, 4 channels of the part)");
  // flattened (segment, split) index -> workspace slot
  auto slot = [&](int f) {
    return ((first + f / p.splits_total) * p.Hkv + h) * p.splits_total + f % p.splits_total;
  };
  // splits without work wrote (-inf, 0) and no output
  auto ml_at = [&](int f) { return *reinterpret_cast<const float2 *>(p.ws_ml + (slot(f) * 16 + row) * 2); };
  // pass 1: this thread's slots, four loads in flight, then the row's 8 threads
  float M = kNegInf, L = 0.0f;
  for (int f0 = j; f0 < nflat; f0 += 4 * kCombineLanes) {
    float2 ml[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int f = f0 + u * kCombineLanes;
      ml[u] = f < nflat ? ml_at(f) : make_float2(kNegInf, 0.0f);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) ml_fold(M, L, ml[u].x, ml[u].y);
  }
#pragma unroll
  for (int o = 1; o < kCombineLanes; o <<= 1) {
    const float m2 = __shfl_xor(M, o, kWave), l2 = __shfl_xor(L, o, kWave);
    ml_fold(M, L, m2, l2);
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  const bool active = row < p.rows;
  if (active && part == 0 && j == 0 && it.lse != nullptr) {
    const int64_t g = row / p.Lq, i = row % p.Lq;
    it.lse[(h * p.group + g) * p.Lq + i] = L > 0.0f ? (M + log2f(L)) * kLn2 : kNegInf;
  }
  // pass 2: 4 channels of this part over every slot
  const int c4 = (part * kCombineLanes + j) * 4;
  float o[4] = {0, 0, 0, 0};
  if (active) {
    for (int f0 = 0; f0 < nflat; f0 += 8) {
      h4 v[8];
      float w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int f = f0 + u < nflat ? f0 + u : f0;
        const float2 ml = ml_at(f);
        w[u] = (f0 + u < nflat && ml.y > 0.0f && ml.x != kNegInf) ? ml.y * exp2f(ml.x - M) * inv : 0.0f;
        v[u] = *reinterpret_cast<const h4 *>(p.ws_o + (slot(f) * 16 + row) * kD + c4);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = w[u] != 0.0f ? fmaf(float(v[u][c]), w[u], o[c]) : o[c];
    }
    const int64_t g = row / p.Lq, i = row % p.Lq;
#pragma unroll
    for (int c = 0; c < 4; ++c) store_dyn(it.out, (i * p.Hq + h * p.group + g) * kD + c4 + c, o[c], p.od);
  }
}

}  // namespace

// Packed tokens per split of the MFMA decode for `bits` (super-tiles per
// split x tokens per super-tile).
int64_t decode_mfma_split_tokens(int bits, int64_t nst) { return nst * 16 * (32 / bits); }

int64_t decode_mfma_res_split_tokens() { return kWaves * kResWaveTokens; }

// Splits per (item, KV head): packed splits, then residual splits.
int64_t decode_mfma_num_splits(int bits, int64_t nst, int64_t max_tq, int64_t max_tr) {
  return ceil_div(max_tq, decode_mfma_split_tokens(bits, nst)) + ceil_div(max_tr, decode_mfma_res_split_tokens());
}

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
                       int out_dtype, float sm_scale, int64_t max_tq, int64_t max_tr, int64_t nst, int64_t segs,
                       void *workspace, int64_t workspace_bytes, hipStream_t stream) {
  // Twice the super-tiles per split when that fits the launch into one round of
  // workgroup slots (4 per CU) and `nst` does not: a batch-1 32k context then
  // runs as one full round instead of ~1.9 (+3 % measured).  Fewer splits, so
  // the workspace sized for `nst` still fits.
  {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) {
      const int64_t units = n_items * Hkv, round = 4 * int64_t(cus);
      if (units * decode_mfma_num_splits(bits, nst, max_tq, max_tr) > round &&
          units * decode_mfma_num_splits(bits, 2 * nst, max_tq, max_tr) <= round)
        nst *= 2;
    }
  }
  const int64_t s_tok = decode_mfma_split_tokens(bits, nst);
  MfmaParams p{};
  p.Hq = Hq; p.Hkv = Hkv; p.Lq = Lq; p.group = Hq / Hkv; p.rows = p.group * Lq;
  p.splits_packed = ceil_div(max_tq, s_tok);
  p.splits_total = decode_mfma_num_splits(bits, nst, max_tq, max_tr);
  p.nst = nst;
  p.segs = segs;
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
  p.units = n_items * Hkv;
  p.super_tokens = 16 * (32 / bits);
  p.xcd_grouped = p.units >= 4 * kXcds;  // at most one unit of imbalance per XCD in four
  const dim3 grid(static_cast<unsigned>((p.xcd_grouped ? ceil_div(p.units, int64_t(kXcds)) * kXcds : p.units) *
                                        p.splits_total));
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
  UC_REQUIRE(segs >= 1 && n_items % segs == 0, "decode: %lld items do not form groups of %lld segments",
             (long long)n_items, (long long)segs);
  if (table)
    hipLaunchKernelGGL((decode_mfma_combine<true>), dim3(Hkv, n_items / segs, kCombineParts), dim3(kCombineThreads),
                       0, stream, items_dev, one, p);
  else
    hipLaunchKernelGGL((decode_mfma_combine<false>), dim3(Hkv, n_items, kCombineParts), dim3(kCombineThreads), 0,
                       stream, items_dev, one, p);
  return check_launch("decode (MFMA combine)");
}

}  // namespace uc
