// MFMA split-K decode over KIVI-packed KV (head_dim 128, 2/4-bit codes).
//
// Storage is token-major (a super-tile of one KV head is one contiguous run of
// every stream: key words, key stats, value words, value stats).  One
// workgroup (4 waves) owns a packed split of one unit (item, KV head) --
// every S-th super-tile (16 key words per channel: 256 tokens at 2-bit)
// starting at the split index -- or a residual split of 256 dense tokens.
// Wave w loads, stages (in its own LDS area, no workgroup barrier in the loop)
// and computes tokens 64w .. 64w + 63 of each super-tile; the next
// super-tile's loads are issued before the current one is computed.  The
// <= 16 query rows of a KV head (query heads x query length) form the N = 16
// columns of every MFMA, so each packed byte is read once per unit.
//
// Keys (S^T = K Q^T on v_mfma_f32_16x16x32_f16).  MFMA rows are the 16 tokens
// of a tile, which lie in one quantization group, so
//     logit = sum_c (q_c s_c) code_c + sum_c q_c m_c :
// the key scale is folded into the B operand once per group (B' = q * s), and
// the minimum term is one MFMA set per wave whose A rows hold the minima of
// the wave's groups.  Staging spreads the words of two channels byte by byte:
// one dword holds byte k of both words in its two 16-bit halves, so each A
// register is one AND (fused with the DPP quad exchange) that leaves
// code << BITS*e in each half: an fp16 value code * 2^(BITS*e - 24), which the
// MFMA multiplies exactly.  The row's power of two, the softmax scale and the
// minimum term are applied in one FMA per logit.
//
// Values (O^T += V^T P^T).  MFMA rows are 16 channels, K = 32 tokens (two
// tiles), staged the same way by token pairs; the power of two of each output
// channel is undone once at the end.  The value scale rides in the B operand
// (P * scale, per channel group); one MFMA per K block adds the minima and, in
// a row of ones, the softmax denominator sum_t P.
//
// Column-folded form (2-bit, G = 32, at most 8 query rows): MFMA columns 0-7
// serve the wave's first 32-token group and columns 8-15 its second, so the
// B' products, logit FMAs and exponentials are halved; the two halves merge
// by a lane exchange at the end of the split.
//
// Each split writes a normalised fp16 partial of its query rows with its
// (max, sum); decode_mfma_combine merges the splits by log-sum-exp.
#include "uc_common.h"
#include "uc_decode.h"
#include "uc_mfma.h"


namespace uc {
namespace {

using namespace mf;

constexpr int kXcds = 8;  // XCDs of an MI355X; workgroup i of a launch runs on XCD i % 8
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
// Residual tokens per wave of a residual split: 32 (2 tiles) when every
// item's residual fits one split that way (the usual R = 128 window: all four
// waves busy), else 64 (4 tiles; long dense segments then need half the splits).
constexpr int kResWaveTokensShort = 32, kResWaveTokensLong = 64;
inline int64_t res_wave_tokens(int64_t max_tr) {
  return max_tr <= kWaves * kResWaveTokensShort ? kResWaveTokensShort : kResWaveTokensLong;
}
constexpr int kWgPerCu = 3;         // resident workgroups per CU (LDS: ~51 KB each; <= 168 VGPRs)
constexpr float kLazyLog2 = 8.0f;   // softmax reference slack (log2 units)

// Tile geometry of `BITS`-bit codes with groups of G tokens / channels.
template <int BITS, int G>
struct Tiles {
  static constexpr int TPW = 32 / BITS;       // codes per word
  static constexpr int CPB = 8 / BITS;        // codes per byte = lanes that share one staged dword
  static constexpr int NPL = 4 / CPB;         // dwords of a 4-dword A fragment one lane reads
  static constexpr int ST = 16 * TPW;         // tokens per super-tile (16 key words)
  static constexpr int NT = ST / 16;          // 16-token tiles per super-tile
  static constexpr int TW = NT / kWaves;      // tiles per wave
  static constexpr int KG = ST / G;           // key groups per super-tile
  static constexpr int GW = (16 * TW) / G > 0 ? (16 * TW) / G : 1;  // key groups per wave
  static constexpr int NGD = kD / G;          // value groups per token
  static constexpr int VWPT = kD / TPW;       // value words per token
  static constexpr int HW = 16 / TPW;         // value words per 16-channel block
  static constexpr int NTP = ST / 2;          // token pairs per super-tile
  static constexpr uint32_t MASK = (1u << BITS) - 1u;
  // Staged words are "byte spread": dword (byte k of word a, byte k of word
  // b) at bits 0-7 and 16-23, so a code sits at most 6 bits up its 16-bit
  // half and the AND leaves an fp16 denormal (or small normal) that is
  // exactly code * 2^(BITS e - 24).
  //
  // Each wave stages and reads only its own WT tokens, so the waves of a
  // workgroup never wait for each other inside the loop.
  //
  // Key words: row (word j, byte k) of 64 dwords, dword 4q + kb = channel
  // pair 16 kb + q.  Lane (row r, slice kap) of a tile needs the four pairs
  // 16 kb + 4 kap + (0..3) of its row's (j, k) for every kb; the CPB lanes
  // that share (j, k) each read NPL 16-byte pieces (all kb of NPL pairs) and
  // exchange them with DPP.  Rows of odd k are rotated by 32 dwords, which
  // keeps the four k rows one tile reads on different banks.
  static constexpr int WT = 16 * TW;          // tokens per wave per super-tile
  static constexpr int JW = WT / TPW;         // key word rows per wave
  // Value words: row (byte k, word-in-block h) of WT/32 blocks x 128 dwords;
  // in a block (32 tokens = 16 token pairs), dword 64 (blk / 4) + 4 slot +
  // blk % 4 holds 16-channel block blk of token pair slot.  Slot 4 kap + jj
  // holds the pair whose tokens lane slice kap needs in place jj of its
  // fragment (pairs 2 kap, 2 kap + 1 of the first tile, then of the second),
  // so a lane's NPL pairs are contiguous; odd k rotated as for the keys.
  static constexpr int VRKW = (WT / 32) * 128;
  // value-stat rows [group][token] padded so the cmin MFMA's minima rows
  // (one per group) sit on different banks
  static constexpr int VSP = WT + (BITS == 2 ? 32 : 16);
  static_assert(TW >= 2 && TW % 2 == 0, "a wave owns whole 32-token value blocks");
  static_assert(KG >= 1 && G % 16 == 0, "a tile lies in one group");
  static_assert(GW == 1 || GW == 2, "the bias MFMA holds one or two groups per wave");
  static_assert(WT <= 64, "the cmin ones row covers a wave's tokens");
};

// v_perm selector: byte k of src1 at byte 0, byte k of src0 at byte 2, zeros elsewhere.
__device__ __forceinline__ constexpr uint32_t byte_spread_sel(int k) {
  return uint32_t(k) | (0x0cu << 8) | (uint32_t(4 + k) << 16) | (0x0cu << 24);
}

// Dword offset of a 4-dword piece at `off` (a multiple of 4) in row k.
__device__ __forceinline__ uint32_t rot_row(uint32_t off, int k) { return (off + 32u * (k & 1)) & 63u; }

// Slot of token pair p (0..15) of a 32-token block: pairs 2 kap, 2 kap + 1,
// 2 kap + 8, 2 kap + 9 go to slots 4 kap .. 4 kap + 3.
__device__ __forceinline__ uint32_t pair_slot(uint32_t p) { return 4 * ((p % 8) / 2) + p % 2 + 2 * (p / 8); }

// One wave's staging area for one super-tile.
template <int BITS, int G>
struct WaveStage {
  using Tl = Tiles<BITS, G>;
  uint32_t kw[Tl::JW * 4 * 64];
  uint32_t vw[4 * Tl::HW * Tl::VRKW];
  // rows padded by 16 dwords: the two key-minimum rows of the bias MFMA sit
  // on different banks
  _Float16 ks[Tl::GW][kD + 32], km[Tl::GW][kD + 32];    // key stats [group][channel]
  _Float16 vs[Tl::NGD][Tl::VSP], vm[Tl::NGD][Tl::VSP];  // value stats [group][token]
};

template <int BITS, int G>
struct DecShared {
  union {
    WaveStage<BITS, G> st[kWaves];
    struct {
      // rows padded by 4 dwords so the 16 query rows of one store hit distinct banks
      float o[kWaves - 1][16][kD + 4];  // waves 1.. : scaled partial outputs [query row][channel]
      float ml[kWaves][16][2];          // every wave's (max, sum) per query row
    } mrg;
  };
};

// Items passed by value in the kernel arguments (calls that name at most
// kArgItems items from host memory); the kernels index them like a table.
constexpr int kArgItems = 8;
struct ArgItems {
  uc_kivi_item v[kArgItems];
};

struct MfmaParams {
  int64_t Hq, Hkv, Lq, group, rows;
  int64_t splits_packed, splits_total, nst;  // nst: super-tiles per packed split
  int64_t segs;                              // consecutive items that share one query and output
  int64_t res_wave;                          // residual tokens per wave of a residual split (32 or 64)
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
  return split >= splits_res ? (split - splits_res) * p.super_tokens < tq : split * kWaves * p.res_wave < tr;
}

// Online-softmax state of one wave.  The output is accumulated transposed
// (O^T = V^T P^T): lane (n, k) owns query column n and output channels
// 16 b + 4 k + v of accumulator b, so every rescale is lane-local.
struct WaveState {
  f4 o[8];
  f4 cmin;  // packed splits: row g < groups: sum_t P * value minimum of group g; row NGD: sum_t P
  float m;  // running max of query n (log2 units), equal across the k-slices
  float l;  // residual splits: this lane's share of the running sum (reduced over the k-slices at the end)
};

// Fold NP tiles of base-2 logits (acc[i][v]: token 16 i + 4 k + v of the
// wave's tiles, column = query) into the running state; acc returns holding
// the probabilities and the output is rescaled.  `valid_rows` tokens of the
// wave's tiles are real (the rest of the last super-tile reads past the end).
// SUM: keep the running sum in st.l (the packed path sums P by MFMA instead).
// tile_base: the wave-tile index of acc[0] (the column-folded path gives each
// half of the columns its own tiles).
template <int NP, bool SUM>
__device__ __forceinline__ void softmax_tiles(f4 (&acc)[NP], int valid_rows, WaveState &st, int kap,
                                              int tile_base = 0) {
  if (valid_rows < 16 * (NP + tile_base)) {
#pragma unroll
    for (int i = 0; i < NP; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (16 * (tile_base + i) + 4 * kap + v >= valid_rows) acc[i][v] = kNegInf;
  }
  float mx = kNegInf;
#pragma unroll
  for (int i = 0; i < NP; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) mx = fmaxf(mx, acc[i][v]);
  mx = max_over_slices(mx);
  // The reference m is raised only when a logit exceeds it by more than
  // kLazyLog2 (-inf + kLazyLog2 = -inf: the first finite tile raises it), so
  // the output is rarely rescaled and probabilities stay <= 2^kLazyLog2, well
  // inside fp16.  (m, l) stay a consistent pair: l = sum 2^(x - m).
  const bool raise = mx > st.m + kLazyLog2;
  const float m_new = raise ? mx : st.m;
  const float m_ref = m_new == kNegInf ? 0.0f : m_new;  // keeps -inf - m_ref at -inf (exp 0), never NaN
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < NP; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float e = fast_exp2(acc[i][v] - m_ref);
      acc[i][v] = e;
      if constexpr (SUM) sum += e;
    }
  const float alpha = raise ? fast_exp2(st.m - m_ref) : 1.0f;
  if constexpr (SUM) st.l = st.l * alpha + sum;
  st.m = m_new;
  if (__any(raise)) {
#pragma unroll
    for (int b = 0; b < 8; ++b) st.o[b] *= alpha;
    st.cmin *= alpha;
  }
}

// ------------------------------------------------------------ packed path --
// Query rows of the KV head staged once per workgroup as fp16 [row][channel]
// (rows padded to 72 dwords: the 16 rows of one fragment read hit distinct
// banks); lane (n, k-slice) reads its B fragment of block kb from here.
constexpr int kQPad = kD + 16;
constexpr int kOnesLen = 64;  // >= the tokens a wave computes per super-tile (WT)

template <int QD>
__device__ __forceinline__ void stage_queries_t(_Float16 (*sq)[kQPad], const void *query, int64_t h,
                                                const MfmaParams &p, bool fold) {
  // 16 rows x 128 channels; thread t < 128 converts 16 consecutive channels of
  // row t/8 (rows 8-15 repeat rows 0-7 for the column-folded packed path)
  if (threadIdx.x >= 128) return;
  const int n = threadIdx.x / 8, d0 = (threadIdx.x % 8) * 16;
  const int src = fold ? (n & 7) : n;
  uint4 raw[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
  if (src < p.rows) {
    const int lq = static_cast<int>(p.Lq), g32 = src / lq;
    const int64_t g = g32, i = src - g32 * lq;
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
                                              const MfmaParams &p, bool fold) {
  if (p.qd == UC_BF16) {
    stage_queries_t<UC_BF16>(sq, query, h, p, fold);
  } else if (p.qd == UC_FP16) {
    stage_queries_t<UC_FP16>(sq, query, h, p, fold);
  } else {
    for (int idx = threadIdx.x; idx < 16 * kD; idx += kThreads) {
      const int n = idx / kD, d = idx % kD, src = fold ? (n & 7) : n;
      float v = 0.0f;
      if (src < p.rows) {
        const int64_t g = src / p.Lq, i = src % p.Lq;
        v = static_cast<const float *>(query)[(i * p.Hq + h * p.group + g) * kD + d];
      }
      sq[n][d] = to_h(v);
    }
  }
}

__device__ __forceinline__ h8 query_frag(const _Float16 (*sq)[kQPad], int kb, int lane) {
  return *reinterpret_cast<const h8 *>(&sq[lane & 15][32 * kb + 8 * (lane >> 4)]);
}

// Everything one super-tile reads from HBM, held in registers so the next
// super-tile's loads overlap this one's MFMAs.  The packed tensors are
// token-major, so every stream of a super-tile is one contiguous run of the
// head's rows.  Thread t loads:
//   key words: channel pairs 16 kb + q (q = t % 16, kb = 0..3) of word t / 16;
//   value words: word quad t % NQ of tokens 2tp, 2tp+1 (tp = t / NQ);
//   key stats: 8 channels (t % 16) of group (t % 128) / 16, scales (t < 128)
//     or minima;
//   value stats: 16 bytes of the scales (t < 128) or minima.
template <int BITS, int G>
struct Prefetch {
  uint2 kw[4];
  uint4 vw[2];
  uint4 ks, vs;
};

struct PackedRegion {
  Rsrc kcode, kscale, kmin, vcode, vscale, vmin;
};

// Issue this wave's loads of the super-tile starting at token t0 (a
// multiple of ST): tokens t0 + WT wave ...  Rows past the packed tokens fall
// outside the buffer resources and read as 0.  Lane l loads
//   key words: channel pairs 16 kb + (l % 16), kb = 0..3, of word row l / 16;
//   value words: word quad l % NQ of token pair l / NQ;
//   key stats: 16 bytes of the wave's group rows, scales then minima;
//   value stats: 16 bytes of the wave's tokens, scales then minima.
template <int BITS, int G>
__device__ __forceinline__ void issue_loads(Prefetch<BITS, G> &pf, const PackedRegion &rg, uint32_t t0, int wave) {
  using Tl = Tiles<BITS, G>;
  const int lane = threadIdx.x & 63;
  const uint32_t tw = t0 + Tl::WT * wave;
  {  // key words [word][D]: JW rows of 512 bytes
    const uint32_t base = ((tw / Tl::TPW + (lane >> 4)) * kD + 2 * (lane & 15)) * 4u;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) pf.kw[kb] = bload64(rg.kcode, base + 128u * kb);
  }
  {  // value words of two neighbouring tokens
    constexpr uint32_t NQ = Tl::VWPT / 4;
    const uint32_t tp = lane / NQ, wq = lane % NQ;
    const uint32_t tok = tw + 2 * tp;
    pf.vw[0] = bload128(rg.vcode, (tok * Tl::VWPT + 4 * wq) * 4u);
    pf.vw[1] = bload128(rg.vcode, ((tok + 1) * Tl::VWPT + 4 * wq) * 4u);
  }
  // Statistics: lanes of stat 0 load scales, of stat 1 minima.  The compiler
  // merges the two branches into one load whose resource is chosen per lane,
  // i.e. a loop over its two values (readfirstlane, compare, masked load).
  // That form is the fastest measured: two loads masked to their halves and
  // OR-ed ran 5-7 % slower on the decode lines, and two full-wave loads with
  // an out-of-range offset for the other half 3-7 % slower.
  {  // key stats [group][D]: GW rows of 256 bytes per stat
    constexpr int NKS = Tl::GW * 16;  // 16-byte chunks per stat
    const int i = lane % NKS, stat = lane / NKS;
    const uint32_t off = (tw / G) * kD * 2u + 16u * i;
    pf.ks = make_uint4(0, 0, 0, 0);
    if (stat == 0) pf.ks = bload128(rg.kscale, off);
    else if (stat == 1) pf.ks = bload128(rg.kmin, off);
  }
  {  // value stats [Tq][NGD]
    constexpr int NVC = Tl::WT * Tl::NGD / 8;  // 16-byte chunks per stat
    const int i = lane % NVC, stat = lane / NVC;
    const uint32_t off = (tw * Tl::NGD + 8 * i) * 2u;
    pf.vs = make_uint4(0, 0, 0, 0);
    if (stat == 0) pf.vs = bload128(rg.vscale, off);
    else if (stat == 1) pf.vs = bload128(rg.vmin, off);
  }
}

// Move this wave's landed prefetch into its byte-spread / transposed LDS
// layouts.
template <int BITS, int G>
__device__ __forceinline__ void stage_lds(WaveStage<BITS, G> &ws, const Prefetch<BITS, G> &pf) {
  using Tl = Tiles<BITS, G>;
  const int lane = threadIdx.x & 63;
  constexpr uint32_t kLo = 0x05040100u, kHi = 0x07060302u;  // low / high halves of (a, b)
  {  // pairs 16 kb + q of word row j: dwords 4q .. 4q + 3 of row (j, k)
    const uint32_t j = lane >> 4, q = lane & 15;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint4 d;
      d.x = __builtin_amdgcn_perm(pf.kw[0].y, pf.kw[0].x, byte_spread_sel(k));
      d.y = __builtin_amdgcn_perm(pf.kw[1].y, pf.kw[1].x, byte_spread_sel(k));
      d.z = __builtin_amdgcn_perm(pf.kw[2].y, pf.kw[2].x, byte_spread_sel(k));
      d.w = __builtin_amdgcn_perm(pf.kw[3].y, pf.kw[3].x, byte_spread_sel(k));
      *reinterpret_cast<uint4 *>(&ws.kw[(4 * j + k) * 64 + rot_row(4 * q, k)]) = d;
    }
  }
  {  // words 4 wq + i of token pair tp: block tp / 16, slot of pair tp % 16
    constexpr uint32_t NQ = Tl::VWPT / 4;
    const uint32_t tp = lane / NQ, wq = lane % NQ;
    const uint32_t a[4] = {pf.vw[0].x, pf.vw[0].y, pf.vw[0].z, pf.vw[0].w};
    const uint32_t b[4] = {pf.vw[1].x, pf.vw[1].y, pf.vw[1].z, pf.vw[1].w};
    const uint32_t in_block = (tp / 16) * 128, slot4 = 4 * pair_slot(tp % 16);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (Tl::HW == 1) {  // 2-bit: word = block blk = 4 wq + i
        const uint4 d = make_uint4(__builtin_amdgcn_perm(b[0], a[0], byte_spread_sel(k)),
                                   __builtin_amdgcn_perm(b[1], a[1], byte_spread_sel(k)),
                                   __builtin_amdgcn_perm(b[2], a[2], byte_spread_sel(k)),
                                   __builtin_amdgcn_perm(b[3], a[3], byte_spread_sel(k)));
        *reinterpret_cast<uint4 *>(&ws.vw[k * Tl::VRKW + in_block + wq * 64 + rot_row(slot4, k)]) = d;
      } else {  // 4-bit: word 4 wq + i = block 2 wq + i / 2, half i % 2
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const uint2 d = make_uint2(__builtin_amdgcn_perm(b[hh], a[hh], byte_spread_sel(k)),
                                     __builtin_amdgcn_perm(b[2 + hh], a[2 + hh], byte_spread_sel(k)));
          *reinterpret_cast<uint2 *>(&ws.vw[(2 * k + hh) * Tl::VRKW + in_block + (wq / 2) * 64 +
                                            rot_row(slot4, k) + 2 * (wq % 2)]) = d;
        }
      }
    }
  }
  {  // key stats arrive as [group][channel] rows already
    constexpr int NKS = Tl::GW * 16;
    const int i = lane % NKS, stat = lane / NKS;
    if (stat < 2) {
      _Float16(*dst)[kD + 32] = stat == 0 ? ws.ks : ws.km;
      *reinterpret_cast<uint4 *>(&dst[i / 16][8 * (i % 16)]) = pf.ks;
    }
  }
  {
    constexpr int NVC = Tl::WT * Tl::NGD / 8;
    const int i = lane % NVC, stat = lane / NVC;
    if (stat < 2) {
      _Float16(*dst)[Tl::VSP] = stat == 0 ? ws.vs : ws.vm;
      const uint32_t w[4] = {pf.vs.x, pf.vs.y, pf.vs.z, pf.vs.w};
      if constexpr (Tl::NGD == 4) {  // tokens 2i, 2i+1 x groups 0..3
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<uint32_t *>(&dst[g][2 * i]) =
              __builtin_amdgcn_perm(w[2 + g / 2], w[g / 2], (g & 1) ? kHi : kLo);
      } else if constexpr (Tl::NGD == 2) {  // tokens 4i .. 4i+3 x groups 0, 1
#pragma unroll
        for (int g = 0; g < 2; ++g)
          *reinterpret_cast<uint2 *>(&dst[g][4 * i]) =
              make_uint2(__builtin_amdgcn_perm(w[1], w[0], g ? kHi : kLo),
                         __builtin_amdgcn_perm(w[3], w[2], g ? kHi : kLo));
      } else {  // one group: tokens 8i .. 8i+7
        *reinterpret_cast<uint4 *>(&dst[0][8 * i]) = pf.vs;
      }
    }
  }
}

// Order this wave's LDS writes before its later reads (and reads before
// later writes) without waiting for the other waves.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-lane constants of the compute loop.
template <int BITS, int G>
struct LaneConst {
  uint32_t kaddr;   // key read offset (dwords) of the wave's first tile
  uint32_t kmask;   // AND mask that leaves the row's codes of two channels
  float pw[4];      // 2^(24 - BITS e) * softmax scale of logit row 4k + v
  uint32_t vmask;   // AND mask of the lane's value row (channel) within a word half
  uint32_t vaddr;   // value read offset (dwords) of the wave's first block
};

template <int BITS, int G>
__device__ __forceinline__ LaneConst<BITS, G> lane_const(int lane, float scale_log2) {
  using Tl = Tiles<BITS, G>;
  LaneConst<BITS, G> lc;
  const int r = lane & 15, kap = lane >> 4, e = r % Tl::CPB;
  {  // tile i of the wave starts 16 i / TPW word rows after its first tile
    const int j = r / Tl::TPW, k = (r % Tl::TPW) / Tl::CPB;  // row r of the wave's first tile
    lc.kaddr = (4 * j + k) * 64 + rot_row(4 * (4 * kap + Tl::NPL * e), k);
    lc.kmask = (Tl::MASK << (BITS * e)) * 0x10001u;
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int ev = ((4 * kap + v) % Tl::TPW) % Tl::CPB;  // tile row 4k + v: position in word, then in byte
    lc.pw[v] = float(1 << (24 - BITS * ev)) * scale_log2;
  }
  {  // channel 16 blk + r: word-in-block r / TPW, byte (r % TPW) / CPB
    const int k = (r % Tl::TPW) / Tl::CPB, hh = r / Tl::TPW;
    lc.vmask = (Tl::MASK << (BITS * e)) * 0x10001u;
    lc.vaddr = (Tl::HW * k + hh) * Tl::VRKW + rot_row(4 * (4 * kap + Tl::NPL * e), k);
  }
  return lc;
}

// quad_perm control that gives lane (4a + b) dword jj of its CPB-lane group:
// lanes of a group hold NPL consecutive dwords each.
template <int CPB, int JJ>
__device__ __forceinline__ constexpr int group_bcast_ctrl() {
  constexpr int NPL = 4 / CPB;
  int ctrl = 0;
  for (int b = 0; b < 4; ++b) ctrl |= ((b / CPB) * CPB + JJ / NPL) << (2 * b);
  return ctrl;
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_and(uint32_t x, uint32_t m) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xf, 0xf, false)) & m;
}

// A fragment of pair dwords jj = 0..3 from the CPB-lane group: piece[s] holds
// this lane's dwords s (NPL of them) of one kb / block.
template <int CPB>
__device__ __forceinline__ h8 gather_and(const uint32_t (&piece)[4 / CPB], uint32_t m) {
  constexpr int NPL = 4 / CPB;
  uint4 x;
  x.x = dpp_and<group_bcast_ctrl<CPB, 0>()>(piece[0 % NPL], m);
  x.y = dpp_and<group_bcast_ctrl<CPB, 1>()>(piece[1 % NPL], m);
  x.z = dpp_and<group_bcast_ctrl<CPB, 2>()>(piece[2 % NPL], m);
  x.w = dpp_and<group_bcast_ctrl<CPB, 3>()>(piece[3 % NPL], m);
  return __builtin_bit_cast(h8, x);
}

// Logits, softmax and P.V of this wave's tiles of the staged super-tile.
template <int BITS, int G>
__device__ __forceinline__ void compute_tile(const WaveStage<BITS, G> &ws, const h8 (&qf)[4],
                                             const LaneConst<BITS, G> &lc, int valid_rows, float scale_log2,
                                             const _Float16 *ones, WaveState &st) {
  using Tl = Tiles<BITS, G>;
  constexpr int NPL = Tl::NPL, CPB = Tl::CPB;
  const int lane = threadIdx.x & 63, r = lane & 15, kap = lane >> 4;
  constexpr int GT = G / 16;  // tiles per group

  // ---- key minimum term of the wave's groups: A row r = minima of the
  // wave's group r % GW, so element v of every lane holds group v % GW's bias
  f4 mb = f4{0, 0, 0, 0};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
    mb = mfma32(*reinterpret_cast<const h8 *>(&ws.km[r % Tl::GW][32 * kb + 8 * kap]), qf[kb], mb);

  // ---- keys: logits of the wave's TW tiles (16 tokens x 16 query rows each)
  f4 acc[Tl::TW];
  h8 bp[4];
#pragma unroll
  for (int i = 0; i < Tl::TW; ++i) {
    if (i % GT == 0) {  // first tile of a group: B' = q * key scale
      const int g = ((16 * i) / G) % Tl::GW;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        bp[kb] = qf[kb] * *reinterpret_cast<const h8 *>(&ws.ks[g][32 * kb + 8 * kap]);
    }
    // NPL pieces of 4 kb each: pairs 16 kb + 4 kap + NPL e + s
    uint32_t pc[NPL][4];
#pragma unroll
    for (int s = 0; s < NPL; ++s) {
      const uint4 x = *reinterpret_cast<const uint4 *>(&ws.kw[lc.kaddr + (16 * i / Tl::TPW) * 256 + 4 * s]);
      pc[s][0] = x.x; pc[s][1] = x.y; pc[s][2] = x.z; pc[s][3] = x.w;
    }
    f4 a = f4{0, 0, 0, 0};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      uint32_t piece[NPL];
#pragma unroll
      for (int s = 0; s < NPL; ++s) piece[s] = pc[s][kb];
      a = mfma32(gather_and<CPB>(piece, lc.kmask), bp[kb], a);
    }
    const float bias = mb[((16 * i) / G) % Tl::GW] * scale_log2;
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[i][v] = __builtin_fmaf(a[v], lc.pw[v], bias);
  }
  softmax_tiles<Tl::TW, false>(acc, valid_rows, st, kap);

  // ---- values: O^T += V^T P^T over 32-token blocks (tiles 2kc, 2kc + 1):
  // K slot 8k + j is token 4k + j of the first tile (j < 4) or 4k + j - 4 of
  // the second, the layout of the two logit accumulators
#pragma unroll
  for (int kc = 0; kc < Tl::TW / 2; ++kc) {
    const int ta = 2 * kc;  // first tile of the block within the wave's tokens
    const h4 pa4 = cvt4(acc[2 * kc]), pb4 = cvt4(acc[2 * kc + 1]);
    const h8 p8 = h8{pa4[0], pa4[1], pa4[2], pa4[3], pb4[0], pb4[1], pb4[2], pb4[3]};
    {  // A rows g < NGD: the value minima of group g; rows from NGD on read a
       // row of ones, so row NGD accumulates the sum of P (rows past it are unused)
      const _Float16 *mrow = r < Tl::NGD ? &ws.vm[r][0] : ones;
      const h4 ma = *reinterpret_cast<const h4 *>(mrow + 16 * ta + 4 * kap);
      const h4 mb4 = *reinterpret_cast<const h4 *>(mrow + 16 * ta + 16 + 4 * kap);
      st.cmin = mfma32(h8{ma[0], ma[1], ma[2], ma[3], mb4[0], mb4[1], mb4[2], mb4[3]}, p8, st.cmin);
    }
    // this lane's NPL pairs of every 16-channel block: dwords blk of NPL slots
    uint32_t pv[NPL][8];
#pragma unroll
    for (int s = 0; s < NPL; ++s)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint4 x = *reinterpret_cast<const uint4 *>(&ws.vw[lc.vaddr + kc * 128 + half * 64 + 4 * s]);
        pv[s][4 * half + 0] = x.x; pv[s][4 * half + 1] = x.y; pv[s][4 * half + 2] = x.z; pv[s][4 * half + 3] = x.w;
      }
    h8 ps;  // P * value scale of the current group, formed at its first block
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      if ((16 * blk) % G == 0) {
        const int g = (16 * blk) / G;
        const h4 sa = *reinterpret_cast<const h4 *>(&ws.vs[g][16 * ta + 4 * kap]);
        const h4 sb = *reinterpret_cast<const h4 *>(&ws.vs[g][16 * ta + 16 + 4 * kap]);
        ps = p8 * h8{sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
      }
      uint32_t piece[NPL];
#pragma unroll
      for (int s = 0; s < NPL; ++s) piece[s] = pv[s][blk];
      st.o[blk] = mfma32(gather_and<CPB>(piece, lc.vmask), ps, st.o[blk]);
    }
  }
}

// Per-lane constants of the column-folded path.
struct FoldConst {
  int half;               // 0: columns 0-7 (the wave's first 32 tokens), 1: columns 8-15 (the next 32)
  const _Float16 *mrow;   // A row of the cmin MFMA (minima of the row's group and half, or ones)
  int voff[2];            // value-stat read offset of block kc: the block's tokens, or a zeroed pad
};

// Column-folded variant of compute_tile for 2-bit codes in 32-token groups
// with at most 8 query rows (decode at GQA 7:1): MFMA column n < 8 is query
// row n over the wave's first group (tiles 0 and 1), column n + 8 the same
// query row over its second group (tiles 2 and 3).  One B operand carries each
// half's key scale; every lane keeps the logits of its own half's two tiles,
// so its softmax covers 32 tokens, not 64.  The value products of a 32-token
// block get zeros in the other half's columns (those value scales are read
// from a zeroed pad of the stat rows), and one cmin MFMA serves both halves
// (A rows 0-3: minima of the first block's tokens per group, rows 4-7: of the
// second block's, row 8: ones).  The two halves of a column are merged once,
// after the split's last super-tile.
template <int BITS, int G>
__device__ __forceinline__ void compute_tile_fold(const WaveStage<BITS, G> &ws, const h8 (&qf)[4],
                                                  const LaneConst<BITS, G> &lc, const FoldConst &fc,
                                                  int valid_rows, float scale_log2, WaveState &st) {
  using Tl = Tiles<BITS, G>;
  static_assert(Tl::TW == 4 && Tl::GW == 2 && Tl::NPL == 1 && Tl::NGD == 4 && Tl::TPW == 16,
                "the folded path is the 2-bit, 32-token-group layout");
  const int lane = threadIdx.x & 63, r = lane & 15, kap = lane >> 4;

  // ---- key minimum term: A row r = minima of group r % 2, so element v
  // holds group v % 2's bias for every column
  f4 mb = f4{0, 0, 0, 0};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
    mb = mfma32(*reinterpret_cast<const h8 *>(&ws.km[r % 2][32 * kb + 8 * kap]), qf[kb], mb);
  const float bias = (fc.half ? mb[1] : mb[0]) * scale_log2;

  // ---- keys: B' = q * key scale of this lane's half, then all four tiles
  h8 bp[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) bp[kb] = qf[kb] * *reinterpret_cast<const h8 *>(&ws.ks[fc.half][32 * kb + 8 * kap]);
  f4 a[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 x = *reinterpret_cast<const uint4 *>(&ws.kw[lc.kaddr + i * 256]);
    const uint32_t pc[4] = {x.x, x.y, x.z, x.w};
    a[i] = f4{0, 0, 0, 0};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const uint32_t piece[1] = {pc[kb]};
      a[i] = mfma32(gather_and<Tl::CPB>(piece, lc.kmask), bp[kb], a[i]);
    }
  }
  f4 acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[j][v] = __builtin_fmaf(fc.half ? a[j + 2][v] : a[j][v], lc.pw[v], bias);
  softmax_tiles<2, false>(acc, valid_rows, st, kap, 2 * fc.half);

  const h4 pa4 = cvt4(acc[0]), pb4 = cvt4(acc[1]);
  const h8 p8 = h8{pa4[0], pa4[1], pa4[2], pa4[3], pb4[0], pb4[1], pb4[2], pb4[3]};
  {
    const h4 ma = *reinterpret_cast<const h4 *>(fc.mrow);
    const h4 mb4 = *reinterpret_cast<const h4 *>(fc.mrow + 16);
    st.cmin = mfma32(h8{ma[0], ma[1], ma[2], ma[3], mb4[0], mb4[1], mb4[2], mb4[3]}, p8, st.cmin);
  }
  // ---- values: O^T += V^T P^T over the two 32-token blocks; block kc counts
  // only in the columns of half kc (the other half's P * scale is zero)
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) {
    uint32_t pv[8];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const uint4 x = *reinterpret_cast<const uint4 *>(&ws.vw[lc.vaddr + kc * 128 + hb * 64]);
      pv[4 * hb + 0] = x.x; pv[4 * hb + 1] = x.y; pv[4 * hb + 2] = x.z; pv[4 * hb + 3] = x.w;
    }
    h8 ps;
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      if ((16 * blk) % G == 0) {
        const int g = (16 * blk) / G;
        const h4 sa = *reinterpret_cast<const h4 *>(&ws.vs[g][fc.voff[kc]]);
        const h4 sb = *reinterpret_cast<const h4 *>(&ws.vs[g][fc.voff[kc] + 16]);
        ps = p8 * h8{sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
      }
      const uint32_t piece[1] = {pv[blk]};
      st.o[blk] = mfma32(gather_and<Tl::CPB>(piece, lc.vmask), ps, st.o[blk]);
    }
  }
}

template <int BITS, int G, bool FOLD>
__device__ __forceinline__ void packed_split(DecShared<BITS, G> &sh, const _Float16 (*sq)[kQPad],
                                             const _Float16 *ones, const uc_kivi_item &it, int64_t h,
                                             int64_t split, const MfmaParams &p, WaveState &st) {
  using Tl = Tiles<BITS, G>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t Tq = it.quantized_tokens;
  const int64_t cap = it.packed_capacity > 0 ? it.packed_capacity : Tq;  // tokens between heads
  // each resource covers the head's Tq packed tokens: rows past them read as 0
  const int64_t kcode_row = int64_t(kD) * 4 / Tl::TPW, kstat_row = int64_t(kD) * 2 / G;  // bytes per token
  const int64_t vcode_row = Tl::VWPT * 4, vstat_row = Tl::NGD * 2;
  PackedRegion rg;
  rg.kcode = make_rsrc(static_cast<const char *>(it.key_code) + h * cap * kcode_row, Tq * kcode_row);
  rg.kscale = make_rsrc(static_cast<const char *>(it.key_scale) + h * cap * kstat_row, Tq * kstat_row);
  rg.kmin = make_rsrc(static_cast<const char *>(it.key_min) + h * cap * kstat_row, Tq * kstat_row);
  rg.vcode = make_rsrc(static_cast<const char *>(it.value_code) + h * cap * vcode_row, Tq * vcode_row);
  rg.vscale = make_rsrc(static_cast<const char *>(it.value_scale) + h * cap * vstat_row, Tq * vstat_row);
  rg.vmin = make_rsrc(static_cast<const char *>(it.value_min) + h * cap * vstat_row, Tq * vstat_row);
  const LaneConst<BITS, G> lc = lane_const<BITS, G>(lane, p.scale_log2);
  h8 qf[4];  // this lane's query fragments, for the whole split
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) qf[kb] = query_frag(sq, kb, lane);
  WaveStage<BITS, G> &ws = sh.st[wave];
  FoldConst fc{};
  if constexpr (FOLD) {
    const int r = lane & 15, kap = lane >> 4;
    fc.half = r >> 3;
    fc.mrow = r < 4 ? &ws.vm[r][4 * kap] : r < 8 ? &ws.vm[r - 4][32 + 4 * kap] : ones + 4 * kap;
    fc.voff[0] = fc.half == 0 ? 4 * kap : 64 + 4 * kap;
    fc.voff[1] = fc.half == 1 ? 32 + 4 * kap : 64 + 4 * kap;
    // the value-scale pads [64, 96) of every group row read as zeros
    static_assert(Tiles<BITS, G>::VSP >= 96, "value-stat rows carry a 32-entry pad");
    reinterpret_cast<uint32_t *>(&ws.vs[lane >> 4][64])[lane & 15] = 0u;
    wave_lds_sync();
  }
  // super-tiles split, split + S, split + 2S, ... (S = packed splits); wave
  // w stages and computes tokens WT w .. WT w + WT - 1 of each on its own
  const int64_t n_super = (Tq + Tl::ST - 1) / Tl::ST;
  const int64_t stride = p.splits_packed * Tl::ST;
  const int n_it = static_cast<int>(min<int64_t>(p.nst, (n_super - split + p.splits_packed - 1) / p.splits_packed));
  Prefetch<BITS, G> pf;
  issue_loads<BITS, G>(pf, rg, static_cast<uint32_t>(split * Tl::ST), wave);
  for (int i = 0; i < n_it; ++i) {
    const uint32_t t0 = static_cast<uint32_t>((split + int64_t(i) * p.splits_packed) * Tl::ST);
    wave_lds_sync();  // this wave is done reading its previous super-tile
    stage_lds<BITS, G>(ws, pf);
    wave_lds_sync();
    if (i + 1 < n_it) issue_loads<BITS, G>(pf, rg, static_cast<uint32_t>(t0 + stride), wave);  // lands during compute
    const int valid = static_cast<int>(min<int64_t>(int64_t(Tl::WT), Tq - t0 - int64_t(Tl::WT) * wave));
    if (valid > 0) {
      if constexpr (FOLD)
        compute_tile_fold<BITS, G>(ws, qf, lc, fc, valid, p.scale_log2, st);
      else
        compute_tile<BITS, G>(ws, qf, lc, valid, p.scale_log2, ones, st);
    }
  }
  if constexpr (FOLD) {
    // finish each half's column as below, then merge the halves of a column
    // (lanes n and n ^ 8 hold the same query row over different tokens)
    const int n = lane & 15, kap = lane >> 4, half = n >> 3;
    float cm[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) cm[g] = __shfl(st.cmin[g], n + 16 * half, kWave);  // row g + 4 half
    const float l_half = __shfl(st.cmin[0], n + 32, kWave);                      // row 8: sum of P
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int e = (4 * kap + v) % Tl::CPB;
      const float undo = float(1 << (24 - BITS * e));
#pragma unroll
      for (int b = 0; b < 8; ++b) st.o[b][v] = st.o[b][v] * undo + cm[(16 * b) / G];
    }
    const float m_o = __shfl_xor(st.m, 8, kWave), l_o = __shfl_xor(l_half, 8, kWave);
    const float M = fmaxf(st.m, m_o), M_ref = M == kNegInf ? 0.0f : M;
    const float a_s = fast_exp2(st.m - M_ref), a_o = fast_exp2(m_o - M_ref);
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) st.o[b][v] = st.o[b][v] * a_s + __shfl_xor(st.o[b][v], 8, kWave) * a_o;
    st.m = M;
    st.l = kap == 0 ? l_half * a_s + l_o * a_o : 0.0f;  // the merge sums the k-slices
    return;
  }
  // undo the denormal code scaling 2^(BITS e - 24) of each output channel
  // (channel 16 b + 4 k + v: e depends on k and v only) and add the value
  // minima: sum_t P min of the channel's group sits in row g of cmin, held by
  // lane (n, k = g / 4) as element g % 4; the sum of P sits in row NGD
  const int n = lane & 15, kap = lane >> 4;
  float cm[Tl::NGD];
#pragma unroll
  for (int g = 0; g < Tl::NGD; ++g) cm[g] = __shfl(st.cmin[g % 4], n + 16 * (g / 4), kWave);
  const float l_all = __shfl(st.cmin[Tl::NGD % 4], n + 16 * (Tl::NGD / 4), kWave);
  st.l = kap == 0 ? l_all : 0.0f;  // the merge sums the k-slices
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int e = ((4 * kap + v) % Tl::TPW) % Tl::CPB;
    const float undo = float(1 << (24 - BITS * e));
#pragma unroll
    for (int b = 0; b < 8; ++b) st.o[b][v] = st.o[b][v] * undo + cm[(16 * b) / G];
  }
}

// --------------------------------------------------------- residual path --
// Dense residual tokens [tw, tw + RWT) of this wave ([Tr, Hkv, 128]
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

// Selection B operand that moves channel 16 par + n of a 32-channel A
// fragment into column n: B[k][n] = (k == 16 par + n).
__device__ __forceinline__ h8 channel_selector(int lane, int par) {
  const int n = lane & 15, kap = lane >> 4;
  h8 b;
#pragma unroll
  for (int j = 0; j < 8; ++j) b[j] = to_h(8 * kap + j == 16 * par + n ? 1.0f : 0.0f);
  return b;
}

template <int RD, int RWT>
__device__ __forceinline__ void residual_split(const _Float16 (*sq)[kQPad], const uc_kivi_item &it, int64_t h,
                                               int64_t tr0, const MfmaParams &p, WaveState &st) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kap = lane >> 4;
  const int64_t Tr = it.residual_tokens;
  int64_t ts, hs;  // token and head strides of the rows (elements)
  residual_strides(it, p.Hkv, kD, ts, hs);
  const int64_t bytes = ((Tr - 1) * ts + (p.Hkv - 1) * hs + kD) * 2;  // extent of the rows (Tr >= 1 here)
  const Rsrc rk = make_rsrc(it.residual_key, bytes), rv = make_rsrc(it.residual_value, bytes);
  // byte offset of token row t of this head; rows past Tr repeat the last row
  // (their probabilities are 0, and its values are finite data)
  const auto row_off = [&](int64_t t) { return static_cast<uint32_t>((min(t, Tr - 1) * ts + h * hs) * 2); };
  const int64_t tw = tr0 + wave * RWT;
  constexpr int kTiles = RWT / 16;
  const h8 csel[2] = {channel_selector(lane, 0), channel_selector(lane, 1)};
  f4 acc[kTiles];
#pragma unroll
  for (int b = 0; b < kTiles; ++b) {
    acc[b] = f4{0, 0, 0, 0};
    const uint32_t base = row_off(tw + 16 * b + r);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      acc[b] = mfma32(load8_h<RD>(rk, base + (32 * kb + 8 * kap) * 2), query_frag(sq, kb, lane), acc[b]);
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[b][v] *= p.scale_log2;
  }
  const int valid = static_cast<int>(min<int64_t>(int64_t(RWT), Tr - tw));
  softmax_tiles<kTiles, true>(acc, valid, st, kap);
  // O^T += V^T P^T: a lane loads 8 channels of one token per 32-channel
  // block; a selection MFMA turns a tile of them into the A layout of
  // accumulator b (row = channel 16 b + n, 4 tokens per lane)
#pragma unroll
  for (int j = 0; j < kTiles / 2; ++j) {
    const h4 pa4 = cvt4(acc[2 * j]), pb4 = cvt4(acc[2 * j + 1]);
    const h8 p8 = h8{pa4[0], pa4[1], pa4[2], pa4[3], pb4[0], pb4[1], pb4[2], pb4[3]};
    const uint32_t base0 = row_off(tw + 32 * j + r);
    const uint32_t base1 = row_off(tw + 32 * j + 16 + r);
#pragma unroll
    for (int b2 = 0; b2 < 4; ++b2) {
      const h8 v0 = load8_h<RD>(rv, base0 + (32 * b2 + 8 * kap) * 2);
      const h8 v1 = load8_h<RD>(rv, base1 + (32 * b2 + 8 * kap) * 2);
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const h4 a0 = cvt4(mfma32(v0, csel[par], f4{0, 0, 0, 0})), a1 = cvt4(mfma32(v1, csel[par], f4{0, 0, 0, 0}));
        st.o[2 * b2 + par] = mfma32(h8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]}, p8, st.o[2 * b2 + par]);
      }
    }
  }
}

// ------------------------------------------------------------------ kernel --
template <int BITS, int G, int RD, bool TABLE, bool FOLD>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) void decode_mfma_kernel(
    const uc_kivi_item *items, ArgItems ai, MfmaParams p) {
  __shared__ __align__(16) DecShared<BITS, G> sh;
  __shared__ __align__(16) _Float16 sq[16][kQPad];
  __shared__ __align__(16) _Float16 sones[kOnesLen];  // the ones rows of the cmin MFMA
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Workgroup i runs on XCD i % 8; with enough units its k = i / 8-th
  // workgroup there is split k % S of unit (item, KV head) u = 8 (k / S) + i % 8,
  // so the S splits of a unit are dispatched back to back on one XCD and share
  // its L2.  A launch of few units spreads each unit's splits over the XCDs.
  // 32-bit index arithmetic (the launch keeps the grid below 2^31; a 64-bit
  // division costs the scalar unit a few hundred instructions)
  const uint32_t splits = static_cast<uint32_t>(p.splits_total), hkv = static_cast<uint32_t>(p.Hkv);
  uint32_t u32, split32;
  if (p.xcd_grouped) {
    const uint32_t x = blockIdx.x % kXcds, k = blockIdx.x / kXcds, q = k / splits;
    u32 = q * kXcds + x;
    split32 = k - q * splits;
  } else {
    u32 = blockIdx.x / splits;
    split32 = blockIdx.x - u32 * splits;
  }
  if (u32 >= static_cast<uint32_t>(p.units)) return;  // uniform: the whole workgroup leaves
  const int64_t split = split32;
  const uint32_t item32 = u32 / hkv;
  const int64_t item = item32;
  const uc_kivi_item it = TABLE ? items[item] : ai.v[item];
  const int64_t h = u32 - item32 * hkv;
  if (!split_has_work(split, it.quantized_tokens, it.residual_tokens, p)) {  // uniform
    // only the statistics: (-inf, 0) gives the split weight 0 in the combine,
    // which then never reads its (unwritten) partial output
    if (tid < 16) {
      const int64_t slot = (item * p.Hkv + h) * p.splits_total + split;
      reinterpret_cast<float2 *>(p.ws_ml)[slot * 16 + tid] = make_float2(kNegInf, 0.0f);
    }
    return;
  }

  stage_queries(sq, it.query, h, p, FOLD);
  if (tid < kOnesLen / 2) reinterpret_cast<uint32_t *>(sones)[tid] = 0x3c003c00u;  // fp16 1.0 pairs
  WaveState st;
#pragma unroll
  for (int b = 0; b < 8; ++b) st.o[b] = f4{0, 0, 0, 0};
  st.cmin = f4{0, 0, 0, 0};
  st.m = kNegInf;
  st.l = 0.0f;
  __syncthreads();

  // residual splits first, so their short runs are spread over the launch
  // instead of forming its tail
  const int64_t splits_res = p.splits_total - p.splits_packed;
  if (split >= splits_res) {
    packed_split<BITS, G, FOLD>(sh, sq, sones, it, h, split - splits_res, p, st);
  } else {
    const int64_t tr0 = split * kWaves * p.res_wave;
    if (tr0 + wave * p.res_wave < it.residual_tokens) {
      if (p.res_wave == kResWaveTokensShort) residual_split<RD, kResWaveTokensShort>(sq, it, h, tr0, p, st);
      else residual_split<RD, kResWaveTokensLong>(sq, it, h, tr0, p, st);
    }
  }

  // ---- merge the waves; lane (n, k) holds query n, channels 16 b + 4 k + v
  const int kap = lane >> 4, n = lane & 15;
  const float l_all = sum_over_slices(st.l);
  __syncthreads();  // the staging area becomes the merge area
  if (kap == 0) {
    sh.mrg.ml[wave][n][0] = st.m;
    sh.mrg.ml[wave][n][1] = l_all;
  }
  __syncthreads();
  float M = kNegInf;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sh.mrg.ml[w][n][0]);
  const float M_ref = M == kNegInf ? 0.0f : M;
  float L = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) L += sh.mrg.ml[w][n][1] * fast_exp2(sh.mrg.ml[w][n][0] - M_ref);
  const float mine = fast_exp2(st.m - M_ref);
  if (wave > 0) {
#pragma unroll
    for (int b = 0; b < 8; ++b)
      *reinterpret_cast<f4 *>(&sh.mrg.o[wave - 1][n][16 * b + 4 * kap]) = st.o[b] * mine;
  }
  __syncthreads();
  if (wave == 0) {
    const int64_t slot = (item * p.Hkv + h) * p.splits_total + split;
    _Float16 *po = p.ws_o + slot * 16 * kD;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    if (n < p.rows) {  // rows past the query rows are never read: not written
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        f4 s = st.o[b] * mine;
#pragma unroll
        for (int w = 0; w < kWaves - 1; ++w) s += *reinterpret_cast<const f4 *>(&sh.mrg.o[w][n][16 * b + 4 * kap]);
        *reinterpret_cast<h4 *>(&po[n * kD + 16 * b + 4 * kap]) = cvt4(s * inv);
      }
    }
    if (kap == 0) {
      p.ws_ml[(slot * 16 + n) * 2 + 0] = M;
      p.ws_ml[(slot * 16 + n) * 2 + 1] = L;
    }
  }
}

// Merge the split partials of one (query group, KV head) -- every split of the
// p.segs items that share the query.  Thread (row = t / 16, c = t % 16) of a
// part owns channels 8c .. 8c + 7 of one query row, so a row's 16 threads read
// each partial row as one contiguous 256-byte run; a part has only the threads
// of the query rows (rounded to whole waves).  The splits are dealt to
// `parts` (1, 2 or 4) parts of the block in contiguous runs; a part takes its
// run in rounds of kCombineRound, every load of a round issued before any
// arithmetic, with an online (M, L): a round that raises the maximum rescales
// the sums first.  The parts then merge through LDS, part 0 writes the output
// and the LSE of the group's first item.  Splits without work wrote (-inf, 0)
// and no partial: their weight is 0 and their partial is not read.
constexpr int kCombineRound = 16;
constexpr int kCombineMaxThreads = 1024;

// Eight channels of output element `idx` on, from fp32 (one 16-byte store for
// 16-bit outputs).
__device__ __forceinline__ void store_out8(void *out, int64_t idx, const float *v, int od) {
  if (od == UC_FP32) {
    float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + idx);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
    return;
  }
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t lo = od == UC_BF16 ? f32_to_bf16_bits(v[2 * k]) : f32_to_f16_bits(v[2 * k]);
    const uint32_t hi = od == UC_BF16 ? f32_to_bf16_bits(v[2 * k + 1]) : f32_to_f16_bits(v[2 * k + 1]);
    w[k] = lo | (hi << 16);
  }
  *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + idx) = make_uint4(w[0], w[1], w[2], w[3]);
}

template <bool TABLE>
__global__ __launch_bounds__(kCombineMaxThreads) void decode_mfma_combine(const uc_kivi_item *items, ArgItems ai,
                                                                          MfmaParams p, int parts) {
  extern __shared__ float red[];  // per thread of parts 1..: M, L, 8 sums (10 floats)
  const int64_t first = blockIdx.x * p.segs;
  const int64_t h = blockIdx.y;
  const int span = int(blockDim.x) / parts;  // threads per part (whole waves)
  const int part = int(threadIdx.x) / span, t = int(threadIdx.x) % span;
  const int r = t >> 4, c8 = (t & 15) * 8;
  const bool active = r < p.rows;
  const int splits = int(p.splits_total), nflat = int(p.segs) * splits;
  const int run = (nflat + parts - 1) / parts, f_lo = part * run, f_hi = min(nflat, f_lo + run);
  // (segment, split) f -> workspace slot: segment f / splits of the group
  auto slot = [&](int f) { return ((first + f / splits) * p.Hkv + h) * p.splits_total + f % splits; };
  float M = kNegInf, L = 0.0f;
  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
  for (int f0 = f_lo; active && f0 < f_hi; f0 += kCombineRound) {
    float2 ml[kCombineRound];
    uint4 v[kCombineRound];
#pragma unroll
    for (int u = 0; u < kCombineRound; ++u) {
      if (f0 + u < f_hi) {
        const int64_t sl = slot(f0 + u);
        ml[u] = *reinterpret_cast<const float2 *>(p.ws_ml + (sl * 16 + r) * 2);
        v[u] = *reinterpret_cast<const uint4 *>(p.ws_o + (sl * 16 + r) * kD + c8);
      } else {
        ml[u] = make_float2(kNegInf, 0.0f);
      }
    }
    float mr = M;
#pragma unroll
    for (int u = 0; u < kCombineRound; ++u)
      if (ml[u].y > 0.0f && ml[u].x != kNegInf) mr = fmaxf(mr, ml[u].x);
    if (mr > M) {  // rescale what earlier rounds summed
      const float sc = M == kNegInf ? 0.0f : exp2f(M - mr);
      L *= sc;
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] *= sc;
      M = mr;
    }
#pragma unroll
    for (int u = 0; u < kCombineRound; ++u) {
      if (!(ml[u].y > 0.0f) || ml[u].x == kNegInf) continue;
      const float w = ml[u].y * exp2f(ml[u].x - M);
      L += w;
      const uint32_t wd[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] = fmaf(f16_bits_to_f32(uint16_t(wd[e] & 0xffffu)), w, acc[2 * e]);
        acc[2 * e + 1] = fmaf(f16_bits_to_f32(uint16_t(wd[e] >> 16)), w, acc[2 * e + 1]);
      }
    }
  }
  if (parts > 1) {  // uniform
    if (part > 0) {
      float *e = red + (threadIdx.x - span) * 10;
      e[0] = M;
      e[1] = L;
#pragma unroll
      for (int c = 0; c < 8; ++c) e[2 + c] = acc[c];
    }
    __syncthreads();
    if (part > 0) return;
    for (int q = 1; q < parts; ++q) {
      const float *e = red + ((q - 1) * span + t) * 10;
      const float m2 = e[0], l2 = e[1];
      if (!(l2 > 0.0f)) continue;
      const float mn = fmaxf(M, m2);
      const float s1 = M == kNegInf ? 0.0f : exp2f(M - mn), s2 = exp2f(m2 - mn);
      L = L * s1 + l2 * s2;
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = acc[c] * s1 + e[2 + c] * s2;
      M = mn;
    }
  }
  if (!active) return;
  const uc_kivi_item it = TABLE ? items[first] : ai.v[first];
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] *= inv;
  const int64_t g = r / p.Lq, i = r % p.Lq;
  if (c8 == 0 && it.lse != nullptr) it.lse[(h * p.group + g) * p.Lq + i] = L > 0.0f ? (M + log2f(L)) * kLn2 : kNegInf;
  store_out8(it.out, (i * p.Hq + h * p.group + g) * kD + c8, acc, p.od);
}

}  // namespace

// Packed tokens per split of the MFMA decode for `bits` (super-tiles per
// split x tokens per super-tile).
int64_t decode_mfma_split_tokens(int bits, int64_t nst) { return nst * 16 * (32 / bits); }

int64_t decode_mfma_res_split_tokens(int64_t max_tr) { return kWaves * res_wave_tokens(max_tr); }

// Splits per (item, KV head): packed splits, then residual splits.
int64_t decode_mfma_num_splits(int bits, int64_t nst, int64_t max_tq, int64_t max_tr) {
  return ceil_div(max_tq, decode_mfma_split_tokens(bits, nst)) + ceil_div(max_tr, decode_mfma_res_split_tokens(max_tr));
}

bool decode_mfma_supported(int bits, int group, int64_t D, int64_t rows) {
  return (bits == 2 || bits == 4) && (group == 32 || group == 64 || group == 128) && D == kD && rows <= 16;
}

int64_t decode_mfma_workspace_bytes(int64_t n_items, int64_t heads_kv, int64_t splits) {
  const int64_t slots = n_items * heads_kv * splits;
  return slots * 16 * kD * int64_t(sizeof(_Float16)) + slots * 16 * 2 * int64_t(sizeof(float));
}

// The column-folded packed path: 2-bit codes, 32-token groups, <= 8 query rows.
template <int BITS, int G>
constexpr bool kFoldable = BITS == 2 && G == 32;

template <int BITS, int G, int RD>
static void launch_typed(bool table, dim3 grid, hipStream_t stream, const uc_kivi_item *items_dev,
                         const ArgItems &one, const MfmaParams &p) {
  if constexpr (kFoldable<BITS, G>) {
    if (p.rows <= 8) {
      if (table)
        hipLaunchKernelGGL((decode_mfma_kernel<BITS, G, RD, true, true>), grid, dim3(kThreads), 0, stream, items_dev,
                           one, p);
      else
        hipLaunchKernelGGL((decode_mfma_kernel<BITS, G, RD, false, true>), grid, dim3(kThreads), 0, stream, items_dev,
                           one, p);
      return;
    }
  }
  if (table)
    hipLaunchKernelGGL((decode_mfma_kernel<BITS, G, RD, true, false>), grid, dim3(kThreads), 0, stream, items_dev,
                       one, p);
  else
    hipLaunchKernelGGL((decode_mfma_kernel<BITS, G, RD, false, false>), grid, dim3(kThreads), 0, stream, items_dev,
                       one, p);
}

template <int BITS, int G>
static void launch_group(bool table, int rd, dim3 grid, hipStream_t stream, const uc_kivi_item *items_dev,
                         const ArgItems &one, const MfmaParams &p) {
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
  // workgroup slots (kWgPerCu per CU) and `nst` does not: a batch-1 32k context then
  // runs as one full round instead of ~1.9 (+3 % measured).  Fewer splits, so
  // the workspace sized for `nst` still fits.
  {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) {
      const int64_t units = n_items * Hkv, round = kWgPerCu * int64_t(cus);
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
  p.res_wave = res_wave_tokens(max_tr);
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
  UC_REQUIRE(table || (single != nullptr && n_items <= kArgItems), "decode: at most %d items from host memory",
             kArgItems);
  ArgItems one{};
  if (!table)
    for (int64_t i = 0; i < n_items; ++i) one.v[i] = single[i];
  p.units = n_items * Hkv;
  p.super_tokens = 16 * (32 / bits);
  p.xcd_grouped = p.units >= 4 * kXcds;  // at most one unit of imbalance per XCD in four
  const int64_t n_groups = (p.xcd_grouped ? ceil_div(p.units, int64_t(kXcds)) * kXcds : p.units) * p.splits_total;
  UC_REQUIRE(n_groups < (int64_t(1) << 31), "decode: grid too large (%lld workgroups)", (long long)n_groups);
  const dim3 grid(static_cast<unsigned>(n_groups));
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
  // one block per (query group, KV head): `parts` runs of about 12 splits each
  // (at most 4), each part with the threads of the query rows
  const int64_t nflat = segs * p.splits_total;
  const int parts = nflat > 36 ? 4 : nflat > 12 ? 2 : 1;
  const dim3 cgrid(static_cast<unsigned>(n_items / segs), static_cast<unsigned>(Hkv));
  const dim3 cblock(static_cast<unsigned>(parts * ceil_div(p.rows * 16, int64_t(kWave)) * kWave));
  const size_t lds = size_t(cblock.x / parts) * (parts - 1) * 10 * sizeof(float);
  if (table)
    hipLaunchKernelGGL((decode_mfma_combine<true>), cgrid, cblock, lds, stream, items_dev, one, p, parts);
  else
    hipLaunchKernelGGL((decode_mfma_combine<false>), cgrid, cblock, lds, stream, items_dev, one, p, parts);
  return check_launch("decode (MFMA combine)");
}

}  // namespace uc
