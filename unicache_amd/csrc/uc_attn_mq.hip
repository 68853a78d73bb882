// Multi-query attention over one KIVI-packed segment plus its dense residual
// (head_dim 128, 2/4-bit codes): the long-query case of UniCache's packed
// attention (image editing: ~1088 queries x 7 query heads per KV head).
//
// Two kernels.  mq_stage_kernel dequantizes the packed keys/values once per
// KV head into an fp16 workspace -- keys [Hkv][Tp][128], values transposed
// [Hkv][128][Tp] (Tp = keys rounded up to 64, zero tail) -- and converts the
// residual into the same arrays; every query block then reads fp16 tiles
// instead of re-dequantizing them (a fused version re-did the dequant for each
// of the ~60 query blocks per head and was VALU-bound).
//
// mq_attention_kernel: one workgroup (4 waves) owns 128 query rows of one KV
// head; each wave keeps 32 rows (two 16-row blocks) in registers and streams
// the keys in 64-key tiles through double-buffered LDS (one barrier per tile,
// the next tile's global loads in flight during the current tile's MFMAs):
//   S^T = K Q^T   (v_mfma_f32_16x16x32_f16, rows = keys, columns = queries)
//   online base-2 softmax over the key rows,
//   O  += P V     (v_mfma_f32_16x16x32_f16, A = P straight from the S^T
//                  accumulators, B = two 4-key runs of the value tile).
// Output: normalised O (written through LDS as whole rows) and the
// natural-log LSE.
#include <type_traits>
#include <utility>

#include "uc_common.h"
#include "uc_mfma.h"

namespace uc {
namespace {

using namespace mf;

constexpr int kXcds = 8;  // XCDs of an MI355X; launch index i runs on XCD i % 8
constexpr int kMqWaves = 4;
constexpr int kMqThreads = kMqWaves * kWave;
constexpr int kRowsPerWave = 32;
constexpr int kMqRows = kMqWaves * kRowsPerWave;  // query rows per workgroup
constexpr int kTile = 64;                         // keys per iteration
constexpr int kKPad = kD + 8;   // key row in halves: 68 dwords, 16 rows on distinct banks
constexpr int kVPad = kTile + 4;  // value row in halves: 34 dwords

struct MqTile {
  _Float16 kt[kTile][kKPad];  // keys [token][channel]
  _Float16 vt[kD][kVPad];     // values [channel][token]
};

struct MqParams {
  int64_t Hq, Hkv, Lq, group, rows;  // rows = group * Lq query rows per KV head
  int64_t keys, keys_pad;            // Tq + Tr and its multiple of 64
  float scale_log2;
  const _Float16 *wk;  // [Hkv][keys_pad][128]
  const _Float16 *wv;  // [Hkv][128][keys_pad]
  int64_t row_blocks, per_xcd;  // row blocks per KV head; work items per XCD
  FastDiv lq;                   // row -> (query head of the group, query position)
};

struct StageParams {
  int64_t Hkv, keys, keys_pad;
  _Float16 *wk, *wv;
};

// Up to kMqMaxBatch segments (one query block each) in one stage launch and
// one attention launch, passed by value as kernel arguments.  Item i owns
// stage tiles [stage_begin[i], stage_begin[i+1]) and attention work items
// (row block x KV head) [attn_begin[i], attn_begin[i+1]).  Work items are
// launched in that order, longest segments first: each one fills a CU, and
// starting the long ones first shortens the tail when the segments differ in
// length.
constexpr int kMqMaxBatch = 8;
struct MqBatch {
  uc_kivi_item it[kMqMaxBatch];
  MqParams p[kMqMaxBatch];
  StageParams sp[kMqMaxBatch];
  int64_t stage_begin[kMqMaxBatch + 1], attn_begin[kMqMaxBatch + 1];
  int n;
};
static_assert(sizeof(MqBatch) <= 4096, "the batch table fits the kernel argument space");

// Item of a batch that owns index x of a cumulative range table (uniform).
__device__ __forceinline__ int batch_item(const int64_t *begin, int n, int64_t x) {
  int i = 0;
  while (i + 1 < n && x >= begin[i + 1]) ++i;
  return i;
}

// Packed words and stats of one 64-key tile, per thread.
template <int BITS>
struct TilePf {
  static constexpr int NW = (kTile / Geo<BITS>::TPW) * kD / 2 / kMqThreads;  // key word pairs (1 or 2)
  static constexpr int NV = kTile / 2 * Geo<BITS>::VW / kMqThreads;          // value word pairs (1 or 2)
  uint32_t kwa[NW], kwb[NW];  // key words of channels 2cp, 2cp+1
  uint32_t ks[NW], km[NW];    // their scales / minima, packed (channel 2cp | 2cp+1 << 16)
  uint32_t vwa[NV], vwb[NV];  // value words of tokens 2tp, 2tp+1
  uint32_t vs[NV], vm[NV];    // their scales / minima, packed (token 2tp | 2tp+1 << 16)
};

// One head's packed tensors (token-major: key words [word][D], key stats
// [group][D], values [token][...]); each resource covers the Tq packed tokens.
struct PackedSrc {
  Rsrc kcode, kscale, kmin, vcode, vscale, vmin;
};

template <int BITS, int G>
__device__ __forceinline__ void issue_tile(TilePf<BITS> &pf, const PackedSrc &src, uint32_t t0, int tid) {
  using Gm = Geo<BITS>;
#pragma unroll
  for (int i = 0; i < TilePf<BITS>::NW; ++i) {
    const int e = i * kMqThreads + tid;
    const int cp = e % (kD / 2), j = e / (kD / 2);  // channel pair, word of the tile
    const uint32_t J = t0 / Gm::TPW + j;
    const uint32_t g = (t0 + j * Gm::TPW) / G;
    const uint2 w = bload64(src.kcode, (J * kD + 2 * cp) * 4u);  // channels 2cp, 2cp+1 are neighbours
    pf.kwa[i] = w.x;
    pf.kwb[i] = w.y;
    pf.ks[i] = bload32(src.kscale, (g * kD + 2 * cp) * 2u);
    pf.km[i] = bload32(src.kmin, (g * kD + 2 * cp) * 2u);
  }
#pragma unroll
  for (int i = 0; i < TilePf<BITS>::NV; ++i) {
    const int e = i * kMqThreads + tid;
    const int tp = e % (kTile / 2), w = e / (kTile / 2);  // token pair, value word
    const uint32_t t = t0 + 2 * tp;
    const int g = (w * Gm::TPW) / G;
    constexpr int NGD = kD / G;
    pf.vwa[i] = bload32(src.vcode, (t * Gm::VW + w) * 4u);
    pf.vwb[i] = bload32(src.vcode, ((t + 1) * Gm::VW + w) * 4u);
    pf.vs[i] = bload16(src.vscale, (t * NGD + g) * 2u) | (bload16(src.vscale, ((t + 1) * NGD + g) * 2u) << 16);
    pf.vm[i] = bload16(src.vmin, (t * NGD + g) * 2u) | (bload16(src.vmin, ((t + 1) * NGD + g) * 2u) << 16);
  }
}

// Dequantize the TPW codes of two words whose 16-bit halves are paired by
// `perm`: out[p] = (code_a(p), code_b(p)) * scale + min, p = code position.
template <int BITS>
__device__ __forceinline__ void dequant_pair(uint32_t wa, uint32_t wb, uint32_t s2, uint32_t m2,
                                             h2 (&out)[Geo<BITS>::TPW]) {
  using Gm = Geo<BITS>;
  constexpr int HALF = Gm::TPW / 2;
  const h2 sp = as_h2(s2), mp = as_h2(m2);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const uint32_t y = __builtin_amdgcn_perm(wb, wa, half ? 0x07060302u : 0x05040100u);
#pragma unroll
    for (int pq = 0; pq < HALF; ++pq) {
      const bool direct = pq <= Gm::PMAX;
      const int pe = direct ? pq : pq - (Gm::PMAX + 1);
      const _Float16 inv = to_h(1.0f / float(1u << (BITS * pe)));
      const h2 x = code_pair<BITS>(direct ? y : (y >> Gm::SH), pe);
      out[half * HALF + pq] = __builtin_elementwise_fma(x, sp * h2{inv, inv}, mp);
    }
  }
}


// ------------------------------------------------------------- stage pass --
// Workgroup (tile, KV head): keys [64*tile, 64*tile + 64) of the combined
// sequence [packed | residual | zero tail].
// The tile's 256 work items are spread over four one-wave workgroups
// (blockIdx.z), which spreads the pass over more CUs.
constexpr int kStageThreads = kWave;

template <int BITS, int G, int RD>
__device__ __forceinline__ void mq_stage_body(const uc_kivi_item &it, const StageParams &sp, int64_t tile) {
  using Gm = Geo<BITS>;
  const int tid = blockIdx.z * kStageThreads + threadIdx.x;  // work item of the tile, 0..255
  const int64_t h = blockIdx.y;
  const int64_t x0 = tile * kTile;  // first key of the tile
  const int64_t Tq = it.quantized_tokens, Tr = it.residual_tokens, T = Tq + Tr;
  _Float16 *wk = sp.wk + h * sp.keys_pad * kD;
  _Float16 *wv = sp.wv + h * kD * sp.keys_pad;

  if (x0 < Tq) {  // packed words (Tq is a multiple of G >= 32, so words never straddle it)
    PackedSrc src;
    const int64_t cap = it.packed_capacity > 0 ? it.packed_capacity : Tq;  // tokens between heads
    const int64_t kcode_row = int64_t(kD) * 4 / Gm::TPW, kstat_row = int64_t(kD) * 2 / G;  // bytes per token
    const int64_t vcode_row = Gm::VW * 4, vstat_row = (kD / G) * 2;
    src.kcode = make_rsrc(static_cast<const char *>(it.key_code) + h * cap * kcode_row, Tq * kcode_row);
    src.kscale = make_rsrc(static_cast<const char *>(it.key_scale) + h * cap * kstat_row, Tq * kstat_row);
    src.kmin = make_rsrc(static_cast<const char *>(it.key_min) + h * cap * kstat_row, Tq * kstat_row);
    src.vcode = make_rsrc(static_cast<const char *>(it.value_code) + h * cap * vcode_row, Tq * vcode_row);
    src.vscale = make_rsrc(static_cast<const char *>(it.value_scale) + h * cap * vstat_row, Tq * vstat_row);
    src.vmin = make_rsrc(static_cast<const char *>(it.value_min) + h * cap * vstat_row, Tq * vstat_row);
    TilePf<BITS> pf;
    issue_tile<BITS, G>(pf, src, static_cast<uint32_t>(x0), tid);
#pragma unroll
    for (int i = 0; i < TilePf<BITS>::NW; ++i) {
      const int e = i * kMqThreads + tid;
      const int cp = e % (kD / 2), j = e / (kD / 2);
      const int64_t t = x0 + j * Gm::TPW;
      if (t >= Tq) continue;
      h2 v[Gm::TPW];
      dequant_pair<BITS>(pf.kwa[i], pf.kwb[i], pf.ks[i], pf.km[i], v);
#pragma unroll
      for (int p = 0; p < Gm::TPW; ++p) *reinterpret_cast<h2 *>(&wk[(t + p) * kD + 2 * cp]) = v[p];
    }
#pragma unroll
    for (int i = 0; i < TilePf<BITS>::NV; ++i) {
      const int e = i * kMqThreads + tid;
      const int tp = e % (kTile / 2), w = e / (kTile / 2);
      const int64_t t = x0 + 2 * tp;
      if (t >= Tq) continue;
      h2 v[Gm::TPW];
      dequant_pair<BITS>(pf.vwa[i], pf.vwb[i], pf.vs[i], pf.vm[i], v);
#pragma unroll
      for (int p = 0; p < Gm::TPW; ++p) *reinterpret_cast<h2 *>(&wv[(w * Gm::TPW + p) * sp.keys_pad + t]) = v[p];
    }
  }
  if (x0 + kTile > Tq) {  // residual keys and the zero tail
    const int64_t row_stride = sp.Hkv * kD;
    {
      const int tok = tid / 4, cq = tid % 4;  // 32 channels of one key
      const int64_t x = x0 + tok;
      if (x >= Tq) {
        h8 o[4];
        if (x < T) {
          const uint16_t *src = static_cast<const uint16_t *>(it.residual_key) + (x - Tq) * row_stride + h * kD + 32 * cq;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint4 raw = *reinterpret_cast<const uint4 *>(src + 8 * q);
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              o[q][2 * j] = to_h(half_bits_to_f32<RD>(w[j]));
              o[q][2 * j + 1] = to_h(half_bits_to_f32<RD>(w[j] >> 16));
            }
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) o[q] = h8{0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<h8 *>(&wk[x * kD + 32 * cq + 8 * q]) = o[q];
      }
    }
    {
      const int tp = tid % (kTile / 2), ce = tid / (kTile / 2);  // key pair, 16-channel block
      const int64_t xa = x0 + 2 * tp;
      if (xa >= Tq) {
        float va[16], vb[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) va[c] = vb[c] = 0.0f;
        const uint16_t *rv = static_cast<const uint16_t *>(it.residual_value);
        if (xa < T) {
          const uint16_t *src = rv + (xa - Tq) * row_stride + h * kD + 16 * ce;
#pragma unroll
          for (int c = 0; c < 16; ++c) va[c] = half_bits_to_f32<RD>(src[c]);
        }
        if (xa + 1 < T) {
          const uint16_t *src = rv + (xa + 1 - Tq) * row_stride + h * kD + 16 * ce;
#pragma unroll
          for (int c = 0; c < 16; ++c) vb[c] = half_bits_to_f32<RD>(src[c]);
        }
#pragma unroll
        for (int c = 0; c < 16; ++c)
          *reinterpret_cast<h2 *>(&wv[(16 * ce + c) * sp.keys_pad + xa]) = h2{to_h(va[c]), to_h(vb[c])};
      }
    }
  }
}

template <int BITS, int G, int RD>
__global__ __launch_bounds__(kStageThreads) void mq_stage_kernel(uc_kivi_item it, StageParams sp) {
  mq_stage_body<BITS, G, RD>(it, sp, blockIdx.x);
}

template <int BITS, int G, int RD>
__global__ __launch_bounds__(kStageThreads) void mq_stage_batch_kernel(MqBatch b) {
  const int64_t tile = blockIdx.x;
  const int i = batch_item(b.stage_begin, b.n, tile);
  mq_stage_body<BITS, G, RD>(b.it[i], b.sp[i], tile - b.stage_begin[i]);
}

// --------------------------------------------------------- attention pass --
// Output is kept transposed (O^T = V^T P^T) so that every lane owns one query
// column: the softmax rescale needs no cross-lane traffic.
struct MqState {
  f4 o[2][8];        // [query block][channel block]: lane (n, k) -> query n, channels 16*cb + 4k + v
  float m[2], l[2];  // lane (n, k): running max of query n; l = this lane's share of the sum
};

// Global fp16 data of one 64-key tile, per thread of a 256-thread key half:
// 64 B of keys, 64 B of values.
struct TileRegs {
  uint4 k[4], v[4];
};

__device__ __forceinline__ void load_tile(TileRegs &tr, Rsrc rk, Rsrc rv, int64_t keys_pad, int64_t x0, int tid) {
  const int tok = tid / 4, kq = tid % 4;  // key rows: 4 threads x 64 B
  const int ch = tid / 2, vh = tid % 2;   // value rows (per channel): 2 threads x 64 B
  const uint32_t ko = static_cast<uint32_t>(((x0 + tok) * kD + 32 * kq) * 2);
  const uint32_t vo = static_cast<uint32_t>((ch * keys_pad + x0 + 32 * vh) * 2);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    tr.k[q] = bload128(rk, ko + 16 * q);
    tr.v[q] = bload128(rv, vo + 16 * q);
  }
}

__device__ __forceinline__ void store_tile(MqTile &t, const TileRegs &tr, int tid) {
  const int tok = tid / 4, kq = tid % 4;
  const int ch = tid / 2, vh = tid % 2;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    *reinterpret_cast<uint4 *>(&t.kt[tok][32 * kq + 8 * q]) = tr.k[q];
    *reinterpret_cast<uint2 *>(&t.vt[ch][32 * vh + 8 * q]) = make_uint2(tr.v[q].x, tr.v[q].y);
    *reinterpret_cast<uint2 *>(&t.vt[ch][32 * vh + 8 * q + 4]) = make_uint2(tr.v[q].z, tr.v[q].w);
  }
}

// One tile: logits, online softmax, P.V for the wave's 32 query rows.
__device__ __forceinline__ void compute_tile(const MqTile &sh, const h8 (&qf)[2][4], int valid_keys,
                                             float scale_log2, MqState &st) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, kap = lane >> 4;
  f4 acc[4][2];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) acc[tb][qb] = f4{0, 0, 0, 0};
  // key fragments of k-block kb+1 are read while the MFMAs of kb run
  h8 ka[2][4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) ka[0][tb] = *reinterpret_cast<const h8 *>(&sh.kt[16 * tb + r][8 * kap]);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    if (kb + 1 < 4) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
        ka[(kb + 1) & 1][tb] = *reinterpret_cast<const h8 *>(&sh.kt[16 * tb + r][32 * (kb + 1) + 8 * kap]);
    }
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) acc[tb][qb] = mfma32(ka[kb & 1][tb], qf[qb][kb], acc[tb][qb]);
  }
  if (valid_keys < kTile) {  // last tile: keys past the end do not exist
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (16 * tb + 4 * kap + v >= valid_keys) acc[tb][0][v] = acc[tb][1][v] = kNegInf;
  }
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float mx = kNegInf;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int v = 0; v < 4; ++v) mx = fmaxf(mx, acc[tb][qb][v]);
    mx = max_over_slices(mx);
    const float m_new = fmaxf(st.m[qb], mx * scale_log2);  // logits in log2 units
    const float m_ref = m_new == kNegInf ? 0.0f : m_new;
    float sum = 0.0f;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float e = fast_exp2(__builtin_fmaf(acc[tb][qb][v], scale_log2, -m_ref));
        acc[tb][qb][v] = e;
        sum += e;
      }
    const float alpha = fast_exp2(st.m[qb] - m_ref);
    st.l[qb] = st.l[qb] * alpha + sum;  // reduced over the k-slices once, at the end
    st.m[qb] = m_new;
    if (__any(alpha != 1.0f)) {  // the running max moved for some query of this block
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) st.o[qb][cb] *= alpha;
    }
  }
#pragma unroll
  for (int tp = 0; tp < 2; ++tp) {
    // A: 16 channels x the 8 keys this k-slice holds in P (two 4-key runs),
    // all eight channel blocks read before the MFMAs
    h8 va[8];
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const h4 lo = *reinterpret_cast<const h4 *>(&sh.vt[16 * cb + r][32 * tp + 4 * kap]);
      const h4 hi = *reinterpret_cast<const h4 *>(&sh.vt[16 * cb + r][32 * tp + 16 + 4 * kap]);
      va[cb] = h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    h8 ap[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const h4 lo = cvt4(acc[2 * tp][qb]), hi = cvt4(acc[2 * tp + 1][qb]);
      ap[qb] = h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) st.o[qb][cb] = mfma32(va[cb], ap[qb], st.o[qb][cb]);
    // keep the 16 LDS reads ahead of the 16 MFMAs (the scheduler otherwise
    // pairs each read with its two MFMAs and waits on every read)
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
  }
}

// 8 waves: waves 0-3 and 4-7 take the first and second half of the key tiles
// for the same 128 query rows (32 per wave), so each SIMD runs two waves whose
// softmax VALU work and MFMAs overlap; the halves merge through LDS at the end.
constexpr int kAttnWaves = 8;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kHalfThreads = kAttnThreads / 2;
static_assert(kHalfThreads == 256, "tile loads map 256 threads per key half");
constexpr int kMergeFloats = 2 * 8 * 4 + 4;  // O^T (2 query blocks x 8 channel blocks x 4) + m[2], l[2]

// Work item w = h * row_blocks + rb of one segment: 128 query rows of KV head h.
template <int QD, int OD>
__device__ __forceinline__ void mq_attention_body(const uc_kivi_item &it, const MqParams &p, int64_t w) {
  __shared__ MqTile sh[2][2];  // [key half][buffer]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = wave / 4, rw = wave % 4, tid_h = tid % kHalfThreads;
  const int r = lane & 15, kap = lane >> 4;
  const int64_t h = w / p.row_blocks;
  const int64_t row0 = (w % p.row_blocks) * kMqRows + rw * kRowsPerWave;

  // query rows of this wave as the B operand of S^T = K Q^T (bf16/fp16 -> fp16 is
  // exact for these magnitudes; the softmax scale is applied to the fp32 logits);
  // rows are contiguous 128-element vectors, read 16 bytes at a time
  h8 qf[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int64_t row = row0 + 16 * qb + r;
    const bool ok = row < p.rows;
    const uint32_t gq = ok ? fast_div(static_cast<uint32_t>(row), p.lq) : 0;
    const int64_t g = gq, i = ok ? row - int64_t(gq) * p.Lq : 0;
    const int64_t base = (i * p.Hq + h * p.group + g) * kD;
    const uint16_t *q16 = static_cast<const uint16_t *>(it.query) + base + 8 * kap;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      qf[qb][kb] = halves_to_h8<QD>(ok ? *reinterpret_cast<const uint4 *>(q16 + 32 * kb) : make_uint4(0, 0, 0, 0));
  }

  MqState st;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) st.o[qb][cb] = f4{0, 0, 0, 0};
    st.m[qb] = kNegInf;
    st.l[qb] = 0.0f;
  }

  const int64_t head_bytes = p.keys_pad * kD * 2;
  const Rsrc rk = make_rsrc(p.wk + h * p.keys_pad * kD, head_bytes);
  const Rsrc rv = make_rsrc(p.wv + h * kD * p.keys_pad, head_bytes);
  const int n_tiles = static_cast<int>(p.keys_pad / kTile);
  const int n0 = (n_tiles + 1) / 2;                 // tiles of the first half (the longer one)
  const int first = half ? n0 : 0;
  const int count = half ? n_tiles - n0 : n0;
  MqTile *buf = sh[half];
  TileRegs tr;
  if (count > 0) {
    load_tile(tr, rk, rv, p.keys_pad, int64_t(first) * kTile, tid_h);
    store_tile(buf[0], tr, tid_h);
  }
  __syncthreads();
  for (int i = 0; i < n0; ++i) {  // both halves step together: the barrier is shared
    const bool active = i < count, more = i + 1 < count;
    if (more) load_tile(tr, rk, rv, p.keys_pad, int64_t(first + i + 1) * kTile, tid_h);
    if (active) {
      const int valid = static_cast<int>(min<int64_t>(kTile, p.keys - int64_t(first + i) * kTile));
      compute_tile(buf[i & 1], qf, valid, p.scale_log2, st);
    }
    if (more) store_tile(buf[(i + 1) & 1], tr, tid_h);  // that buffer was last read in tile i-1
    __syncthreads();
  }

  // merge: the second half hands (O^T, m, l) of its lanes to the wave with the
  // same rows in the first half
  float *mg = reinterpret_cast<float *>(&sh[1][0]) + rw * kMergeFloats * kWave;
  static_assert(sizeof(float) * kMergeFloats * kWave * 4 <= sizeof(MqTile) * 2, "merge fits the second half");
  if (half == 1) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
      for (int cb = 0; cb < 8; ++cb)
#pragma unroll
        for (int v = 0; v < 4; ++v) mg[((qb * 8 + cb) * 4 + v) * kWave + lane] = st.o[qb][cb][v];
      mg[(64 + qb) * kWave + lane] = st.m[qb];
      mg[(66 + qb) * kWave + lane] = st.l[qb];
    }
  }
  __syncthreads();
  typedef typename DtypeOf<OD>::T OutT;
  constexpr int kRowPad = kD + 8;
  OutT *ob = reinterpret_cast<OutT *>(&sh[0][0]) + rw * kRowsPerWave * kRowPad;
  static_assert(sizeof(OutT) * kMqRows * kRowPad <= sizeof(MqTile) * 2, "output staging fits the first half");
  if (half == 0) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const float m2 = mg[(64 + qb) * kWave + lane], l2 = mg[(66 + qb) * kWave + lane];
      const float M = fmaxf(st.m[qb], m2);
      const float M_ref = M == kNegInf ? 0.0f : M;
      const float a1 = fast_exp2(st.m[qb] - M_ref), a2 = fast_exp2(m2 - M_ref);
      const float l = sum_over_slices(st.l[qb] * a1 + l2 * a2);
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
      for (int cb = 0; cb < 8; ++cb)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float o = st.o[qb][cb][v] * a1 + mg[((qb * 8 + cb) * 4 + v) * kWave + lane] * a2;
          store_from_f32<OD>(ob, (16 * qb + r) * kRowPad + 16 * cb + 4 * kap + v, o * inv);
        }
      const int64_t row = row0 + 16 * qb + r;
      if (kap == 0 && row < p.rows && it.lse != nullptr) {
        // (h * group + g) * Lq + i = h * rows + row
        it.lse[h * p.rows + row] = l > 0.0f ? (M + log2f(l)) * kLn2 : kNegInf;
      }
    }
  }
  __syncthreads();
  if (half == 0) {
    constexpr int kChunk = 16 / sizeof(OutT);  // elements per 16-byte store
    constexpr int kPerRow = kD / kChunk;
#pragma unroll
    for (int q = 0; q < kRowsPerWave * kPerRow / kWave; ++q) {
      const int idx = q * kWave + lane, rr = idx / kPerRow, cc = (idx % kPerRow) * kChunk;
      const int64_t row = row0 + rr;
      if (row >= p.rows) continue;
      const uint32_t gq = fast_div(static_cast<uint32_t>(row), p.lq);
      const int64_t g = gq, i = row - int64_t(gq) * p.Lq;
      *reinterpret_cast<uint4 *>(static_cast<OutT *>(it.out) + (i * p.Hq + h * p.group + g) * kD + cc) =
          *reinterpret_cast<const uint4 *>(&ob[rr * kRowPad + cc]);
    }
  }
}

// Workgroups are dealt to the 8 XCDs round-robin by launch index; work item w
// goes to index 8 * (w % per_xcd) + w / per_xcd, so each XCD serves a
// contiguous run of row blocks -- mostly of one KV head of one segment, whose
// staged keys and values its own L2 then holds.
template <int QD, int OD>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void mq_attention_kernel(
    uc_kivi_item it, MqParams p) {
  const int64_t id = blockIdx.x, w = (id % kXcds) * p.per_xcd + id / kXcds;
  if (w >= p.row_blocks * p.Hkv) return;  // uniform: the whole workgroup leaves
  mq_attention_body<QD, OD>(it, p, w);
}

template <int QD, int OD>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void mq_attention_batch_kernel(
    MqBatch b) {
  const int64_t w = blockIdx.x;
  const int i = batch_item(b.attn_begin, b.n, w);
  mq_attention_body<QD, OD>(b.it[i], b.p[i], w - b.attn_begin[i]);
}

}  // namespace
}  // namespace uc

using namespace uc;

extern "C" int64_t uc_kivi_mq_workspace_bytes(int64_t heads_kv, int64_t head_dim, int64_t quantized_tokens,
                                              int64_t residual_tokens) {
  if (heads_kv <= 0 || head_dim <= 0 || quantized_tokens < 0 || residual_tokens < 0) return -1;
  const int64_t keys_pad = ceil_div(quantized_tokens + residual_tokens, int64_t(kTile)) * kTile;
  return heads_kv * keys_pad * head_dim * 2 * int64_t(sizeof(_Float16));
}

namespace uc {
namespace {

template <int V>
using IC = std::integral_constant<int, V>;

// Calls f(IC<bits>, IC<group>, IC<residual dtype>) for the stage kernels.
template <class F>
void stage_config(int bits, int group_size, int res_dtype, F &&f) {
  auto by_rd = [&](auto b, auto g) {
    if (res_dtype == UC_FP16) f(b, g, IC<UC_FP16>{});
    else f(b, g, IC<UC_BF16>{});
  };
  auto by_group = [&](auto b) {
    if (group_size == 32) by_rd(b, IC<32>{});
    else if (group_size == 64) by_rd(b, IC<64>{});
    else by_rd(b, IC<128>{});
  };
  if (bits == 2) by_group(IC<2>{});
  else by_group(IC<4>{});
}

// Calls f(IC<query dtype>, IC<out dtype>) for the attention kernels.
template <class F>
void attn_config(int q_dtype, int out_dtype, F &&f) {
  auto by_out = [&](auto qd) {
    if (out_dtype == UC_BF16) f(qd, IC<UC_BF16>{});
    else if (out_dtype == UC_FP16) f(qd, IC<UC_FP16>{});
    else f(qd, IC<UC_FP32>{});
  };
  if (q_dtype == UC_FP16) by_out(IC<UC_FP16>{});
  else by_out(IC<UC_BF16>{});
}

int mq_check_config(int bits, int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim, int q_dtype,
                    int res_dtype, int out_dtype) {
  UC_REQUIRE(bits == 2 || bits == 4, "attn_mq: bits must be 2 or 4 (got %d)", bits);
  UC_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
             "attn_mq: group_size must be 32, 64 or 128 (got %d)", group_size);
  UC_REQUIRE(head_dim == mf::kD, "attn_mq: head_dim must be 128 (got %lld)", (long long)head_dim);
  UC_REQUIRE(heads_kv > 0 && heads_q > 0 && heads_q % heads_kv == 0,
             "attn_mq: query heads (%lld) must be a multiple of KV heads (%lld)", (long long)heads_q,
             (long long)heads_kv);
  UC_REQUIRE((q_dtype == UC_BF16 || q_dtype == UC_FP16) && (res_dtype == UC_BF16 || res_dtype == UC_FP16),
             "attn_mq: query and residual must be bf16 or fp16");
  UC_REQUIRE(out_dtype == UC_BF16 || out_dtype == UC_FP16 || out_dtype == UC_FP32, "attn_mq: bad out dtype");
  return UC_OK;
}

int mq_check_item(const uc_kivi_item &it, int group_size, int64_t heads_q, int64_t heads_kv, int64_t query_len) {
  UC_REQUIRE(query_len > 0 && query_len * (heads_q / heads_kv) < (int64_t(1) << 31),
             "attn_mq: query_len must be positive and query rows per KV head below 2^31");
  UC_REQUIRE(it.quantized_tokens >= 0 && it.residual_tokens >= 0 && it.quantized_tokens % group_size == 0,
             "attn_mq: quantized tokens must be a non-negative multiple of group_size");
  UC_REQUIRE(it.quantized_tokens + it.residual_tokens > 0, "attn_mq: empty segment");
  UC_REQUIRE(it.packed_capacity == 0 ||
                 (it.packed_capacity >= it.quantized_tokens && it.packed_capacity % group_size == 0),
             "attn_mq: packed_capacity must be 0 or a multiple of group_size >= quantized_tokens");
  UC_REQUIRE(it.query != nullptr && it.out != nullptr, "attn_mq: query/out are NULL");
  UC_REQUIRE((reinterpret_cast<uintptr_t>(it.query) & 15) == 0 && (reinterpret_cast<uintptr_t>(it.out) & 15) == 0,
             "attn_mq: query and out must be 16-byte aligned");
  UC_REQUIRE(it.quantized_tokens == 0 || (it.key_code && it.key_scale && it.key_min && it.value_code &&
                                          it.value_scale && it.value_min),
             "attn_mq: packed tensors are NULL");
  UC_REQUIRE(it.residual_tokens == 0 || (it.residual_key && it.residual_value), "attn_mq: residual is NULL");
  const int64_t keys_pad = ceil_div(it.quantized_tokens + it.residual_tokens, int64_t(kTile)) * kTile;
  UC_REQUIRE(keys_pad * mf::kD * 2 < (int64_t(1) << 31) && it.quantized_tokens * 64 < (int64_t(1) << 31),
             "attn_mq: segment too long for 32-bit buffer offsets");
  return UC_OK;
}

// Stage and attention parameters of one segment whose staged K and V start at ws.
void mq_fill(const uc_kivi_item &it, int64_t heads_q, int64_t heads_kv, int64_t query_len, float sm_scale,
             _Float16 *ws, StageParams &sp, MqParams &p) {
  sp = StageParams{};
  sp.Hkv = heads_kv;
  sp.keys = it.quantized_tokens + it.residual_tokens;
  sp.keys_pad = ceil_div(sp.keys, int64_t(kTile)) * kTile;
  sp.wk = ws;
  sp.wv = ws + heads_kv * sp.keys_pad * mf::kD;
  p = MqParams{};
  p.Hq = heads_q;
  p.Hkv = heads_kv;
  p.Lq = query_len;
  p.group = heads_q / heads_kv;
  p.rows = p.group * query_len;
  p.keys = sp.keys;
  p.keys_pad = sp.keys_pad;
  p.scale_log2 = sm_scale * kLog2e;
  p.wk = sp.wk;
  p.wv = sp.wv;
  p.row_blocks = ceil_div(p.rows, int64_t(kMqRows));
  p.lq = make_fastdiv(static_cast<uint32_t>(query_len));
  p.per_xcd = ceil_div(p.row_blocks * heads_kv, int64_t(kXcds));
}

}  // namespace
}  // namespace uc

extern "C" int uc_kivi_attn_mq(const uc_kivi_item *item_host, int bits, int group_size, int64_t heads_q,
                               int64_t heads_kv, int64_t head_dim, int64_t query_len, int q_dtype, int res_dtype,
                               int out_dtype, float sm_scale, void *workspace, int64_t workspace_bytes,
                               uc_stream_t stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  UC_REQUIRE(item_host != nullptr, "attn_mq: item is NULL");
  const uc_kivi_item it = *item_host;
  int rc = mq_check_config(bits, group_size, heads_q, heads_kv, head_dim, q_dtype, res_dtype, out_dtype);
  if (rc != UC_OK) return rc;
  rc = mq_check_item(it, group_size, heads_q, heads_kv, query_len);
  if (rc != UC_OK) return rc;
  const int64_t need = uc_kivi_mq_workspace_bytes(heads_kv, head_dim, it.quantized_tokens, it.residual_tokens);
  UC_REQUIRE(workspace != nullptr && workspace_bytes >= need, "attn_mq: workspace too small (%lld < %lld bytes)",
             (long long)workspace_bytes, (long long)need);
  StageParams sp;
  MqParams p;
  mq_fill(it, heads_q, heads_kv, query_len, sm_scale, static_cast<_Float16 *>(workspace), sp, p);
  const dim3 sgrid(static_cast<unsigned>(sp.keys_pad / kTile), static_cast<unsigned>(heads_kv),
                   static_cast<unsigned>(kMqThreads / kStageThreads));
  stage_config(bits, group_size, res_dtype, [&](auto b, auto g, auto rd) {
    hipLaunchKernelGGL((mq_stage_kernel<decltype(b)::value, decltype(g)::value, decltype(rd)::value>), sgrid,
                       dim3(kStageThreads), 0, stream, it, sp);
  });
  rc = check_launch("attn_mq (stage)");
  if (rc != UC_OK) return rc;
  const dim3 grid(static_cast<unsigned>(p.per_xcd * kXcds));
  attn_config(q_dtype, out_dtype, [&](auto qd, auto od) {
    hipLaunchKernelGGL((mq_attention_kernel<decltype(qd)::value, decltype(od)::value>), grid, dim3(kAttnThreads), 0,
                       stream, it, p);
  });
  return check_launch("attn_mq");
}

extern "C" int uc_kivi_attn_mq_batch(const uc_kivi_item *items_host, const int64_t *query_lens, int n_items,
                                     int bits, int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                                     int q_dtype, int res_dtype, int out_dtype, float sm_scale, void *workspace,
                                     int64_t workspace_bytes, uc_stream_t stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  UC_REQUIRE(n_items >= 1 && n_items <= kMqMaxBatch, "attn_mq_batch: n_items must be 1..%d (got %d)", kMqMaxBatch,
             n_items);
  UC_REQUIRE(items_host != nullptr && query_lens != nullptr, "attn_mq_batch: items or query_lens is NULL");
  int rc = mq_check_config(bits, group_size, heads_q, heads_kv, head_dim, q_dtype, res_dtype, out_dtype);
  if (rc != UC_OK) return rc;
  int64_t need = 0;
  for (int i = 0; i < n_items; ++i) {
    rc = mq_check_item(items_host[i], group_size, heads_q, heads_kv, query_lens[i]);
    if (rc != UC_OK) return rc;
    need += uc_kivi_mq_workspace_bytes(heads_kv, head_dim, items_host[i].quantized_tokens,
                                       items_host[i].residual_tokens);
  }
  UC_REQUIRE(workspace != nullptr && workspace_bytes >= need,
             "attn_mq_batch: workspace too small (%lld < %lld bytes)", (long long)workspace_bytes, (long long)need);
  // longest segments first: their work items start first on every XCD
  int order[kMqMaxBatch];
  for (int i = 0; i < n_items; ++i) order[i] = i;
  const auto keys_of = [&](int i) { return items_host[i].quantized_tokens + items_host[i].residual_tokens; };
  for (int i = 1; i < n_items; ++i)
    for (int j = i; j > 0 && keys_of(order[j]) > keys_of(order[j - 1]); --j) std::swap(order[j], order[j - 1]);
  MqBatch b{};
  b.n = n_items;
  _Float16 *ws = static_cast<_Float16 *>(workspace);
  for (int i = 0; i < n_items; ++i) {
    const int src = order[i];
    b.it[i] = items_host[src];
    mq_fill(items_host[src], heads_q, heads_kv, query_lens[src], sm_scale, ws, b.sp[i], b.p[i]);
    ws += 2 * heads_kv * b.sp[i].keys_pad * mf::kD;  // staged K and V of segment i
    b.stage_begin[i + 1] = b.stage_begin[i] + b.sp[i].keys_pad / kTile;
    b.attn_begin[i + 1] = b.attn_begin[i] + b.p[i].row_blocks * heads_kv;
  }
  UC_REQUIRE(b.stage_begin[n_items] < (int64_t(1) << 31) && b.attn_begin[n_items] < (int64_t(1) << 31),
             "attn_mq_batch: launch too large");
  const dim3 sgrid(static_cast<unsigned>(b.stage_begin[n_items]), static_cast<unsigned>(heads_kv),
                   static_cast<unsigned>(kMqThreads / kStageThreads));
  stage_config(bits, group_size, res_dtype, [&](auto bb, auto g, auto rd) {
    hipLaunchKernelGGL((mq_stage_batch_kernel<decltype(bb)::value, decltype(g)::value, decltype(rd)::value>), sgrid,
                       dim3(kStageThreads), 0, stream, b);
  });
  rc = check_launch("attn_mq_batch (stage)");
  if (rc != UC_OK) return rc;
  const dim3 grid(static_cast<unsigned>(b.attn_begin[n_items]));
  attn_config(q_dtype, out_dtype, [&](auto qd, auto od) {
    hipLaunchKernelGGL((mq_attention_batch_kernel<decltype(qd)::value, decltype(od)::value>), grid,
                       dim3(kAttnThreads), 0, stream, b);
  });
  return check_launch("attn_mq_batch");
}
