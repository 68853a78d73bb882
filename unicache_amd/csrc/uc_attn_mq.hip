// Multi-query attention over one KIVI-packed segment plus its dense keys
// (head_dim 128, 2/4-bit codes): the long-query case of UniCache's packed
// attention (image editing: ~1088 queries x 7 query heads per KV head).
//
// Two kernels.  mq_stage_kernel dequantizes the packed prefix of every KV head
// once into a workspace of fp16 rows, keys and values alike [Hkv][Tq][128]
// (code * scale + minimum in fp32, then one rounding to fp16); the ~60 query
// blocks of a head then read fp16 rows instead of re-dequantizing the codes.
// The dense keys (the segment's residual, or the bf16 tokens riding with it)
// are not copied: the attention kernel reads their [T, Hkv, 128] rows where
// they lie.
//
// mq_attention_kernel: one workgroup (8 waves) owns 128 query rows of one KV
// head; waves 0-3 take the first half of the 64-key tiles and waves 4-7 the
// second, 32 query rows per wave.  Tiles of keys and values stream into
// double-buffered LDS slots by buffer-to-LDS loads (no registers held), one
// barrier per tile, and each wave runs
//   S^T = K Q^T    (v_mfma_f32_16x16x32, rows = keys, columns = queries),
//   online base-2 softmax over the key rows against a lazily raised reference,
//   O^T += V^T P^T (v_mfma_f32_16x16x32; the V^T fragments come straight from
//                   the value rows through the transposing LDS read
//                   ds_read_b64_tr_b16, P^T straight from the S^T accumulators).
// Prefix tiles use fp16 operands.  Dense tiles use the dense keys' own dtype:
// bf16 tokens enter the matrix cores unrounded and keep their range.
// Output: normalised O (written through LDS as whole rows) and the natural-log
// LSE.
#include <type_traits>
#include <utility>

#include "uc_common.h"
#include "uc_mfma.h"

namespace uc {
namespace {

using namespace mf;

typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __fp16 lds_h4 __attribute__((ext_vector_type(4)));
// Fragments as clang vectors (natural alignment, kept whole in registers).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16x16x32 MFMA on eight 16-bit operands per lane of dtype DT (raw bits), and
// the rounding of fp32 probabilities to that dtype (nearest even).
template <int DT>
struct Mma;
template <>
struct Mma<UC_FP16> {
  static __device__ __forceinline__ f4 run(u32x4 a, u32x4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ u32x2 pack(f4 v) { return __builtin_bit_cast(u32x2, cvt4(v)); }
  // c + the two packed elements of x, in fp32
  static __device__ __forceinline__ float sum2(uint32_t x, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x), h2{to_h(1.0f), to_h(1.0f)}, c, false);
  }
};
template <>
struct Mma<UC_BF16> {
  static __device__ __forceinline__ f4 run(u32x4 a, u32x4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0,
                                                   0);
  }
  static __device__ __forceinline__ u32x2 pack(f4 v) {
    return __builtin_bit_cast(u32x2, __builtin_convertvector(v, bf4));
  }
  static __device__ __forceinline__ float sum2(uint32_t x, float c) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, x), bf2{__bf16(1.0f), __bf16(1.0f)}, c, false);
  }
};

// Eight 16-bit elements of dtype FROM as dtype TO (identity when equal).
template <int FROM, int TO>
__device__ __forceinline__ u32x4 convert8(u32x4 raw) {
  if constexpr (FROM == TO) {
    return raw;
  } else {
    const uint32_t w[4] = {raw[0], raw[1], raw[2], raw[3]};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = half_bits_to_f32<FROM>(w[j]), hi = half_bits_to_f32<FROM>(w[j] >> 16);
      o[j] = TO == UC_BF16 ? (uint32_t(f32_to_bf16_bits(lo)) | (uint32_t(f32_to_bf16_bits(hi)) << 16))
                           : (uint32_t(f32_to_f16_bits(lo)) | (uint32_t(f32_to_f16_bits(hi)) << 16));
    }
    return u32x4{o[0], o[1], o[2], o[3]};
  }
}

constexpr int kXcds = 8;  // XCDs of an MI355X; launch index i runs on XCD i % 8
constexpr int kTile = 64;  // keys per tile
constexpr int kHalfWaves = 4;
constexpr int kAttnWaves = 2 * kHalfWaves;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kRowsPerWave = 32;
constexpr int kMqRows = kHalfWaves * kRowsPerWave;  // query rows per workgroup
constexpr int kStageThreads = kWave;
constexpr int kStageSplit = 4;  // one-wave workgroups per (tile, KV head) of the stage pass
// The reference of a query column is raised only when a logit exceeds it by
// more than kSlack (log2 units): probabilities stay below 2^kSlack, and most
// tiles need no rescale of the output accumulators.
constexpr float kSlack = 8.0f;

// One 64-key tile in LDS: 64 rows of 256 B (16 chunks of 16 B) of keys and of
// values.  Key row t keeps chunk c at position c ^ (t & 15): the 16 rows one
// key fragment read touches (16 lanes, one chunk each) sit in 16 different
// bank groups.  Value row t keeps chunk c at position c ^ (2t & 15): a
// transposing read of 32 lanes covers 8 rows x 32 B, which then fill all 64
// banks once.
constexpr int kSlotBytes = 2 * kTile * 256;
constexpr int kValueBytes = kTile * 256;  // values start after the keys of a slot
constexpr int kMergeFloats = 2 * 8 * 4 + 4;  // O^T (2 query blocks x 8 channel blocks x 4) + m[2], l[2]
constexpr int kRowPad = kD + 8;              // output staging row, in elements
struct MqShared {
  union {
    uint32_t slot[2][2][kSlotBytes / 4];  // [key half][buffer]: the tiles
    struct {                              // after the last tile:
      float mg[kHalfWaves][kMergeFloats * kWave];  // (O^T, m, l) of the second half's waves
      uint32_t ob[kMqRows * kRowPad];              // normalised output rows (fp32 size)
    } ep;
  };
};
static_assert(sizeof(MqShared) <= 160 * 1024, "fits the LDS of a workgroup");

struct MqParams {
  int64_t Hq, Hkv, Lq, group, rows;  // rows = group * Lq query rows per KV head
  int64_t Tq, Tr;                    // packed prefix and dense tokens
  int nq, nd;                        // their 64-key tiles
  float scale_log2;
  const _Float16 *wk, *wv;           // staged prefix rows [Hkv][Tq][128]
  int64_t row_blocks, per_xcd;       // row blocks per KV head; work items per XCD
  FastDiv lq;                        // row -> (query head of the group, query position)
};

struct StageParams {
  int64_t Tq;
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

// ------------------------------------------------------------- stage pass --
// Workgroup (tile, KV head, quarter): tokens [64*tile, 64*tile + 64) of the
// packed prefix; the tile's 256 work items are spread over kStageSplit
// one-wave workgroups (blockIdx.z).  Arithmetic as uc_kivi_dequant: a rounded
// multiply and a rounded add in fp32, then the cast to fp16.
template <int BITS, int G>
__device__ __forceinline__ void mq_stage_body(const uc_kivi_item &it, const StageParams &sp, int64_t tile) {
  constexpr int TPW = 32 / BITS;        // codes per word
  constexpr int KW = kTile / TPW;       // key words per channel in a tile
  constexpr int VW = kD / TPW;          // value words per token
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const int tid = blockIdx.z * kStageThreads + threadIdx.x;
  const int64_t h = blockIdx.y;
  const int64_t t0 = tile * kTile, Tq = sp.Tq;
  const int64_t cap = it.packed_capacity > 0 ? it.packed_capacity : Tq;  // tokens between heads
  const uint32_t *kc = static_cast<const uint32_t *>(it.key_code) + h * (cap / TPW) * kD;
  const uint16_t *ks = static_cast<const uint16_t *>(it.key_scale) + h * (cap / G) * kD;
  const uint16_t *km = static_cast<const uint16_t *>(it.key_min) + h * (cap / G) * kD;
  const uint32_t *vc = static_cast<const uint32_t *>(it.value_code) + h * cap * VW;
  const uint16_t *vs = static_cast<const uint16_t *>(it.value_scale) + h * cap * (kD / G);
  const uint16_t *vm = static_cast<const uint16_t *>(it.value_min) + h * cap * (kD / G);
  uint32_t *wk = reinterpret_cast<uint32_t *>(sp.wk + h * Tq * kD);
  _Float16 *wv = sp.wv + h * Tq * kD;

  // Every load of the thread is issued before any arithmetic: the packed
  // words are cold in HBM and each thread has only a few of them.
  // keys: item (word j of the tile, channel pair cp); a wave writes whole
  // 256-byte rows, one per token of the word
  constexpr int kItems = kStageSplit * kStageThreads;
  constexpr int NK = KW * (kD / 2) / kItems, NV = kTile * VW / kItems;
  static_assert(NK >= 1 && NV >= 1 && KW * (kD / 2) % kItems == 0 && kTile * VW % kItems == 0, "stage items");
  uint2 kw[NK];
  uint32_t ks2[NK], km2[NK], vw[NV];
  uint16_t vs1[NV], vm1[NV];
#pragma unroll
  for (int q = 0; q < NK; ++q) {
    const int e = q * kItems + tid, cp = e % (kD / 2), j = e / (kD / 2);
    const int64_t t = min(t0 + j * TPW, Tq - TPW);  // first token of the word (Tq is a multiple of G >= TPW)
    const int64_t w = t / TPW, g = t / G;
    kw[q] = *reinterpret_cast<const uint2 *>(kc + w * kD + 2 * cp);
    ks2[q] = *reinterpret_cast<const uint32_t *>(ks + g * kD + 2 * cp);
    km2[q] = *reinterpret_cast<const uint32_t *>(km + g * kD + 2 * cp);
  }
#pragma unroll
  for (int q = 0; q < NV; ++q) {
    const int e = q * kItems + tid, w = e % VW;
    const int64_t t = min(t0 + e / VW, Tq - 1);
    const int g = (w * TPW) / G;
    vw[q] = vc[t * VW + w];
    vs1[q] = vs[t * (kD / G) + g];
    vm1[q] = vm[t * (kD / G) + g];
  }
#pragma unroll
  for (int q = 0; q < NK; ++q) {
    const int e = q * kItems + tid, cp = e % (kD / 2), j = e / (kD / 2);
    const int64_t t = t0 + j * TPW;
    if (t >= Tq) continue;
    const float s0 = f16_bits_to_f32(ks2[q] & 0xffffu), s1 = f16_bits_to_f32(ks2[q] >> 16);
    const float m0 = f16_bits_to_f32(km2[q] & 0xffffu), m1 = f16_bits_to_f32(km2[q] >> 16);
#pragma unroll
    for (int p = 0; p < TPW; ++p) {
      const float v0 = add_rn(mul_rn(float((kw[q].x >> (p * BITS)) & kMask), s0), m0);
      const float v1 = add_rn(mul_rn(float((kw[q].y >> (p * BITS)) & kMask), s1), m1);
      wk[(t + p) * (kD / 2) + cp] = uint32_t(f32_to_f16_bits(v0)) | (uint32_t(f32_to_f16_bits(v1)) << 16);
    }
  }
  // values: item (token of the tile, word); TPW contiguous channels out
#pragma unroll
  for (int q = 0; q < NV; ++q) {
    const int e = q * kItems + tid, w = e % VW;
    const int64_t t = t0 + e / VW;
    if (t >= Tq) continue;
    const float s = f16_bits_to_f32(vs1[q]), m = f16_bits_to_f32(vm1[q]);
    uint32_t o[TPW / 2];
#pragma unroll
    for (int p = 0; p < TPW; p += 2) {
      const float v0 = add_rn(mul_rn(float((vw[q] >> (p * BITS)) & kMask), s), m);
      const float v1 = add_rn(mul_rn(float((vw[q] >> ((p + 1) * BITS)) & kMask), s), m);
      o[p / 2] = uint32_t(f32_to_f16_bits(v0)) | (uint32_t(f32_to_f16_bits(v1)) << 16);
    }
    uint4 *dst = reinterpret_cast<uint4 *>(wv + t * kD + w * TPW);
#pragma unroll
    for (int q2 = 0; q2 < TPW / 8; ++q2) dst[q2] = make_uint4(o[4 * q2], o[4 * q2 + 1], o[4 * q2 + 2], o[4 * q2 + 3]);
  }
}

template <int BITS, int G>
__global__ __launch_bounds__(kStageThreads) void mq_stage_kernel(uc_kivi_item it, StageParams sp) {
  mq_stage_body<BITS, G>(it, sp, blockIdx.x);
}

template <int BITS, int G>
__global__ __launch_bounds__(kStageThreads) void mq_stage_batch_kernel(MqBatch b) {
  const int64_t tile = blockIdx.x;
  const int i = batch_item(b.stage_begin, b.n, tile);
  mq_stage_body<BITS, G>(b.it[i], b.sp[i], tile - b.stage_begin[i]);
}

// --------------------------------------------------------- attention pass --
// Output is kept transposed (O^T = V^T P^T) so that every lane owns one query
// column: the softmax rescale needs no cross-lane traffic.
struct MqState {
  f4 o[2][8];        // [query block][channel block]: lane (n, k) -> query n, channels 16*cb + 4k + v
  float m[2], l[2];  // lane (n, k): reference of query n (log2 units); l = this lane's share of the sum
};

// The rows of one KV head in one key source: the staged prefix (fp16 rows of
// 256 B) or the dense keys and values ([T, Hkv, 128] rows Hkv * 256 B apart).
struct RowSrc {
  Rsrc k, v;
  uint32_t row_bytes;
  int64_t rows;
};

__device__ __forceinline__ RowSrc make_src(const void *k, const void *v, int64_t rows, int64_t row_bytes) {
  RowSrc s;
  const int64_t bytes = rows > 0 ? (rows - 1) * row_bytes + kD * 2 : 0;
  s.k = make_rsrc(k, bytes);
  s.v = make_rsrc(v, bytes);
  s.row_bytes = static_cast<uint32_t>(row_bytes);
  s.rows = rows;
  return s;
}

// Lane part of the buffer-to-LDS loads of the source: lane L of the wave's
// load j lands in tile row 16 * hw + 4 * j + L / 16 at chunk position L % 16
// and so fetches source chunk (L % 16) ^ (row & 15) for keys and
// (L % 16) ^ (2 row & 15) for values; row & 15 = 4j + L/16.  Offsets of load
// j: key base ^ 64 j, value base ^ 128 (j & 1).
struct DmaLane {
  uint32_t kbase, vbase;
};

__device__ __forceinline__ DmaLane dma_lane(uint32_t row_bytes) {
  const uint32_t lane = threadIdx.x & 63, rq = lane >> 4, c = lane & 15;
  return DmaLane{rq * row_bytes + 16u * (c ^ rq), rq * row_bytes + 16u * (c ^ (2u * rq))};
}

// Tile rows [r0, r0 + valid) of `src` into `slot` (keys, then values); wave hw
// of the half fills tile rows 16 hw .. 16 hw + 15.  Rows past `valid` repeat
// the last valid row, so every value row that meets a zero probability holds
// finite data.
__device__ __forceinline__ void issue_tile(uint4 *slot, const RowSrc &src, const DmaLane &dl, int64_t r0, int valid,
                                           int hw) {
  typedef __attribute__((address_space(3))) void *lds_ptr;
  const uint32_t lane = threadIdx.x & 63;
  if (valid == kTile) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t so = static_cast<uint32_t>(r0 + 16 * hw + 4 * j) * src.row_bytes;
      uint4 *dst = slot + (16 * hw + 4 * j) * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.k, (lds_ptr)dst, 16, dl.kbase ^ (64u * j), so, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.v, (lds_ptr)(dst + kValueBytes / 16), 16,
                                               dl.vbase ^ (128u * (j & 1)), so, 0, 0);
    }
  } else {
    uint32_t ln = lane;  // recomputed here, not kept from the loop's start
    asm volatile("" : "+v"(ln));
    const uint32_t so = static_cast<uint32_t>(r0) * src.row_bytes, c = ln & 15;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t row = 16 * hw + 4 * j + (ln >> 4), rl = row & 15;
      const uint32_t base = min(row, static_cast<uint32_t>(valid - 1)) * src.row_bytes;
      uint4 *dst = slot + (16 * hw + 4 * j) * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.k, (lds_ptr)dst, 16, base + 16u * (c ^ rl), so, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.v, (lds_ptr)(dst + kValueBytes / 16), 16,
                                               base + 16u * (c ^ ((2u * rl) & 15u)), so, 0, 0);
    }
  }
}

// LDS byte addresses of the fragment reads in buffer 0 of the wave's half
// (buffer 1 adds kSlotBytes):
//   key fragment (tb, kb): row 16 tb + n, chunk 4 kb + k (lane (n, k)), at
//     position (4 kb + k) ^ n: ak[kb] + 4096 tb;
//   V^T fragment (tp, hi, cb) by ds_read_b64_tr_b16: lane i of 16-lane group k
//     names row 32 tp + 16 hi + 4 k + i / 4, channels 16 cb + 4 (i % 4) .. + 3,
//     and receives channel 16 cb + i of rows 32 tp + 16 hi + 4 k .. + 3:
//     av[cb] + 8192 tp + 4096 hi.
struct FragLane {
  uint32_t ak[4], av[8];
};

__device__ __forceinline__ FragLane frag_lane(uint32_t half_base) {
  const uint32_t lane = threadIdx.x & 63, n = lane & 15, k = lane >> 4;
  FragLane f;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) f.ak[kb] = half_base + n * 256u + 16u * ((4u * kb + k) ^ n);
  const uint32_t row = 4 * k + n / 4;  // row within the 16-row run
  const uint32_t y2 = row & 7;         // (2 row & 15) / 2: the swizzle of chunk pairs
#pragma unroll
  for (int cb = 0; cb < 8; ++cb)
    f.av[cb] = half_base + kValueBytes + row * 256u + 32u * (cb ^ y2) + 16u * ((n >> 1) & 1u) + 8u * (n & 1u);
  return f;
}

typedef __attribute__((address_space(3))) const u32x4 *lds_u4p;
typedef __attribute__((address_space(3))) lds_h4 *lds_h4p;

__device__ __forceinline__ u32x4 read_k(uint32_t addr) { return *(lds_u4p)(uintptr_t)addr; }

__device__ __forceinline__ u32x2 read_vt(uint32_t addr) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_h4p)(uintptr_t)addr));
}

// One tile: logits, lazy online softmax, P.V for the wave's 32 query rows,
// operands of dtype DT.
template <int DT, int BUF>
__device__ __forceinline__ void compute_tile(FragLane fl, const u32x4 (&qf)[2][4], int valid, float scale_log2,
                                             MqState &st) {
  constexpr uint32_t kBuf = BUF * kSlotBytes;
  // opaque to loop-invariant code motion: the constant parts of the addresses
  // below stay next to their reads and fold into the instructions' offsets
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+v"(fl.ak[kb]));
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) asm volatile("" : "+v"(fl.av[cb]));
  using Op = Mma<DT>;
  const int lane = threadIdx.x & 63;
  const int kap = lane >> 4;
  f4 acc[4][2];  // [tb][qb]: lane (n, k) -> keys 16 tb + 4 k + v of query 16 qb + n
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) acc[tb][qb] = f4{0, 0, 0, 0};
  // The two waves of a SIMD run the same phases at the same time; the wave in
  // a matrix-core phase takes issue priority over the one in the softmax, so
  // whichever gets ahead keeps the matrix cores fed.
  __builtin_amdgcn_s_setprio(3);
  // key fragments of k-block kb+1 are read while the MFMAs of kb run
  u32x4 ka[2][4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) ka[0][tb] = read_k(fl.ak[0] + kBuf + 4096 * tb);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    if (kb + 1 < 4) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) ka[(kb + 1) & 1][tb] = read_k(fl.ak[kb + 1] + kBuf + 4096 * tb);
    }
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) acc[tb][qb] = Op::run(ka[kb & 1][tb], qf[qb][kb], acc[tb][qb]);
  }
  __builtin_amdgcn_s_setprio(0);
  if (valid < kTile) {  // keys past the end of the source do not exist
    int k4 = 4 * kap;  // key 16 tb + 4 k + v exists while 4 k < valid - 16 tb - v
    asm volatile("" : "+v"(k4));
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (k4 >= valid - 16 * tb - v) acc[tb][0][v] = acc[tb][1][v] = kNegInf;
  }
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float mx = kNegInf;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int v = 0; v < 4; ++v) mx = fmaxf(mx, acc[tb][qb][v]);
    mx = max_over_slices(mx) * scale_log2;  // the column's tile max, log2 units
    if (__any(mx > st.m[qb] + kSlack)) {    // some column outgrew its reference: move it to the tile max
      // (a wave-uniform branch; inside it every lane scales, by 1 where nothing moved)
      const float m_new = fmaxf(st.m[qb], mx);
      const float alpha = m_new == st.m[qb] ? 1.0f : fast_exp2(st.m[qb] - m_new);  // 0 while nothing is accumulated
      st.l[qb] *= alpha;
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) st.o[qb][cb] *= alpha;
      st.m[qb] = m_new;
    }
  }
  // probabilities, rounded to the operand dtype; the row sums add the rounded
  // values (the weights P.V uses) with fp32 dot products
  u32x2 pp[4][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float m_ref = st.m[qb] == kNegInf ? 0.0f : st.m[qb];
    float sum = st.l[qb];  // reduced over the k-slices once, at the end
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      f4 e;
#pragma unroll
      for (int v = 0; v < 4; ++v) e[v] = fast_exp2(__builtin_fmaf(acc[tb][qb][v], scale_log2, -m_ref));
      pp[tb][qb] = Op::pack(e);
      sum = Op::sum2(pp[tb][qb][0], Op::sum2(pp[tb][qb][1], sum));
    }
    st.l[qb] = sum;
  }
  __builtin_amdgcn_s_setprio(3);
#pragma unroll
  for (int tp = 0; tp < 2; ++tp) {
    // B: P^T of the 32 keys 32 tp .. 32 tp + 31, two 4-key runs per k-slice
    u32x4 ap[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) ap[qb] = u32x4{pp[2 * tp][qb][0], pp[2 * tp][qb][1], pp[2 * tp + 1][qb][0],
                                                  pp[2 * tp + 1][qb][1]};
    // A: 16 channels x the same 8 keys of each k-slice, all eight channel
    // blocks read before the MFMAs
    u32x4 va[8];
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const u32x2 lo = read_vt(fl.av[cb] + kBuf + 8192 * tp);
      const u32x2 hi = read_vt(fl.av[cb] + kBuf + 8192 * tp + 4096);
      va[cb] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) st.o[qb][cb] = Op::run(va[cb], ap[qb], st.o[qb][cb]);
    // keep the 16 LDS reads ahead of the 16 MFMAs (the scheduler otherwise
    // pairs each read with its MFMAs and waits on every read)
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
  }
  __builtin_amdgcn_s_setprio(0);
}

// Query fragments of the wave's rows, raw (dtype QD), as the B operand of
// S^T = K Q^T: lane (n, k) holds row row0 + 16 qb + n, channels 32 kb + 8 k ..
// + 7.  Rows past the end are zero.
__device__ __forceinline__ void load_queries(u32x4 (&qf)[2][4], const uc_kivi_item &it, const MqParams &p, int64_t h,
                                             int64_t row0) {
  const int lane = threadIdx.x & 63, r = lane & 15, kap = lane >> 4;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int64_t row = row0 + 16 * qb + r;
    const bool ok = row < p.rows;
    const uint32_t gq = ok ? fast_div(static_cast<uint32_t>(row), p.lq) : 0;
    const int64_t g = gq, i = ok ? row - int64_t(gq) * p.Lq : 0;
    const uint16_t *q16 = static_cast<const uint16_t *>(it.query) + (i * p.Hq + h * p.group + g) * kD + 8 * kap;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      qf[qb][kb] = ok ? *reinterpret_cast<const u32x4 *>(q16 + 32 * kb) : u32x4{0, 0, 0, 0};
  }
}

template <int FROM, int TO>
__device__ __forceinline__ void convert_queries(u32x4 (&qf)[2][4]) {
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) qf[qb][kb] = convert8<FROM, TO>(qf[qb][kb]);
}

// Work item w = h * row_blocks + rb of one segment: 128 query rows of KV head h.
// Tiles [0, nq) are the staged prefix (fp16), tiles [nq, nq + nd) the dense
// keys (dtype RD).
template <int QD, int RD, int OD>
__device__ __forceinline__ void mq_attention_body(const uc_kivi_item &it, const MqParams &p, int64_t w) {
  __shared__ __align__(16) MqShared sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: tile choices stay scalar
  const int half = wave / kHalfWaves, hw = wave % kHalfWaves;
  const int r = lane & 15, kap = lane >> 4;
  const int64_t h = w / p.row_blocks;
  const int64_t row0 = (w % p.row_blocks) * kMqRows + hw * kRowsPerWave;

  const RowSrc pre = make_src(p.wk + h * p.Tq * kD, p.wv + h * p.Tq * kD, p.Tq, kD * 2);
  const RowSrc den = p.Tr > 0 ? make_src(static_cast<const uint16_t *>(it.residual_key) + h * kD,
                                         static_cast<const uint16_t *>(it.residual_value) + h * kD, p.Tr,
                                         p.Hkv * kD * 2)
                              : pre;
  const int n_tiles = p.nq + p.nd;
  const int n0 = (n_tiles + 1) / 2;  // tiles of the first half (the longer one)
  const int first = half ? n0 : 0;
  const int count = half ? n_tiles - n0 : n0;
  const uint32_t sh_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char *)&sh));
  const FragLane fl = frag_lane(sh_base + half * 2 * kSlotBytes);

  MqState st;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) st.o[qb][cb] = f4{0, 0, 0, 0};
    st.m[qb] = kNegInf;
    st.l[qb] = 0.0f;
  }

  // tile t: its source, first source row and valid rows
  auto tile_src = [&](int t, int64_t &r0, int &valid) -> const RowSrc & {
    const bool d = t >= p.nq;
    r0 = int64_t(d ? t - p.nq : t) * kTile;
    valid = static_cast<int>(min<int64_t>(kTile, (d ? p.Tr : p.Tq) - r0));
    return d ? den : pre;
  };
  const DmaLane dl_pre = dma_lane(pre.row_bytes), dl_den = dma_lane(den.row_bytes);
  auto issue = [&](int t, int buf) {
    int64_t r0;
    int valid;
    const RowSrc &s = tile_src(t, r0, valid);
    issue_tile(reinterpret_cast<uint4 *>(sh.slot[half][buf]), s, t >= p.nq ? dl_den : dl_pre, r0, valid, hw);
  };
  // The first half loads the rows' query fragments and hands them to the
  // wave with the same rows in the second half through LDS (buffer 1 of the
  // first half, free until step 0), so each query row is read once.
  u32x4 qf[2][4];
  if (count > 0) issue(first, 0);
  {
    u32x4 *qs = reinterpret_cast<u32x4 *>(sh.slot[0][1]) + hw * 8 * kWave + lane;
    if (half == 0) {
      load_queries(qf, it, p, h, row0);
#pragma unroll
      for (int j = 0; j < 8; ++j) qs[j * kWave] = qf[j / 4][j % 4];
    }
    __syncthreads();
    if (half == 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[j / 4][j % 4] = qs[j * kWave];
    }
  }
  const bool dense_first = first >= p.nq;  // this half starts with dense tiles
  if (dense_first) convert_queries<QD, RD>(qf);
  else convert_queries<QD, UC_FP16>(qf);

  // Step i: wait for tile first + i, start loading tile first + i + 1 into
  // the other buffer, compute tile first + i (steps past `count` only keep
  // the barrier count of the two halves equal).
  auto step = [&](int i, auto dt_tag, auto buf_tag) {
    constexpr int DT = decltype(dt_tag)::value, BUF = decltype(buf_tag)::value;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's loads of tile i are in LDS
    __syncthreads();                     // ... and everyone's; buffer BUF ^ 1 is free again
    if (i + 1 < count) issue(first + i + 1, BUF ^ 1);
    if (i < count) {
      int64_t r0;
      int valid;
      tile_src(first + i, r0, valid);
      compute_tile<DT, BUF>(fl, qf, valid, p.scale_log2, st);
    }
  };
  // steps [i, end) with operands of dtype DT, buffer i & 1, two per round
  int i = 0;
  auto run = [&](auto dt_tag, int end) {
    if (i < end && (i & 1)) step(i++, dt_tag, std::integral_constant<int, 1>{});
    for (; i + 1 < end; i += 2) {
      step(i, dt_tag, std::integral_constant<int, 0>{});
      step(i + 1, dt_tag, std::integral_constant<int, 1>{});
    }
    if (i < end) step(i++, dt_tag, std::integral_constant<int, 0>{});
  };
  // both halves run n0 steps (the barrier is shared): the prefix tiles of this
  // half with fp16 operands, then its dense tiles in their own dtype (the
  // fp16 fragments go back to the dense dtype: exact when it is fp16, and for
  // bf16 queries whose values fp16 holds)
  const int n_pre = static_cast<int>(max(0, min(count, p.nq - first)));
  run(std::integral_constant<int, UC_FP16>{}, n_pre);
  if (n_pre < count && !dense_first) convert_queries<UC_FP16, RD>(qf);
  run(std::integral_constant<int, RD>{}, n0);
  __syncthreads();  // every wave is done reading its last tile

  // merge: the second half hands (O^T, m, l) of its lanes to the wave with the
  // same rows in the first half
  float *mg = sh.ep.mg[hw];
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
  OutT *ob = reinterpret_cast<OutT *>(sh.ep.ob) + hw * kRowsPerWave * kRowPad;
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
  {  // each half writes 16 of the 32 rows
    constexpr int kChunk = 16 / sizeof(OutT);  // elements per 16-byte store
    constexpr int kPerRow = kD / kChunk;
    const OutT *obw = reinterpret_cast<const OutT *>(sh.ep.ob) + hw * kRowsPerWave * kRowPad;
#pragma unroll
    for (int q = 0; q < kRowsPerWave / 2 * kPerRow / kWave; ++q) {
      const int idx = q * kWave + lane, rr = half * (kRowsPerWave / 2) + idx / kPerRow, cc = (idx % kPerRow) * kChunk;
      const int64_t row = row0 + rr;
      if (row >= p.rows) continue;
      const uint32_t gq = fast_div(static_cast<uint32_t>(row), p.lq);
      const int64_t g = gq, i = row - int64_t(gq) * p.Lq;
      *reinterpret_cast<uint4 *>(static_cast<OutT *>(it.out) + (i * p.Hq + h * p.group + g) * kD + cc) =
          *reinterpret_cast<const uint4 *>(&obw[rr * kRowPad + cc]);
    }
  }
}

// Workgroups are dealt to the 8 XCDs round-robin by launch index; work item w
// goes to index 8 * (w % per_xcd) + w / per_xcd, so each XCD serves a
// contiguous run of row blocks -- mostly of one KV head of one segment, whose
// keys and values its own L2 then holds.
template <int QD, int RD, int OD>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void mq_attention_kernel(
    uc_kivi_item it, MqParams p) {
  const int64_t id = blockIdx.x, w = (id % kXcds) * p.per_xcd + id / kXcds;
  if (w >= p.row_blocks * p.Hkv) return;  // uniform: the whole workgroup leaves
  mq_attention_body<QD, RD, OD>(it, p, w);
}

template <int QD, int RD, int OD>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void mq_attention_batch_kernel(
    MqBatch b) {
  const int64_t w = blockIdx.x;
  const int i = batch_item(b.attn_begin, b.n, w);
  mq_attention_body<QD, RD, OD>(b.it[i], b.p[i], w - b.attn_begin[i]);
}

}  // namespace
}  // namespace uc

using namespace uc;

extern "C" int64_t uc_kivi_mq_workspace_bytes(int64_t heads_kv, int64_t head_dim, int64_t quantized_tokens,
                                              int64_t residual_tokens) {
  if (heads_kv <= 0 || head_dim <= 0 || quantized_tokens < 0 || residual_tokens < 0) return -1;
  return 2 * heads_kv * quantized_tokens * head_dim * int64_t(sizeof(_Float16));
}

namespace uc {
namespace {

template <int V>
using IC = std::integral_constant<int, V>;

// Calls f(IC<bits>, IC<group>) for the stage kernels.
template <class F>
void stage_config(int bits, int group_size, F &&f) {
  auto by_group = [&](auto b) {
    if (group_size == 32) f(b, IC<32>{});
    else if (group_size == 64) f(b, IC<64>{});
    else f(b, IC<128>{});
  };
  if (bits == 2) by_group(IC<2>{});
  else by_group(IC<4>{});
}

// Calls f(IC<query dtype>, IC<dense dtype>, IC<out dtype>) for the attention kernels.
template <class F>
void attn_config(int q_dtype, int res_dtype, int out_dtype, F &&f) {
  auto by_out = [&](auto qd, auto rd) {
    if (out_dtype == UC_BF16) f(qd, rd, IC<UC_BF16>{});
    else if (out_dtype == UC_FP16) f(qd, rd, IC<UC_FP16>{});
    else f(qd, rd, IC<UC_FP32>{});
  };
  auto by_res = [&](auto qd) {
    if (res_dtype == UC_FP16) by_out(qd, IC<UC_FP16>{});
    else by_out(qd, IC<UC_BF16>{});
  };
  if (q_dtype == UC_FP16) by_res(IC<UC_FP16>{});
  else by_res(IC<UC_BF16>{});
}

int mq_check_config(int bits, int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim, int q_dtype,
                    int res_dtype, int out_dtype, float sm_scale) {
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
  UC_REQUIRE(sm_scale > 0.0f && sm_scale < __builtin_inff(), "attn_mq: sm_scale must be positive and finite");
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
  UC_REQUIRE(it.residual_tokens == 0 || ((reinterpret_cast<uintptr_t>(it.residual_key) & 15) == 0 &&
                                         (reinterpret_cast<uintptr_t>(it.residual_value) & 15) == 0),
             "attn_mq: residual keys and values must be 16-byte aligned");
  // buffer offsets are 32-bit: a head's staged rows and the dense rows' span
  UC_REQUIRE(it.quantized_tokens * mf::kD * 2 < (int64_t(1) << 31) &&
                 it.residual_tokens * heads_kv * mf::kD * 2 < (int64_t(1) << 31),
             "attn_mq: segment too long for 32-bit buffer offsets");
  return UC_OK;
}

// Stage and attention parameters of one segment whose staged K and V start at ws.
void mq_fill(const uc_kivi_item &it, int64_t heads_q, int64_t heads_kv, int64_t query_len, float sm_scale,
             _Float16 *ws, StageParams &sp, MqParams &p) {
  sp = StageParams{};
  sp.Tq = it.quantized_tokens;
  sp.wk = ws;
  sp.wv = ws + heads_kv * sp.Tq * mf::kD;
  p = MqParams{};
  p.Hq = heads_q;
  p.Hkv = heads_kv;
  p.Lq = query_len;
  p.group = heads_q / heads_kv;
  p.rows = p.group * query_len;
  p.Tq = it.quantized_tokens;
  p.Tr = it.residual_tokens;
  p.nq = static_cast<int>(ceil_div(p.Tq, int64_t(kTile)));
  p.nd = static_cast<int>(ceil_div(p.Tr, int64_t(kTile)));
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
  int rc = mq_check_config(bits, group_size, heads_q, heads_kv, head_dim, q_dtype, res_dtype, out_dtype, sm_scale);
  if (rc != UC_OK) return rc;
  rc = mq_check_item(it, group_size, heads_q, heads_kv, query_len);
  if (rc != UC_OK) return rc;
  const int64_t need = uc_kivi_mq_workspace_bytes(heads_kv, head_dim, it.quantized_tokens, it.residual_tokens);
  UC_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need &&
                           (reinterpret_cast<uintptr_t>(workspace) & 15) == 0),
             "attn_mq: workspace too small or misaligned (%lld < %lld bytes)", (long long)workspace_bytes,
             (long long)need);
  StageParams sp;
  MqParams p;
  mq_fill(it, heads_q, heads_kv, query_len, sm_scale, static_cast<_Float16 *>(workspace), sp, p);
  if (p.nq > 0) {
    const dim3 sgrid(static_cast<unsigned>(p.nq), static_cast<unsigned>(heads_kv), kStageSplit);
    stage_config(bits, group_size, [&](auto b, auto g) {
      hipLaunchKernelGGL((mq_stage_kernel<decltype(b)::value, decltype(g)::value>), sgrid, dim3(kStageThreads), 0,
                         stream, it, sp);
    });
    rc = check_launch("attn_mq (stage)");
    if (rc != UC_OK) return rc;
  }
  const dim3 grid(static_cast<unsigned>(p.per_xcd * kXcds));
  attn_config(q_dtype, res_dtype, out_dtype, [&](auto qd, auto rd, auto od) {
    hipLaunchKernelGGL((mq_attention_kernel<decltype(qd)::value, decltype(rd)::value, decltype(od)::value>), grid,
                       dim3(kAttnThreads), 0, stream, it, p);
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
  int rc = mq_check_config(bits, group_size, heads_q, heads_kv, head_dim, q_dtype, res_dtype, out_dtype, sm_scale);
  if (rc != UC_OK) return rc;
  int64_t need = 0;
  for (int i = 0; i < n_items; ++i) {
    rc = mq_check_item(items_host[i], group_size, heads_q, heads_kv, query_lens[i]);
    if (rc != UC_OK) return rc;
    need += uc_kivi_mq_workspace_bytes(heads_kv, head_dim, items_host[i].quantized_tokens,
                                       items_host[i].residual_tokens);
  }
  UC_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need &&
                           (reinterpret_cast<uintptr_t>(workspace) & 15) == 0),
             "attn_mq_batch: workspace too small or misaligned (%lld < %lld bytes)", (long long)workspace_bytes,
             (long long)need);
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
    ws += 2 * heads_kv * b.sp[i].Tq * mf::kD;  // staged K and V of segment i
    b.stage_begin[i + 1] = b.stage_begin[i] + b.p[i].nq;
    b.attn_begin[i + 1] = b.attn_begin[i] + b.p[i].row_blocks * heads_kv;
  }
  UC_REQUIRE(b.stage_begin[n_items] < (int64_t(1) << 31) && b.attn_begin[n_items] < (int64_t(1) << 31),
             "attn_mq_batch: launch too large");
  if (b.stage_begin[n_items] > 0) {
    const dim3 sgrid(static_cast<unsigned>(b.stage_begin[n_items]), static_cast<unsigned>(heads_kv), kStageSplit);
    stage_config(bits, group_size, [&](auto bb, auto g) {
      hipLaunchKernelGGL((mq_stage_batch_kernel<decltype(bb)::value, decltype(g)::value>), sgrid,
                         dim3(kStageThreads), 0, stream, b);
    });
    rc = check_launch("attn_mq_batch (stage)");
    if (rc != UC_OK) return rc;
  }
  const dim3 grid(static_cast<unsigned>(b.attn_begin[n_items]));
  attn_config(q_dtype, res_dtype, out_dtype, [&](auto qd, auto rd, auto od) {
    hipLaunchKernelGGL((mq_attention_batch_kernel<decltype(qd)::value, decltype(rd)::value, decltype(od)::value>),
                       grid, dim3(kAttnThreads), 0, stream, b);
  });
  return check_launch("attn_mq_batch");
}
