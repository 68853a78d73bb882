// Multi-query attention over KIVI-packed segments and dense 16-bit segments
// (head_dim 128, 2/4-bit codes): the long-query case of UniCache's packed
// attention (image editing: ~1088 queries x 7 query heads per KV head), one
// softmax over every segment of a query in one launch.
//
// mq_attention_kernel: one workgroup (8 waves) owns 128 query rows of one KV
// head; waves 0-3 take half of the 64-key tiles (half of the packed tiles,
// then part of the dense ones) and waves 4-7 the rest, 32 query rows per wave.
// A tile's keys and values reach double-buffered LDS slots as fp16 or 16-bit
// dense rows in one swizzled layout, one barrier per tile:
//   packed tiles: the half's 256 threads load the tile's code words and fp16
//     scales and minima into registers (issued before the previous tile's
//     math), dequantize them (code * scale + minimum, one fp16 fma) and write
//     the key and value rows -- the codes are read from HBM, never staged;
//   dense tiles: buffer-to-LDS loads of the rows where they lie (any token
//     and head stride), no registers held.
// Then each wave runs
//   S^T = K Q^T    (v_mfma_f32_16x16x32, rows = keys, columns = queries),
//   online base-2 softmax over the key rows against a lazily raised reference,
//   O^T += V^T P^T (v_mfma_f32_16x16x32; the V^T fragments come straight from
//                   the value rows through the transposing LDS read
//                   ds_read_b64_tr_b16, P^T straight from the S^T accumulators).
// Packed tiles use fp16 operands.  Dense tiles use the dense keys' own dtype:
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
constexpr int kHalfThreads = kHalfWaves * kWave;
constexpr int kAttnWaves = 2 * kHalfWaves;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kRowsPerWave = 32;
constexpr int kMqRows = kHalfWaves * kRowsPerWave;  // query rows per workgroup
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

// ------------------------------------------------------------ launch table --
// Everything a launch needs travels by value in the kernel arguments: up to
// kMqMaxQueries queries, each attending its own run of packed and dense
// segments of the table.
constexpr int kMqMaxQueries = 8;
constexpr int kMqMaxPacked = 8;
constexpr int kMqMaxDense = 16;

// A packed prefix: head 0 of the six native tensors (token-major words,
// packed_capacity tokens between heads) and its token count.
struct PackedSeg {
  const char *kc, *ks, *km, *vc, *vs, *vm;
  int64_t cap;
  int tokens;  // a multiple of the group size
};

// A dense segment: key row (token t, head h) at k + t * tok_bytes + h * head_bytes.
struct DenseSeg {
  const char *k, *v;
  int64_t tok_bytes, head_bytes;
  int tokens;
};

struct MqQuery {
  const void *query;  // [Lq, Hq, 128]
  void *out;          // [Lq, Hq, 128]
  float *lse;         // [Hq, Lq] or null
  int64_t Lq, rows;   // rows = group * Lq query rows per KV head
  FastDiv lq;         // row -> (query head of the group, query position)
  int row_blocks;     // 128-row blocks per KV head
  int per_xcd;        // work items (row block x KV head) per XCD
  int slot0;          // the query's first launch slot on every XCD
  int p0, np, d0, nd;  // its packed segments [p0, p0 + np) and dense ones [d0, d0 + nd)
  int pt, dt;          // its packed and dense 64-key tiles
};

struct MqTable {
  PackedSeg ps[kMqMaxPacked];
  DenseSeg ds[kMqMaxDense];
  MqQuery q[kMqMaxQueries];
  int n_queries, Hkv, group, gshift;  // gshift = log2(group size)
  int64_t Hq;
  float scale_log2;
};
static_assert(sizeof(MqTable) <= 4096, "the launch table fits the kernel argument space");

struct TileRef {
  int seg, r0, valid;  // segment, first token, tokens of the tile that exist
};

// A pointer the compiler must treat as wave-uniform (buffer resources are
// scalar: a value it cannot prove uniform would cost a loop over the lanes).
__device__ __forceinline__ const char *uniform_ptr(const char *p) {
  const uint64_t x = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x >> 32));
  return reinterpret_cast<const char *>((uint64_t(hi) << 32) | lo);
}

// Tile f of a run of segments of `tokens` tokens each (uniform scan).
template <class Seg>
__device__ __forceinline__ TileRef find_tile(const Seg *segs, int first, int n, int f) {
  int s = first;
  const int last = first + n - 1;
  while (s < last) {
    const int tiles = (segs[s].tokens + kTile - 1) / kTile;
    if (f < tiles) break;
    f -= tiles;
    ++s;
  }
  const int r0 = f * kTile;
  return TileRef{s, r0, min(kTile, segs[s].tokens - r0)};
}

// ---------------------------------------------------------- packed tiles --
// A half's 256 threads turn the codes of one packed 64-token tile into fp16
// key and value rows in the tile's LDS slot.
//   Keys: thread (cb = tid % 16, tq = tid / 16) writes tokens 4 tq .. 4 tq + 3,
//     channels 8 cb .. 8 cb + 7 (one chunk per token): it loads the eight
//     channels' words of the word row holding those tokens and their fp16
//     scale and minimum pairs.  A byte permute puts the four tokens' codes of
//     two channels into the two 16-bit halves of one register; each code pair
//     is OR-ed into the mantissa of 1024, 1024 is subtracted exactly and one
//     packed fp16 fma applies scale and minimum.  The 16 lanes of a store hit
//     one whole row: no bank conflict.
//   Values: thread (c8 = tid % 8, t = tid / 8) writes channels 16 c8 ..
//     16 c8 + 15 (two chunks) of tokens t and t + 32 from one word pair (4-bit)
//     or word (2-bit) per token and the token's scale and minimum.  Even and
//     odd channels are split into two registers whose bytes a permute
//     interleaves, giving code pairs (2j, 2j + 1) of a chunk.  A thread stores
//     its chunks 2 c8 and 2 c8 + 1 in the order given by bit 2 of c8 and the
//     token's parity: each 8 lanes of a store then cover 8 chunk positions
//     that differ modulo 8, and each 16 lanes all 16 -- no bank conflict
//     whether the LDS serves 128 or 256 bytes of a store per cycle.
// Rows past the end of the segment repeat the last valid word row or token:
// finite values under a probability of exactly zero.
template <int BITS>
struct PackedRegs;
template <>
struct PackedRegs<2> {
  u32x4 kw[2], ks, km;       // 8 key words; 8 scales and 8 minima (fp16 pairs)
  uint32_t vw[2];            // value word of tokens t and t + 32
  uint32_t vs[2], vm[2];     // the aligned dwords holding their fp16 scale and minimum
  uint32_t vhi;              // bit k: token k's stats are the dword's upper half
};
template <>
struct PackedRegs<4> {
  u32x4 kw[2], ks, km;
  u32x2 vw[2];               // value word pair of tokens t and t + 32
  uint32_t vs[2], vm[2];
  uint32_t vhi;
};

// Lane constants of the dequantizing stores (slot-relative LDS byte offsets).
struct DeqLane {
  uint32_t ksel;      // permute selector: the thread's four tokens of two channels
  uint32_t kaddr[4];  // key chunk of token 4 tq + i
  uint32_t vsel[2];   // 2-bit: permute selector of store b; 4-bit: word of store b
  uint32_t vaddr[2];  // value chunk of store b, token t (token t + 32: + 8192)
};

template <int BITS>
__device__ __forceinline__ DeqLane deq_lane(int tid_h) {
  constexpr int TPW = 32 / BITS;
  const uint32_t cb = tid_h & 15, tq = tid_h >> 4;
  const uint32_t a = 4 * (tq % (TPW / 4));  // first token of the thread within its word
  DeqLane d;
  if constexpr (BITS == 2)  // byte a/4 of each channel's word: tokens a .. a+3
    d.ksel = (a / 4) | (0x0cu << 8) | ((4 + a / 4) << 16) | (0x0cu << 24);
  else  // bytes a/2, a/2+1: tokens a .. a+3
    d.ksel = (a / 2) | ((a / 2 + 1) << 8) | ((4 + a / 2) << 16) | ((5 + a / 2) << 24);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t row = 4 * tq + i;
    d.kaddr[i] = row * 256u + 16u * (cb ^ (row & 15u));
  }
  const uint32_t c8 = tid_h & 7, t = tid_h >> 3, flip = ((c8 >> 2) ^ t) & 1;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const uint32_t half8 = flip ^ b;  // store b writes chunk 2 c8 + half8
    d.vsel[b] = BITS == 2 ? (half8 ? 0x07060302u : 0x05040100u) : half8;
    d.vaddr[b] = kValueBytes + t * 256u + 16u * ((2 * c8 + half8) ^ ((2 * t) & 15u));
  }
  return d;
}

// One KV head of a packed segment: the first byte of each tensor's rows and
// the token count.
struct PackedHead {
  const char *kc, *ks, *km, *vc, *vs, *vm;
  int tokens;
};

template <int BITS>
__device__ __forceinline__ PackedHead packed_head(const PackedSeg &ps, int64_t h, int gshift) {
  constexpr int TPW = 32 / BITS, VW = kD / TPW;
  const int64_t cap = ps.cap, vstat = (kD >> gshift) * 2;
  return PackedHead{ps.kc + h * (cap / TPW) * 512, ps.ks + h * (cap >> gshift) * 256,
                    ps.km + h * (cap >> gshift) * 256, ps.vc + h * cap * VW * 4,
                    ps.vs + h * cap * vstat,        ps.vm + h * cap * vstat,
                    ps.tokens};
}

// Loads of the packed tile of rows [r0, r0 + valid) of head `ph` into registers.
template <int BITS>
__device__ __forceinline__ void load_packed(PackedRegs<BITS> &pr, const PackedHead &ph, int r0, int valid, int gshift,
                                            int tid_h) {
  constexpr int TPW = 32 / BITS, VW = kD / TPW;
  const int64_t Tq = ph.tokens;
  const int vstat = (kD >> gshift) * 2;  // bytes of a token's value stats
  const Rsrc kc = make_rsrc(ph.kc, (Tq / TPW) * 512);
  const Rsrc ks = make_rsrc(ph.ks, (Tq >> gshift) * 256);
  const Rsrc km = make_rsrc(ph.km, (Tq >> gshift) * 256);
  const Rsrc vc = make_rsrc(ph.vc, Tq * VW * 4);
  const Rsrc vs = make_rsrc(ph.vs, Tq * vstat);
  const Rsrc vm = make_rsrc(ph.vm, Tq * vstat);
  const uint32_t cb = tid_h & 15, tq = tid_h >> 4;
  const uint32_t tqc = min(tq, static_cast<uint32_t>(valid / 4 - 1));  // last existing token quad
  // keys: word row jc of the tile, channels 8 cb ..; stats of token r0 + 4 tqc
  // (r0 is a multiple of 64, so its group offset separates for every group size)
  const uint32_t jc = tqc / (TPW / 4);
  const int kso = (r0 / TPW) * 512;
  const uint32_t kvo = jc * 512u + 32u * cb;
  pr.kw[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kc, kvo, kso, 0));
  pr.kw[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kc, kvo + 16u, kso, 0));
  const int sso = (r0 >> gshift) * 256;
  const uint32_t svo = ((4u * tqc) >> gshift) * 256u + 16u * cb;
  pr.ks = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ks, svo, sso, 0));
  pr.km = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(km, svo, sso, 0));
  // values: tokens t and t + 32 (the latter clamped), channels 16 c8 ..
  const uint32_t c8 = tid_h & 7, t = tid_h >> 3;
  const uint32_t t1 = min(t + 32u, static_cast<uint32_t>(valid - 1));
  const int vso = r0 * VW * 4, vsso = r0 * vstat;
  const uint32_t g = (16u * c8) >> gshift;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t tok = k ? t1 : t;
    if constexpr (BITS == 2)
      pr.vw[k] = __builtin_amdgcn_raw_buffer_load_b32(vc, tok * (VW * 4) + 4u * c8, vso, 0);
    else
      pr.vw[k] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(vc, tok * (VW * 4) + 8u * c8, vso, 0));
    // the stats' dword (the tensors' sizes are multiples of 4 bytes, so the
    // aligned dword stays in range): no 16-bit load, whose widening would
    // wait for the load right away
    const uint32_t so = tok * vstat + 2u * g;
    pr.vs[k] = __builtin_amdgcn_raw_buffer_load_b32(vs, so & ~3u, vsso, 0);
    pr.vm[k] = __builtin_amdgcn_raw_buffer_load_b32(vm, so & ~3u, vsso, 0);
    if (k == 0) pr.vhi = (so >> 1) & 1u;
    else pr.vhi |= so & 2u;
  }
}

// code pair (low BITS of each 16-bit half of x) -> code * scale + minimum.
// `magic` holds 0x64006400 in a register, so that mask and OR are one
// v_and_or_b32 (an instruction takes one literal).
template <int BITS>
__device__ __forceinline__ uint32_t deq2(uint32_t x, h2 s, h2 m, uint32_t magic) {
  constexpr uint32_t mask = ((1u << BITS) - 1u) * 0x00010001u;
  const h2 c = as_h2((x & mask) | magic) - h2{to_h(1024.0f), to_h(1024.0f)};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, s, m));
}

typedef __attribute__((address_space(3))) u32x4 *lds_u4w;

__device__ __forceinline__ void write_chunk(uint32_t addr, u32x4 v) { *(lds_u4w)(uintptr_t)addr = v; }

// Dequantize the key (store_keys) or value (store_values) registers into the
// slot at LDS byte address `slot`.
template <int BITS>
__device__ __forceinline__ void store_keys(const PackedRegs<BITS> &pr, int tid_h, uint32_t slot, uint32_t magic) {
  DeqLane dl = deq_lane<BITS>(tid_h);
  u32x4 o[4];  // [token i][channel pair]
#pragma unroll
  for (int pi = 0; pi < 4; ++pi) {
    const uint32_t w0 = pr.kw[pi >> 1][2 * (pi & 1)], w1 = pr.kw[pi >> 1][2 * (pi & 1) + 1];
    const uint32_t u = __builtin_amdgcn_perm(w1, w0, dl.ksel);
    const h2 s = as_h2(pr.ks[pi]), m = as_h2(pr.km[pi]);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i][pi] = deq2<BITS>(u >> (BITS * i), s, m, magic);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) write_chunk(slot + dl.kaddr[i], o[i]);
}

template <int BITS>
__device__ __forceinline__ void store_values(const PackedRegs<BITS> &pr, int tid_h, uint32_t slot, uint32_t magic) {
  DeqLane dl = deq_lane<BITS>(tid_h);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    // the token's fp16 scale and minimum in both halves
    const uint32_t sel = 0x01000100u + ((pr.vhi >> k) & 1u) * 0x02020202u;
    const h2 s = as_h2(__builtin_amdgcn_perm(pr.vs[k], pr.vs[k], sel));
    const h2 m = as_h2(__builtin_amdgcn_perm(pr.vm[k], pr.vm[k], sel));
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      u32x4 o;
      if constexpr (BITS == 2) {
        // channel 2j at bits 4j of ye, 2j+1 at bits 4j of yo; the permute
        // takes the chunk's half of both
        const uint32_t w = pr.vw[k];
        const uint32_t ye = w & 0x33333333u, yo = (w >> 2) & 0x33333333u;
        const uint32_t z = __builtin_amdgcn_perm(yo, ye, dl.vsel[b]);
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = deq2<2>(z >> (4 * j), s, m, magic);
      } else {
        // one word per chunk: channel 2j at byte j of ye, 2j+1 at byte j of yo
        const uint32_t w = dl.vsel[b] ? pr.vw[k][1] : pr.vw[k][0];
        const uint32_t ye = w & 0x0f0f0f0fu, yo = (w >> 4) & 0x0f0f0f0fu;
        const uint32_t za = __builtin_amdgcn_perm(yo, ye, 0x05040100u), zb = __builtin_amdgcn_perm(yo, ye, 0x07060302u);
        o[0] = deq2<4>(za, s, m, magic);
        o[1] = deq2<4>(za >> 8, s, m, magic);
        o[2] = deq2<4>(zb, s, m, magic);
        o[3] = deq2<4>(zb >> 8, s, m, magic);
      }
      write_chunk(slot + dl.vaddr[b] + 8192u * k, o);
    }
  }
}

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
// operands of dtype DT.  With HOOK, hook(tp) adds independent vector work
// (the next tile's dequantization) that is interleaved with the 16 P.V MFMAs
// of key half tp, so that it issues while the matrix cores are busy.
template <int DT, int BUF, bool HOOK, class Hook>
__device__ __forceinline__ void compute_tile(FragLane fl, const u32x4 (&qf)[2][4], int valid, float scale_log2,
                                             MqState &st, Hook &&hook) {
  constexpr uint32_t kBuf = BUF * kSlotBytes;
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
    if constexpr (HOOK) {
      hook(tp);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x200, 4, 0);
    } else {
      __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
    }
  }
  __builtin_amdgcn_s_setprio(0);
}

// Query fragments of the wave's rows, raw (dtype QD), as the B operand of
// S^T = K Q^T: lane (n, k) holds row row0 + 16 qb + n, channels 32 kb + 8 k ..
// + 7.  Rows past the end are zero.
__device__ __forceinline__ void load_queries(u32x4 (&qf)[2][4], const MqQuery &Q, const MqTable &tb, int64_t h,
                                             int64_t row0) {
  const int lane = threadIdx.x & 63, r = lane & 15, kap = lane >> 4;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int64_t row = row0 + 16 * qb + r;
    const bool ok = row < Q.rows;
    const uint32_t gq = ok ? fast_div(static_cast<uint32_t>(row), Q.lq) : 0;
    const int64_t g = gq, i = ok ? row - int64_t(gq) * Q.Lq : 0;
    const uint16_t *q16 = static_cast<const uint16_t *>(Q.query) + (i * tb.Hq + h * tb.group + g) * kD + 8 * kap;
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

// Work item of query Q: 128 query rows (row block rb) of KV head h over every
// segment of the query.  Each half takes half of the packed tiles (fp16
// operands) and then dense tiles (dtype RD) up to n0 = ceil(tiles / 2) for
// the first half.
template <int BITS, int QD, int RD, int OD>
__device__ __forceinline__ void mq_attention_body(const MqTable &tb, const MqQuery &Q, int64_t h, int64_t rb) {
  __shared__ __align__(16) MqShared sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: tile choices stay scalar
  const int half = wave / kHalfWaves, hw = wave % kHalfWaves;
  const int tid_h = tid - half * kHalfThreads;
  const int r = lane & 15, kap = lane >> 4;
  const int64_t row0 = rb * kMqRows + hw * kRowsPerWave;

  const int n_tiles = Q.pt + Q.dt, n0 = (n_tiles + 1) / 2;
  const int q0 = (Q.pt + 1) / 2, d0 = n0 - q0;  // the first half's packed and dense tiles
  const int pb = half ? q0 : 0, db = half ? d0 : 0;
  const int n_pre = half ? Q.pt - q0 : q0;
  const int count = n_pre + (half ? Q.dt - d0 : d0);
  const uint32_t sh_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char *)&sh));
  const uint32_t half_base = sh_base + half * 2 * kSlotBytes;
  const FragLane fl = frag_lane(half_base);

  MqState st;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) st.o[qb][cb] = f4{0, 0, 0, 0};
    st.m[qb] = kNegInf;
    st.l[qb] = 0.0f;
  }

  // Cursors over the half's tiles, kept in registers: the dense segment and
  // first row of the next dense tile, the packed segment (its head) and first
  // row of the next packed tile.  Segment records are read from the launch
  // table only when a cursor enters a new segment.
  int dseg = Q.d0, dr0 = 0, drows = 0, dbytes = 0;
  const char *dk = nullptr, *dv = nullptr;
  auto dense_seg = [&](int sidx) {
    const DenseSeg &ds = tb.ds[sidx];
    dk = ds.k + h * ds.head_bytes;
    dv = ds.v + h * ds.head_bytes;
    drows = ds.tokens;
    dbytes = static_cast<int>(ds.tok_bytes);
  };
  if (count > n_pre) {
    const TileRef tr = find_tile(tb.ds, Q.d0, Q.nd, db);
    dseg = tr.seg;
    dr0 = tr.r0;
    dense_seg(dseg);
  }
  // next dense tile into buffer buf; returns its valid rows
  auto issue_dense = [&](int buf) {
    const int rows = __builtin_amdgcn_readfirstlane(drows), row_bytes = __builtin_amdgcn_readfirstlane(dbytes);
    const int r0 = __builtin_amdgcn_readfirstlane(dr0);
    const RowSrc src = make_src(uniform_ptr(dk), uniform_ptr(dv), rows, row_bytes);
    const int valid = min(kTile, rows - r0);
    issue_tile(reinterpret_cast<uint4 *>(sh.slot[half][buf]), src, dma_lane(src.row_bytes), r0, valid, hw);
    dr0 = r0 + kTile;
    if (dr0 >= rows && dseg + 1 < Q.d0 + Q.nd) {
      dr0 = 0;
      dense_seg(++dseg);
    }
    return valid;
  };
  int pseg = Q.p0, pr0 = 0;
  PackedHead ph{};
  if (n_pre > 0) {
    const TileRef tr = find_tile(tb.ps, Q.p0, Q.np, pb);
    pseg = tr.seg;
    pr0 = tr.r0;
    ph = packed_head<BITS>(tb.ps[pseg], h, tb.gshift);
  }
  PackedRegs<BITS> pr;
  // loads of the next packed tile; returns its valid rows
  auto load_tile = [&]() {
    const PackedHead u{uniform_ptr(ph.kc), uniform_ptr(ph.ks), uniform_ptr(ph.km), uniform_ptr(ph.vc),
                       uniform_ptr(ph.vs), uniform_ptr(ph.vm), __builtin_amdgcn_readfirstlane(ph.tokens)};
    const int r0 = __builtin_amdgcn_readfirstlane(pr0);
    const int valid = min(kTile, u.tokens - r0);
    load_packed<BITS>(pr, u, r0, valid, tb.gshift, tid_h);
    pr0 = r0 + kTile;
    if (pr0 >= u.tokens && pseg + 1 < Q.p0 + Q.np) {
      pr0 = 0;
      ph = packed_head<BITS>(tb.ps[++pseg], h, tb.gshift);
    }
    return valid;
  };

  // The first half loads the rows' query fragments and hands them to the
  // wave with the same rows in the second half through LDS (buffer 1 of the
  // first half, free until step 0), so each query row is read once.
  uint32_t magic = 0x64006400u;  // fp16 1024 in both halves, held in a register
  asm volatile("" : "+v"(magic));
  const int n_dense = count - n_pre;
  // Each half runs its packed tiles first, then its dense ones.  The first
  // half loads the rows' query fragments and hands them to the wave with the
  // same rows in the second half through LDS (buffer 1 of the first half,
  // free until step 0), so each query row is read once.
  int cur_valid = 0;  // rows of the tile in the buffer the next step computes
  if (n_pre > 0) cur_valid = load_tile();
  else if (count > 0) cur_valid = issue_dense(0);
  u32x4 qf[2][4];
  {
    u32x4 *qs = reinterpret_cast<u32x4 *>(sh.slot[0][1]) + hw * 8 * kWave + lane;
    if (half == 0) {
      load_queries(qf, Q, tb, h, row0);
#pragma unroll
      for (int j = 0; j < 8; ++j) qs[j * kWave] = qf[j / 4][j % 4];
    }
    if (n_pre > 0) {
      store_keys<BITS>(pr, tid_h, half_base, magic);
      store_values<BITS>(pr, tid_h, half_base, magic);
    }
    __syncthreads();
    if (half == 1) {
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[j / 4][j % 4] = qs[j * kWave];
    }
  }
  if (n_pre > 0) convert_queries<QD, UC_FP16>(qf);
  else convert_queries<QD, RD>(qf);

  // Step i: wait for tile i (in buffer i & 1), start bringing tile i + 1 into
  // the other buffer (packed: its loads now, its dequantizing stores
  // interleaved with tile i's P.V MFMAs), compute tile i (steps past `count`
  // only keep the barrier count of the two halves equal).  NEXT_PACKED: tile
  // i + 1 is packed.
  auto step = [&](int i, auto dt_tag, auto buf_tag, auto packed_tag) {
    constexpr int DT = decltype(dt_tag)::value, BUF = decltype(buf_tag)::value;
    constexpr bool NEXT_PACKED = decltype(packed_tag)::value;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's loads of tile i are in LDS
    __syncthreads();                     // ... and everyone's; buffer BUF ^ 1 is free again
    int next_valid = 0;
    if constexpr (NEXT_PACKED) next_valid = load_tile();
    else if (i + 1 < count) next_valid = issue_dense(BUF ^ 1);
    const uint32_t next_slot = half_base + (BUF ^ 1) * kSlotBytes;
    auto hook = [&](int tp) {
      if (tp == 0) store_keys<BITS>(pr, tid_h, next_slot, magic);
      else store_values<BITS>(pr, tid_h, next_slot, magic);
    };
    if (i < count) {
      // a packed tile's dequantization rides in the P.V MFMAs of the
      // previous (packed) tile
      compute_tile<DT, BUF, NEXT_PACKED>(fl, qf, cur_valid, tb.scale_log2, st, hook);
    }
    cur_valid = next_valid;
  };
  // steps [i, end) with operands of dtype DT, buffer i & 1, two per round
  int i = 0;
  auto run = [&](auto dt_tag, auto packed_tag, int end) {
    if (i < end && (i & 1)) step(i++, dt_tag, std::integral_constant<int, 1>{}, packed_tag);
    for (; i + 1 < end; i += 2) {
      step(i, dt_tag, std::integral_constant<int, 0>{}, packed_tag);
      step(i + 1, dt_tag, std::integral_constant<int, 1>{}, packed_tag);
    }
    if (i < end) step(i++, dt_tag, std::integral_constant<int, 0>{}, packed_tag);
  };
  // both halves run n0 steps (the barrier is shared): the packed tiles of this
  // half with fp16 operands, then its dense tiles in their own dtype (the
  // fp16 fragments go back to the dense dtype: exact when it is fp16, and for
  // bf16 queries whose values fp16 holds)
  using F16 = std::integral_constant<int, UC_FP16>;
  using DR = std::integral_constant<int, RD>;
  run(F16{}, std::true_type{}, n_pre - 1);
  run(F16{}, std::false_type{}, n_pre);
  if (n_pre > 0 && n_dense > 0) convert_queries<UC_FP16, RD>(qf);
  run(DR{}, std::false_type{}, n0);
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
      if (kap == 0 && row < Q.rows && Q.lse != nullptr) {
        // (h * group + g) * Lq + i = h * rows + row
        Q.lse[h * Q.rows + row] = l > 0.0f ? (M + log2f(l)) * kLn2 : kNegInf;
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
      if (row >= Q.rows) continue;
      const uint32_t gq = fast_div(static_cast<uint32_t>(row), Q.lq);
      const int64_t g = gq, i = row - int64_t(gq) * Q.Lq;
      *reinterpret_cast<uint4 *>(static_cast<OutT *>(Q.out) + (i * tb.Hq + h * tb.group + g) * kD + cc) =
          *reinterpret_cast<const uint4 *>(&obw[rr * kRowPad + cc]);
    }
  }
}

// Launch slot id runs on XCD x = id % 8 as that XCD's slot j = id / 8.  Each
// query owns slots [slot0, slot0 + per_xcd) of every XCD, and XCD x serves its
// work items x * per_xcd .. (row blocks of KV head h at h * row_blocks ..): a
// contiguous run, mostly of one KV head, whose keys and values its own L2
// then holds, and one eighth of every query.  Queries come longest first.
template <int BITS, int QD, int RD, int OD>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void mq_attention_kernel(
    MqTable tb) {
  const int x = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
  int qi = 0;
  while (qi + 1 < tb.n_queries && j >= tb.q[qi + 1].slot0) ++qi;
  const MqQuery &Q = tb.q[qi];
  const int w = x * Q.per_xcd + (j - Q.slot0);
  if (w >= Q.row_blocks * tb.Hkv) return;  // uniform: the whole workgroup leaves
  mq_attention_body<BITS, QD, RD, OD>(tb, Q, w / Q.row_blocks, w % Q.row_blocks);
}

}  // namespace
}  // namespace uc

using namespace uc;

extern "C" int64_t uc_kivi_mq_workspace_bytes(int64_t heads_kv, int64_t head_dim, int64_t quantized_tokens,
                                              int64_t residual_tokens) {
  if (heads_kv <= 0 || head_dim <= 0 || quantized_tokens < 0 || residual_tokens < 0) return -1;
  return 0;  // the packed codes are dequantized inside the attention kernel
}

namespace uc {
namespace {

template <int V>
using IC = std::integral_constant<int, V>;

// Calls f(IC<bits>, IC<query dtype>, IC<dense dtype>, IC<out dtype>).
template <class F>
void attn_config(int bits, int q_dtype, int res_dtype, int out_dtype, F &&f) {
  auto by_out = [&](auto b, auto qd, auto rd) {
    if (out_dtype == UC_BF16) f(b, qd, rd, IC<UC_BF16>{});
    else if (out_dtype == UC_FP16) f(b, qd, rd, IC<UC_FP16>{});
    else f(b, qd, rd, IC<UC_FP32>{});
  };
  auto by_res = [&](auto b, auto qd) {
    if (res_dtype == UC_FP16) by_out(b, qd, IC<UC_FP16>{});
    else by_out(b, qd, IC<UC_BF16>{});
  };
  auto by_q = [&](auto b) {
    if (q_dtype == UC_FP16) by_res(b, IC<UC_FP16>{});
    else by_res(b, IC<UC_BF16>{});
  };
  if (bits == 2) by_q(IC<2>{});
  else by_q(IC<4>{});
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

constexpr int64_t kOffsetLimit = int64_t(1) << 31;  // buffer offsets are 32-bit

// Launch table under construction: segments are appended per query.
struct TableBuilder {
  MqTable t{};
  int64_t heads_q, heads_kv;
  int group_size;

  int add_packed(const uc_kivi_item &it) {
    UC_REQUIRE(it.quantized_tokens >= 0 && it.quantized_tokens % group_size == 0,
               "attn_mq: quantized tokens must be a non-negative multiple of group_size");
    if (it.quantized_tokens == 0) return UC_OK;
    UC_REQUIRE(it.packed_capacity == 0 ||
                   (it.packed_capacity >= it.quantized_tokens && it.packed_capacity % group_size == 0),
               "attn_mq: packed_capacity must be 0 or a multiple of group_size >= quantized_tokens");
    UC_REQUIRE(it.key_code && it.key_scale && it.key_min && it.value_code && it.value_scale && it.value_min,
               "attn_mq: packed tensors are NULL");
    const uintptr_t any_odd = reinterpret_cast<uintptr_t>(it.key_code) | reinterpret_cast<uintptr_t>(it.key_scale) |
                              reinterpret_cast<uintptr_t>(it.key_min) | reinterpret_cast<uintptr_t>(it.value_code) |
                              reinterpret_cast<uintptr_t>(it.value_scale) | reinterpret_cast<uintptr_t>(it.value_min);
    UC_REQUIRE((any_odd & 3) == 0, "attn_mq: packed tensors must be 4-byte aligned");
    // largest per-head extent: 4-bit value words, 64 bytes per token
    UC_REQUIRE(it.quantized_tokens * 64 < kOffsetLimit, "attn_mq: packed segment too long for 32-bit offsets");
    int n = 0;
    for (int q = 0; q < t.n_queries; ++q) n += t.q[q].np;
    UC_REQUIRE(n < kMqMaxPacked, "attn_mq: more than %d packed segments in one call", kMqMaxPacked);
    PackedSeg &s = t.ps[n];
    s.kc = static_cast<const char *>(it.key_code);
    s.ks = static_cast<const char *>(it.key_scale);
    s.km = static_cast<const char *>(it.key_min);
    s.vc = static_cast<const char *>(it.value_code);
    s.vs = static_cast<const char *>(it.value_scale);
    s.vm = static_cast<const char *>(it.value_min);
    s.cap = it.packed_capacity > 0 ? it.packed_capacity : it.quantized_tokens;
    s.tokens = static_cast<int>(it.quantized_tokens);
    MqQuery &q = t.q[t.n_queries - 1];
    ++q.np;
    q.pt += static_cast<int>(ceil_div(it.quantized_tokens, kTile));
    return UC_OK;
  }

  // dense rows; strides in bytes
  int add_dense(const void *k, const void *v, int64_t tokens, int64_t tok_bytes, int64_t head_bytes) {
    UC_REQUIRE(tokens >= 0, "attn_mq: negative dense token count");
    if (tokens == 0) return UC_OK;
    UC_REQUIRE(k != nullptr && v != nullptr, "attn_mq: dense keys or values are NULL");
    UC_REQUIRE((reinterpret_cast<uintptr_t>(k) & 15) == 0 && (reinterpret_cast<uintptr_t>(v) & 15) == 0 &&
                   tok_bytes % 16 == 0 && head_bytes % 16 == 0 && tok_bytes > 0 && head_bytes >= 0,
               "attn_mq: dense keys and values must be 16-byte aligned with 16-byte token and head strides");
    UC_REQUIRE((tokens - 1) * tok_bytes + mf::kD * 2 < kOffsetLimit,
               "attn_mq: dense segment too long for 32-bit offsets");
    int n = 0;
    for (int q = 0; q < t.n_queries; ++q) n += t.q[q].nd;
    UC_REQUIRE(n < kMqMaxDense, "attn_mq: more than %d dense segments in one call", kMqMaxDense);
    DenseSeg &s = t.ds[n];
    s.k = static_cast<const char *>(k);
    s.v = static_cast<const char *>(v);
    s.tok_bytes = tok_bytes;
    s.head_bytes = head_bytes;
    s.tokens = static_cast<int>(tokens);
    MqQuery &q = t.q[t.n_queries - 1];
    ++q.nd;
    q.dt += static_cast<int>(ceil_div(tokens, kTile));
    return UC_OK;
  }

  int begin_query(const void *query, void *out, float *lse, int64_t query_len) {
    UC_REQUIRE(t.n_queries < kMqMaxQueries, "attn_mq: more than %d queries in one call", kMqMaxQueries);
    UC_REQUIRE(query_len > 0 && query_len * (heads_q / heads_kv) < kOffsetLimit,
               "attn_mq: query_len must be positive and query rows per KV head below 2^31");
    UC_REQUIRE(query != nullptr && out != nullptr, "attn_mq: query/out are NULL");
    UC_REQUIRE((reinterpret_cast<uintptr_t>(query) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "attn_mq: query and out must be 16-byte aligned");
    UC_REQUIRE((reinterpret_cast<uintptr_t>(lse) & 3) == 0, "attn_mq: lse must be 4-byte aligned");
    int p0 = 0, d0 = 0;
    for (int q = 0; q < t.n_queries; ++q) {
      p0 += t.q[q].np;
      d0 += t.q[q].nd;
    }
    MqQuery &q = t.q[t.n_queries++];
    q = MqQuery{};
    q.query = query;
    q.out = out;
    q.lse = lse;
    q.Lq = query_len;
    q.rows = (heads_q / heads_kv) * query_len;
    q.lq = make_fastdiv(static_cast<uint32_t>(query_len));
    q.p0 = p0;
    q.d0 = d0;
    return UC_OK;
  }

  // Adds the packed prefix and residual of `it` to the current query.
  int add_item(const uc_kivi_item &it) {
    UC_REQUIRE(it.residual_tokens >= 0, "attn_mq: negative residual token count");
    int rc = add_packed(it);
    if (rc != UC_OK) return rc;
    int64_t ts, hs;
    residual_strides(it, heads_kv, mf::kD, ts, hs);
    return add_dense(it.residual_key, it.residual_value, it.residual_tokens, ts * 2, hs * 2);
  }

  int end_query() {
    MqQuery &q = t.q[t.n_queries - 1];
    UC_REQUIRE(q.pt + q.dt > 0, "attn_mq: empty segment");
    const int64_t row_blocks = ceil_div(q.rows, int64_t(kMqRows));
    UC_REQUIRE(row_blocks * heads_kv < kOffsetLimit, "attn_mq: launch too large");
    q.row_blocks = static_cast<int>(row_blocks);
    q.per_xcd = static_cast<int>(ceil_div(row_blocks * heads_kv, int64_t(kXcds)));
    return UC_OK;
  }

  // Orders the queries longest first (segments stay where they are), assigns
  // the launch slots and returns the grid size.
  int64_t finish(float sm_scale) {
    const auto work = [](const MqQuery &q) { return int64_t(q.pt + q.dt) * q.rows; };
    for (int i = 1; i < t.n_queries; ++i)
      for (int j = i; j > 0 && work(t.q[j]) > work(t.q[j - 1]); --j) std::swap(t.q[j], t.q[j - 1]);
    int slots = 0;
    for (int i = 0; i < t.n_queries; ++i) {
      t.q[i].slot0 = slots;
      slots += t.q[i].per_xcd;
    }
    t.Hkv = static_cast<int>(heads_kv);
    t.Hq = heads_q;
    t.group = static_cast<int>(heads_q / heads_kv);
    t.gshift = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
    t.scale_log2 = sm_scale * kLog2e;
    return int64_t(slots) * kXcds;
  }
};

int mq_launch(TableBuilder &b, int bits, int q_dtype, int res_dtype, int out_dtype, float sm_scale,
              hipStream_t stream, const char *what) {
  const int64_t grid = b.finish(sm_scale);
  UC_REQUIRE(grid < kOffsetLimit, "%s: launch too large", what);
  attn_config(bits, q_dtype, res_dtype, out_dtype, [&](auto bb, auto qd, auto rd, auto od) {
    hipLaunchKernelGGL((mq_attention_kernel<decltype(bb)::value, decltype(qd)::value, decltype(rd)::value,
                                            decltype(od)::value>),
                       dim3(static_cast<unsigned>(grid)), dim3(kAttnThreads), 0, stream, b.t);
  });
  return check_launch(what);
}

}  // namespace
}  // namespace uc

extern "C" int uc_kivi_attn_mq(const uc_kivi_item *item_host, int bits, int group_size, int64_t heads_q,
                               int64_t heads_kv, int64_t head_dim, int64_t query_len, int q_dtype, int res_dtype,
                               int out_dtype, float sm_scale, void *workspace, int64_t workspace_bytes,
                               uc_stream_t stream_) {
  (void)workspace;
  (void)workspace_bytes;
  UC_REQUIRE(item_host != nullptr, "attn_mq: item is NULL");
  int rc = mq_check_config(bits, group_size, heads_q, heads_kv, head_dim, q_dtype, res_dtype, out_dtype, sm_scale);
  if (rc != UC_OK) return rc;
  TableBuilder b;
  b.heads_q = heads_q;
  b.heads_kv = heads_kv;
  b.group_size = group_size;
  const uc_kivi_item &it = *item_host;
  if ((rc = b.begin_query(it.query, it.out, it.lse, query_len)) != UC_OK) return rc;
  if ((rc = b.add_item(it)) != UC_OK) return rc;
  if ((rc = b.end_query()) != UC_OK) return rc;
  return mq_launch(b, bits, q_dtype, res_dtype, out_dtype, sm_scale, static_cast<hipStream_t>(stream_), "attn_mq");
}

extern "C" int uc_kivi_attn_mq_batch(const uc_kivi_item *items_host, const int64_t *query_lens, int n_items,
                                     int bits, int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                                     int q_dtype, int res_dtype, int out_dtype, float sm_scale, void *workspace,
                                     int64_t workspace_bytes, uc_stream_t stream_) {
  (void)workspace;
  (void)workspace_bytes;
  UC_REQUIRE(n_items >= 1 && n_items <= kMqMaxQueries, "attn_mq_batch: n_items must be 1..%d (got %d)",
             kMqMaxQueries, n_items);
  UC_REQUIRE(items_host != nullptr && query_lens != nullptr, "attn_mq_batch: items or query_lens is NULL");
  int rc = mq_check_config(bits, group_size, heads_q, heads_kv, head_dim, q_dtype, res_dtype, out_dtype, sm_scale);
  if (rc != UC_OK) return rc;
  TableBuilder b;
  b.heads_q = heads_q;
  b.heads_kv = heads_kv;
  b.group_size = group_size;
  for (int i = 0; i < n_items; ++i) {
    const uc_kivi_item &it = items_host[i];
    if ((rc = b.begin_query(it.query, it.out, it.lse, query_lens[i])) != UC_OK) return rc;
    if ((rc = b.add_item(it)) != UC_OK) return rc;
    if ((rc = b.end_query()) != UC_OK) return rc;
  }
  return mq_launch(b, bits, q_dtype, res_dtype, out_dtype, sm_scale, static_cast<hipStream_t>(stream_),
                   "attn_mq_batch");
}

extern "C" int uc_kivi_attn_mq_segments(const uc_kivi_item *packed_host, int n_packed,
                                        const uc_dense_segment *dense_host, int n_dense, const void *query, void *out,
                                        float *lse, int bits, int group_size, int64_t heads_q, int64_t heads_kv,
                                        int64_t head_dim, int64_t query_len, int q_dtype, int dense_dtype,
                                        int out_dtype, float sm_scale, uc_stream_t stream_) {
  UC_REQUIRE(n_packed >= 0 && n_dense >= 0 && (n_packed == 0 || packed_host) && (n_dense == 0 || dense_host),
             "attn_mq_segments: bad segment arrays");
  int rc = mq_check_config(bits, group_size, heads_q, heads_kv, head_dim, q_dtype, dense_dtype, out_dtype, sm_scale);
  if (rc != UC_OK) return rc;
  TableBuilder b;
  b.heads_q = heads_q;
  b.heads_kv = heads_kv;
  b.group_size = group_size;
  if ((rc = b.begin_query(query, out, lse, query_len)) != UC_OK) return rc;
  for (int i = 0; i < n_packed; ++i)
    if ((rc = b.add_item(packed_host[i])) != UC_OK) return rc;
  for (int i = 0; i < n_dense; ++i) {
    const uc_dense_segment &d = dense_host[i];
    if ((rc = b.add_dense(d.key, d.value, d.tokens, d.token_stride * 2, d.head_stride * 2)) != UC_OK) return rc;
  }
  if ((rc = b.end_query()) != UC_OK) return rc;
  return mq_launch(b, bits, q_dtype, dense_dtype, out_dtype, sm_scale, static_cast<hipStream_t>(stream_),
                   "attn_mq_segments");
}

extern "C" int uc_kivi_attn_mq_table(const uc_mq_query *queries_host, int n_queries, const uc_kivi_item *packed_host,
                                     int n_packed, const uc_dense_segment *dense_host, int n_dense, int bits,
                                     int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim, int q_dtype,
                                     int dense_dtype, int out_dtype, float sm_scale, uc_stream_t stream_) {
  UC_REQUIRE(n_queries >= 1 && n_queries <= kMqMaxQueries && queries_host != nullptr,
             "attn_mq_table: n_queries must be 1..%d", kMqMaxQueries);
  UC_REQUIRE(n_packed >= 0 && n_dense >= 0 && (n_packed == 0 || packed_host) && (n_dense == 0 || dense_host),
             "attn_mq_table: bad segment arrays");
  int rc = mq_check_config(bits, group_size, heads_q, heads_kv, head_dim, q_dtype, dense_dtype, out_dtype, sm_scale);
  if (rc != UC_OK) return rc;
  TableBuilder b;
  b.heads_q = heads_q;
  b.heads_kv = heads_kv;
  b.group_size = group_size;
  for (int qi = 0; qi < n_queries; ++qi) {
    const uc_mq_query &q = queries_host[qi];
    UC_REQUIRE(q.packed_begin >= 0 && q.n_packed >= 0 && int64_t(q.packed_begin) + q.n_packed <= n_packed &&
                   q.dense_begin >= 0 && q.n_dense >= 0 && int64_t(q.dense_begin) + q.n_dense <= n_dense,
               "attn_mq_table: query %d names segments outside the arrays", qi);
    if ((rc = b.begin_query(q.query, q.out, q.lse, q.query_len)) != UC_OK) return rc;
    for (int i = 0; i < q.n_packed; ++i)
      if ((rc = b.add_item(packed_host[q.packed_begin + i])) != UC_OK) return rc;
    for (int i = 0; i < q.n_dense; ++i) {
      const uc_dense_segment &d = dense_host[q.dense_begin + i];
      if ((rc = b.add_dense(d.key, d.value, d.tokens, d.token_stride * 2, d.head_stride * 2)) != UC_OK) return rc;
    }
    if ((rc = b.end_query()) != UC_OK) return rc;
  }
  return mq_launch(b, bits, q_dtype, dense_dtype, out_dtype, sm_scale, static_cast<hipStream_t>(stream_),
                   "attn_mq_table");
}
