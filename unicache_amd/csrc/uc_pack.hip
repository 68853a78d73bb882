// KIVI quantize/pack, dequantize and fake-quant kernels (HBM-bound byte work).
//
// Bit-exactness contract (physical.py:160-175, 190-201; builtin.py:42-53):
// every value is widened to fp32; min/max are exact and, like torch.amin /
// amax and clamp_min, turn a group containing NaN into NaN stats (whose codes
// are then 0: the fp32 code is NaN and the clamp to [0, 2^b-1] yields 0,
// which is also what torch's NaN -> uint8 cast gives on x86); the subtraction,
// division (IEEE correctly rounded, the HIP default) and round-half-even
// (v_rndne_f32) happen once each, in the same order as the torch code, and
// dequantisation is a rounded multiply followed by a rounded add (never an
// FMA: the library is built with -ffp-contract=off and these use __f*_rn).
#include "uc_common.h"
#include "uc_mfma.h"

#include <type_traits>

namespace uc {
namespace {

// ----------------------------------------------------------------- keys --
// One lane owns a channel pair (c, c+1) of one head and quantizes one token
// group per iteration: keys are grouped along tokens, so the min/max
// reduction stays inside the lane and a wave reads whole 256-byte head rows.
template <int IN, int BITS, int G, bool VEC>
__device__ void pack_key_group(const void *__restrict__ key, int64_t st, int64_t sh, int64_t sd,
                               int64_t h, int64_t c, int64_t g, int64_t head_dim,
                               void *__restrict__ code, int64_t kc_sh, int64_t kc_sd, int64_t kc_sw,
                               void *__restrict__ kscale, void *__restrict__ kmin, int stats_dtype,
                               int64_t ks_sh, int64_t ks_sd, int64_t ks_sg) {
  constexpr float kMaxCode = float((1 << BITS) - 1);
  const bool has1 = (c + 1) < head_dim;
  float x0[G], x1[G];
  const int64_t t0 = g * G;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int64_t off = (t0 + i) * st + h * sh + c * sd;
    if constexpr (VEC) {
      const uint32_t pair = *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(key) + off);
      x0[i] = half_bits_to_f32<IN>(pair);
      x1[i] = half_bits_to_f32<IN>(pair >> 16);
    } else {
      x0[i] = load_as_f32<IN>(key, off);
      x1[i] = has1 ? load_as_f32<IN>(key, off + sd) : 0.0f;
    }
  }
  GroupRange r0, r1;
  r0.init(x0[0]);
  r1.init(x1[0]);
#pragma unroll
  for (int i = 1; i < G; ++i) {
    r0.add(x0[i]);
    r1.add(x1[i]);
  }
  r0.finish();
  r1.finish();
  const float mn0 = r0.mn, mn1 = r1.mn;
  const float s0 = clamp_min_nan(div_rn(sub_rn(r0.mx, mn0), kMaxCode), kEps);
  const float s1 = clamp_min_nan(div_rn(sub_rn(r1.mx, mn1), kMaxCode), kEps);
  const float rcp_s0 = __builtin_amdgcn_rcpf(s0), rcp_s1 = __builtin_amdgcn_rcpf(s1);

  if constexpr (BITS == 8) {
    uint8_t *out = static_cast<uint8_t *>(code);
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const float q0 = fminf(fmaxf(quant_rint(sub_rn(x0[i], mn0), s0, rcp_s0), 0.0f), kMaxCode);
      out[h * kc_sh + c * kc_sd + (t0 + i) * kc_sw] = static_cast<uint8_t>(q0);
      if (has1) {
        const float q1 = fminf(fmaxf(quant_rint(sub_rn(x1[i], mn1), s1, rcp_s1), 0.0f), kMaxCode);
        out[h * kc_sh + (c + 1) * kc_sd + (t0 + i) * kc_sw] = static_cast<uint8_t>(q1);
      }
    }
  } else {
    constexpr int kPerWord = 32 / BITS;
    constexpr int kWords = G / kPerWord;
    int32_t *out = static_cast<int32_t *>(code);
#pragma unroll
    for (int w = 0; w < kWords; ++w) {
      uint32_t w0 = 0, w1 = 0;
#pragma unroll
      for (int j = 0; j < kPerWord; ++j) {
        const int i = w * kPerWord + j;
        const uint32_t q0 = static_cast<uint32_t>(
            fminf(fmaxf(quant_rint(sub_rn(x0[i], mn0), s0, rcp_s0), 0.0f), kMaxCode));
        const uint32_t q1 = static_cast<uint32_t>(
            fminf(fmaxf(quant_rint(sub_rn(x1[i], mn1), s1, rcp_s1), 0.0f), kMaxCode));
        w0 |= q0 << (j * BITS);
        w1 |= q1 << (j * BITS);
      }
      const int64_t wi = g * kWords + w;
      out[h * kc_sh + c * kc_sd + wi * kc_sw] = static_cast<int32_t>(w0);
      if (has1) out[h * kc_sh + (c + 1) * kc_sd + wi * kc_sw] = static_cast<int32_t>(w1);
    }
  }
  const int64_t so0 = h * ks_sh + c * ks_sd + g * ks_sg;
  const int64_t so1 = so0 + ks_sd;
  if (stats_dtype == UC_FP16) {
    store_from_f32<UC_FP16>(kscale, so0, s0);
    store_from_f32<UC_FP16>(kmin, so0, mn0);
    if (has1) {
      store_from_f32<UC_FP16>(kscale, so1, s1);
      store_from_f32<UC_FP16>(kmin, so1, mn1);
    }
  } else if (stats_dtype == UC_BF16) {
    store_from_f32<UC_BF16>(kscale, so0, s0);
    store_from_f32<UC_BF16>(kmin, so0, mn0);
    if (has1) {
      store_from_f32<UC_BF16>(kscale, so1, s1);
      store_from_f32<UC_BF16>(kmin, so1, mn1);
    }
  } else {
    store_from_f32<UC_FP32>(kscale, so0, s0);
    store_from_f32<UC_FP32>(kmin, so0, mn0);
    if (has1) {
      store_from_f32<UC_FP32>(kscale, so1, s1);
      store_from_f32<UC_FP32>(kmin, so1, mn1);
    }
  }
}

// ---------------------------------------------------------------- values --
// One lane owns 16 consecutive channels of one (head, token); a value group
// of G channels spans G/16 neighbouring lanes, reduced with shuffles.  The 16
// codes of a lane form exactly one 2-bit word / two 4-bit words.
template <int IN, bool VEC>
__device__ __forceinline__ void load_value_chunk(const void *__restrict__ value, int64_t st, int64_t sh, int64_t sd,
                                                 int64_t h, int64_t t, int64_t chunk, bool active, float (&x)[16]) {
  if (active) {
    const int64_t base = t * st + h * sh + chunk * 16 * sd;
    if constexpr (VEC) {
      const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(value) + base);
      const uint4 a = p[0], b = p[1];
      const uint32_t words[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x[2 * i] = half_bits_to_f32<IN>(words[i]);
        x[2 * i + 1] = half_bits_to_f32<IN>(words[i] >> 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = load_as_f32<IN>(value, base + i * sd);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = 0.0f;
  }
}

template <int BITS, int G>
__device__ __forceinline__ void quant_value_chunk(const float (&x)[16], int64_t h, int64_t t, int64_t chunk,
                                                  bool active, void *__restrict__ code, int64_t vc_sh,
                                                  int64_t vc_st, int64_t vc_sw, void *__restrict__ vscale,
                                                  void *__restrict__ vmin, int stats_dtype, int64_t vs_sh,
                                                  int64_t vs_st, int64_t vs_sg) {
  constexpr float kMaxCode = float((1 << BITS) - 1);
  constexpr int kLanesPerGroup = G / 16;
  GroupRange r;
  r.init(x[0]);
#pragma unroll
  for (int i = 1; i < 16; ++i) r.add(x[i]);
#pragma unroll
  for (int o = 1; o < kLanesPerGroup; o <<= 1) r.merge_xor(o);
  if (!active) return;
  r.finish();
  const float mn = r.mn, mx = r.mx;
  const float s = clamp_min_nan(div_rn(sub_rn(mx, mn), kMaxCode), kEps);
  const float rcp_s = __builtin_amdgcn_rcpf(s);
  uint32_t q[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    q[i] = static_cast<uint32_t>(fminf(fmaxf(quant_rint(sub_rn(x[i], mn), s, rcp_s), 0.0f), kMaxCode));

  if constexpr (BITS == 8) {
    uint8_t *out = static_cast<uint8_t *>(code);
#pragma unroll
    for (int i = 0; i < 16; ++i) out[h * vc_sh + t * vc_st + (chunk * 16 + i) * vc_sw] = static_cast<uint8_t>(q[i]);
  } else {
    constexpr int kPerWord = 32 / BITS;
    constexpr int kWords = 16 / kPerWord;
    int32_t *out = static_cast<int32_t *>(code);
#pragma unroll
    for (int w = 0; w < kWords; ++w) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < kPerWord; ++j) word |= q[w * kPerWord + j] << (j * BITS);
      out[h * vc_sh + t * vc_st + (chunk * kWords + w) * vc_sw] = static_cast<int32_t>(word);
    }
  }
  if ((chunk % kLanesPerGroup) == 0) {
    const int64_t so = h * vs_sh + t * vs_st + (chunk / kLanesPerGroup) * vs_sg;
    if (stats_dtype == UC_FP16) {
      store_from_f32<UC_FP16>(vscale, so, s);
      store_from_f32<UC_FP16>(vmin, so, mn);
    } else if (stats_dtype == UC_BF16) {
      store_from_f32<UC_BF16>(vscale, so, s);
      store_from_f32<UC_BF16>(vmin, so, mn);
    } else {
      store_from_f32<UC_FP32>(vscale, so, s);
      store_from_f32<UC_FP32>(vmin, so, mn);
    }
  }
}

struct PackArgs {
  const void *key;
  int64_t k_st, k_sh, k_sd;
  const void *value;
  int64_t v_st, v_sh, v_sd;
  int64_t tokens, heads, head_dim;
  int stats_dtype;
  void *key_code;
  int64_t kc_sh, kc_sd, kc_sw;
  void *key_scale, *key_min;
  int64_t ks_sh, ks_sd, ks_sg;
  void *value_code;
  int64_t vc_sh, vc_st, vc_sw;
  void *value_scale, *value_min;
  int64_t vs_sh, vs_st, vs_sg;
  int64_t key_waves;   // waves doing key work (first part of the grid)
  int64_t value_waves; // waves doing value work
};

constexpr int kPackThreads = 256;

// wave -> (head, group, 128-channel slab); lane -> channel pair
template <int IN, int KB, int G, bool VEC>
__device__ __forceinline__ void pack_key_block(const PackArgs &a, int64_t block) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = block * (kPackThreads / kWave) + (threadIdx.x / kWave);
  if (wave >= a.key_waves) return;
  const int64_t slabs = (a.head_dim + 127) / 128;
  const int64_t groups = a.tokens / G;
  const int64_t slab = wave % slabs;
  const int64_t g = (wave / slabs) % groups;
  const int64_t h = wave / (slabs * groups);
  const int64_t c = slab * 128 + 2 * lane;
  if (c < a.head_dim)
    pack_key_group<IN, KB, G, VEC>(a.key, a.k_st, a.k_sh, a.k_sd, h, c, g, a.head_dim, a.key_code, a.kc_sh,
                                   a.kc_sd, a.kc_sw, a.key_scale, a.key_min, a.stats_dtype, a.ks_sh, a.ks_sd,
                                   a.ks_sg);
}

// wave -> (head, kVRuns consecutive runs of tokens); lane -> (token in run,
// 16-channel chunk).  The loads of all the wave's runs are issued before any
// run is quantized.
constexpr int kVRuns = 2;

template <int IN, int VB, int G, bool VEC>
__device__ __forceinline__ void pack_value_block(const PackArgs &a, int64_t block) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t vw = block * (kPackThreads / kWave) + (threadIdx.x / kWave);
  if (vw >= a.value_waves) return;
  const int64_t lanes_per_token = a.head_dim / 16;
  const int64_t tokens_per_wave = kWave / lanes_per_token;
  const int64_t runs = (a.tokens + tokens_per_wave - 1) / tokens_per_wave;
  const int64_t groups = (runs + kVRuns - 1) / kVRuns;
  const int64_t h = vw / groups;
  const int64_t chunk = lane % lanes_per_token;
  int64_t t[kVRuns];
  bool active[kVRuns];
  float x[kVRuns][16];
#pragma unroll
  for (int k = 0; k < kVRuns; ++k) {
    t[k] = ((vw % groups) * kVRuns + k) * tokens_per_wave + lane / lanes_per_token;
    active[k] = (lane < tokens_per_wave * lanes_per_token) && t[k] < a.tokens;
    load_value_chunk<IN, VEC>(a.value, a.v_st, a.v_sh, a.v_sd, h, t[k], chunk, active[k], x[k]);
  }
#pragma unroll
  for (int k = 0; k < kVRuns; ++k)
    quant_value_chunk<VB, G>(x[k], h, t[k], chunk, active[k], a.value_code, a.vc_sh, a.vc_st, a.vc_sw,
                             a.value_scale, a.value_min, a.stats_dtype, a.vs_sh, a.vs_st, a.vs_sg);
}

template <int IN, int KB, int G, bool VEC>
__global__ __launch_bounds__(kPackThreads) void kivi_pack_key_kernel(PackArgs a) {
  pack_key_block<IN, KB, G, VEC>(a, blockIdx.x);
}

template <int IN, int VB, int G, bool VEC>
__global__ __launch_bounds__(kPackThreads) void kivi_pack_value_kernel(PackArgs a) {
  pack_value_block<IN, VB, G, VEC>(a, blockIdx.x);
}

// Keys and values of equal bits in one launch: the first key_blocks
// workgroups pack keys, the rest values (one launch instead of two).
template <int IN, int BITS, int G>
__global__ __launch_bounds__(kPackThreads) void kivi_pack_kv_kernel(PackArgs a, int64_t key_blocks) {
  const int64_t b = blockIdx.x;
  if (b < key_blocks)
    pack_key_block<IN, BITS, G, true>(a, b);
  else
    pack_value_block<IN, BITS, G, true>(a, b - key_blocks);
}

int64_t wave_blocks(int64_t waves) { return (waves + (kPackThreads / kWave) - 1) / (kPackThreads / kWave); }

// ------------------------------------------------------ fast 2/4-bit pack --
// Keys and values of equal 2/4 bits, head_dim 128, 16-bit rows with unit
// channel stride into token-major storage (unit channel / word strides).  A
// key unit is one token group of one head (lane = channel pair, G loads of 4
// bytes), a value unit VR runs of 8 tokens of one head (lane = token of the
// run and 16-channel chunk, two 16-byte loads per run); heads are the fastest
// index, so the four waves of a workgroup read whole token rows.  Wave w of
// the grid takes unit w: key units first, then value units.  A lane's raw
// 16-bit pairs stay in registers: read once for the range, once for the codes.
//
// The range uses IEEE minimum/maximum (v_minimum3 / v_maximum3, two elements
// per instruction), which propagate NaN as torch.amin / amax do.  Codes are
// rint((x - mn) * rcp(scale)), with the correctly rounded division only for
// elements near a half step (code_of), and are converted and byte-packed by
// v_cvt_pk_u8_f32 (exact for these integer values): byte m of dword c holds
// code m * (8 / b) + c, so shifting the dwords together puts code j at bit
// b * j, LSB first (physical.py:72-85).  A group with NaN or inf, or a scale
// past 2^126, takes the generic arithmetic (quant_rint and the clamp).
template <int IN>
__device__ __forceinline__ float lo16(uint32_t r) {
  if constexpr (IN == UC_BF16) return __uint_as_float(r << 16);
  else return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r)));
}
template <int IN>
__device__ __forceinline__ float hi16(uint32_t r) {
  if constexpr (IN == UC_BF16) return __uint_as_float(r & 0xffff0000u);
  else return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r >> 16)));
}
__device__ __forceinline__ float min_nan(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Integer-valued code q (0..255) into byte m of d.
__device__ __forceinline__ uint32_t put_code_byte(int m, float q, uint32_t d) {
  switch (m) {
    case 0: return __builtin_amdgcn_cvt_pk_u8_f32(q, 0, d);
    case 1: return __builtin_amdgcn_cvt_pk_u8_f32(q, 1, d);
    case 2: return __builtin_amdgcn_cvt_pk_u8_f32(q, 2, d);
    default: return __builtin_amdgcn_cvt_pk_u8_f32(q, 3, d);
  }
}

// Scale of a group from its range (physical.py:160-175); a NaN range gives
// the canonical NaN statistics of GroupRange.
template <int BITS>
__device__ __forceinline__ float group_scale(float &mn, float &mx) {
  if (mn != mn) {
    mn = __builtin_nanf("");
    mx = mn;
  }
  return clamp_min_nan(div_rn(sub_rn(mx, mn), float((1 << BITS) - 1)), kEps);
}

// Code of one element of a group whose scale s is finite with a normal
// reciprocal r: y = (x - mn) * r lies in [0, 2^b - 1 + 2^-20], so rint(y)
// needs no clamp, and it is the code of the correctly rounded quotient
// whenever y is farther than 2^b 2^-20 >= |y| 2^-20 from a half-integer (the
// argument of quant_rint).  Inside that band -- about one element in a
// thousand for bf16 data, whose groups often hold exact half steps -- the
// correctly rounded division decides, for the lanes that need it.
template <int BITS>
__device__ __forceinline__ float code_of(float x, float mn, float s, float r) {
  constexpr float kNearHalf = 0.5f - float(1 << BITS) * 0x1p-20f;
  const float d = sub_rn(x, mn);
  const float y = mul_rn(d, r);
  float q = rintf(y);
  if (fabsf(sub_rn(y, q)) >= kNearHalf) q = rintf(div_rn(d, s));
  return q;
}

// Groups the fast codes serve: finite scale (no NaN or inf in the group) with
// a normal reciprocal.  Others take the generic arithmetic (quant_rint, clamp).
__device__ __forceinline__ bool fast_group(float s, float r) { return s <= 3.0e38f && r >= 0x1p-126f; }

// Word k of the codes from the byte dwords d (code m * (8 / BITS) + c of the
// word in byte m of d[c]).
template <int BITS>
__device__ __forceinline__ uint32_t merge_code_bytes(const uint32_t (&d)[8 / BITS]) {
  uint32_t w = d[0];
#pragma unroll
  for (int c = 1; c < 8 / BITS; ++c) w |= d[c] << (BITS * c);
  return w;
}

// The codes of one word by the generic kernels' arithmetic (quant_rint, clamp).
template <int BITS>
__device__ __forceinline__ uint32_t exact_code_word(const float (&x)[32 / BITS], float mn, float s, float r) {
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 32 / BITS; ++j) {
    const float q = fminf(fmaxf(quant_rint(sub_rn(x[j], mn), s, r), 0.0f), float((1 << BITS) - 1));
    word |= static_cast<uint32_t>(q) << (j * BITS);
  }
  return word;
}

__device__ __forceinline__ uint32_t stat_bits(float v, int stats_dtype) {
  return stats_dtype == UC_FP16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v);
}

template <int IN, int BITS, int G>
__device__ __forceinline__ void fast_key_unit(const PackArgs &a, int64_t unit, int lane) {
  constexpr int kPer = 32 / BITS, kPerByte = 8 / BITS, kWords = G / kPer;
  // heads fastest: the waves of a workgroup read whole token rows
  const int64_t h = unit % a.heads, g = unit / a.heads;
  const uint16_t *src = static_cast<const uint16_t *>(a.key) + g * G * a.k_st + h * a.k_sh;
  const mf::Rsrc rs = mf::make_rsrc(src, (G - 1) * a.k_st * 2 + 256);
  const uint32_t row = static_cast<uint32_t>(a.k_st * 2);
  uint32_t raw[G];
#pragma unroll
  for (int i = 0; i < G; ++i) raw[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, 4u * lane, i * row, 0);
  float mn0 = lo16<IN>(raw[0]), mx0 = mn0, mn1 = hi16<IN>(raw[0]), mx1 = mn1;
#pragma unroll
  for (int i = 1; i < G; ++i) {
    const float x0 = lo16<IN>(raw[i]), x1 = hi16<IN>(raw[i]);
    mn0 = min_nan(mn0, x0);
    mx0 = max_nan(mx0, x0);
    mn1 = min_nan(mn1, x1);
    mx1 = max_nan(mx1, x1);
  }
  const float s0 = group_scale<BITS>(mn0, mx0), s1 = group_scale<BITS>(mn1, mx1);
  const float r0 = __builtin_amdgcn_rcpf(s0), r1 = __builtin_amdgcn_rcpf(s1);
  // converting again costs less than keeping the range pass's 2G floats live
#pragma unroll
  for (int i = 0; i < G; ++i) asm volatile("" : "+v"(raw[i]));
  // both channels element by element, so each raw pair dies at its last use
  const bool fast0 = fast_group(s0, r0), fast1 = fast_group(s1, r1);
  uint32_t w0[kWords], w1[kWords];
  if (fast0 && fast1) {
#pragma unroll
    for (int k = 0; k < kWords; ++k) {
      uint32_t d0[kPerByte], d1[kPerByte];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int c = 0; c < kPerByte; ++c) {
          const uint32_t v = raw[k * kPer + m * kPerByte + c];
          d0[c] = put_code_byte(m, code_of<BITS>(lo16<IN>(v), mn0, s0, r0), m ? d0[c] : 0u);
          d1[c] = put_code_byte(m, code_of<BITS>(hi16<IN>(v), mn1, s1, r1), m ? d1[c] : 0u);
        }
      }
      w0[k] = merge_code_bytes<BITS>(d0);
      w1[k] = merge_code_bytes<BITS>(d1);
    }
  } else {
    // rare (NaN or inf in a group, a scale past 2^126): both channels by the
    // generic arithmetic
#pragma unroll
    for (int k = 0; k < kWords; ++k) {
      float x0[kPer], x1[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        x0[j] = lo16<IN>(raw[k * kPer + j]);
        x1[j] = hi16<IN>(raw[k * kPer + j]);
      }
      w0[k] = exact_code_word<BITS>(x0, mn0, s0, r0);
      w1[k] = exact_code_word<BITS>(x1, mn1, s1, r1);
    }
  }
  const int64_t c = 2 * lane;
  uint32_t *kc = static_cast<uint32_t *>(a.key_code) + h * a.kc_sh + g * kWords * a.kc_sw + c;
#pragma unroll
  for (int w = 0; w < kWords; ++w) *reinterpret_cast<uint2 *>(kc + w * a.kc_sw) = make_uint2(w0[w], w1[w]);
  const int64_t so = h * a.ks_sh + g * a.ks_sg + c;
  *reinterpret_cast<uint32_t *>(static_cast<uint16_t *>(a.key_scale) + so) =
      stat_bits(s0, a.stats_dtype) | (stat_bits(s1, a.stats_dtype) << 16);
  *reinterpret_cast<uint32_t *>(static_cast<uint16_t *>(a.key_min) + so) =
      stat_bits(mn0, a.stats_dtype) | (stat_bits(mn1, a.stats_dtype) << 16);
}

template <int IN, int BITS, int G, int VR>
__device__ __forceinline__ void fast_value_unit(const PackArgs &a, int64_t unit, int lane) {
  constexpr int kRuns = VR;       // runs of 8 tokens per unit
  constexpr int kLanes = G / 16;  // lanes of one value group
  constexpr int kPer = 32 / BITS, kPerByte = 8 / BITS, kWords = 16 / kPer;
  const int64_t h = unit % a.heads, g = unit / a.heads;
  const int tok = lane >> 3, chunk = lane & 7;
  const uint16_t *src = static_cast<const uint16_t *>(a.value) + g * (8 * VR) * a.v_st + h * a.v_sh;
  const mf::Rsrc rs = mf::make_rsrc(src, (8 * VR - 1) * a.v_st * 2 + 256);
  const uint32_t voff = static_cast<uint32_t>((tok * a.v_st + chunk * 16) * 2);
  const uint32_t run = static_cast<uint32_t>(8 * a.v_st * 2);
  uint4 raw[kRuns][2];
#pragma unroll
  for (int r = 0; r < kRuns; ++r) {
    raw[r][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, r * run, 0));
    raw[r][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16u, r * run, 0));
  }
#pragma unroll
  for (int r = 0; r < kRuns; ++r) {
    const uint32_t p[8] = {raw[r][0].x, raw[r][0].y, raw[r][0].z, raw[r][0].w,
                           raw[r][1].x, raw[r][1].y, raw[r][1].z, raw[r][1].w};
    auto x = [&](int i) { return (i & 1) ? hi16<IN>(p[i >> 1]) : lo16<IN>(p[i >> 1]); };
    float mn = x(0), mx = mn;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      mn = min_nan(mn, x(i));
      mx = max_nan(mx, x(i));
    }
#pragma unroll
    for (int o = 1; o < kLanes; o <<= 1) {
      mn = min_nan(mn, __shfl_xor(mn, o, kWave));
      mx = max_nan(mx, __shfl_xor(mx, o, kWave));
    }
    const float s = group_scale<BITS>(mn, mx);
    const float rc = __builtin_amdgcn_rcpf(s);
    uint32_t w[kWords];
    if (fast_group(s, rc)) {
#pragma unroll
      for (int k = 0; k < kWords; ++k) {
        uint32_t d[kPerByte];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
          for (int c = 0; c < kPerByte; ++c)
            d[c] = put_code_byte(m, code_of<BITS>(x(k * kPer + m * kPerByte + c), mn, s, rc), m ? d[c] : 0u);
        }
        w[k] = merge_code_bytes<BITS>(d);
      }
    } else {
#pragma unroll
      for (int k = 0; k < kWords; ++k) {
        float xs[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) xs[j] = x(k * kPer + j);
        w[k] = exact_code_word<BITS>(xs, mn, s, rc);
      }
    }
    const int64_t t = g * (8 * VR) + r * 8 + tok;
    uint32_t *vc = static_cast<uint32_t *>(a.value_code) + h * a.vc_sh + t * a.vc_st + chunk * kWords;
    if constexpr (kWords == 1) *vc = w[0];
    else *reinterpret_cast<uint2 *>(vc) = make_uint2(w[0], w[1]);
    if ((chunk % kLanes) == 0) {
      const int64_t so = h * a.vs_sh + t * a.vs_st + chunk / kLanes;
      static_cast<uint16_t *>(a.value_scale)[so] = static_cast<uint16_t>(stat_bits(s, a.stats_dtype));
      static_cast<uint16_t *>(a.value_min)[so] = static_cast<uint16_t>(stat_bits(mn, a.stats_dtype));
    }
  }
}

// waves per SIMD the register budget is sized for (G raw key pairs per lane)
template <int G>
constexpr int kFastPackWaves = G <= 16 ? 8 : G <= 32 ? 6 : 3;

template <int IN, int BITS, int G, int VR>
__global__ __launch_bounds__(kPackThreads) __attribute__((amdgpu_waves_per_eu(kFastPackWaves<G>))) void
kivi_pack_fast_kernel(PackArgs a, int64_t key_units, int64_t value_units) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t u = int64_t(blockIdx.x) * (kPackThreads / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (u < key_units)
    fast_key_unit<IN, BITS, G>(a, u, lane);
  else if (u < key_units + value_units)
    fast_value_unit<IN, BITS, G, VR>(a, u - key_units, lane);
}

// Whether uc_kivi_pack's arguments fit kivi_pack_fast_kernel.
bool fast_pack_fits(const PackArgs &a, int in_dtype, int kb, int vb, int group) {
  auto al = [](const void *p, int b) { return (reinterpret_cast<uintptr_t>(p) % b) == 0; };
  const bool shape = a.key && a.value && kb == vb && (kb == 2 || kb == 4) && a.head_dim == 128 &&
                     (group == 16 || group == 32 || group == 64) && (in_dtype == UC_BF16 || in_dtype == UC_FP16) &&
                     (a.stats_dtype == UC_BF16 || a.stats_dtype == UC_FP16);
  if (!shape) return false;
  const bool in = a.k_sd == 1 && a.v_sd == 1 && a.k_st > 0 && a.v_st > 0 && a.k_sh >= 0 && a.v_sh >= 0 &&
                  a.k_st % 2 == 0 && a.k_sh % 2 == 0 && al(a.key, 4) && a.v_st % 8 == 0 && a.v_sh % 8 == 0 &&
                  al(a.value, 16) && int64_t(group) * a.k_st * 2 + 256 < (int64_t(1) << 31) &&
                  int64_t(group) * a.v_st * 2 + 256 < (int64_t(1) << 31);
  const bool kout = a.kc_sd == 1 && a.kc_sw % 2 == 0 && a.kc_sh % 2 == 0 && al(a.key_code, 8) && a.ks_sd == 1 &&
                    a.ks_sg % 2 == 0 && a.ks_sh % 2 == 0 && al(a.key_scale, 4) && al(a.key_min, 4);
  const bool vout = a.vc_sw == 1 && (kb == 2 || (a.vc_st % 2 == 0 && a.vc_sh % 2 == 0 && al(a.value_code, 8))) &&
                    al(a.value_code, 4) && a.vs_sg == 1 && al(a.value_scale, 2) && al(a.value_min, 2);
  return in && kout && vout;
}

template <int IN, int BITS, int G>
void launch_pack_fast_g(const PackArgs &a, hipStream_t stream) {
  const int64_t key_units = a.heads * (a.tokens / G);
  // value runs of 8 tokens per wave: two for launches of a few waves per SIMD
  // (a config-1 sequence: 7.7 against 8.0 us), one above (32k tokens: 20.1
  // against 20.9 us)
  const int vr = a.heads * a.tokens >= 65536 ? 1 : 2;
  const int64_t value_units = a.heads * (a.tokens / (8 * vr));
  const dim3 grid(static_cast<unsigned>(wave_blocks(key_units + value_units)));
  if (vr == 1)
    hipLaunchKernelGGL((kivi_pack_fast_kernel<IN, BITS, G, 1>), grid, dim3(kPackThreads), 0, stream, a, key_units,
                       value_units);
  else
    hipLaunchKernelGGL((kivi_pack_fast_kernel<IN, BITS, G, 2>), grid, dim3(kPackThreads), 0, stream, a, key_units,
                       value_units);
}

template <int IN, int BITS>
void launch_pack_fast(const PackArgs &a, int group, hipStream_t stream) {
  if (group == 16) launch_pack_fast_g<IN, BITS, 16>(a, stream);
  else if (group == 32) launch_pack_fast_g<IN, BITS, 32>(a, stream);
  else launch_pack_fast_g<IN, BITS, 64>(a, stream);
}

template <int IN, int G>
void launch_pack(const PackArgs &a, int kb, int vb, bool kvec, bool vvec, hipStream_t stream) {
  if (kb == vb && kb != 8 && kvec && vvec && a.key_waves > 0 && a.value_waves > 0) {
    const int64_t key_blocks = wave_blocks(a.key_waves);
    const dim3 grid(static_cast<unsigned>(key_blocks + wave_blocks(a.value_waves)));
    if (kb == 2)
      hipLaunchKernelGGL((kivi_pack_kv_kernel<IN, 2, G>), grid, dim3(kPackThreads), 0, stream, a, key_blocks);
    else
      hipLaunchKernelGGL((kivi_pack_kv_kernel<IN, 4, G>), grid, dim3(kPackThreads), 0, stream, a, key_blocks);
    return;
  }
  if (a.key_waves > 0) {
    const dim3 grid(wave_blocks(a.key_waves));
    UC_DISPATCH_BITS(kb, KB, [&] {
      if (kvec)
        hipLaunchKernelGGL((kivi_pack_key_kernel<IN, KB, G, true>), grid, dim3(kPackThreads), 0, stream, a);
      else
        hipLaunchKernelGGL((kivi_pack_key_kernel<IN, KB, G, false>), grid, dim3(kPackThreads), 0, stream, a);
    });
  }
  if (a.value_waves > 0) {
    const dim3 grid(wave_blocks(a.value_waves));
    UC_DISPATCH_BITS(vb, VB, [&] {
      if (vvec)
        hipLaunchKernelGGL((kivi_pack_value_kernel<IN, VB, G, true>), grid, dim3(kPackThreads), 0, stream, a);
      else
        hipLaunchKernelGGL((kivi_pack_value_kernel<IN, VB, G, false>), grid, dim3(kPackThreads), 0, stream, a);
    });
  }
}

bool aligned(const void *p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// ------------------------------------------------------- any group size --
// UniCache's reference backend takes any positive group size
// (physical.py:247-248): a value row of head_dim channels may end in a partial
// group (physical.py:151-158), and one code word may hold codes of several
// groups.  One thread owns a span of lcm(G, codes per word) positions of a key
// row (one head and channel, along tokens) or a value row (one head and token,
// along channels) -- whole groups and whole words -- and walks its groups in
// order: the group's exact range, its fp32 scale and minimum (stored rounded to
// the stats dtype), then each code into the current word, stored when the word
// is full or the row ends (zero-padded, as physical.py:72-85 pads).
struct GenericPackArgs {
  PackArgs p;
  int group, kb, vb;
  int64_t kspan, vspan;        // positions per thread
  int64_t kthreads, vthreads;  // threads doing key / value rows
};

template <int IN>
__device__ void pack_generic_row(const void *src, int64_t base, int64_t stride, int64_t length, int64_t begin,
                                 int64_t end, int group, int bits, void *code, int64_t code_base,
                                 int64_t code_stride, void *scale, void *minimum, int64_t stat_base,
                                 int64_t stat_stride, int stats_dtype) {
  const float max_code = float((1 << bits) - 1);
  const int per_word = bits == 8 ? 1 : 32 / bits;
  uint32_t word = 0;
  for (int64_t g0 = begin; g0 < end; g0 += group) {
    const int64_t g1 = min(g0 + int64_t(group), length);
    GroupRange r;
    r.init(load_as_f32<IN>(src, base + g0 * stride));
    for (int64_t i = g0 + 1; i < g1; ++i) r.add(load_as_f32<IN>(src, base + i * stride));
    r.finish();
    const float mn = r.mn;
    const float s = clamp_min_nan(div_rn(sub_rn(r.mx, mn), max_code), kEps);
    const int64_t so = stat_base + (g0 / group) * stat_stride;
    store_dyn(scale, so, s, stats_dtype);
    store_dyn(minimum, so, mn, stats_dtype);
    const float rcp = __builtin_amdgcn_rcpf(s);
    for (int64_t i = g0; i < g1; ++i) {
      const float x = load_as_f32<IN>(src, base + i * stride);
      const uint32_t q = static_cast<uint32_t>(fminf(fmaxf(quant_rint(sub_rn(x, mn), s, rcp), 0.0f), max_code));
      if (bits == 8) {
        static_cast<uint8_t *>(code)[code_base + i * code_stride] = static_cast<uint8_t>(q);
        continue;
      }
      const int pos = static_cast<int>(i % per_word);
      word |= q << (pos * bits);
      if (pos == per_word - 1 || i == length - 1) {
        static_cast<int32_t *>(code)[code_base + (i / per_word) * code_stride] = static_cast<int32_t>(word);
        word = 0;
      }
    }
  }
}

template <int IN>
__global__ __launch_bounds__(kPackThreads) void kivi_pack_generic_kernel(GenericPackArgs g) {
  const PackArgs &a = g.p;
  int64_t idx = int64_t(blockIdx.x) * kPackThreads + threadIdx.x;
  if (idx < g.kthreads) {
    const int64_t chunks = (a.tokens + g.kspan - 1) / g.kspan;
    const int64_t c = idx % chunks, d = (idx / chunks) % a.head_dim, h = idx / (chunks * a.head_dim);
    const int64_t begin = c * g.kspan, end = min(a.tokens, begin + g.kspan);
    pack_generic_row<IN>(a.key, h * a.k_sh + d * a.k_sd, a.k_st, a.tokens, begin, end, g.group, g.kb, a.key_code,
                         h * a.kc_sh + d * a.kc_sd, a.kc_sw, a.key_scale, a.key_min, h * a.ks_sh + d * a.ks_sd,
                         a.ks_sg, a.stats_dtype);
    return;
  }
  idx -= g.kthreads;
  if (idx < g.vthreads) {
    const int64_t chunks = (a.head_dim + g.vspan - 1) / g.vspan;
    const int64_t c = idx % chunks, t = (idx / chunks) % a.tokens, h = idx / (chunks * a.tokens);
    const int64_t begin = c * g.vspan, end = min(a.head_dim, begin + g.vspan);
    pack_generic_row<IN>(a.value, h * a.v_sh + t * a.v_st, a.v_sd, a.head_dim, begin, end, g.group, g.vb,
                         a.value_code, h * a.vc_sh + t * a.vc_st, a.vc_sw, a.value_scale, a.value_min,
                         h * a.vs_sh + t * a.vs_st, a.vs_sg, a.stats_dtype);
  }
}

int64_t gcd64(int64_t x, int64_t y) {
  while (y) {
    const int64_t r = x % y;
    x = y;
    y = r;
  }
  return x;
}

// The group sizes the tuned pack / dequant kernels take.
bool tuned_group(int group, int64_t head_dim) {
  return (group == 16 || group == 32 || group == 64 || group == 128) && head_dim % group == 0;
}

// -------------------------------------------------------------- dequant --
struct DequantArgs {
  const void *key_code;
  int64_t kc_sh, kc_sd, kc_sw;
  const void *key_scale, *key_min;
  int64_t ks_sh, ks_sd, ks_sg;
  const void *value_code;
  int64_t vc_sh, vc_st, vc_sw;
  const void *value_scale, *value_min;
  int64_t vs_sh, vs_st, vs_sg;
  int64_t heads, head_dim, start, count;
  void *out_key, *out_value;
  int64_t o_st, o_sh, o_sd, offset;
  int lg;         // log2(group_size) (tuned group sizes)
  int64_t group;  // group_size (any)
  int sd, od;     // stats and output dtype codes
};

// One thread per output element (token, head, channel); keys and values are
// restored by separate halves of the grid.
template <int KB, int VB>
__global__ __launch_bounds__(256) void kivi_dequant_kernel(DequantArgs a) {
  const int64_t per_tensor = a.count * a.heads * a.head_dim;
  int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool is_value = idx >= per_tensor;
  if (is_value) idx -= per_tensor;
  if (idx >= per_tensor) return;
  const int64_t d = idx % a.head_dim;
  const int64_t h = (idx / a.head_dim) % a.heads;
  const int64_t n = idx / (a.head_dim * a.heads);
  const int64_t t = a.start + n;
  float out;
  if (!is_value) {
    if (a.key_code == nullptr) return;
    constexpr int kPerWord = KB == 8 ? 1 : 32 / KB;
    const uint32_t c = read_code<KB>(a.key_code, h * a.kc_sh + d * a.kc_sd + (t / kPerWord) * a.kc_sw,
                                     t % kPerWord);
    const int64_t so = h * a.ks_sh + d * a.ks_sd + (t / a.group) * a.ks_sg;
    const float s = load_dyn(a.key_scale, so, a.sd);
    const float m = load_dyn(a.key_min, so, a.sd);
    out = add_rn(mul_rn(float(c), s), m);
    store_dyn(a.out_key, (a.offset + n) * a.o_st + h * a.o_sh + d * a.o_sd, out, a.od);
  } else {
    if (a.value_code == nullptr) return;
    constexpr int kPerWord = VB == 8 ? 1 : 32 / VB;
    const uint32_t c = read_code<VB>(a.value_code, h * a.vc_sh + t * a.vc_st + (d / kPerWord) * a.vc_sw,
                                     d % kPerWord);
    const int64_t so = h * a.vs_sh + t * a.vs_st + (d / a.group) * a.vs_sg;
    const float s = load_dyn(a.value_scale, so, a.sd);
    const float m = load_dyn(a.value_min, so, a.sd);
    out = add_rn(mul_rn(float(c), s), m);
    store_dyn(a.out_value, (a.offset + n) * a.o_st + h * a.o_sh + d * a.o_sd, out, a.od);
  }
}

// Native 2/4-bit layout (words contiguous along tokens for keys, along
// channels for values; unit channel stride in the output).  Same arithmetic
// as kivi_dequant_kernel, laid out for whole-row stores.
template <int OD>
__device__ __forceinline__ void store_pair(void *out, int64_t off, float v0, float v1) {
  if constexpr (OD == UC_FP32) {
    *reinterpret_cast<float2 *>(static_cast<float *>(out) + off) = make_float2(v0, v1);
  } else {
    const uint32_t lo = OD == UC_BF16 ? f32_to_bf16_bits(v0) : f32_to_f16_bits(v0);
    const uint32_t hi = OD == UC_BF16 ? f32_to_bf16_bits(v1) : f32_to_f16_bits(v1);
    *reinterpret_cast<uint32_t *>(static_cast<uint16_t *>(out) + off) = lo | (hi << 16);
  }
}

constexpr int kDqRunWords = 4;  // key words per lane and channel

// Keys: lane = (head, run of 4 words, channel pair), channel pairs fastest, so
// a wave writes whole 128-channel head rows for each token of its run.
template <int BITS, int OD>
__global__ __launch_bounds__(256) void dequant_key_native_kernel(DequantArgs a, int64_t runs) {
  constexpr int TPW = 32 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const int64_t pairs = a.head_dim / 2;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= a.heads * runs * pairs) return;
  const int64_t cp = idx % pairs, run = (idx / pairs) % runs, h = idx / (pairs * runs);
  const int64_t c = 2 * cp, stop = a.start + a.count;
  const int64_t w0 = a.start / TPW + run * kDqRunWords, w_end = (stop + TPW - 1) / TPW;
  const uint32_t *kc = static_cast<const uint32_t *>(a.key_code) + h * a.kc_sh + c * a.kc_sd;
  uint32_t wa[kDqRunWords], wb[kDqRunWords];
  float s0[kDqRunWords], m0[kDqRunWords], s1[kDqRunWords], m1[kDqRunWords];
  // every load of the run first (a word lies inside one group: TPW <= group_size)
#pragma unroll
  for (int j = 0; j < kDqRunWords; ++j) {
    const bool ok = w0 + j < w_end;
    wa[j] = ok ? kc[(w0 + j) * a.kc_sw] : 0u;
    wb[j] = ok ? kc[a.kc_sd + (w0 + j) * a.kc_sw] : 0u;
    const int64_t so = h * a.ks_sh + c * a.ks_sd + (((ok ? w0 + j : w0) * TPW) >> a.lg) * a.ks_sg;
    s0[j] = load_dyn(a.key_scale, so, a.sd);
    m0[j] = load_dyn(a.key_min, so, a.sd);
    s1[j] = load_dyn(a.key_scale, so + a.ks_sd, a.sd);
    m1[j] = load_dyn(a.key_min, so + a.ks_sd, a.sd);
  }
#pragma unroll
  for (int j = 0; j < kDqRunWords; ++j) {
    const int64_t w = w0 + j;
    if (w >= w_end) break;
#pragma unroll
    for (int p = 0; p < TPW; ++p) {
      const int64_t t = w * TPW + p;
      if (t < a.start || t >= stop) continue;
      const float v0 = add_rn(mul_rn(float((wa[j] >> (p * BITS)) & kMask), s0[j]), m0[j]);
      const float v1 = add_rn(mul_rn(float((wb[j] >> (p * BITS)) & kMask), s1[j]), m1[j]);
      store_pair<OD>(a.out_key, (a.offset + t - a.start) * a.o_st + h * a.o_sh + c, v0, v1);
    }
  }
}

// Keys from token-major storage (channel stride 1 for words and stats) into
// 16-bit rows with 16-byte alignment: lane = (key word, head, 8 channels),
// channel octets fastest, then heads.  A lane loads its octet's words of the
// run (two 16-byte loads per word) and their groups' scales and minima (16
// bytes each), then writes one 16-byte store per token: a wave writes whole
// 256-byte head rows, four times the bytes per store of the pairwise kernel.
constexpr int kDqOctetWords = 1;  // key words per lane of the octet kernel: enough lanes to fill the chip

template <int BITS, int OD, int SD>
__device__ __forceinline__ void dequant_key_octet_block(const DequantArgs &a, int64_t runs, int64_t block) {
  constexpr int TPW = 32 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const int64_t octets = a.head_dim / 8;
  const int64_t idx = block * 256 + threadIdx.x;
  if (idx >= a.heads * runs * octets) return;
  // octets, then heads fastest: the lanes of a wave write whole token rows
  // (32-bit divisions: the launch keeps the index below 2^31)
  const uint32_t i32 = static_cast<uint32_t>(idx), oct32 = static_cast<uint32_t>(octets);
  const uint32_t hd32 = static_cast<uint32_t>(a.heads), q = i32 / oct32, r32 = q / hd32;
  const int64_t oc = i32 - q * oct32, h = q - r32 * hd32, run = r32;
  const int64_t c = 8 * oc, stop = a.start + a.count;
  const int64_t w0 = a.start / TPW + run * kDqOctetWords, w_end = (stop + TPW - 1) / TPW;
  const uint32_t *kc = static_cast<const uint32_t *>(a.key_code) + h * a.kc_sh + c;
  uint32_t wd[kDqOctetWords][8];
  float sc[kDqOctetWords][8], mn[kDqOctetWords][8];
#pragma unroll
  for (int j = 0; j < kDqOctetWords; ++j) {
    const bool ok = w0 + j < w_end;
    const int64_t w = ok ? w0 + j : w0;
    const uint4 lo = *reinterpret_cast<const uint4 *>(kc + w * a.kc_sw);
    const uint4 hi = *reinterpret_cast<const uint4 *>(kc + w * a.kc_sw + 4);
    wd[j][0] = lo.x; wd[j][1] = lo.y; wd[j][2] = lo.z; wd[j][3] = lo.w;
    wd[j][4] = hi.x; wd[j][5] = hi.y; wd[j][6] = hi.z; wd[j][7] = hi.w;
    const int64_t so = h * a.ks_sh + c + ((w * TPW) >> a.lg) * a.ks_sg;
    const uint4 sv = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.key_scale) + so);
    const uint4 mv = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.key_min) + so);
    const uint32_t s4[4] = {sv.x, sv.y, sv.z, sv.w}, m4[4] = {mv.x, mv.y, mv.z, mv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      sc[j][2 * k] = half_bits_to_f32<SD>(s4[k]);
      sc[j][2 * k + 1] = half_bits_to_f32<SD>(s4[k] >> 16);
      mn[j][2 * k] = half_bits_to_f32<SD>(m4[k]);
      mn[j][2 * k + 1] = half_bits_to_f32<SD>(m4[k] >> 16);
    }
  }
#pragma unroll
  for (int j = 0; j < kDqOctetWords; ++j) {
    const int64_t w = w0 + j;
    if (w >= w_end) break;
#pragma unroll
    for (int p = 0; p < TPW; ++p) {
      const int64_t t = w * TPW + p;
      if (t < a.start || t >= stop) continue;
      uint32_t out[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float v0 = add_rn(mul_rn(float((wd[j][2 * k] >> (p * BITS)) & kMask), sc[j][2 * k]), mn[j][2 * k]);
        const float v1 =
            add_rn(mul_rn(float((wd[j][2 * k + 1] >> (p * BITS)) & kMask), sc[j][2 * k + 1]), mn[j][2 * k + 1]);
        const uint32_t b0 = OD == UC_BF16 ? f32_to_bf16_bits(v0) : f32_to_f16_bits(v0);
        const uint32_t b1 = OD == UC_BF16 ? f32_to_bf16_bits(v1) : f32_to_f16_bits(v1);
        out[k] = b0 | (b1 << 16);
      }
      *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.out_key) + (a.offset + t - a.start) * a.o_st +
                                 h * a.o_sh + c) = make_uint4(out[0], out[1], out[2], out[3]);
    }
  }
}

// Values: lane = (token, head, word), words fastest, then heads: one 4-byte
// word and its group's stats in, 16 (2-bit) or 8 (4-bit) contiguous channels
// out.
template <int BITS, int OD, int SD>
__global__ __launch_bounds__(256) void dequant_key_octet_kernel(DequantArgs a, int64_t runs) {
  dequant_key_octet_block<BITS, OD, SD>(a, runs, blockIdx.x);
}

template <int BITS, int OD, bool VEC>
__device__ __forceinline__ void dequant_value_native_block(const DequantArgs &a, int64_t block) {
  constexpr int CPW = 32 / BITS;  // channels per word
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const int64_t words = a.head_dim / CPW;
  const int64_t idx = block * 256 + threadIdx.x;
  if (idx >= a.heads * a.count * words) return;
  // words, then heads fastest: the lanes of a wave write whole token rows
  // (32-bit divisions: the launch keeps the index below 2^31)
  const uint32_t i32 = static_cast<uint32_t>(idx), wd32 = static_cast<uint32_t>(words);
  const uint32_t hd32 = static_cast<uint32_t>(a.heads), q = i32 / wd32, n32 = q / hd32;
  const int64_t w = i32 - q * wd32, h = q - n32 * hd32, n = n32;
  const int64_t t = a.start + n;
  const uint32_t word = static_cast<const uint32_t *>(a.value_code)[h * a.vc_sh + t * a.vc_st + w];
  const int64_t so = h * a.vs_sh + t * a.vs_st + ((w * CPW) >> a.lg) * a.vs_sg;
  const float s = load_dyn(a.value_scale, so, a.sd), m = load_dyn(a.value_min, so, a.sd);
  const int64_t o = (a.offset + n) * a.o_st + h * a.o_sh + w * CPW;
  float v[CPW];
#pragma unroll
  for (int p = 0; p < CPW; ++p) v[p] = add_rn(mul_rn(float((word >> (p * BITS)) & kMask), s), m);
  if (VEC) {  // CPW contiguous outputs as whole 16-byte stores
    constexpr int kPer16 = OD == UC_FP32 ? 4 : 8;
#pragma unroll
    for (int q = 0; q < CPW / kPer16; ++q) {
      uint32_t r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (OD == UC_FP32) {
          r[e] = __float_as_uint(v[q * 4 + e]);
        } else {
          const float lo = v[q * 8 + 2 * e], hi = v[q * 8 + 2 * e + 1];
          r[e] = (OD == UC_BF16 ? f32_to_bf16_bits(lo) : f32_to_f16_bits(lo)) |
                 (uint32_t(OD == UC_BF16 ? f32_to_bf16_bits(hi) : f32_to_f16_bits(hi)) << 16);
        }
      }
      *reinterpret_cast<uint4 *>(static_cast<char *>(a.out_value) + (o + q * kPer16) * (OD == UC_FP32 ? 4 : 2)) =
          make_uint4(r[0], r[1], r[2], r[3]);
    }
  } else {
#pragma unroll
    for (int p = 0; p < CPW; p += 2) store_pair<OD>(a.out_value, o + p, v[p], v[p + 1]);
  }
}

template <int BITS, int OD, bool VEC>
__global__ __launch_bounds__(256) void dequant_value_native_kernel(DequantArgs a) {
  dequant_value_native_block<BITS, OD, VEC>(a, blockIdx.x);
}

// Keys (the first key_blocks workgroups, octet form) and values of equal bits
// in one launch.
template <int BITS, int OD, int SD, bool VEC>
__global__ __launch_bounds__(256) void dequant_kv_kernel(DequantArgs a, int64_t runs, int64_t key_blocks) {
  const int64_t b = blockIdx.x;
  if (b < key_blocks)
    dequant_key_octet_block<BITS, OD, SD>(a, runs, b);
  else
    dequant_value_native_block<BITS, OD, VEC>(a, b - key_blocks);
}

// ----------------------------------------------------------- fake quant --
struct FakeQuantArgs {
  const void *data;
  int64_t st, sh, sd;
  int64_t tokens, heads, head_dim;
  int dim;
  int64_t group;  // effective group width min(group_size, length)
  float max_code;
  void *out;
};

// One thread per (group, fixed coordinates): two passes over the group
// (min/max, then quantize-dequantize), following builtin.py:42-53.
template <int DT>
__global__ __launch_bounds__(256) void fake_quant_kernel(FakeQuantArgs a) {
  const int64_t length = a.dim == 0 ? a.tokens : a.head_dim;
  const int64_t groups = (length + a.group - 1) / a.group;
  // fixed coordinates: (heads, head_dim) for dim 0, (tokens, heads) for dim 2
  const int64_t fixed = a.dim == 0 ? a.heads * a.head_dim : a.tokens * a.heads;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= fixed * groups) return;
  const int64_t f = idx % fixed;  // fixed coordinate varies fastest for coalescing
  const int64_t g = idx / fixed;
  int64_t base, step;
  if (a.dim == 0) {
    const int64_t d = f % a.head_dim, h = f / a.head_dim;
    base = h * a.sh + d * a.sd;
    step = a.st;
  } else {
    const int64_t h = f % a.heads, t = f / a.heads;
    base = t * a.st + h * a.sh;
    step = a.sd;
  }
  const int64_t start = g * a.group;
  const int64_t stop = min(length, start + a.group);
  GroupRange r;
  r.init(load_as_f32<DT>(a.data, base + start * step));
  for (int64_t i = start + 1; i < stop; ++i) r.add(load_as_f32<DT>(a.data, base + i * step));
  r.finish();
  const float mn = r.mn;
  const float scale = div_rn(clamp_min_nan(sub_rn(r.mx, mn), kEps), a.max_code);
  const float rcp_scale = __builtin_amdgcn_rcpf(scale);
  for (int64_t i = start; i < stop; ++i) {
    const float x = load_as_f32<DT>(a.data, base + i * step);
    const float code = fminf(fmaxf(quant_rint(sub_rn(x, mn), scale, rcp_scale), 0.0f), a.max_code);
    store_from_f32<DT>(a.out, base + i * step, add_rn(mul_rn(code, scale), mn));
  }
}

// Groups along tokens, 16-bit data with unit channel stride: lane = (group,
// head, channel pair), channel pairs fastest, the group's values held in
// registers (one read, one write of every element).
template <int DT, int GM>
__global__ __launch_bounds__(256) void fake_quant_tokens_kernel(FakeQuantArgs a) {
  const int64_t pairs = a.head_dim / 2, groups = (a.tokens + a.group - 1) / a.group;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= groups * a.heads * pairs) return;
  const int64_t cp = idx % pairs, h = (idx / pairs) % a.heads, g = idx / (pairs * a.heads);
  const int64_t t0 = g * a.group, n = min(a.group, a.tokens - t0);
  const int64_t base = t0 * a.st + h * a.sh + 2 * cp;
  float x0[GM], x1[GM];
#pragma unroll
  for (int i = 0; i < GM; ++i) {
    const uint32_t pair = i < n ? *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(a.data) + base +
                                                                       i * a.st)
                                : 0u;
    x0[i] = half_bits_to_f32<DT>(pair);
    x1[i] = half_bits_to_f32<DT>(pair >> 16);
  }
  GroupRange r0, r1;
  r0.init(x0[0]);
  r1.init(x1[0]);
#pragma unroll
  for (int i = 1; i < GM; ++i) {
    if (i < n) {
      r0.add(x0[i]);
      r1.add(x1[i]);
    }
  }
  r0.finish();
  r1.finish();
  const float mn0 = r0.mn, mn1 = r1.mn;
  const float s0 = div_rn(clamp_min_nan(sub_rn(r0.mx, mn0), kEps), a.max_code);
  const float s1 = div_rn(clamp_min_nan(sub_rn(r1.mx, mn1), kEps), a.max_code);
  const float rcp_s0 = __builtin_amdgcn_rcpf(s0), rcp_s1 = __builtin_amdgcn_rcpf(s1);
#pragma unroll
  for (int i = 0; i < GM; ++i) {
    if (i < n) {
      const float c0 = fminf(fmaxf(quant_rint(sub_rn(x0[i], mn0), s0, rcp_s0), 0.0f), a.max_code);
      const float c1 = fminf(fmaxf(quant_rint(sub_rn(x1[i], mn1), s1, rcp_s1), 0.0f), a.max_code);
      store_pair<DT>(a.out, base + i * a.st, add_rn(mul_rn(c0, s0), mn0), add_rn(mul_rn(c1, s1), mn1));
    }
  }
}

// Fake-quant value of one element of a group whose scale s is finite with a
// normal reciprocal r (builtin.py:42-53): the code is rint((x - mn) * r), the
// correctly rounded division deciding within (max_code + 1) 2^-20 of a half
// step, as in code_of (y lies in [0, max_code + 2^-20] here, so no clamp);
// then code * s + mn with two roundings.  `near` = 0.5 - (max_code + 1) 2^-20.
__device__ __forceinline__ float fake_value(float x, float mn, float s, float r, float near) {
  const float d = sub_rn(x, mn);
  const float y = mul_rn(d, r);
  float q = rintf(y);
  if (fabsf(sub_rn(y, q)) >= near) q = rintf(div_rn(d, s));
  return add_rn(mul_rn(q, s), mn);
}

// The generic arithmetic (quant_rint and the clamp) for the other groups.
__device__ __forceinline__ float fake_value_generic(float x, float mn, float s, float r, float max_code) {
  const float q = fminf(fmaxf(quant_rint(sub_rn(x, mn), s, r), 0.0f), max_code);
  return add_rn(mul_rn(q, s), mn);
}

// fake quant's scale (builtin.py:50: clamp, then divide) from a NaN-propagating
// range; a NaN range gives the canonical NaN of GroupRange
__device__ __forceinline__ float fake_scale(float &mn, float &mx, float max_code) {
  if (mn != mn) {
    mn = __builtin_nanf("");
    mx = mn;
  }
  return div_rn(clamp_min_nan(sub_rn(mx, mn), kEps), max_code);
}

// Two 16-bit results packed, each rounded to nearest even (NaN canonical for
// bf16, as torch's casts).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float v0, float v1) {
  return DT == UC_BF16 ? (uint32_t(f32_to_bf16_bits(v0)) | (uint32_t(f32_to_bf16_bits(v1)) << 16))
                       : (uint32_t(f32_to_f16_bits(v0)) | (uint32_t(f32_to_f16_bits(v1)) << 16));
}

// The same for head_dim 128 with the group's tokens split over the four
// waves of a workgroup (workgroup = (group, head), lane = channel pair): each
// wave holds TPW tokens in registers as raw 16-bit pairs, the four partial
// ranges (IEEE minimum / maximum, NaN-propagating) meet in LDS, then every wave
// quantizes its own tokens.
template <int DT, int TPW>
__global__ __launch_bounds__(256) void fake_quant_tokens_split_kernel(FakeQuantArgs a) {
  __shared__ float rmn[4][2 * kWave], rmx[4][2 * kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t g = blockIdx.x / a.heads, h = blockIdx.x % a.heads;
  const int64_t t0 = g * a.group, n = min(a.group, a.tokens - t0);
  const int64_t w0 = int64_t(wave) * TPW;  // this wave's first token of the group
  const int64_t base = (t0 + w0) * a.st + h * a.sh + 2 * lane;
  uint32_t raw[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i)
    raw[i] = w0 + i < n ? *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(a.data) + base +
                                                              i * a.st)
                        : 0u;
  float mn0 = __builtin_inff(), mx0 = -__builtin_inff(), mn1 = __builtin_inff(), mx1 = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    if (w0 + i < n) {
      const float x0 = half_bits_to_f32<DT>(raw[i]), x1 = half_bits_to_f32<DT>(raw[i] >> 16);
      mn0 = min_nan(mn0, x0);
      mx0 = max_nan(mx0, x0);
      mn1 = min_nan(mn1, x1);
      mx1 = max_nan(mx1, x1);
    }
  }
  rmn[wave][2 * lane] = mn0;
  rmn[wave][2 * lane + 1] = mn1;
  rmx[wave][2 * lane] = mx0;
  rmx[wave][2 * lane + 1] = mx1;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mn0 = min_nan(mn0, rmn[w][2 * lane]);
    mn1 = min_nan(mn1, rmn[w][2 * lane + 1]);
    mx0 = max_nan(mx0, rmx[w][2 * lane]);
    mx1 = max_nan(mx1, rmx[w][2 * lane + 1]);
  }
  const float s0 = fake_scale(mn0, mx0, a.max_code), s1 = fake_scale(mn1, mx1, a.max_code);
  const float r0 = __builtin_amdgcn_rcpf(s0), r1 = __builtin_amdgcn_rcpf(s1);
  const float near = 0.5f - (a.max_code + 1.0f) * 0x1p-20f;
  uint16_t *out = static_cast<uint16_t *>(a.out);
  if (fast_group(s0, r0) && fast_group(s1, r1)) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      if (w0 + i < n) {
        const float v0 = fake_value(half_bits_to_f32<DT>(raw[i]), mn0, s0, r0, near);
        const float v1 = fake_value(half_bits_to_f32<DT>(raw[i] >> 16), mn1, s1, r1, near);
        *reinterpret_cast<uint32_t *>(out + base + i * a.st) = pack2<DT>(v0, v1);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      if (w0 + i < n) {
        const float v0 = fake_value_generic(half_bits_to_f32<DT>(raw[i]), mn0, s0, r0, a.max_code);
        const float v1 = fake_value_generic(half_bits_to_f32<DT>(raw[i] >> 16), mn1, s1, r1, a.max_code);
        *reinterpret_cast<uint32_t *>(out + base + i * a.st) = pack2<DT>(v0, v1);
      }
    }
  }
}

// Groups along channels (8 to 64 channels, dividing head_dim), 16-bit data
// with unit channel stride: lane = 8 channels of one (token, head), a group
// spans group/8 neighbouring lanes reduced with shuffles.
template <int DT>
__global__ __launch_bounds__(256) void fake_quant_channels_kernel(FakeQuantArgs a, int lanes_per_group) {
  const int64_t chunks = a.head_dim / 8;
  const int64_t total = a.tokens * a.heads * chunks;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool active = idx < total;  // whole groups are active or not: total is a multiple of the group lanes
  // 32-bit divisions: the launch keeps tokens * heads * chunks below 2^31
  const uint32_t k = active ? static_cast<uint32_t>(idx) : 0u, c32 = static_cast<uint32_t>(chunks);
  const uint32_t h32 = static_cast<uint32_t>(a.heads), q = k / c32, t32 = q / h32;
  const int64_t ch = k - q * c32, h = q - t32 * h32, t = t32;
  const int64_t off = t * a.st + h * a.sh + 8 * ch;
  const uint4 raw = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.data) + off);
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float x[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = half_bits_to_f32<DT>(w[j]);
    x[2 * j + 1] = half_bits_to_f32<DT>(w[j] >> 16);
  }
  float mn = x[0], mx = x[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) {
    mn = min_nan(mn, x[j]);
    mx = max_nan(mx, x[j]);
  }
  for (int o = 1; o < lanes_per_group; o <<= 1) {
    mn = min_nan(mn, __shfl_xor(mn, o, kWave));
    mx = max_nan(mx, __shfl_xor(mx, o, kWave));
  }
  if (!active) return;
  const float s = fake_scale(mn, mx, a.max_code);
  const float r = __builtin_amdgcn_rcpf(s);
  uint32_t o[4];
  if (fast_group(s, r)) {
    const float near = 0.5f - (a.max_code + 1.0f) * 0x1p-20f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack2<DT>(fake_value(x[2 * j], mn, s, r, near), fake_value(x[2 * j + 1], mn, s, r, near));
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack2<DT>(fake_value_generic(x[2 * j], mn, s, r, a.max_code),
                       fake_value_generic(x[2 * j + 1], mn, s, r, a.max_code));
  }
  *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.out) + off) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace
}  // namespace uc

using namespace uc;

extern "C" int uc_kivi_pack(const void *key, int64_t k_st, int64_t k_sh, int64_t k_sd,
                            const void *value, int64_t v_st, int64_t v_sh, int64_t v_sd,
                            int in_dtype, int64_t tokens, int64_t heads, int64_t head_dim,
                            int k_bits, int v_bits, int group_size, int stats_dtype,
                            void *key_code, int64_t kc_sh, int64_t kc_sd, int64_t kc_sw,
                            void *key_scale, void *key_min, int64_t ks_sh, int64_t ks_sd, int64_t ks_sg,
                            void *value_code, int64_t vc_sh, int64_t vc_st, int64_t vc_sw,
                            void *value_scale, void *value_min, int64_t vs_sh, int64_t vs_st, int64_t vs_sg,
                            uc_stream_t stream) {
  UC_REQUIRE(valid_dtype(in_dtype) && valid_dtype(stats_dtype), "uc_kivi_pack: unknown dtype code");
  UC_REQUIRE(k_bits == 2 || k_bits == 4 || k_bits == 8, "KIVI physical cache supports 2, 4, or 8 bit payloads");
  UC_REQUIRE(v_bits == 2 || v_bits == 4 || v_bits == 8, "KIVI physical cache supports 2, 4, or 8 bit payloads");
  UC_REQUIRE(group_size > 0, "KIVI physical cache group_size must be positive");
  UC_REQUIRE(tokens >= 0 && heads > 0 && head_dim > 0, "uc_kivi_pack: bad shape");
  UC_REQUIRE(tokens % group_size == 0, "uc_kivi_pack: tokens (%lld) must be a multiple of group_size",
             (long long)tokens);
  UC_REQUIRE(head_dim <= 1024, "uc_kivi_pack: head_dim must be <= 1024");
  if (tokens == 0) return UC_OK;
  PackArgs a{};
  a.key = key; a.k_st = k_st; a.k_sh = k_sh; a.k_sd = k_sd;
  a.value = value; a.v_st = v_st; a.v_sh = v_sh; a.v_sd = v_sd;
  a.tokens = tokens; a.heads = heads; a.head_dim = head_dim; a.stats_dtype = stats_dtype;
  a.key_code = key_code; a.kc_sh = kc_sh; a.kc_sd = kc_sd; a.kc_sw = kc_sw;
  a.key_scale = key_scale; a.key_min = key_min; a.ks_sh = ks_sh; a.ks_sd = ks_sd; a.ks_sg = ks_sg;
  a.value_code = value_code; a.vc_sh = vc_sh; a.vc_st = vc_st; a.vc_sw = vc_sw;
  a.value_scale = value_scale; a.value_min = value_min; a.vs_sh = vs_sh; a.vs_st = vs_st; a.vs_sg = vs_sg;
  hipStream_t s = as_stream(stream);
  if (!tuned_group(group_size, head_dim)) {
    // any other group size, and value rows with a partial last group
    GenericPackArgs g{};
    g.p = a;
    g.group = group_size;
    g.kb = k_bits;
    g.vb = v_bits;
    const int64_t kpw = k_bits == 8 ? 1 : 32 / k_bits, vpw = v_bits == 8 ? 1 : 32 / v_bits;
    g.kspan = group_size / gcd64(group_size, kpw) * kpw;
    g.vspan = group_size / gcd64(group_size, vpw) * vpw;
    g.kthreads = key ? heads * head_dim * ((tokens + g.kspan - 1) / g.kspan) : 0;
    g.vthreads = value ? heads * tokens * ((head_dim + g.vspan - 1) / g.vspan) : 0;
    const dim3 grid(static_cast<unsigned>(ceil_div(g.kthreads + g.vthreads, int64_t(kPackThreads))));
    if (in_dtype == UC_BF16)
      hipLaunchKernelGGL((kivi_pack_generic_kernel<UC_BF16>), grid, dim3(kPackThreads), 0, s, g);
    else if (in_dtype == UC_FP16)
      hipLaunchKernelGGL((kivi_pack_generic_kernel<UC_FP16>), grid, dim3(kPackThreads), 0, s, g);
    else
      hipLaunchKernelGGL((kivi_pack_generic_kernel<UC_FP32>), grid, dim3(kPackThreads), 0, s, g);
    return check_launch("uc_kivi_pack");
  }
  if (fast_pack_fits(a, in_dtype, k_bits, v_bits, group_size)) {
    if (in_dtype == UC_BF16) {
      if (k_bits == 2) launch_pack_fast<UC_BF16, 2>(a, group_size, s);
      else launch_pack_fast<UC_BF16, 4>(a, group_size, s);
    } else {
      if (k_bits == 2) launch_pack_fast<UC_FP16, 2>(a, group_size, s);
      else launch_pack_fast<UC_FP16, 4>(a, group_size, s);
    }
    return check_launch("uc_kivi_pack");
  }
  const int64_t slabs = (head_dim + 127) / 128;
  a.key_waves = key ? heads * (tokens / group_size) * slabs : 0;
  const int64_t lanes_per_token = head_dim / 16;
  const int64_t tokens_per_wave = kWave / lanes_per_token;
  a.value_waves = value ? heads * ceil_div(ceil_div(tokens, tokens_per_wave), int64_t(kVRuns)) : 0;
  const bool half = half_dtype(in_dtype);
  const bool kvec = half && k_sd == 1 && (k_st % 2 == 0) && (k_sh % 2 == 0) && aligned(key, 4);
  const bool vvec = half && v_sd == 1 && (v_st % 8 == 0) && (v_sh % 8 == 0) && aligned(value, 16);
  // 16-bit inputs only take the vectorised path; fp32 inputs use scalar loads
  auto go = [&](auto in_tag) {
    constexpr int IN = decltype(in_tag)::value;
    switch (group_size) {
      case 16: launch_pack<IN, 16>(a, k_bits, v_bits, kvec, vvec, s); break;
      case 32: launch_pack<IN, 32>(a, k_bits, v_bits, kvec, vvec, s); break;
      case 64: launch_pack<IN, 64>(a, k_bits, v_bits, kvec, vvec, s); break;
      default: launch_pack<IN, 128>(a, k_bits, v_bits, kvec, vvec, s); break;
    }
  };
  if (in_dtype == UC_BF16) go(std::integral_constant<int, UC_BF16>{});
  else if (in_dtype == UC_FP16) go(std::integral_constant<int, UC_FP16>{});
  else go(std::integral_constant<int, UC_FP32>{});
  return check_launch("uc_kivi_pack");
}

extern "C" int uc_kivi_dequant(const void *key_code, int64_t kc_sh, int64_t kc_sd, int64_t kc_sw,
                               const void *key_scale, const void *key_min, int64_t ks_sh, int64_t ks_sd, int64_t ks_sg,
                               const void *value_code, int64_t vc_sh, int64_t vc_st, int64_t vc_sw,
                               const void *value_scale, const void *value_min, int64_t vs_sh, int64_t vs_st, int64_t vs_sg,
                               int stats_dtype, int64_t heads, int64_t head_dim,
                               int k_bits, int v_bits, int group_size, int64_t start, int64_t stop,
                               void *out_key, void *out_value, int out_dtype,
                               int64_t o_st, int64_t o_sh, int64_t o_sd, int64_t output_offset,
                               uc_stream_t stream) {
  UC_REQUIRE(valid_dtype(stats_dtype) && valid_dtype(out_dtype), "uc_kivi_dequant: unknown dtype code");
  UC_REQUIRE(k_bits == 2 || k_bits == 4 || k_bits == 8, "KIVI physical cache supports 2, 4, or 8 bit payloads");
  UC_REQUIRE(v_bits == 2 || v_bits == 4 || v_bits == 8, "KIVI physical cache supports 2, 4, or 8 bit payloads");
  UC_REQUIRE(group_size > 0, "KIVI physical cache group_size must be positive");
  UC_REQUIRE(heads > 0 && head_dim > 0 && start >= 0 && stop >= start && output_offset >= 0,
             "uc_kivi_dequant: bad range");
  UC_REQUIRE(key_code == nullptr || out_key != nullptr, "uc_kivi_dequant: missing key output");
  UC_REQUIRE(value_code == nullptr || out_value != nullptr, "uc_kivi_dequant: missing value output");
  const int64_t count = stop - start;
  if (count == 0) return UC_OK;
  DequantArgs a{};
  a.key_code = key_code; a.kc_sh = kc_sh; a.kc_sd = kc_sd; a.kc_sw = kc_sw;
  a.key_scale = key_scale; a.key_min = key_min; a.ks_sh = ks_sh; a.ks_sd = ks_sd; a.ks_sg = ks_sg;
  a.value_code = value_code; a.vc_sh = vc_sh; a.vc_st = vc_st; a.vc_sw = vc_sw;
  a.value_scale = value_scale; a.value_min = value_min; a.vs_sh = vs_sh; a.vs_st = vs_st; a.vs_sg = vs_sg;
  a.heads = heads; a.head_dim = head_dim; a.start = start; a.count = count;
  a.out_key = out_key; a.out_value = out_value;
  a.o_st = o_st; a.o_sh = o_sh; a.o_sd = o_sd; a.offset = output_offset;
  const int64_t total = 2 * count * heads * head_dim;
  const int64_t blocks = ceil_div(total, 256);
  a.lg = group_size == 16 ? 4 : group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
  a.group = group_size;
  a.sd = stats_dtype; a.od = out_dtype;
  hipStream_t s = as_stream(stream);
  // native 2/4-bit layout with pairwise-aligned unit-stride output rows
  const int out_bytes = out_dtype == UC_FP32 ? 4 : 2;
  const bool out_ok = o_sd == 1 && o_st % 2 == 0 && o_sh % 2 == 0 && head_dim % 32 == 0 &&
                      (out_key == nullptr || aligned(out_key, 2 * out_bytes)) &&
                      (out_value == nullptr || aligned(out_value, 2 * out_bytes));
  // word-major (UniCache's kernel-native tensors) or token-major (this
  // library's native storage) key codes
  const bool key_native = key_code != nullptr && (k_bits == 2 || k_bits == 4) && (kc_sw == 1 || kc_sd == 1);
  const bool value_native = value_code != nullptr && (v_bits == 2 || v_bits == 4) && vc_sw == 1;
  if (out_ok && tuned_group(group_size, head_dim) && (key_code == nullptr || key_native) &&
      (value_code == nullptr || value_native)) {
    UC_REQUIRE(heads * (count + 64) * head_dim < (int64_t(1) << 31),
               "uc_kivi_dequant: chunk too large for one call (%lld tokens x %lld heads)", (long long)count,
               (long long)heads);
    UC_DISPATCH_DTYPE(out_dtype, OD, [&] {
      // token-major words and stats (channel stride 1), 16-bit stats and
      // output, 16-byte aligned rows: the octet kernel
      const bool octet = key_code != nullptr && kc_sd == 1 && ks_sd == 1 && OD != UC_FP32 && stats_dtype != UC_FP32 &&
                         head_dim % 8 == 0 && kc_sw % 4 == 0 && kc_sh % 4 == 0 && ks_sg % 8 == 0 && ks_sh % 8 == 0 &&
                         o_st % 8 == 0 && o_sh % 8 == 0 && aligned(key_code, 16) && aligned(key_scale, 16) &&
                         aligned(key_min, 16) && aligned(out_key, 16);
      const int64_t per16 = 16 / out_bytes;
      const bool vvec = value_code != nullptr && aligned(out_value, 16) && o_st % per16 == 0 && o_sh % per16 == 0 &&
                        (32 / v_bits) % per16 == 0;
      if (octet && value_code != nullptr && k_bits == v_bits && vvec) {
        // keys and values in one launch
        const int tpw = 32 / k_bits;
        const int64_t words = (start + count + tpw - 1) / tpw - start / tpw;
        const int64_t runs = ceil_div(words, int64_t(kDqOctetWords));
        const int64_t key_blocks = ceil_div(heads * runs * (head_dim / 8), int64_t(256));
        const int64_t value_blocks = ceil_div(heads * count * (head_dim * v_bits / 32), int64_t(256));
        const dim3 grid(static_cast<unsigned>(key_blocks + value_blocks));
        auto go_kv = [&](auto sd_tag) {
          constexpr int SD = decltype(sd_tag)::value;
          if (k_bits == 2)
            hipLaunchKernelGGL((dequant_kv_kernel<2, OD, SD, true>), grid, dim3(256), 0, s, a, runs, key_blocks);
          else
            hipLaunchKernelGGL((dequant_kv_kernel<4, OD, SD, true>), grid, dim3(256), 0, s, a, runs, key_blocks);
        };
        if (stats_dtype == UC_BF16) go_kv(std::integral_constant<int, UC_BF16>{});
        else go_kv(std::integral_constant<int, UC_FP16>{});
        return;
      }
      if (octet) {
        const int tpw = 32 / k_bits;
        const int64_t words = (start + count + tpw - 1) / tpw - start / tpw;
        const int64_t runs = ceil_div(words, int64_t(kDqOctetWords));
        const dim3 grid(static_cast<unsigned>(ceil_div(heads * runs * (head_dim / 8), int64_t(256))));
        auto go_key = [&](auto sd_tag) {
          constexpr int SD = decltype(sd_tag)::value;
          if (k_bits == 2)
            hipLaunchKernelGGL((dequant_key_octet_kernel<2, OD, SD>), grid, dim3(256), 0, s, a, runs);
          else
            hipLaunchKernelGGL((dequant_key_octet_kernel<4, OD, SD>), grid, dim3(256), 0, s, a, runs);
        };
        if (stats_dtype == UC_BF16) go_key(std::integral_constant<int, UC_BF16>{});
        else go_key(std::integral_constant<int, UC_FP16>{});
      } else if (key_code != nullptr) {
        const int tpw = 32 / k_bits;
        const int64_t words = (start + count + tpw - 1) / tpw - start / tpw;
        const int64_t runs = ceil_div(words, int64_t(kDqRunWords));
        const int64_t n = heads * runs * (head_dim / 2);
        if (k_bits == 2)
          hipLaunchKernelGGL((dequant_key_native_kernel<2, OD>), dim3(ceil_div(n, 256)), dim3(256), 0, s, a, runs);
        else
          hipLaunchKernelGGL((dequant_key_native_kernel<4, OD>), dim3(ceil_div(n, 256)), dim3(256), 0, s, a, runs);
      }
      if (value_code != nullptr) {
        const int64_t n = heads * count * (head_dim * v_bits / 32);
        // 16-byte stores when every run of a word's channels starts on 16 bytes
        const bool vec = vvec;
        auto go = [&](auto vec_tag) {
          constexpr bool VEC = decltype(vec_tag)::value;
          if (v_bits == 2)
            hipLaunchKernelGGL((dequant_value_native_kernel<2, OD, VEC>), dim3(ceil_div(n, 256)), dim3(256), 0, s, a);
          else
            hipLaunchKernelGGL((dequant_value_native_kernel<4, OD, VEC>), dim3(ceil_div(n, 256)), dim3(256), 0, s, a);
        };
        if (vec) go(std::true_type{});
        else go(std::false_type{});
      }
    });
    return check_launch("uc_kivi_dequant");
  }
  UC_DISPATCH_BITS(k_bits, KB, [&] {
    UC_DISPATCH_BITS(v_bits, VB, [&] {
      hipLaunchKernelGGL((kivi_dequant_kernel<KB, VB>), dim3(blocks), dim3(256), 0, s, a);
    });
  });
  return check_launch("uc_kivi_dequant");
}

extern "C" int uc_kivi_fake_quant(const void *data, int64_t st, int64_t sh, int64_t sd,
                                  int dtype, int64_t tokens, int64_t heads, int64_t head_dim,
                                  int bits, int dim, int group_size,
                                  void *out, uc_stream_t stream) {
  UC_REQUIRE(valid_dtype(dtype), "uc_kivi_fake_quant: unknown dtype code");
  UC_REQUIRE(bits == 2 || bits == 3 || bits == 4 || bits == 8, "Unsupported fake quant bits: %d", bits);
  UC_REQUIRE(dim == 0 || dim == 2, "uc_kivi_fake_quant: dim must be 0 (tokens) or 2 (channels)");
  UC_REQUIRE(tokens >= 0 && heads >= 0 && head_dim >= 0, "uc_kivi_fake_quant: bad shape");
  const int64_t length = dim == 0 ? tokens : head_dim;
  if (tokens == 0 || heads == 0 || head_dim == 0) return UC_OK;
  FakeQuantArgs a{};
  a.data = data; a.st = st; a.sh = sh; a.sd = sd;
  a.tokens = tokens; a.heads = heads; a.head_dim = head_dim; a.dim = dim;
  a.group = group_size <= 0 ? 1 : (group_size < length ? group_size : length);
  a.max_code = float((1 << bits) - 1);
  a.out = out;
  const int64_t groups = ceil_div(length, a.group);
  const int64_t fixed = dim == 0 ? heads * head_dim : tokens * heads;
  const int64_t blocks = ceil_div(fixed * groups, 256);
  hipStream_t s = as_stream(stream);
  const bool half = dtype == UC_BF16 || dtype == UC_FP16;
  if (half && dim == 0 && sd == 1 && head_dim == 2 * kWave && st % 2 == 0 && sh % 2 == 0 && aligned(data, 4) &&
      aligned(out, 4) && a.group <= 64) {
    const dim3 grid(static_cast<unsigned>(groups * heads));
    UC_DISPATCH_DTYPE(dtype, DT, [&] {
      if constexpr (DT != UC_FP32) {
        if (a.group <= 16)
          hipLaunchKernelGGL((fake_quant_tokens_split_kernel<DT, 4>), grid, dim3(256), 0, s, a);
        else if (a.group <= 32)
          hipLaunchKernelGGL((fake_quant_tokens_split_kernel<DT, 8>), grid, dim3(256), 0, s, a);
        else
          hipLaunchKernelGGL((fake_quant_tokens_split_kernel<DT, 16>), grid, dim3(256), 0, s, a);
      }
    });
    return check_launch("uc_kivi_fake_quant");
  }
  if (half && dim == 0 && sd == 1 && head_dim % 2 == 0 && st % 2 == 0 && sh % 2 == 0 && aligned(data, 4) &&
      aligned(out, 4) && a.group <= 64) {
    const int64_t n = groups * heads * (head_dim / 2);
    const dim3 grid(static_cast<unsigned>(ceil_div(n, 256)));
    UC_DISPATCH_DTYPE(dtype, DT, [&] {
      if constexpr (DT != UC_FP32) {
        if (a.group <= 16)
          hipLaunchKernelGGL((fake_quant_tokens_kernel<DT, 16>), grid, dim3(256), 0, s, a);
        else if (a.group <= 32)
          hipLaunchKernelGGL((fake_quant_tokens_kernel<DT, 32>), grid, dim3(256), 0, s, a);
        else
          hipLaunchKernelGGL((fake_quant_tokens_kernel<DT, 64>), grid, dim3(256), 0, s, a);
      }
    });
    return check_launch("uc_kivi_fake_quant");
  }
  const int64_t lanes = a.group / 8;
  if (half && dim == 2 && sd == 1 && a.group % 8 == 0 && (lanes == 1 || lanes == 2 || lanes == 4 || lanes == 8) &&
      head_dim % a.group == 0 && st % 8 == 0 && sh % 8 == 0 && aligned(data, 16) && aligned(out, 16)) {
    const int64_t n = tokens * heads * (head_dim / 8);
    UC_REQUIRE(tokens * heads * (head_dim / 8) < (int64_t(1) << 31), "uc_kivi_fake_quant: too many elements for one call");
    const dim3 grid(static_cast<unsigned>(ceil_div(n, 256)));
    UC_DISPATCH_DTYPE(dtype, DT, [&] {
      if constexpr (DT != UC_FP32)
        hipLaunchKernelGGL((fake_quant_channels_kernel<DT>), grid, dim3(256), 0, s, a, static_cast<int>(lanes));
    });
    return check_launch("uc_kivi_fake_quant");
  }
  UC_DISPATCH_DTYPE(dtype, DT, [&] {
    hipLaunchKernelGGL((fake_quant_kernel<DT>), dim3(blocks), dim3(256), 0, s, a);
  });
  return check_launch("uc_kivi_fake_quant");
}
