// Shared helpers for the gfx950 kernels of libunicache_hip.so: element
// conversions with explicit rounding, error reporting for the C ABI, and
// wavefront reductions.  Every kernel in this library is written for CDNA4
// (64-lane wavefronts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/unicache_hip.h"

namespace uc {

constexpr int kWave = 64;
constexpr float kEps = 1.1920928955078125e-07f;  // FLT_EPSILON == torch.finfo(float32).eps
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- errors --
void set_error(const char *fmt, ...);
void clear_error();
int check_launch(const char *what);

#define UC_REQUIRE(cond, ...)                 \
  do {                                        \
    if (!(cond)) {                            \
      ::uc::set_error(__VA_ARGS__);           \
      return UC_EINVAL;                       \
    }                                         \
  } while (0)

#define UC_REQUIRE_RT(cond, ...)              \
  do {                                        \
    if (!(cond)) {                            \
      ::uc::set_error(__VA_ARGS__);           \
      return UC_ERUNTIME;                     \
    }                                         \
  } while (0)

inline hipStream_t as_stream(uc_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Residual row strides of an item, in elements (token, KV head): both fields
// 0 mean token-major rows [Tr, Hkv, D].
__host__ __device__ inline void residual_strides(const uc_kivi_item &it, int64_t hkv, int64_t d, int64_t &ts,
                                                 int64_t &hs) {
  if (it.residual_token_stride == 0 && it.residual_head_stride == 0) {
    ts = hkv * d;
    hs = d;
  } else {
    ts = it.residual_token_stride;
    hs = it.residual_head_stride;
  }
}

// Division of n < 2^31 by a launch constant d >= 1 without a divide sequence:
// with l = ceil(log2 d) and m = floor(2^(31+l) / d) + 1 (< 2^32),
// floor(n / d) = (n m) >> (31 + l) exactly (m d - 2^(31+l) is in (0, d] <= 2^l,
// so the error term stays below 1/d).
struct FastDiv {
  uint32_t d, m, shift;
};

inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  const uint64_t m = ((uint64_t(1) << (31 + l)) / d) + 1;
  return FastDiv{d, static_cast<uint32_t>(m), 31 + l};
}

__host__ __device__ __forceinline__ uint32_t fast_div(uint32_t n, FastDiv f) {
  return static_cast<uint32_t>((uint64_t(n) * f.m) >> f.shift);
}

// Group range with the NaN rule of torch.amin / amax: a NaN anywhere in the
// group makes both bounds NaN (fminf / fmaxf alone would skip it).
struct GroupRange {
  float mn, mx;
  bool nan;
  __device__ __forceinline__ void init(float x) {
    mn = x;
    mx = x;
    nan = x != x;
  }
  __device__ __forceinline__ void add(float x) {
    mn = fminf(mn, x);
    mx = fmaxf(mx, x);
    nan = nan || x != x;
  }
  // fold in the range held by lane (lane ^ o)
  __device__ __forceinline__ void merge_xor(int o) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    nan = __shfl_xor(static_cast<int>(nan), o, 64) != 0 || nan;
  }
  __device__ __forceinline__ void finish() {
    if (nan) {
      mn = __builtin_nanf("");
      mx = mn;
    }
  }
};

// torch's clamp_min(v, lo): a NaN stays NaN.
__device__ __forceinline__ float clamp_min_nan(float v, float lo) { return v != v ? v : fmaxf(v, lo); }

inline bool valid_dtype(int d) { return d == UC_BF16 || d == UC_FP16 || d == UC_FP32; }
inline bool half_dtype(int d) { return d == UC_BF16 || d == UC_FP16; }

// ------------------------------------------------------------ conversions --
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// Round-to-nearest-even float -> bfloat16 with canonical NaN, the rounding of
// torch's Float->BFloat16 cast.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, b);
  return static_cast<float>(h);
}

// v_cvt_f16_f32 rounds to nearest even, like torch's Float->Half cast.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

// Load element `i` of a buffer of dtype D as float.
template <int D>
__device__ __forceinline__ float load_as_f32(const void *p, int64_t i) {
  if constexpr (D == UC_BF16) {
    return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  } else if constexpr (D == UC_FP16) {
    return f16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  } else {
    return static_cast<const float *>(p)[i];
  }
}

template <int D>
__device__ __forceinline__ void store_from_f32(void *p, int64_t i, float v) {
  if constexpr (D == UC_BF16) {
    static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
  } else if constexpr (D == UC_FP16) {
    static_cast<uint16_t *>(p)[i] = f32_to_f16_bits(v);
  } else {
    static_cast<float *>(p)[i] = v;
  }
}

// Storage type of a dtype code.
template <int D>
struct DtypeOf {
  typedef uint16_t T;
};
template <>
struct DtypeOf<UC_FP32> {
  typedef float T;
};

// Element `i` of a buffer whose dtype is only known at run time (uniform
// branch; used by the kernels that are not on the hot path).
__device__ __forceinline__ float load_dyn(const void *p, int64_t i, int dt) {
  if (dt == UC_BF16) return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  if (dt == UC_FP16) return f16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  return static_cast<const float *>(p)[i];
}

__device__ __forceinline__ void store_dyn(void *p, int64_t i, float v, int dt) {
  if (dt == UC_BF16) {
    static_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
  } else if (dt == UC_FP16) {
    static_cast<uint16_t *>(p)[i] = f32_to_f16_bits(v);
  } else {
    static_cast<float *>(p)[i] = v;
  }
}

// Value of a 16-bit element (bf16 or fp16) already in a register.
template <int D>
__device__ __forceinline__ float half_bits_to_f32(uint32_t b) {
  if constexpr (D == UC_BF16) {
    return bf16_bits_to_f32(b & 0xffffu);
  } else {
    return f16_bits_to_f32(static_cast<uint16_t>(b & 0xffffu));
  }
}

// Exact IEEE single-rounding arithmetic (never contracted into an FMA).
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float sub_rn(float a, float b) { return __fsub_rn(a, b); }
__device__ __forceinline__ float div_rn(float a, float b) { return __fdiv_rn(a, b); }

// rint(div_rn(d, s)), the code of a quantization step (round half to even),
// with the division replaced by a multiply by r = v_rcp_f32(s) wherever that
// cannot change the code.  r is within one ulp of 1/s, so y = RN(d r) is
// within |y| (2^-23 + 2^-24 + 2^-47) of d/s, and div_rn(d, s) within half an
// ulp (|y| 2^-24) of it: both lie within |y| 2^-22 of each other.  When y is
// farther than |y| 2^-20 from a half-integer they round to the same integer;
// otherwise -- or when y is not finite, or r is not a normal number (v_rcp_f32
// flushes denormal results) -- the correctly rounded division decides.
__device__ __forceinline__ float quant_rint(float d, float s, float r) {
  const float y = d * r;
  const float q = rintf(y);
  const float dist = fabsf(fabsf(y - q) - 0.5f);
  return dist > fabsf(y) * 0x1p-20f && r >= 0x1p-126f ? q : rintf(div_rn(d, s));
}

// Code `pos_in_word` of the word at `word_off` (2/4-bit, LSB first), or the
// byte at `word_off` for 8-bit codes (physical.py:88-104).
template <int BITS>
__device__ __forceinline__ uint32_t read_code(const void *code, int64_t word_off, int64_t pos_in_word) {
  if constexpr (BITS == 8) {
    return static_cast<const uint8_t *>(code)[word_off];
  } else {
    const uint32_t w = static_cast<const uint32_t *>(code)[word_off];
    return (w >> (pos_in_word * BITS)) & ((1u << BITS) - 1u);
  }
}

// ------------------------------------------------------------ reductions --
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Dispatch a runtime dtype code to a template parameter.
#define UC_DISPATCH_DTYPE(code, NAME, ...)                  \
  [&] {                                                     \
    switch (code) {                                         \
      case UC_BF16: { constexpr int NAME = UC_BF16; return __VA_ARGS__(); } \
      case UC_FP16: { constexpr int NAME = UC_FP16; return __VA_ARGS__(); } \
      default: { constexpr int NAME = UC_FP32; return __VA_ARGS__(); }      \
    }                                                       \
  }()

#define UC_DISPATCH_BITS(code, NAME, ...)                   \
  [&] {                                                     \
    switch (code) {                                         \
      case 2: { constexpr int NAME = 2; return __VA_ARGS__(); } \
      case 4: { constexpr int NAME = 4; return __VA_ARGS__(); } \
      default: { constexpr int NAME = 8; return __VA_ARGS__(); } \
    }                                                       \
  }()

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace uc
