// MFMA fragment types, fp16 code extraction and buffer-resource loads shared
// by the packed-attention kernels (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace uc {
namespace mf {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;  // head_dim of the MFMA kernels
constexpr float kNegInf = -__builtin_huge_valf();

// Geometry of `BITS`-bit KIVI words.
template <int BITS>
struct Geo {
  static constexpr int TPW = 32 / BITS;            // tokens per key word = channels per value word
  static constexpr int ST = 16 * TPW;              // tokens of 16 consecutive key words
  static constexpr int VW = kD / TPW;              // value words per token
  static constexpr int PMAX = (10 - BITS) / BITS;  // last position whose code fits the fp16 mantissa
  static constexpr int SH = BITS * (PMAX + 1);     // shift that brings the other positions down
  static constexpr uint32_t MASK = (1u << BITS) - 1u;
};

__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }

__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) { return (x & m) | c; }

// 2^x on the hardware exp unit; -inf gives 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ _Float16 to_h(float x) { return static_cast<_Float16>(x); }

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h4 cvt4(f4 v) { return h4{to_h(v[0]), to_h(v[1]), to_h(v[2]), to_h(v[3])}; }

// Two codes at position `pe` of the 16-bit halves of `src` as fp16
// (code * 2^(BITS*pe)): the bits are OR-ed into the mantissa of 1024 and 1024
// is subtracted exactly.
template <int BITS>
__device__ __forceinline__ h2 code_pair(uint32_t src, int pe) {
  const uint32_t mask = (Geo<BITS>::MASK << (BITS * pe)) | (Geo<BITS>::MASK << (16 + BITS * pe));
  return as_h2(and_or(src, mask, 0x64006400u)) - h2{to_h(1024.0f), to_h(1024.0f)};
}

// Eight 16-bit values (bf16 or fp16, dtype code D) from 16 aligned bytes, as fp16.
template <int D>
__device__ __forceinline__ h8 halves_to_h8(uint4 raw) {
  if constexpr (D == 1) {  // UC_FP16: already fp16
    return __builtin_bit_cast(h8, raw);
  } else {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    h8 out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[2 * j] = to_h(__builtin_bit_cast(float, w[j] << 16));
      out[2 * j + 1] = to_h(__builtin_bit_cast(float, w[j] & 0xffff0000u));
    }
    return out;
  }
}

// Max / sum over the four lanes n, n+16, n+32, n+48 (the k-slices of one
// MFMA column) with the gfx950 lane-swap instructions (VALU, no LDS trip).
__device__ __forceinline__ float max_over_slices(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  const float y = fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(a[0])),
                        __builtin_bit_cast(float, static_cast<uint32_t>(a[1])));
  const auto b = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, y), __builtin_bit_cast(uint32_t, y),
                                                  false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(b[0])),
               __builtin_bit_cast(float, static_cast<uint32_t>(b[1])));
}

__device__ __forceinline__ float sum_over_slices(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  const float y = __builtin_bit_cast(float, static_cast<uint32_t>(a[0])) +
                  __builtin_bit_cast(float, static_cast<uint32_t>(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, y), __builtin_bit_cast(uint32_t, y),
                                                  false, false);
  return __builtin_bit_cast(float, static_cast<uint32_t>(b[0])) +
         __builtin_bit_cast(float, static_cast<uint32_t>(b[1]));
}

// Buffer resources over one region: loads past `bytes` return zero.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kRsrcWord3 = 0x00020000;  // 32-bit data format, raw (stride 0) addressing

__device__ __forceinline__ Rsrc make_rsrc(const void *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), kRsrcWord3);
}
__device__ __forceinline__ uint32_t bload16(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bload32(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint2 bload64(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ uint4 bload128(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

}  // namespace mf
}  // namespace uc
