// mfma_common.h — CDNA4 matrix-core helpers shared by the MFMA kernels:
// operand types, the 32x32x16 bf16/fp16 MFMA, RNE packing of fp32 pairs and
// in-register dequantization of one 32-code chunk.
#pragma once
#include "common.h"

namespace iqmm {

typedef __attribute__((ext_vector_type(8))) __bf16 g_bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 g_f16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) unsigned int g_u32x4_t;
typedef __attribute__((ext_vector_type(2))) float g_f2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 g_bf16x2_t;


template <int XT>
__device__ __forceinline__ f32x16_t mfma32(const g_u32x4_t& a, const g_u32x4_t& b, const f32x16_t& c) {
  if constexpr (XT == BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(g_bf16x8_t, a),
                                                   __builtin_bit_cast(g_bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(g_f16x8_t, a),
                                                  __builtin_bit_cast(g_f16x8_t, b), c, 0, 0, 0);
}

// two fp32 -> packed 16-bit (RNE)
template <int XT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (XT == BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((g_f2_t){lo, hi}, g_bf16x2_t));
  } else {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(lo))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(hi))) << 16);
  }
}

// Dequantize one 32-code chunk into 16 packed 16-bit pairs (natural k order).
// s/b: scale and bias of the chunk's group (for nvfp4 s/s2 cover the halves).
template <int XT, int MODE, int BITS>
__device__ __forceinline__ void dequant32(const uint32_t (&wd)[BITS], float s, float b, float s2,
                                          uint32_t (&o)[16]) {
  if constexpr (MODE == AFFINE && BITS == 4) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = wd[q] & 0x0F0F0F0Fu, hi = (wd[q] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float q0 = static_cast<float>((lo >> (8 * i)) & 0xffu);
        const float q1 = static_cast<float>((hi >> (8 * i)) & 0xffu);
        o[4 * q + i] = pack2<XT>(fmaf(s, q0, b), fmaf(s, q1, b));
      }
    }
  } else if constexpr (MODE == AFFINE && BITS == 8) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint32_t v = wd[q];
      o[2 * q] = pack2<XT>(fmaf(s, static_cast<float>(v & 0xffu), b),
                           fmaf(s, static_cast<float>((v >> 8) & 0xffu), b));
      o[2 * q + 1] = pack2<XT>(fmaf(s, static_cast<float>((v >> 16) & 0xffu), b),
                               fmaf(s, static_cast<float>(v >> 24), b));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = 2 * i + h;
        const uint32_t q = chunk_code<BITS>(wd, j);
        if constexpr (MODE == AFFINE) v[h] = fmaf(s, static_cast<float>(q), b);
        else v[h] = fp_elem<MODE>(q) * (MODE == NVFP4 && j >= 16 ? s2 : s);
      }
      o[i] = pack2<XT>(v[0], v[1]);
    }
  }
}

// byte k of v as fp32 (v_cvt_f32_ubyte{k})
template <int B>
__device__ __forceinline__ float ubyte_f(uint32_t v) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

}  // namespace iqmm
