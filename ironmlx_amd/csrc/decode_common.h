// decode_common.h — helpers shared by the decode-width kernels
// (qmm_decode.hip) and their grouped gather_qmm form (qmm_gather.hip).
#pragma once
#include "mfma_common.h"

namespace iqmm {

typedef __attribute__((ext_vector_type(4))) float f32x4d_t;

template <int XT>
__device__ __forceinline__ f32x4d_t mfma16(const g_u32x4_t& a, const g_u32x4_t& b, const f32x4d_t& c) {
  if constexpr (XT == BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, a),
                                                   __builtin_bit_cast(g_bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(g_f16x8_t, a),
                                                  __builtin_bit_cast(g_f16x8_t, b), c, 0, 0, 0);
}

}  // namespace iqmm
