// gemv_common.h — the M = 1 GEMV arithmetic on packed affine 4-bit codes,
// shared by the decode GEMV (qmv_q4.hip) and the one-token MoE kernels
// (moe.hip).
//
// A 32-code chunk is 16 bytes: lo = w & 0x0F0F0F0F holds n0,n2,n4,n6 (one per
// byte) and hi = (w >> 4) & 0x0F0F0F0F holds n1,n3,n5,n7.  v_perm_b32 against
// a register of bytes E (0x43 for bf16, 0x64 for fp16) builds 16-bit halves
// E:n, i.e. exactly C + n with C = 128.0 (bf16) or 1024.0 (fp16), both of unit
// spacing.  Four such pairs (n0,n4) (n2,n6) (n1,n5) (n3,n7) feed
// v_dot2_f32_{bf16,f16} against x pairs permuted the same way.  With
// d = sum x (C + q) and xs = sum x over the chunk (one quantization group):
//   s * sum(x q) + b * xs = s * (d - C * xs) + b * xs.
#pragma once
#include "common.h"

namespace iqmm {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;

template <int XT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (XT == BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                  c, false);
}

template <int XT>
struct Magic;
template <> struct Magic<BF16> {
  static constexpr uint32_t ebytes = 0x43434343u;  // exponent byte of 128.0 bf16
  static constexpr float c = 128.f;
  static constexpr uint32_t one2 = 0x3f803f80u;    // (1.0, 1.0)
};
template <> struct Magic<F16> {
  static constexpr uint32_t ebytes = 0x64646464u;  // exponent byte of 1024.0 fp16
  static constexpr float c = 1024.f;
  static constexpr uint32_t one2 = 0x3c003c00u;
};

// byte selectors for v_perm_b32(E, v): bytes 0..3 of v, 4..7 of E
constexpr uint32_t SEL_B0B2 = 0x04020400u;  // halves (E:v.b0), (E:v.b2)
constexpr uint32_t SEL_B1B3 = 0x04030401u;  // halves (E:v.b1), (E:v.b3)

// ---------------------------------------------------------------------------
// Shared pieces: DPP row reduction, x pair construction, one chunk's dot.
__device__ __forceinline__ float dpp_sum_to_lane63(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
  return v;
}

template <int XT>
__device__ __forceinline__ void make_pairs(const uint32_t (&X)[16], uint32_t (&P)[16], float& xs) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t A0 = X[4 * q], A1 = X[4 * q + 1], B0 = X[4 * q + 2], B1 = X[4 * q + 3];
    P[4 * q + 0] = __builtin_amdgcn_perm(B0, A0, 0x05040100u);
    P[4 * q + 1] = __builtin_amdgcn_perm(B1, A1, 0x05040100u);
    P[4 * q + 2] = __builtin_amdgcn_perm(B0, A0, 0x07060302u);
    P[4 * q + 3] = __builtin_amdgcn_perm(B1, A1, 0x07060302u);
  }
  xs = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) xs = dot2<XT>(X[i], Magic<XT>::one2, xs);
}

template <int XT>
__device__ __forceinline__ float chunk_dot(const u32x4_t& wv, const uint32_t (&P)[16]) {
  const uint32_t E = Magic<XT>::ebytes;
  const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
  float d = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t lo = wd[q] & 0x0F0F0F0Fu;
    const uint32_t hi = (wd[q] >> 4) & 0x0F0F0F0Fu;
    d = dot2<XT>(__builtin_amdgcn_perm(E, lo, SEL_B0B2), P[4 * q + 0], d);
    d = dot2<XT>(__builtin_amdgcn_perm(E, lo, SEL_B1B3), P[4 * q + 1], d);
    d = dot2<XT>(__builtin_amdgcn_perm(E, hi, SEL_B0B2), P[4 * q + 2], d);
    d = dot2<XT>(__builtin_amdgcn_perm(E, hi, SEL_B1B3), P[4 * q + 3], d);
  }
  return d;
}

// The W half of chunk_dot: the 16 (C + n) pairs of one chunk, reused for
// every x row of a multi-row GEMV.
template <int XT>
__device__ __forceinline__ void chunk_pairs(const u32x4_t& wv, uint32_t (&W)[16]) {
  const uint32_t E = Magic<XT>::ebytes;
  const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t lo = wd[q] & 0x0F0F0F0Fu;
    const uint32_t hi = (wd[q] >> 4) & 0x0F0F0F0Fu;
    W[4 * q + 0] = __builtin_amdgcn_perm(E, lo, SEL_B0B2);
    W[4 * q + 1] = __builtin_amdgcn_perm(E, lo, SEL_B1B3);
    W[4 * q + 2] = __builtin_amdgcn_perm(E, hi, SEL_B0B2);
    W[4 * q + 3] = __builtin_amdgcn_perm(E, hi, SEL_B1B3);
  }
}

}  // namespace iqmm
