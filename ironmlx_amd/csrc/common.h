// common.h — device-side helpers shared by the gfx950 quantized-matmul kernels.
//
// Number formats:
//   - fp16 / bf16 storage is uint16_t; conversions to fp32 are exact, from fp32
//     round to nearest even (bf16 by integer rounding, fp16 by v_cvt_f16_f32,
//     whose default mode is RNE).
//   - quantized rows are LSB-first bit streams of `bits`-wide codes in
//     little-endian uint32 words; a "chunk" is 32 consecutive codes of a row,
//     which occupies exactly `bits` words.
//   - e4m3fn / e2m1 elements decode through fp16 bit patterns (an exact
//     re-biasing: the code's exponent/mantissa fields are placed in an fp16
//     and rescaled by a power of two); e8m0 scales decode to 2^(c-127).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace iqmm {

enum Dt : int { F32 = 0, F16 = 1, BF16 = 2, U32 = 3, U8 = 4, I32 = 5, I64 = 6 };
enum Mode : int { AFFINE = 0, MXFP4 = 1, MXFP8 = 2, NVFP4 = 3 };

// -------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_to_f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ uint16_t f_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float h_to_f(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f_to_h(float f) {
  // Keep the conversion a plain v_cvt_f16_f32: without this the compiler may
  // merge a preceding multiply into v_fma_mix*_f16 with a +0 addend, which
  // turns a -0 product into +0.
  asm volatile("" : "+v"(f));
  uint16_t r = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  // canonical quiet NaN (sign kept), matching the CPU restatement
  if ((r & 0x7c00) == 0x7c00 && (r & 0x3ff)) r = (r & 0x8000) | 0x7e00;
  return r;
}

template <int DT> struct Store;
template <> struct Store<F32> { using T = float; };
template <> struct Store<F16> { using T = uint16_t; };
template <> struct Store<BF16> { using T = uint16_t; };
template <> struct Store<U8> { using T = uint8_t; };

template <int DT>
__device__ __forceinline__ float to_f(typename Store<DT>::T v) {
  if constexpr (DT == F32) return v;
  else if constexpr (DT == F16) return h_to_f(v);
  else return bf16_to_f(v);
}
template <int DT>
__device__ __forceinline__ typename Store<DT>::T from_f(float v) {
  if constexpr (DT == F32) return v;
  else if constexpr (DT == F16) return f_to_h(v);
  else return f_to_bf16(v);
}

// exp(x): Cody-Waite reduction x = n ln2 + r (|r| <= ln2 / 2; ln2 split into
// a 16-bit head, so n * head is exact, and a tail), the degree-7 Taylor
// polynomial of e^r in Horner form with explicit fma, then a 2^n scale.  Each
// step is a correctly rounded IEEE operation, so results are reproducible
// bit for bit on the host (within 2 ulp of exp).
__device__ __forceinline__ float iq_expf(float x) {
  if (x != x) return x;
  if (x > 88.7228394f) return __builtin_inff();
  if (x < -103.972084f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269502f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860682e-6f, r);
  float p = 1.0f / 5040.0f;
  p = __builtin_fmaf(p, r, 1.0f / 720.0f);
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, static_cast<int>(n));
}

// SwiGLU of one (gate, up) pair of fp32 sums, rounded the way the unfused
// composition rounds it: gate and up are first stored in the output type
// (they are quantized_matmul outputs), then silu(g) = g * sigmoid(g) and the
// product with up are separate elementwise ops, each rounded to the output
// type (mlx/src/nn/activations.rs:7-10, mlx/src/nn/mlp.rs:27-33).
template <int DT>
__device__ __forceinline__ typename Store<DT>::T swiglu_out(float g, float u) {
  const float gr = to_f<DT>(from_f<DT>(g)), ur = to_f<DT>(from_f<DT>(u));
  const float sg = to_f<DT>(from_f<DT>(1.0f / (1.0f + iq_expf(-gr))));
  const float a = to_f<DT>(from_f<DT>(gr * sg));
  return from_f<DT>(a * ur);
}

// -------------------------------------------------------------- fp element codes
// e2m1 code (4 bits, sign in bit 3) -> value / 2^14 as fp16 bits
__device__ __forceinline__ float e2m1_to_f(uint32_t c) {
  uint16_t h = static_cast<uint16_t>(((c & 7u) << 9) | ((c & 8u) << 12));
  return h_to_f(h) * 16384.0f;
}
// e4m3fn code (8 bits) -> value; S.1111.111 is NaN
__device__ __forceinline__ float e4m3_to_f(uint32_t c) {
  if ((c & 0x7fu) == 0x7fu) return __uint_as_float(0x7fc00000u);
  uint16_t h = static_cast<uint16_t>(((c & 0x7fu) << 7) | ((c & 0x80u) << 8));
  return h_to_f(h) * 256.0f;
}
// e8m0 code -> 2^(c-127); 255 is NaN
__device__ __forceinline__ float e8m0_to_f(uint32_t c) {
  if (c == 255u) return __uint_as_float(0x7fc00000u);
  if (c == 0u) return __uint_as_float(0x00400000u);
  return __uint_as_float(c << 23);
}

template <int MODE>
__device__ __forceinline__ float fp_elem(uint32_t q) {
  if constexpr (MODE == MXFP8) return e4m3_to_f(q);
  else return e2m1_to_f(q);
}
template <int MODE>
__device__ __forceinline__ float fp_scale(uint32_t c) {
  if constexpr (MODE == NVFP4) return e4m3_to_f(c);
  else return e8m0_to_f(c);
}

// mode constants
template <int MODE> struct ModeInfo;
template <> struct ModeInfo<AFFINE> { static constexpr int GS = 0, BITS = 0; };
template <> struct ModeInfo<MXFP4> { static constexpr int GS = 32, BITS = 4; };
template <> struct ModeInfo<MXFP8> { static constexpr int GS = 32, BITS = 8; };
template <> struct ModeInfo<NVFP4> { static constexpr int GS = 16, BITS = 4; };

// -------------------------------------------------------------- bit stream
// code j (0..31) of a chunk held in `bits` registers
template <int BITS>
__device__ __forceinline__ uint32_t chunk_code(const uint32_t (&wd)[BITS], int j) {
  const int bit = j * BITS;
  const int w = bit >> 5, sh = bit & 31;
  uint32_t v = wd[w] >> sh;
  if (sh + BITS > 32) v |= wd[w + 1] << (32 - sh);
  return v & ((1u << BITS) - 1u);
}

// load one 32-code chunk (BITS words) with the widest aligned vector loads
template <int BITS>
__device__ __forceinline__ void load_chunk(uint32_t (&wd)[BITS], const uint32_t* p) {
  if constexpr (BITS == 4) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    wd[0] = v.x; wd[1] = v.y; wd[2] = v.z; wd[3] = v.w;
  } else if constexpr (BITS == 8) {
    uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
    wd[0] = a.x; wd[1] = a.y; wd[2] = a.z; wd[3] = a.w;
    wd[4] = b.x; wd[5] = b.y; wd[6] = b.z; wd[7] = b.w;
  } else if constexpr (BITS == 2) {
    uint2 v = *reinterpret_cast<const uint2*>(p);
    wd[0] = v.x; wd[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < BITS; ++i) wd[i] = p[i];
  }
}

// -------------------------------------------------------------- batch mapping
// Output batch element b -> (x matrix index, w matrix index).  Dense qmm maps
// through broadcast strides; gather_qmm reads the index arrays (themselves
// addressed through broadcast strides).
struct BatchMap {
  int ndim;
  int64_t shape[8];
  int64_t xs[8];  // stride into x batch (dense) or into lhs indices (gather)
  int64_t ws[8];  // stride into w batch (dense) or into rhs indices (gather)
  const void* lhs;
  const void* rhs;
  int lhs_dt, rhs_dt;  // I32 / U32 / I64
  int64_t nx, nw;      // number of x / w matrices (index bounds)
};

__device__ __forceinline__ int64_t load_index(const void* p, int dt, int64_t i) {
  if (dt == I64) return static_cast<const int64_t*>(p)[i];
  if (dt == U32) return static_cast<int64_t>(static_cast<const uint32_t*>(p)[i]);
  return static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

// Returns false when a gathered index is out of range: the caller then writes
// NaN for that output matrix and touches no x / w memory.
__device__ __forceinline__ bool map_batch(const BatchMap& bm, int64_t b, int64_t& xb, int64_t& wb) {
  int64_t xo = 0, wo = 0, r = b;
  for (int d = bm.ndim - 1; d >= 0; --d) {
    int64_t i = r % bm.shape[d];
    r /= bm.shape[d];
    xo += i * bm.xs[d];
    wo += i * bm.ws[d];
  }
  xb = bm.lhs ? load_index(bm.lhs, bm.lhs_dt, xo) : xo;
  wb = bm.rhs ? load_index(bm.rhs, bm.rhs_dt, wo) : wo;
  return xb >= 0 && xb < bm.nx && wb >= 0 && wb < bm.nw;
}

// -------------------------------------------------------------- wave reduction
__device__ __forceinline__ float wave_sum_width(float v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace iqmm
