// qmv_q4.hip — the decode GEMV fast path: affine 4-bit, transpose=true, M=1,
// bf16 or fp16 activations (the shape every ironmlx decode step runs,
// mlx/src/nn/linear.rs:51-63 with x = [1, 1, K]).
//
// One wave per workgroup owns RB consecutive weight rows.  Lane l walks the
// 32-code chunks c = l, l+64, ... of every row: a chunk is 16 bytes, so each
// row is read with fully coalesced 1 KiB wave loads, non-temporal since every
// weight byte is used once.  The x chunk (32 values) is loaded once per chunk
// and reused for all RB rows.
//
// Unpacking: lo = w & 0x0F0F0F0F holds n0,n2,n4,n6 (one per byte) and
// hi = (w >> 4) & 0x0F0F0F0F holds n1,n3,n5,n7.  v_perm_b32 against a register
// of bytes E (0x43 for bf16, 0x64 for fp16) builds 16-bit halves E:n, i.e.
// exactly C + n with C = 128.0 (bf16) or 1024.0 (fp16), both of unit
// spacing.  Four such pairs (n0,n4) (n2,n6) (n1,n5) (n3,n7) feed
// v_dot2_f32_{bf16,f16} against x pairs permuted the same way, so per 8 codes
// the VALU does 3 bit ops, 4 permutes and 4 dot2.  With d = sum x (C + q) and
// xs = sum x over the chunk (one quantization group):
//   s * sum(x q) + b * xs = s * (d - C * xs) + b * xs.
#include <stdlib.h>

#include "launch.h"

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

template <int XT, int RB>
__global__ __launch_bounds__(64) void qmv_q4_m1_kernel(QmmArgs a, int64_t batch0) {
  using XS = uint16_t;
  const int lane = threadIdx.x;
  const int64_t bb = batch0 + blockIdx.y;
  const int N = a.N, K = a.K;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(N);  // M = 1
  const int row0 = blockIdx.x * RB;

  int64_t xb = 0, wb = 0;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      if (lane < RB && row0 + lane < N) out[row0 + lane] = from_f<XT>(__builtin_nanf(""));
      return;
    }
  }
  const char* xbase = reinterpret_cast<const char*>(static_cast<const XS*>(a.x) + xb * a.x_mat);
  const uint32_t* w = a.w + wb * a.w_mat;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = static_cast<const XS*>(a.b) + wb * a.s_mat;
  const int wpr = K >> 3;  // words per row
  const int G = K / a.gs;
  const int gshift = __builtin_ctz(a.gs);

  // uniform per-row bases; lanes add a 32-bit byte offset
  const char* wrow[RB];
  const XS* srow[RB];
  const XS* brow[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int row = min(row0 + r, N - 1);
    wrow[r] = reinterpret_cast<const char*>(w + static_cast<int64_t>(row) * wpr);
    srow[r] = sp + static_cast<int64_t>(row) * G;
    brow[r] = bp + static_cast<int64_t>(row) * G;
  }

  float acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = 0.f;

  const int C = K >> 5;
  const uint32_t E = Magic<XT>::ebytes;
#pragma unroll 2
  for (int c = lane; c < C; c += 64) {
    const uint32_t off = static_cast<uint32_t>(c) << 4;
    // weights first: RB independent 16-byte streaming loads in flight
    u32x4_t wv[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r)
      wv[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow[r] + off));
    const int g = (c << 5) >> gshift;
    XS sr[RB], br[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      sr[r] = srow[r][g];
      br[r] = brow[r][g];
    }
    // x chunk: 32 values as 16 packed pairs X[i] = x[2i] | x[2i+1] << 16
    uint32_t X[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xbase + (off << 2) + 16 * i);
      X[4 * i] = v.x; X[4 * i + 1] = v.y; X[4 * i + 2] = v.z; X[4 * i + 3] = v.w;
    }
    // x pairs in the order the nibble pairs are built for word q:
    // (x0,x4) (x2,x6) (x1,x5) (x3,x7) relative to 8q
    uint32_t P[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t A0 = X[4 * q], A1 = X[4 * q + 1], B0 = X[4 * q + 2], B1 = X[4 * q + 3];
      P[4 * q + 0] = __builtin_amdgcn_perm(B0, A0, 0x05040100u);  // x0, x4
      P[4 * q + 1] = __builtin_amdgcn_perm(B1, A1, 0x05040100u);  // x2, x6
      P[4 * q + 2] = __builtin_amdgcn_perm(B0, A0, 0x07060302u);  // x1, x5
      P[4 * q + 3] = __builtin_amdgcn_perm(B1, A1, 0x07060302u);  // x3, x7
    }
    float xs = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) xs = dot2<XT>(X[i], Magic<XT>::one2, xs);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const uint32_t wd[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
      float d = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo = wd[q] & 0x0F0F0F0Fu;          // n0 n2 n4 n6
        const uint32_t hi = (wd[q] >> 4) & 0x0F0F0F0Fu;   // n1 n3 n5 n7
        d = dot2<XT>(__builtin_amdgcn_perm(E, lo, SEL_B0B2), P[4 * q + 0], d);  // n0, n4
        d = dot2<XT>(__builtin_amdgcn_perm(E, lo, SEL_B1B3), P[4 * q + 1], d);  // n2, n6
        d = dot2<XT>(__builtin_amdgcn_perm(E, hi, SEL_B0B2), P[4 * q + 2], d);  // n1, n5
        d = dot2<XT>(__builtin_amdgcn_perm(E, hi, SEL_B1B3), P[4 * q + 3], d);  // n3, n7
      }
      const float s = to_f<XT>(sr[r]), b = to_f<XT>(br[r]);
      acc[r] = fmaf(s, fmaf(-Magic<XT>::c, xs, d), fmaf(b, xs, acc[r]));
    }
  }
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = wave_sum_width(acc[r], 64);
  float v = acc[0];
#pragma unroll
  for (int r = 1; r < RB; ++r)
    if (lane == r) v = acc[r];
  if (lane < RB && row0 + lane < N) out[row0 + lane] = from_f<XT>(v);
}

// ---------------------------------------------------------------------------
// Variant 2: 256-thread workgroups; each lane owns a 64-code span of every row
// (32 contiguous bytes: one affine group at gs=64), so each row costs a lane
// two 16-byte weight loads and one scale/bias pair.  x pairs for the span are
// built once per wave (XLDS=false) or once per workgroup through LDS
// (XLDS=true).  Row sums are reduced with DPP.
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

template <int XT, int RB, bool XLDS>
__global__ __launch_bounds__(256) void qmv_q4_m1_v2_kernel(QmmArgs a, int64_t batch0) {
  using XS = uint16_t;
  __shared__ uint32_t xp_lds[XLDS ? 128 * 16 : 1];
  __shared__ float xs_lds[XLDS ? 128 : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bb = batch0 + blockIdx.y;
  const int N = a.N, K = a.K;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(N);
  const int row0 = (blockIdx.x * 4 + wave) * RB;

  int64_t xb = 0, wb = 0;
  bool ok = true;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) ok = map_batch(a.bm, bb, xb, wb);
  if (!ok) {
    if (lane < RB && row0 + lane < N) out[row0 + lane] = from_f<XT>(__builtin_nanf(""));
    return;  // uniform across the workgroup (one batch element per block)
  }
  const char* xbase = reinterpret_cast<const char*>(static_cast<const XS*>(a.x) + xb * a.x_mat);
  const uint32_t* w = a.w + wb * a.w_mat;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = static_cast<const XS*>(a.b) + wb * a.s_mat;
  const int wpr = K >> 3;
  const int G = K / a.gs;
  const int gshift = __builtin_ctz(a.gs);

  const char* wrow[RB];
  const XS* srow[RB];
  const XS* brow[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int row = min(row0 + r, N - 1);
    wrow[r] = reinterpret_cast<const char*>(w + static_cast<int64_t>(row) * wpr);
    srow[r] = sp + static_cast<int64_t>(row) * G;
    brow[r] = bp + static_cast<int64_t>(row) * G;
  }
  float acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = 0.f;

  for (int seg = 0; seg < K; seg += 4096) {
    const int k0 = seg + lane * 64;
    const bool active = k0 < K;
    if constexpr (XLDS) {
      if (seg > 0) __syncthreads();
      if (tid < 128 && seg + tid * 32 < K) {
        uint32_t X[16], P[16];
        float xs;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xbase + 2 * (seg + tid * 32) + 16 * i);
          X[4 * i] = v.x; X[4 * i + 1] = v.y; X[4 * i + 2] = v.z; X[4 * i + 3] = v.w;
        }
        make_pairs<XT>(X, P, xs);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<u32x4_t*>(&xp_lds[tid * 16 + 4 * i]) =
              u32x4_t{P[4 * i], P[4 * i + 1], P[4 * i + 2], P[4 * i + 3]};
        xs_lds[tid] = xs;
      }
      __syncthreads();
    }
    if (active) {
      const uint32_t off = static_cast<uint32_t>(k0) >> 1;  // byte offset of the span
      u32x4_t wv[RB][2];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        wv[r][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow[r] + off));
        wv[r][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow[r] + off + 16));
      }
      const int g0 = k0 >> gshift, g1 = (k0 + 32) >> gshift;
      XS sr[RB][2], br[RB][2];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        sr[r][0] = srow[r][g0];
        br[r][0] = brow[r][g0];
        sr[r][1] = srow[r][g1];
        br[r][1] = brow[r][g1];
      }
      uint32_t P[2][16];
      float xs[2];
      if constexpr (XLDS) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int ci = lane * 2 + h;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&xp_lds[ci * 16 + 4 * i]);
            P[h][4 * i] = v.x; P[h][4 * i + 1] = v.y; P[h][4 * i + 2] = v.z; P[h][4 * i + 3] = v.w;
          }
          xs[h] = xs_lds[ci];
        }
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint32_t X[16];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xbase + 2 * k0 + 64 * h + 16 * i);
            X[4 * i] = v.x; X[4 * i + 1] = v.y; X[4 * i + 2] = v.z; X[4 * i + 3] = v.w;
          }
          make_pairs<XT>(X, P[h], xs[h]);
        }
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float d = chunk_dot<XT>(wv[r][h], P[h]);
          const float s = to_f<XT>(sr[r][h]), b = to_f<XT>(br[r][h]);
          acc[r] = fmaf(s, fmaf(-Magic<XT>::c, xs[h], d), fmaf(b, xs[h], acc[r]));
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = dpp_sum_to_lane63(acc[r]);
  if (lane == 63) {
#pragma unroll
    for (int r = 0; r < RB; ++r)
      if (row0 + r < N) out[row0 + r] = from_f<XT>(acc[r]);
  }
}

// ---------------------------------------------------------------------------
// Variant 3 (streaming): x pairs for the whole K are built once per workgroup
// into LDS; each wave then walks a contiguous range of rows with a two-row
// register double buffer, so the loads of rows r+1, r+2 are in flight while
// row r is reduced.  Lane l owns chunks l, l+64, ... (CPL per row).
template <int XT, int CPL>
__device__ __forceinline__ void load_row(u32x4_t (&wv)[CPL], uint16_t (&sb)[2 * CPL],
                                         const char* wrow, const uint16_t* srow,
                                         const uint16_t* brow, int lane, int C, int gshift) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    const int cc = c < C ? c : C - 1;
    wv[j] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(wrow + (static_cast<uint32_t>(cc) << 4)));
    const int g = (cc << 5) >> gshift;
    sb[2 * j] = srow[g];
    sb[2 * j + 1] = brow[g];
  }
}

template <int XT, int CPL>
__device__ __forceinline__ float row_partial(const u32x4_t (&wv)[CPL], const uint16_t (&sb)[2 * CPL],
                                             const uint32_t* xp_lds, const float* xs_lds, int lane,
                                             int C) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    if (c < C) {
      uint32_t P[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&xp_lds[c * 16 + 4 * i]);
        P[4 * i] = v.x; P[4 * i + 1] = v.y; P[4 * i + 2] = v.z; P[4 * i + 3] = v.w;
      }
      const float xs = xs_lds[c];
      const float d = chunk_dot<XT>(wv[j], P);
      const float s = to_f<XT>(sb[2 * j]), b = to_f<XT>(sb[2 * j + 1]);
      acc = fmaf(s, fmaf(-Magic<XT>::c, xs, d), fmaf(b, xs, acc));
    }
  }
  return acc;
}

template <int XT, int CPL>
__global__ __launch_bounds__(256) void qmv_q4_stream_kernel(QmmArgs a, int rows_per_wave,
                                                            int64_t batch0) {
  using XS = uint16_t;
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t bb = batch0 + blockIdx.y;
  const int N = a.N, K = a.K, C = K >> 5;
  uint32_t* xp_lds = smem;                                   // [C][16]
  float* xs_lds = reinterpret_cast<float*>(smem + C * 16);  // [C]
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(N);

  int64_t xb = 0, wb = 0;
  bool ok = true;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) ok = map_batch(a.bm, bb, xb, wb);
  const int r_begin = (blockIdx.x * 4 + wave) * rows_per_wave;
  const int r_end = min(N, r_begin + rows_per_wave);
  if (!ok) {
    for (int r = r_begin + lane; r < r_end; r += 64) out[r] = from_f<XT>(__builtin_nanf(""));
    return;  // uniform over the workgroup
  }
  const char* xbase = reinterpret_cast<const char*>(static_cast<const XS*>(a.x) + xb * a.x_mat);
  for (int c = tid; c < C; c += 256) {
    uint32_t X[16], P[16];
    float xs;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xbase + (c << 6) + 16 * i);
      X[4 * i] = v.x; X[4 * i + 1] = v.y; X[4 * i + 2] = v.z; X[4 * i + 3] = v.w;
    }
    make_pairs<XT>(X, P, xs);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4_t*>(&xp_lds[c * 16 + 4 * i]) =
          u32x4_t{P[4 * i], P[4 * i + 1], P[4 * i + 2], P[4 * i + 3]};
    xs_lds[c] = xs;
  }
  __syncthreads();
  if (r_begin >= r_end) return;

  const uint32_t* w = a.w + wb * a.w_mat;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = static_cast<const XS*>(a.b) + wb * a.s_mat;
  const int wpr = K >> 3, G = K / a.gs, gshift = __builtin_ctz(a.gs);
  auto wrow = [&](int r) { return reinterpret_cast<const char*>(w + static_cast<int64_t>(r) * wpr); };
  auto srow = [&](int r) { return sp + static_cast<int64_t>(r) * G; };
  auto brow = [&](int r) { return bp + static_cast<int64_t>(r) * G; };

  u32x4_t w0[CPL], w1[CPL];
  uint16_t sb0[2 * CPL], sb1[2 * CPL];
  int r = r_begin;
  const int rl = r_end - 1;
  load_row<XT, CPL>(w0, sb0, wrow(r), srow(r), brow(r), lane, C, gshift);
  {
    const int r1 = min(r + 1, rl);
    load_row<XT, CPL>(w1, sb1, wrow(r1), srow(r1), brow(r1), lane, C, gshift);
  }
  for (; r < r_end; r += 2) {
    float p0 = row_partial<XT, CPL>(w0, sb0, xp_lds, xs_lds, lane, C);
    {
      const int rn = min(r + 2, rl);
      load_row<XT, CPL>(w0, sb0, wrow(rn), srow(rn), brow(rn), lane, C, gshift);
    }
    p0 = dpp_sum_to_lane63(p0);
    if (lane == 63) out[r] = from_f<XT>(p0);
    if (r + 1 < r_end) {
      float p1 = row_partial<XT, CPL>(w1, sb1, xp_lds, xs_lds, lane, C);
      const int rn = min(r + 3, rl);
      load_row<XT, CPL>(w1, sb1, wrow(rn), srow(rn), brow(rn), lane, C, gshift);
      p1 = dpp_sum_to_lane63(p1);
      if (lane == 63) out[r + 1] = from_f<XT>(p1);
    }
  }
}

// ---------------------------------------------------------------------------
// Ordered single-pass kernel (the default).  One wave per workgroup owns RB
// rows; lane l owns chunks l, l+64, ... (CPL per row).  Loads are issued in
// the order they are consumed -- x first (cache-resident), then for each row
// its weight chunks followed by its scales and biases -- so that, with
// in-order vmcnt accounting, row r's arithmetic and DPP reduction run while
// the loads of rows r+1.. are still in flight.
template <int XT, int RB, int CPL>
__global__ __launch_bounds__(64) void qmv_q4_ord_kernel(QmmArgs a, int64_t batch0) {
  using XS = uint16_t;
  const int lane = threadIdx.x;
  const int64_t bb = batch0 + blockIdx.y;
  const int N = a.N, K = a.K, C = K >> 5;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(N);
  const int row0 = blockIdx.x * RB;

  int64_t xb = 0, wb = 0;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      if (lane < RB && row0 + lane < N) out[row0 + lane] = from_f<XT>(__builtin_nanf(""));
      return;
    }
  }
  const char* xbase = reinterpret_cast<const char*>(static_cast<const XS*>(a.x) + xb * a.x_mat);
  const uint32_t* w = a.w + wb * a.w_mat;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = static_cast<const XS*>(a.b) + wb * a.s_mat;
  const int wpr = K >> 3, G = K / a.gs, gshift = __builtin_ctz(a.gs);

  // chunk index per slot (clamped; out-of-range slots are masked at the end)
  int cidx[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) cidx[j] = min(lane + 64 * j, C - 1);

  // 1. x chunks (cache-resident) first
  uint32_t X[CPL][16];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xbase + (cidx[j] << 6) + 16 * i);
      X[j][4 * i] = v.x; X[j][4 * i + 1] = v.y; X[j][4 * i + 2] = v.z; X[j][4 * i + 3] = v.w;
    }
  // 2. per row: weight chunks, then that row's scales / biases
  u32x4_t wv[RB][CPL];
  XS sr[RB][CPL], br[RB][CPL];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int row = min(row0 + r, N - 1);
    const char* wr = reinterpret_cast<const char*>(w + static_cast<int64_t>(row) * wpr);
    const XS* srow = sp + static_cast<int64_t>(row) * G;
    const XS* brow = bp + static_cast<int64_t>(row) * G;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      wv[r][j] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(wr + (static_cast<uint32_t>(cidx[j]) << 4)));
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int g = (cidx[j] << 5) >> gshift;
      sr[r][j] = srow[g];
      br[r][j] = brow[g];
    }
  }
  // 3. x pairs and chunk sums (overlaps the weight loads)
  uint32_t P[CPL][16];
  float xs[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    make_pairs<XT>(X[j], P[j], xs[j]);
    if (lane + 64 * j >= C) xs[j] = 0.f;  // masked slot contributes nothing
  }
  // 4. rows in load order
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float d = chunk_dot<XT>(wv[r][j], P[j]);
      if (lane + 64 * j >= C) d = 0.f;
      const float s = to_f<XT>(sr[r][j]), b = to_f<XT>(br[r][j]);
      acc = fmaf(s, fmaf(-Magic<XT>::c, xs[j], d), fmaf(b, xs[j], acc));
    }
    acc = dpp_sum_to_lane63(acc);
    if (lane == 63 && row0 + r < N) out[row0 + r] = from_f<XT>(acc);
  }
}

bool qmv_q4_m1_supported(const QmmArgs& a) {
  return a.transpose && a.M == 1 && a.mode == AFFINE && a.bits == 4 &&
         (a.xdt == BF16 || a.xdt == F16);
}

namespace {
int tune_rb() {
  static const int v = [] {
    const char* e = getenv("IQMM_TUNE_QMV_RB");
    return e ? atoi(e) : 0;
  }();
  return v;
}
int tune_variant() {
  static const int v = [] {
    const char* e = getenv("IQMM_TUNE_QMV_VARIANT");
    return e ? atoi(e) : 0;
  }();
  return v;
}

template <int XT, int RB, bool XLDS>
hipError_t launch_v2(const QmmArgs& a) {
  const int64_t nblk = (a.N + 4 * RB - 1) / (4 * RB);
  if (nblk <= 0 || a.nbatch <= 0) return hipSuccess;
  for (int64_t b0 = 0; b0 < a.nbatch; b0 += 65535) {
    const int64_t nb = a.nbatch - b0 < 65535 ? a.nbatch - b0 : 65535;
    hipLaunchKernelGGL((qmv_q4_m1_v2_kernel<XT, RB, XLDS>),
                       dim3(static_cast<unsigned>(nblk), static_cast<unsigned>(nb)), dim3(256), 0,
                       a.stream, a, b0);
  }
  return hipGetLastError();
}

template <int XT, int RB>
hipError_t launch_rb(const QmmArgs& a) {
  const int64_t nrb = (a.N + RB - 1) / RB;
  if (nrb <= 0 || a.nbatch <= 0) return hipSuccess;
  // batch rides on grid.y (at most 65535 per launch)
  for (int64_t b0 = 0; b0 < a.nbatch; b0 += 65535) {
    const int64_t nb = a.nbatch - b0 < 65535 ? a.nbatch - b0 : 65535;
    hipLaunchKernelGGL((qmv_q4_m1_kernel<XT, RB>), dim3(static_cast<unsigned>(nrb), static_cast<unsigned>(nb)),
                       dim3(64), 0, a.stream, a, b0);
  }
  return hipGetLastError();
}

template <int XT, int CPL>
hipError_t launch_stream(const QmmArgs& a) {
  const int C = a.K >> 5;
  // spread rows over ~4 waves per SIMD (256 CUs x 4 SIMDs)
  const int target_waves = 4096;
  int rpw = static_cast<int>((a.N * a.nbatch + target_waves - 1) / target_waves);
  if (rpw < 2) rpw = 2;
  if (tune_rb()) rpw = tune_rb();
  const int64_t nwaves = (a.N + rpw - 1) / rpw;
  const int64_t nblk = (nwaves + 3) / 4;
  const size_t lds = static_cast<size_t>(C) * 68;
  for (int64_t b0 = 0; b0 < a.nbatch; b0 += 65535) {
    const int64_t nb = a.nbatch - b0 < 65535 ? a.nbatch - b0 : 65535;
    hipLaunchKernelGGL((qmv_q4_stream_kernel<XT, CPL>),
                       dim3(static_cast<unsigned>(nblk), static_cast<unsigned>(nb)), dim3(256), lds,
                       a.stream, a, rpw, b0);
  }
  return hipGetLastError();
}

template <int XT, int RB, int CPL>
hipError_t launch_ord(const QmmArgs& a) {
  const int64_t nrb = (a.N + RB - 1) / RB;
  if (nrb <= 0 || a.nbatch <= 0) return hipSuccess;
  for (int64_t b0 = 0; b0 < a.nbatch; b0 += 65535) {
    const int64_t nb = a.nbatch - b0 < 65535 ? a.nbatch - b0 : 65535;
    hipLaunchKernelGGL((qmv_q4_ord_kernel<XT, RB, CPL>),
                       dim3(static_cast<unsigned>(nrb), static_cast<unsigned>(nb)), dim3(64), 0,
                       a.stream, a, b0);
  }
  return hipGetLastError();
}

template <int XT, int CPL>
hipError_t launch_ord_cpl(const QmmArgs& a) {
  // rows per wave: 4 while that leaves >= 2048 waves, else fewer
  int rb = tune_rb();
  if (rb == 0) {
    const int64_t rows = a.N * a.nbatch;
    rb = rows >= 4 * 2048 ? 4 : rows >= 2 * 2048 ? 2 : 1;
    if (CPL >= 4 && rb > 2) rb = 2;
  }
  switch (rb) {
    case 4: return launch_ord<XT, 4, CPL>(a);
    case 2: return launch_ord<XT, 2, CPL>(a);
    default: return launch_ord<XT, 1, CPL>(a);
  }
}

template <int XT>
hipError_t launch_xt(const QmmArgs& a) {
  const int var = tune_variant();
  const int cpl = ((a.K >> 5) + 63) / 64;
  if (var == 0 && a.K >= 1024 && cpl <= 8) {
    switch (cpl) {
      case 1: return launch_ord_cpl<XT, 1>(a);
      case 2: return launch_ord_cpl<XT, 2>(a);
      case 3: return launch_ord_cpl<XT, 3>(a);
      case 4: return launch_ord_cpl<XT, 4>(a);
      case 5: return launch_ord_cpl<XT, 5>(a);
      case 6: return launch_ord_cpl<XT, 6>(a);
      case 7: return launch_ord_cpl<XT, 7>(a);
      default: return launch_ord_cpl<XT, 8>(a);
    }
  }
  if (var == 3 && a.K <= 16384) {
    switch (cpl) {
      case 1: return launch_stream<XT, 1>(a);
      case 2: return launch_stream<XT, 2>(a);
      case 3: return launch_stream<XT, 3>(a);
      case 4: return launch_stream<XT, 4>(a);
      case 5: return launch_stream<XT, 5>(a);
      case 6: return launch_stream<XT, 6>(a);
      case 7: return launch_stream<XT, 7>(a);
      default: return launch_stream<XT, 8>(a);
    }
  }
  if (var == 1 || var == 2) {
    int rb = tune_rb() ? tune_rb() : 4;
    const bool lds = var == 2;
    switch (rb) {
      case 8: return lds ? launch_v2<XT, 8, true>(a) : launch_v2<XT, 8, false>(a);
      case 2: return lds ? launch_v2<XT, 2, true>(a) : launch_v2<XT, 2, false>(a);
      case 1: return lds ? launch_v2<XT, 1, true>(a) : launch_v2<XT, 1, false>(a);
      default: return lds ? launch_v2<XT, 4, true>(a) : launch_v2<XT, 4, false>(a);
    }
  }
  // rows per wave: as many as keep >= ~4 waves per CU resident (256 CUs)
  int rb = tune_rb();
  if (rb == 0) {
    const int64_t rows = a.N * a.nbatch;
    rb = rows >= 8 * 1024 ? 8 : rows >= 4 * 1024 ? 4 : rows >= 2 * 1024 ? 2 : 1;
  }
  switch (rb) {
    case 8: return launch_rb<XT, 8>(a);
    case 4: return launch_rb<XT, 4>(a);
    case 2: return launch_rb<XT, 2>(a);
    default: return launch_rb<XT, 1>(a);
  }
}
}  // namespace

hipError_t launch_qmv_q4_m1(const QmmArgs& a) {
  return a.xdt == BF16 ? launch_xt<BF16>(a) : launch_xt<F16>(a);
}

}  // namespace iqmm
