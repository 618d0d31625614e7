// qmv_q4.hip — the decode GEMV fast path: affine 4-bit, transpose=true, M=1,
// bf16 or fp16 activations (the shape every ironmlx decode step runs,
// mlx/src/nn/linear.rs:51-63 with x = [1, 1, K]).
//
// One wave per workgroup owns RB (1, 2 or 4) consecutive weight rows.  Lane
// l owns the 32-code chunks c = l, l+64, ... (CPL of them) of every row: a
// chunk is 16 bytes, so each row is read with fully coalesced 1 KiB wave
// loads, non-temporal since every weight byte is used once.  Each x chunk is
// loaded once and reused for all RB rows.
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
  // K in [1024, 16384]: one to eight 32-code chunks per lane per row
  return a.transpose && a.M == 1 && a.mode == AFFINE && a.bits == 4 &&
         (a.xdt == BF16 || a.xdt == F16) && a.K >= 1024 && a.K <= 16384;
}

namespace {
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
  const int64_t rows = a.N * a.nbatch;
  int rb = rows >= 4 * 2048 ? 4 : rows >= 2 * 2048 ? 2 : 1;
  if (CPL >= 4 && rb > 2) rb = 2;
  switch (rb) {
    case 4: return launch_ord<XT, 4, CPL>(a);
    case 2: return launch_ord<XT, 2, CPL>(a);
    default: return launch_ord<XT, 1, CPL>(a);
  }
}

template <int XT>
hipError_t launch_xt(const QmmArgs& a) {
  switch (((a.K >> 5) + 63) / 64) {
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
}  // namespace

hipError_t launch_qmv_q4_m1(const QmmArgs& a) {
  return a.xdt == BF16 ? launch_xt<BF16>(a) : launch_xt<F16>(a);
}

}  // namespace iqmm
