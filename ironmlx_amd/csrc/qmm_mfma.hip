// qmm_mfma.hip — prefill-shaped quantized matmul on CDNA4 matrix cores.
//
// out[M, N] = x[M, K] . deq(W)^T  (transpose)  or  x . deq(W)  (!transpose)
// x is bf16 or fp16.  A 256-thread workgroup owns a BM x BN output tile and
// walks K in BK steps:
//   - the x tile is copied global -> LDS with 16-byte loads;
//   - the packed W tile is read once (one 32-code chunk per thread),
//     dequantized in registers with the same arithmetic as `dequantize`
//     (rn(rn(s*q)+b), then RNE to x's 16-bit type) and written to LDS in
//     [n][k] order;
//   - four waves (2 x 2) each accumulate a 64 x 64 sub-tile with
//     v_mfma_f32_16x16x32_{bf16,f16} (fp32 accumulate).
// Reference op: mlx/src/ops.rs:695-727 at prefill (x = [1, L, K],
// mlx/src/generate/mod.rs:76-80).
#include "launch.h"

namespace iqmm {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

template <int XT>
__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, const f32x4_t& c) {
  if constexpr (XT == BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

#pragma clang fp contract(off)
// dequantized value of code j of a chunk, as x's 16-bit type
template <int XT, int MODE, int BITS>
__device__ __forceinline__ uint16_t deq16(const uint32_t (&wd)[BITS], int j, float s, float b) {
  const uint32_t q = chunk_code<BITS>(wd, j);
  float v;
  if constexpr (MODE == AFFINE) {
    const float p = s * static_cast<float>(q);
    v = p + b;
  } else {
    v = fp_elem<MODE>(q) * s;
  }
  return from_f<XT>(v);
}
#pragma clang fp contract(on)

constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;

template <int XT, int MODE, int BITS, bool TRANS>
__global__ __launch_bounds__(256) void qmm_mfma_kernel(QmmArgs a, int64_t ntn, int64_t ntm) {
  using XS = uint16_t;
  constexpr bool AFF = MODE == AFFINE;
  constexpr int SUBG = MODE == NVFP4 ? 16 : 32;
  constexpr int NSUB = 32 / SUBG;
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDK];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int64_t blk = blockIdx.x;
  const int64_t tn = blk % ntn, tm = (blk / ntn) % ntm, bb = blk / (ntn * ntm);
  const int M = a.M, N = a.N, K = a.K;
  const int m0 = static_cast<int>(tm) * BM, n0 = static_cast<int>(tn) * BN;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;

  int64_t xb, wb;
  const bool ok = map_batch(a.bm, bb, xb, wb);
  if (!ok) {
    for (int i = t; i < BM * BN; i += 256) {
      const int r = m0 + i / BN, c = n0 + i % BN;
      if (r < M && c < N) out[static_cast<int64_t>(r) * N + c] = from_f<XT>(__builtin_nanf(""));
    }
    return;
  }
  const XS* x = static_cast<const XS*>(a.x) + xb * a.x_mat;
  const uint32_t* w = a.w + wb * a.w_mat;
  const int gs = AFF ? a.gs : SUBG;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = AFF ? static_cast<const XS*>(a.b) + wb * a.s_mat : nullptr;
  const uint8_t* s8 = static_cast<const uint8_t*>(a.s) + wb * a.s_mat;

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += BK) {
    // ---- x tile: BM x BK, 8 elements (16 B) per load
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = t + 256 * i, r = idx >> 3, cv = (idx & 7) * 8;
      const int gm = m0 + r, gk = k0 + cv;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (gm < M && gk < K) v = *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(gm) * K + gk);
      *reinterpret_cast<uint4*>(&As[r * LDK + cv]) = v;
    }
    // ---- W tile, dequantized into Bs[n][k]
    if constexpr (TRANS) {
      const int n = t >> 1, h = t & 1;
      const int gn = n0 + n, gk = k0 + 32 * h;
      uint16_t v[32];
      if (gn < N && gk < K) {
        const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
        uint32_t wd[BITS];
        load_chunk<BITS>(wd, w + gn * wpr + (gk >> 5) * BITS);
        const int G = K / gs;
#pragma unroll
        for (int hs = 0; hs < NSUB; ++hs) {
          float s, b = 0.f;
          const int64_t gi = static_cast<int64_t>(gn) * G + (gk + hs * SUBG) / gs;
          if constexpr (AFF) {
            s = to_f<XT>(sp[gi]);
            b = to_f<XT>(bp[gi]);
          } else {
            s = fp_scale<MODE>(s8[gi]);
          }
#pragma unroll
          for (int j = 0; j < SUBG; ++j) v[hs * SUBG + j] = deq16<XT, MODE, BITS>(wd, hs * SUBG + j, s, b);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = 0;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint4 u;
        u.x = v[8 * i] | (static_cast<uint32_t>(v[8 * i + 1]) << 16);
        u.y = v[8 * i + 2] | (static_cast<uint32_t>(v[8 * i + 3]) << 16);
        u.z = v[8 * i + 4] | (static_cast<uint32_t>(v[8 * i + 5]) << 16);
        u.w = v[8 * i + 6] | (static_cast<uint32_t>(v[8 * i + 7]) << 16);
        *reinterpret_cast<uint4*>(&Bs[n * LDK + 32 * h + 8 * i]) = u;
      }
    } else {
      // W is [K, N]: row k holds the codes of all n; one chunk = 32 n at fixed k
      const int kk = t >> 2, nc = t & 3;
      const int gk = k0 + kk, gn = n0 + 32 * nc;
      uint16_t v[32];
      if (gk < K && gn < N) {
        const int64_t wpr = static_cast<int64_t>(N) * BITS / 32;
        uint32_t wd[BITS];
        load_chunk<BITS>(wd, w + gk * wpr + (gn >> 5) * BITS);
        const int G = N / gs;
#pragma unroll
        for (int hs = 0; hs < NSUB; ++hs) {
          float s, b = 0.f;
          const int64_t gi = static_cast<int64_t>(gk) * G + (gn + hs * SUBG) / gs;
          if constexpr (AFF) {
            s = to_f<XT>(sp[gi]);
            b = to_f<XT>(bp[gi]);
          } else {
            s = fp_scale<MODE>(s8[gi]);
          }
#pragma unroll
          for (int j = 0; j < SUBG; ++j) v[hs * SUBG + j] = deq16<XT, MODE, BITS>(wd, hs * SUBG + j, s, b);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = 0;
      }
#pragma unroll
      for (int j = 0; j < 32; ++j) Bs[(32 * nc + j) * LDK + kk] = v[j];
    }
    __syncthreads();

    // ---- MFMA over the BK slice: lane l feeds row (l & 15), k = 8 * (l >> 4) .. +8
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      uint4 af[4], bf[4];
      const int koff = ks * 32 + 8 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const uint4*>(&As[(wm * 64 + i * 16 + (lane & 15)) * LDK + koff]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = *reinterpret_cast<const uint4*>(&Bs[(wn * 64 + j * 16 + (lane & 15)) * LDK + koff]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<XT>(af[i], bf[j], acc[i][j]);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds C[4 * (l >> 4) + r][l & 15] of each 16 x 16 block
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
        const int col = n0 + wn * 64 + j * 16 + (lane & 15);
        if (row < M && col < N) out[static_cast<int64_t>(row) * N + col] = from_f<XT>(acc[i][j][r]);
      }
}

bool qmm_mfma_supported(const QmmArgs& a) {
  return (a.xdt == BF16 || a.xdt == F16) && a.K % 32 == 0 && (a.transpose || a.N % 32 == 0);
}

namespace {
template <int XT, int MODE, int BITS>
hipError_t mfma_launch_t(const QmmArgs& a) {
  const int64_t ntn = (a.N + BN - 1) / BN, ntm = (a.M + BM - 1) / BM;
  const int64_t nblk = ntn * ntm * a.nbatch;
  if (nblk <= 0) return hipSuccess;
  if (nblk > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  dim3 grid(static_cast<unsigned>(nblk));
  if (a.transpose)
    hipLaunchKernelGGL((qmm_mfma_kernel<XT, MODE, BITS, true>), grid, dim3(256), 0, a.stream, a, ntn, ntm);
  else
    hipLaunchKernelGGL((qmm_mfma_kernel<XT, MODE, BITS, false>), grid, dim3(256), 0, a.stream, a, ntn, ntm);
  return hipGetLastError();
}

template <int XT>
hipError_t mfma_by_mode(const QmmArgs& a) {
  switch (a.mode) {
    case AFFINE:
      switch (a.bits) {
        case 2: return mfma_launch_t<XT, AFFINE, 2>(a);
        case 3: return mfma_launch_t<XT, AFFINE, 3>(a);
        case 4: return mfma_launch_t<XT, AFFINE, 4>(a);
        case 5: return mfma_launch_t<XT, AFFINE, 5>(a);
        case 6: return mfma_launch_t<XT, AFFINE, 6>(a);
        case 8: return mfma_launch_t<XT, AFFINE, 8>(a);
      }
      break;
    case MXFP4: return mfma_launch_t<XT, MXFP4, 4>(a);
    case MXFP8: return mfma_launch_t<XT, MXFP8, 8>(a);
    case NVFP4: return mfma_launch_t<XT, NVFP4, 4>(a);
  }
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_qmm_mfma(const QmmArgs& a) {
  if (a.xdt == BF16) return mfma_by_mode<BF16>(a);
  if (a.xdt == F16) return mfma_by_mode<F16>(a);
  return hipErrorInvalidValue;
}

}  // namespace iqmm
