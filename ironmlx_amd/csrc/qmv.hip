// qmv.hip — decode-shaped quantized matmul on the vector ALUs (small M).
//
//   qmv: transpose=true,  out[m, n] = sum_k x[m, k] * deq(W)[n, k]
//   qvm: transpose=false, out[m, n] = sum_k x[m, k] * deq(W)[k, n]
//
// qmv streams each weight row once: lanes of a row-slot walk the row's
// 32-code chunks with coalesced 16-byte loads (4-bit), decode codes in
// registers and accumulate in fp32 in the factored form
//   sum_g [ s_g * sum_{k in g} x_k q_k  +  b_g * sum_{k in g} x_k ]
// so the affine rescale costs two FMAs per 32 codes, not per code.  A wave
// owns (64 / LPR) row-slots of NR rows each; NR rows share every x chunk
// load.  Partial sums are reduced across the LPR lanes of a slot with
// cross-lane shuffles.  Reference op: mlx/src/ops.rs:695-727 (decode calls
// from mlx/src/nn/linear.rs:51-63 are always M=1, batch.rs:323-333).
#include "launch.h"

namespace iqmm {

template <int XT>
__device__ __forceinline__ void load_x32(float (&xf)[32], const typename Store<XT>::T* p) {
  if constexpr (XT == F32) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float4 v = reinterpret_cast<const float4*>(p)[i];
      xf[4 * i] = v.x; xf[4 * i + 1] = v.y; xf[4 * i + 2] = v.z; xf[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint4 v = reinterpret_cast<const uint4*>(p)[i];
      uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xf[8 * i + 2 * j] = to_f<XT>(static_cast<uint16_t>(u[j] & 0xffffu));
        xf[8 * i + 2 * j + 1] = to_f<XT>(static_cast<uint16_t>(u[j] >> 16));
      }
    }
  }
}

// value of code j of a chunk as the float the dot product uses: the integer
// code (affine) or the decoded element (fp modes)
template <int MODE, int BITS>
__device__ __forceinline__ float code_value(const uint32_t (&wd)[BITS], int j) {
  const uint32_t q = chunk_code<BITS>(wd, j);
  if constexpr (MODE == AFFINE) return static_cast<float>(q);
  else return fp_elem<MODE>(q);
}

template <int XT, int MODE, int BITS, int MT, int NR>
__global__ __launch_bounds__(256) void qmv_kernel(QmmArgs a, int lpr_log2, int64_t nrb,
                                                  int64_t nmt) {
  using XS = typename Store<XT>::T;
  constexpr bool AFF = MODE == AFFINE;
  constexpr int SUBG = MODE == NVFP4 ? 16 : 32;  // codes of a chunk sharing a scale
  constexpr int NSUB = 32 / SUBG;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int LPR = 1 << lpr_log2, spw = 64 >> lpr_log2;
  const int slot = lane >> lpr_log2, sub = lane & (LPR - 1);

  const int64_t blk = blockIdx.x;
  const int64_t rb = blk % nrb, mt = (blk / nrb) % nmt, bb = blk / (nrb * nmt);
  const int M = a.M, N = a.N, K = a.K;
  const int64_t row0 = ((rb * 4 + wave) * spw + slot) * NR;
  const int m0 = static_cast<int>(mt) * MT;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;

  int64_t xb, wb;
  if (!map_batch(a.bm, bb, xb, wb)) {
    if (sub == 0)
      for (int r = 0; r < NR; ++r)
        for (int m = 0; m < MT; ++m)
          if (row0 + r < N && m0 + m < M)
            out[static_cast<int64_t>(m0 + m) * N + row0 + r] = from_f<XT>(__builtin_nanf(""));
    return;
  }
  const XS* x = static_cast<const XS*>(a.x) + xb * a.x_mat;
  const uint32_t* w = a.w + wb * a.w_mat;
  const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
  const int gs = AFF ? a.gs : SUBG;
  const int G = K / gs;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = AFF ? static_cast<const XS*>(a.b) + wb * a.s_mat : nullptr;
  const uint8_t* s8 = static_cast<const uint8_t*>(a.s) + wb * a.s_mat;

  int64_t rows[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) rows[r] = min(row0 + r, static_cast<int64_t>(N - 1));

  float acc[MT][NR];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[m][r] = 0.f;

  const int C = K >> 5;
#pragma unroll 2
  for (int c = sub; c < C; c += LPR) {
    uint32_t wd[NR][BITS];
#pragma unroll
    for (int r = 0; r < NR; ++r) load_chunk<BITS>(wd[r], w + rows[r] * wpr + c * BITS);
    float xf[MT][32];
    float xs[MT][NSUB];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m0 + m < M) {
        load_x32<XT>(xf[m], x + static_cast<int64_t>(m0 + m) * K + c * 32);
      } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) xf[m][j] = 0.f;
      }
      if constexpr (AFF) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j) t += xf[m][j];
        xs[m][0] = t;
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float sc[NSUB], bi = 0.f;
      if constexpr (AFF) {
        const int64_t gi = rows[r] * G + (c * 32) / gs;
        sc[0] = to_f<XT>(sp[gi]);
        bi = to_f<XT>(bp[gi]);
      } else {
#pragma unroll
        for (int h = 0; h < NSUB; ++h) sc[h] = fp_scale<MODE>(s8[rows[r] * G + c * NSUB + h]);
      }
#pragma unroll
      for (int h = 0; h < NSUB; ++h) {
        float d[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) d[m] = 0.f;
#pragma unroll
        for (int j = 0; j < SUBG; ++j) {
          const float q = code_value<MODE, BITS>(wd[r], h * SUBG + j);
#pragma unroll
          for (int m = 0; m < MT; ++m) d[m] = fmaf(xf[m][h * SUBG + j], q, d[m]);
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if constexpr (AFF) acc[m][r] += fmaf(sc[0], d[m], bi * xs[m][0]);
          else acc[m][r] = fmaf(sc[h], d[m], acc[m][r]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[m][r] = wave_sum_width(acc[m][r], LPR);
  if (sub == 0) {
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (row0 + r < N && m0 + m < M)
          out[static_cast<int64_t>(m0 + m) * N + row0 + r] = from_f<XT>(acc[m][r]);
  }
}

// transpose=false: a thread owns one 32-column chunk of W's packed rows and a
// slice of the k range; slices are summed through LDS.
template <int XT, int MODE, int BITS>
__global__ __launch_bounds__(256) void qvm_kernel(QmmArgs a, int cw_log2, int64_t nnb) {
  using XS = typename Store<XT>::T;
  constexpr bool AFF = MODE == AFFINE;
  constexpr int SUBG = MODE == NVFP4 ? 16 : 32;
  constexpr int NSUB = 32 / SUBG;
  __shared__ float red[256 * 33];
  const int CW = 1 << cw_log2, KS = 256 >> cw_log2;
  const int t = threadIdx.x, cl = t & (CW - 1), ks = t >> cw_log2;
  const int M = a.M, N = a.N, K = a.K;
  const int64_t blk = blockIdx.x;
  const int64_t nb = blk % nnb, m = (blk / nnb) % M, bb = blk / (nnb * M);
  const int64_t cc = nb * CW + cl;
  const int CN = N >> 5;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N + m * N;

  int64_t xb, wb;
  const bool ok = map_batch(a.bm, bb, xb, wb);
  float acc[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) acc[j] = 0.f;
  if (ok && cc < CN) {
    const XS* x = static_cast<const XS*>(a.x) + xb * a.x_mat + m * K;
    const uint32_t* w = a.w + wb * a.w_mat;
    const int64_t wpr = static_cast<int64_t>(N) * BITS / 32;
    const int gs = AFF ? a.gs : SUBG;
    const int G = N / gs;
    const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
    const XS* bp = AFF ? static_cast<const XS*>(a.b) + wb * a.s_mat : nullptr;
    const uint8_t* s8 = static_cast<const uint8_t*>(a.s) + wb * a.s_mat;
    for (int k = ks; k < K; k += KS) {
      uint32_t wd[BITS];
      load_chunk<BITS>(wd, w + k * wpr + cc * BITS);
      const float xv = to_f<XT>(x[k]);
      if constexpr (AFF) {
        const int64_t gi = static_cast<int64_t>(k) * G + (cc * 32) / gs;
        const float t1 = xv * to_f<XT>(sp[gi]), t2 = xv * to_f<XT>(bp[gi]);
#pragma unroll
        for (int j = 0; j < 32; ++j)
          acc[j] += fmaf(t1, static_cast<float>(chunk_code<BITS>(wd, j)), t2);
      } else {
#pragma unroll
        for (int h = 0; h < NSUB; ++h) {
          const float t1 = xv * fp_scale<MODE>(s8[static_cast<int64_t>(k) * G + cc * NSUB + h]);
#pragma unroll
          for (int j = 0; j < SUBG; ++j)
            acc[h * SUBG + j] = fmaf(t1, fp_elem<MODE>(chunk_code<BITS>(wd, h * SUBG + j)),
                                     acc[h * SUBG + j]);
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 32; ++j) red[(ks * CW + cl) * 33 + j] = acc[j];
  __syncthreads();
  for (int o = t; o < CW * 32; o += 256) {
    const int c2 = o >> 5, j = o & 31;
    float v = 0.f;
    for (int s = 0; s < KS; ++s) v += red[(s * CW + c2) * 33 + j];
    const int64_t col = (nb * CW + c2) * 32 + j;
    if (col < N) out[col] = from_f<XT>(ok ? v : __builtin_nanf(""));
  }
}

// ------------------------------------------------------------------ dispatch
namespace {
int ilog2_floor(int64_t v) {
  int l = 0;
  while ((int64_t(1) << (l + 1)) <= v) ++l;
  return l;
}

template <int XT, int MODE, int BITS>
hipError_t qmv_launch_t(const QmmArgs& a) {
  const int C = a.K / 32;
  const int lpr_log2 = C >= 64 ? 6 : ilog2_floor(C > 0 ? C : 1);
  const int spw = 64 >> lpr_log2;
  const int mt_size = a.M == 1 ? 1 : 4;
  const int64_t nmt = (a.M + mt_size - 1) / mt_size;
  // NR=4 rows per slot when that still leaves >= ~2 waves of work per CU
  const int64_t rows_nr4 = 4LL * spw * 4;
  const bool big = ((a.N + rows_nr4 - 1) / rows_nr4) * nmt * a.nbatch >= 512;
  const int nr = big ? 4 : 1;
  const int64_t rows_per_blk = 4LL * spw * nr;
  const int64_t nrb = (a.N + rows_per_blk - 1) / rows_per_blk;
  const int64_t nblk = nrb * nmt * a.nbatch;
  if (nblk <= 0) return hipSuccess;
  if (nblk > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  dim3 grid(static_cast<unsigned>(nblk)), block(256);
  if (mt_size == 1) {
    if (nr == 4) hipLaunchKernelGGL((qmv_kernel<XT, MODE, BITS, 1, 4>), grid, block, 0, a.stream, a, lpr_log2, nrb, nmt);
    else hipLaunchKernelGGL((qmv_kernel<XT, MODE, BITS, 1, 1>), grid, block, 0, a.stream, a, lpr_log2, nrb, nmt);
  } else {
    if (nr == 4) hipLaunchKernelGGL((qmv_kernel<XT, MODE, BITS, 4, 4>), grid, block, 0, a.stream, a, lpr_log2, nrb, nmt);
    else hipLaunchKernelGGL((qmv_kernel<XT, MODE, BITS, 4, 1>), grid, block, 0, a.stream, a, lpr_log2, nrb, nmt);
  }
  return hipGetLastError();
}

template <int XT, int MODE, int BITS>
hipError_t qvm_launch_t(const QmmArgs& a) {
  const int64_t CN = a.N / 32;
  int cw_log2 = 0;
  while (cw_log2 < 6 && (int64_t(1) << cw_log2) < CN) ++cw_log2;
  const int64_t nnb = (CN + (1 << cw_log2) - 1) >> cw_log2;
  const int64_t nblk = nnb * a.M * a.nbatch;
  if (nblk <= 0) return hipSuccess;
  if (nblk > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((qvm_kernel<XT, MODE, BITS>), dim3(static_cast<unsigned>(nblk)), dim3(256), 0,
                     a.stream, a, cw_log2, nnb);
  return hipGetLastError();
}

template <int XT>
hipError_t qmv_by_mode(const QmmArgs& a, bool trans) {
#define IQMM_CASE(MODE, BITS) \
  return trans ? qmv_launch_t<XT, MODE, BITS>(a) : qvm_launch_t<XT, MODE, BITS>(a)
  switch (a.mode) {
    case AFFINE:
      switch (a.bits) {
        case 2: IQMM_CASE(AFFINE, 2);
        case 3: IQMM_CASE(AFFINE, 3);
        case 4: IQMM_CASE(AFFINE, 4);
        case 5: IQMM_CASE(AFFINE, 5);
        case 6: IQMM_CASE(AFFINE, 6);
        case 8: IQMM_CASE(AFFINE, 8);
      }
      break;
    case MXFP4: IQMM_CASE(MXFP4, 4);
    case MXFP8: IQMM_CASE(MXFP8, 8);
    case NVFP4: IQMM_CASE(NVFP4, 4);
  }
#undef IQMM_CASE
  return hipErrorInvalidValue;
}

hipError_t qmv_any(const QmmArgs& a, bool trans) {
  switch (a.xdt) {
    case F32: return qmv_by_mode<F32>(a, trans);
    case F16: return qmv_by_mode<F16>(a, trans);
    case BF16: return qmv_by_mode<BF16>(a, trans);
  }
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_qmv(const QmmArgs& a) { return qmv_any(a, true); }
hipError_t launch_qvm(const QmmArgs& a) { return qmv_any(a, false); }

}  // namespace iqmm
