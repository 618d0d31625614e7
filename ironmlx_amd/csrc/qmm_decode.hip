// qmm_decode.hip — affine 4-bit quantized matmul at decode widths (transpose,
// 1 <= M <= 32 x rows, gs 32 / 64 / 128) on CDNA4 matrix cores: the batched
// decode step of mlx/src/nn/linear.rs:51-63 with x = [B, 1, K] (B sequences
// that mlx/src/generate/batch.rs:313-339 would run as B separate M = 1 calls).
//
// The weights enter v_mfma_f32_16x16x32 undequantized: v_perm_b32 turns each
// nibble n into the 16-bit value C + n (C = 128 bf16 / 1024 fp16, unit
// spacing) and x is permuted to the same pair order; per quantization group
//   sum x (s q + b) = s D + (b - C s) X,   D = sum x (C + q),  X = sum x,
// with X from the same MFMA against an all-ones operand.  K slots are
// chunk-major: MFMA j of a 128-code block takes chunk 4p + j (inside one
// group for gs >= 32) and lane (r, q) its 8-code piece q, so an x load is 64
// contiguous bytes per row; each lane loads one 16-byte weight chunk and a
// 4 x 4 dword transpose across the lanes q (v_permlane32_swap, then
// v_permlane16_swap) hands it out.
//
// A workgroup owns NT 16-row tiles (NC = 16 NT output columns) and its S waves
// split K into S ranges of KB blocks each (KB is a template argument: the
// K loop is fully unrolled and every offset is an immediate).  Each wave reads
// the scale / bias words of its whole K range for its NT rows once (every lane
// of a row loads the same words), keeps D blocks of x and weights in flight,
// and leaves NT x MT 16 x 16 fp32 partial tiles that meet in LDS.  Rows past M
// read the last x row and produce output rows that are never stored, so no
// per-element masking is needed.  GLU: the weight holds 2N rows (gate rows
// [0, N), up rows [N, 2N)); tiles [0, NT/2) take gate rows and [NT/2, NT) the
// matching up rows, and the epilogue writes silu(gate) * up (NC = 8 NT).
//
// Measured against the previous decode-width kernel on MI355X (bf16, gs 64):
// K = 4096, N = 14336: M = 4 / 16 / 32 17.9 / 20.2 / 23.5 -> 12.1 / 13.8 /
// 17.5 us; N = 4096, K = 14336: M = 4 / 16 21.4 / 27.7 -> 13.6 / 19.2 us.
#include <type_traits>

#include "launch.h"
#include "mfma_common.h"
#include "decode_common.h"

namespace iqmm {
namespace {

template <int XT, int NT, int MT, int GB, int S, int D, int KB, bool GLU, bool MAPPED>
__global__ __launch_bounds__(64 * S) void qmm_decode_kernel(QmmArgs a) {
  static_assert(!GLU || NT % 2 == 0, "GLU pairs gate tiles with up tiles");
  constexpr int NC = GLU ? 8 * NT : 16 * NT;  // output columns per workgroup
  using XS = uint16_t;
  constexpr float CM = XT == BF16 ? 128.f : 1024.f;
  constexpr uint32_t EB = XT == BF16 ? 0x43434343u : 0x64646464u;
  constexpr uint32_t ONE2 = XT == BF16 ? 0x3f803f80u : 0x3c003c00u;
  constexpr int JG = 4 / GB;         // MFMAs per group
  constexpr int SH = KB * GB;        // 16-bit scale halves per row in the wave's K range
  constexpr int SW = (SH + 1) / 2;   // 32-bit words holding them
  __shared__ float red[S > 1 ? S * NT * MT * 256 : 1];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int M = a.M, N = a.N, K = a.K;
  const int n0 = blockIdx.x * NC;
  const int64_t bb = blockIdx.y;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;
  int64_t xb = bb, wb = bb;
  if constexpr (MAPPED) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      for (int i = t; i < M * NC; i += 64 * S) {
        const int m = i / NC, n = n0 + i % NC;
        if (n < N) out[static_cast<int64_t>(m) * N + n] = from_f<XT>(__builtin_nanf(""));
      }
      return;
    }
  }
  const int gshift = __builtin_ctz(a.gs);
  const int64_t wrow = K / 2, srow = (K >> gshift) * 2, xrow = static_cast<int64_t>(K) * 2;
  const int r = lane & 15, q = lane >> 4;
  const int pb = KB * wave;  // first 128-code block of this wave
  const char* xbase = reinterpret_cast<const char*>(static_cast<const XS*>(a.x) + xb * a.x_mat);
  const char* xr[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) xr[i] = xbase + min(i * 16 + r, M - 1) * xrow + pb * 256 + 16 * q;
  const char* w = reinterpret_cast<const char*>(a.w + wb * a.w_mat);
  const char* sp = reinterpret_cast<const char*>(static_cast<const XS*>(a.s) + wb * a.s_mat);
  const char* bp = reinterpret_cast<const char*>(static_cast<const XS*>(a.b) + wb * a.s_mat);
  const char* wr[NT];
  uint32_t sw[NT][SW], bw[NT][SW];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int64_t n = GLU ? static_cast<int64_t>(tt / (NT / 2)) * N + min(n0 + 16 * (tt % (NT / 2)) + r, N - 1)
                          : min(n0 + 16 * tt + r, N - 1);
    wr[tt] = w + n * wrow + pb * 64 + 16 * q;
    // the scale halves of [pb, pb + KB) start at half pb * GB; pb * GB is even
    // unless GB = 1 and KB is odd, which the launcher excludes
    const char* s0 = sp + n * srow + pb * GB * 2;
    const char* b0 = bp + n * srow + pb * GB * 2;
#pragma unroll
    for (int h = 0; h < SW; ++h) {
      sw[tt][h] = *reinterpret_cast<const uint32_t*>(s0 + 4 * h);
      bw[tt][h] = *reinterpret_cast<const uint32_t*>(b0 + 4 * h);
    }
  }
  struct Blk {
    g_u32x4_t xa[MT][4];
    g_u32x4_t wv[NT];
  };
  auto load = [&](int b, Blk& B) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) B.xa[i][j] = *reinterpret_cast<const g_u32x4_t*>(xr[i] + b * 256 + 64 * j);
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
      B.wv[tt] = __builtin_nontemporal_load(reinterpret_cast<const g_u32x4_t*>(wr[tt] + b * 64));
  };
  f32x4d_t Y[NT][MT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int i = 0; i < MT; ++i) Y[tt][i] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  const g_u32x4_t ones = {ONE2, ONE2, ONE2, ONE2};
  auto compute = [&](const Blk& B, int b) {
    g_u32x4_t A[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // (x0,x4) (x1,x5) (x2,x6) (x3,x7), the pair order of the weights below
        const g_u32x4_t v = B.xa[i][j];
        A[i][j] = g_u32x4_t{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                            __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
      }
    f32x4d_t XG[MT][GB];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        XG[i][g] = mfma16<XT>(A[i][g * JG], ones, f32x4d_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int j = 1; j < JG; ++j) XG[i][g] = mfma16<XT>(A[i][g * JG + j], ones, XG[i][g]);
      }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      uint32_t wd[4] = {B.wv[tt].x, B.wv[tt].y, B.wv[tt].z, B.wv[tt].w};
      // 4 x 4 transpose over the lanes q: afterwards wd[j] of lane q is dword
      // q of the chunk that lane j loaded (chunk 4p + j)
      auto s02 = __builtin_amdgcn_permlane32_swap(wd[0], wd[2], false, false);
      auto s13 = __builtin_amdgcn_permlane32_swap(wd[1], wd[3], false, false);
      auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
      auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
      wd[0] = s01[0]; wd[1] = s01[1]; wd[2] = s23[0]; wd[3] = s23[1];
      g_u32x4_t Wp[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = wd[j] & 0x0F0F0F0Fu, hi = (wd[j] >> 4) & 0x0F0F0F0Fu;
        Wp[j] = g_u32x4_t{__builtin_amdgcn_perm(EB, lo, 0x04020400u), __builtin_amdgcn_perm(EB, hi, 0x04020400u),
                          __builtin_amdgcn_perm(EB, lo, 0x04030401u), __builtin_amdgcn_perm(EB, hi, 0x04030401u)};
      }
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        const int hf = b * GB + g;  // scale half of this group within the range
        const float s = to_f<XT>(static_cast<XS>(sw[tt][hf >> 1] >> (16 * (hf & 1))));
        const float bs = to_f<XT>(static_cast<XS>(bw[tt][hf >> 1] >> (16 * (hf & 1))));
        const float cb = fmaf(-CM, s, bs);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          f32x4d_t Dd = mfma16<XT>(A[i][g * JG], Wp[g * JG], f32x4d_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int j = 1; j < JG; ++j) Dd = mfma16<XT>(A[i][g * JG + j], Wp[g * JG + j], Dd);
#pragma unroll
          for (int v = 0; v < 4; ++v) Y[tt][i][v] = fmaf(s, Dd[v], fmaf(cb, XG[i][g][v], Y[tt][i][v]));
        }
      }
    }
  };
  Blk ring[D];
#pragma unroll
  for (int d = 0; d < D && d < KB; ++d) load(d, ring[d]);
#pragma unroll
  for (int b = 0; b < KB; ++b) {
    compute(ring[b % D], b);
    if (b + D < KB) load(b + D, ring[b % D]);
  }
  // lane holds Y[m = 16 i + 4 q + v][n = 16 tt + r] of each tile
  if constexpr (S == 1) {
#pragma unroll
    for (int tt = 0; tt < (GLU ? NT / 2 : NT); ++tt)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = 16 * i + 4 * q + v, n = n0 + 16 * tt + r;
          if (m < M && n < N)
            out[static_cast<int64_t>(m) * N + n] =
                GLU ? swiglu_out<XT>(Y[tt][i][v], Y[tt + NT / 2][i][v]) : from_f<XT>(Y[tt][i][v]);
        }
    return;
  }
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[((wave * NT + tt) * MT + i) * 256 + (4 * q + v) * 16 + r] = Y[tt][i][v];
  __syncthreads();
  for (int idx = t; idx < M * NC; idx += 64 * S) {
    const int m = idx / NC, nn = idx % NC;
    const int i = m >> 4, mr = m & 15;
    if (n0 + nn >= N) continue;
    if constexpr (GLU) {
      float acc[2] = {0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int tt = h * (NT / 2) + (nn >> 4);
#pragma unroll
        for (int w2 = 0; w2 < S; ++w2) acc[h] += red[((w2 * NT + tt) * MT + i) * 256 + mr * 16 + (nn & 15)];
      }
      out[static_cast<int64_t>(m) * N + n0 + nn] = swiglu_out<XT>(acc[0], acc[1]);
    } else {
      const int tt = nn >> 4;
      float acc = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < S; ++w2) acc += red[((w2 * NT + tt) * MT + i) * 256 + mr * 16 + (nn & 15)];
      out[static_cast<int64_t>(m) * N + n0 + nn] = from_f<XT>(acc);
    }
  }
}

// One configuration: NT tiles per workgroup, MT x-row tiles, S waves, D
// blocks in flight, KB blocks per wave (K = 128 KB S).
struct DecCfg {
  int nt, s, d, kb;
};

// Choice per shape (measured on MI355X, bf16, gs 64, M in {4, 8, 16, 32}):
// wide matrices (>= 8192 rows) take four tiles and eight waves of four
// blocks (K = 4096); 6144 rows two tiles; narrower ones one tile and four
// waves of eight blocks so that enough workgroups exist; K = 14336 four waves
// of 28 blocks (M <= 16) or eight of 14 (M > 16).
DecCfg choose(const QmmArgs& a, int64_t rows) {
  const int P = a.K >> 7;
  const bool two_mt = a.M > 16;
  DecCfg c{1, 4, 3, 0};
  if (P == 32) {
    if (rows >= 8192) c = DecCfg{4, 8, 2, 4};
    else if (rows >= 6144) c = DecCfg{2, 8, 2, 4};
    else c = two_mt ? DecCfg{1, 8, 2, 4} : DecCfg{1, 4, 3, 8};
  } else if (P == 112) {
    c = two_mt ? DecCfg{1, 8, 2, 14} : DecCfg{1, 4, 3, 28};
  } else if (P % 8 == 0 && P / 8 <= 32) {
    c = DecCfg{1, 8, 2, P / 8};
  } else if (P % 4 == 0 && P / 4 <= 32) {
    c = DecCfg{1, 4, 3, P / 4};
  } else {
    c.kb = 0;  // unsupported
  }
  if (a.glu && c.nt < 2) c.nt = 2;
  return c;
}

template <int XT, int NT, int MT, int GB, int S, int D, int KB, bool GLU>
hipError_t dec_go(const QmmArgs& a, dim3 grid) {
  if constexpr (GLU && NT % 2 != 0) {
    return hipErrorInvalidValue;  // choose() gives GLU two or more tiles
  } else {
  const bool mapped = a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr;
  if (mapped)
    hipLaunchKernelGGL((qmm_decode_kernel<XT, NT, MT, GB, S, D, KB, GLU, true>), grid, dim3(64 * S), 0, a.stream, a);
  else
    hipLaunchKernelGGL((qmm_decode_kernel<XT, NT, MT, GB, S, D, KB, GLU, false>), grid, dim3(64 * S), 0, a.stream, a);
  return hipGetLastError();
  }
}

// the instantiated (NT, S, D, KB) configurations
template <int XT, int MT, int GB, bool GLU>
hipError_t dec_cfg(const QmmArgs& a, const DecCfg& c, dim3 grid) {
#define IQMM_DEC(NT_, S_, D_, KB_)                                                    \
  if (c.nt == NT_ && c.s == S_ && c.d == D_ && c.kb == KB_)                           \
    return dec_go<XT, NT_, MT, GB, S_, D_, KB_, GLU>(a, grid);
  IQMM_DEC(4, 8, 2, 4)
  IQMM_DEC(2, 8, 2, 4)
  IQMM_DEC(1, 8, 2, 4)
  IQMM_DEC(1, 4, 3, 8)
  IQMM_DEC(2, 4, 3, 8)
  IQMM_DEC(1, 8, 2, 14)
  IQMM_DEC(2, 8, 2, 14)
  IQMM_DEC(1, 4, 3, 28)
  IQMM_DEC(2, 4, 3, 28)
  IQMM_DEC(1, 8, 2, 8)
  IQMM_DEC(2, 8, 2, 8)
  IQMM_DEC(1, 8, 2, 2)
  IQMM_DEC(2, 8, 2, 2)
  IQMM_DEC(1, 8, 2, 16)
  IQMM_DEC(2, 8, 2, 16)
#undef IQMM_DEC
  return hipErrorInvalidValue;
}

bool cfg_instantiated(const DecCfg& c) {
  static const DecCfg known[] = {{4, 8, 2, 4}, {2, 8, 2, 4}, {1, 8, 2, 4}, {1, 4, 3, 8}, {2, 4, 3, 8},
                                 {1, 8, 2, 14}, {2, 8, 2, 14}, {1, 4, 3, 28}, {2, 4, 3, 28}, {1, 8, 2, 8},
                                 {2, 8, 2, 8}, {1, 8, 2, 2}, {2, 8, 2, 2}, {1, 8, 2, 16}, {2, 8, 2, 16}};
  for (const DecCfg& k : known)
    if (k.nt == c.nt && k.s == c.s && k.d == c.d && k.kb == c.kb) return true;
  return false;
}

template <int XT, int GB, bool GLU>
hipError_t dec_launch(const QmmArgs& a) {
  const int64_t rows = static_cast<int64_t>(a.N) * (GLU ? 2 : 1) * a.nbatch;
  const DecCfg c = choose(a, rows);
  const int nc = GLU ? 8 * c.nt : 16 * c.nt;
  const dim3 grid(static_cast<unsigned>((a.N + nc - 1) / nc), static_cast<unsigned>(a.nbatch));
  return a.M > 16 ? dec_cfg<XT, 2, GB, GLU>(a, c, grid) : dec_cfg<XT, 1, GB, GLU>(a, c, grid);
}

template <int XT, bool GLU>
hipError_t dec_launch_gs(const QmmArgs& a) {
  switch (a.gs) {
    case 32: return dec_launch<XT, 4, GLU>(a);
    case 64: return dec_launch<XT, 2, GLU>(a);
    default: return dec_launch<XT, 1, GLU>(a);
  }
}

}  // namespace

bool qmm_decode_supported(const QmmArgs& a) {
  if (!(a.transpose && a.mode == AFFINE && a.bits == 4 && (a.xdt == BF16 || a.xdt == F16) && a.M >= 1 &&
        a.M <= 32 && a.K % 128 == 0 && a.nbatch >= 1 && a.nbatch <= 65535 && a.N >= 1))
    return false;
  if (a.gs != 32 && a.gs != 64 && a.gs != 128) return false;
  const int64_t rows = static_cast<int64_t>(a.N) * (a.glu ? 2 : 1) * a.nbatch;
  const DecCfg c = choose(a, rows);
  if (c.kb == 0 || c.kb * c.s * 128 != a.K || !cfg_instantiated(c)) return false;
  // gs 128: one scale half per block, the wave's first half must start a word
  if (a.gs == 128 && c.kb % 2 != 0) return false;
  // scales / biases are read as aligned 32-bit words
  const bool aligned = (reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 4 == 0 &&
                       ((a.K / a.gs) * 2) % 4 == 0;
  // one matrix below 2^31 bytes of codes (32-bit row arithmetic of x offsets)
  return aligned && static_cast<int64_t>(a.M) * a.K * 2 < (int64_t{1} << 31);
}

hipError_t launch_qmm_decode(const QmmArgs& a) {
  if (a.glu) return a.xdt == BF16 ? dec_launch_gs<BF16, true>(a) : dec_launch_gs<F16, true>(a);
  return a.xdt == BF16 ? dec_launch_gs<BF16, false>(a) : dec_launch_gs<F16, false>(a);
}

}  // namespace iqmm
