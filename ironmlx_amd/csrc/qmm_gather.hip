// qmm_gather.hip — sorted grouped gather_qmm (affine 4-bit, gs 32 / 64 / 128)
// with the factored MFMA arithmetic of qmm_decode.hip.
#include <type_traits>

#include "launch.h"
#include "mfma_common.h"
#include "decode_common.h"

namespace iqmm {
namespace {

// Sorted grouped gather_qmm (sorted_indices; the MoE layer of
// mlx/src/nn/moe.rs:84-170 over the stacked experts of
// mlx/src/model/qwen35.rs:653-775) with the factored arithmetic above.
// Workgroup (column block, expert e) takes the expert's rows [off[e],
// off[e + 1]) of the flattened batch (x rows gathered through lhs), in passes
// of up to 32 rows; each wave streams its K range of the expert's weight rows
// per pass (the first pass from HBM, later ones from L2).  The scale / bias
// words of the wave's range are read once.  Rows whose lhs index is out of
// range are written as NaN; workgroup e = E (one past the experts) writes NaN
// for batch entries outside every expert's segment.
template <int XT, int NT, int GB, int S, int D, int KB, bool GLU>
__global__ __launch_bounds__(64 * S) void gather_decode_kernel(QmmArgs a, int64_t nflat, const int64_t* off) {
  static_assert(!GLU || NT % 2 == 0, "GLU pairs gate tiles with up tiles");
  constexpr int NC = GLU ? 8 * NT : 16 * NT;
  using XS = uint16_t;
  constexpr float CM = XT == BF16 ? 128.f : 1024.f;
  constexpr uint32_t EB = XT == BF16 ? 0x43434343u : 0x64646464u;
  constexpr uint32_t ONE2 = XT == BF16 ? 0x3f803f80u : 0x3c003c00u;
  constexpr int JG = 4 / GB;
  constexpr int SW = (KB * GB + 1) / 2;
  __shared__ float red[S > 1 ? S * NT * 2 * 256 : 1];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int Mx = a.M, N = a.N, K = a.K;
  const int n0 = blockIdx.x * NC;
  const int64_t e = blockIdx.y;
  XS* out = static_cast<XS*>(a.out);
  if (e == a.bm.nw) {
    // offsets are clamped into [0, nflat]: indices that are not sorted as
    // promised give wrong rows, never out-of-range accesses
    const int64_t first_valid = min(max(off[0], int64_t{0}), nflat);
    const int64_t end_valid = min(max(off[e], first_valid), nflat);
    const int64_t nbad = first_valid + (nflat - end_valid);
    for (int64_t i = t; i < nbad * Mx * NC; i += 64 * S) {
      const int64_t rr = i / NC, n = i % NC;
      const int64_t bi = rr / Mx, mrow = rr % Mx;
      const int64_t b = bi < first_valid ? bi : end_valid + (bi - first_valid);
      if (n0 + n < N) out[(b * Mx + mrow) * N + n0 + n] = from_f<XT>(__builtin_nanf(""));
    }
    return;
  }
  const int64_t blo = min(max(off[e], int64_t{0}), nflat);
  const int64_t bhi = min(max(off[e + 1], blo), nflat);
  if (blo >= bhi) return;  // workgroup-uniform
  const int64_t rows_total = (bhi - blo) * Mx;
  const int gshift = __builtin_ctz(a.gs);
  const int64_t wrow = K / 2, srow = (K >> gshift) * 2;
  const int r = lane & 15, q = lane >> 4;
  const int pb = KB * wave;
  const XS* x = static_cast<const XS*>(a.x);
  const char* w = reinterpret_cast<const char*>(a.w + e * a.w_mat);
  const char* sp = reinterpret_cast<const char*>(static_cast<const XS*>(a.s) + e * a.s_mat);
  const char* bp = reinterpret_cast<const char*>(static_cast<const XS*>(a.b) + e * a.s_mat);
  const char* wr[NT];
  uint32_t sw[NT][SW], bw[NT][SW];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int64_t n = GLU ? static_cast<int64_t>(tt / (NT / 2)) * N + min(n0 + 16 * (tt % (NT / 2)) + r, N - 1)
                          : min(n0 + 16 * tt + r, N - 1);
    wr[tt] = w + n * wrow + pb * 64 + 16 * q;
    const char* s0 = sp + n * srow + pb * GB * 2;
    const char* b0 = bp + n * srow + pb * GB * 2;
#pragma unroll
    for (int h = 0; h < SW; ++h) {
      sw[tt][h] = *reinterpret_cast<const uint32_t*>(s0 + 4 * h);
      bw[tt][h] = *reinterpret_cast<const uint32_t*>(b0 + 4 * h);
    }
  }
  const g_u32x4_t ones = {ONE2, ONE2, ONE2, ONE2};
  // one pass over rows [r0, r0 + 16 MT) of the expert
  auto pass = [&](auto mt_c, int64_t r0) {
    constexpr int MT = decltype(mt_c)::value;
    const char* xr[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int64_t rr = min(r0 + 16 * i + r, rows_total - 1);
      const int64_t b = blo + rr / Mx, mrow = rr % Mx;
      const int64_t xm = a.bm.lhs ? load_index(a.bm.lhs, a.bm.lhs_dt, b) : b;
      const int64_t xs = (xm >= 0 && xm < a.bm.nx) ? xm : 0;
      xr[i] = reinterpret_cast<const char*>(x + xs * a.x_mat + mrow * K) + pb * 256 + 16 * q;
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
    auto compute = [&](const Blk& B, int b) {
      g_u32x4_t A[MT][4];
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
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
          const int hf = b * GB + g;
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
    // row rr = r0 + 16 i + 4 q + v of the expert, column n0 + 16 tt + r
    auto store = [&](int64_t rr, int col, float g, float u) {
      const int64_t b = blo + rr / Mx, mrow = rr % Mx;
      const int64_t xm = a.bm.lhs ? load_index(a.bm.lhs, a.bm.lhs_dt, b) : b;
      const bool ok = xm >= 0 && xm < a.bm.nx;
      const auto v = GLU ? swiglu_out<XT>(g, u) : from_f<XT>(g);
      out[(b * Mx + mrow) * N + col] = ok ? v : from_f<XT>(__builtin_nanf(""));
    };
    if constexpr (S == 1) {
#pragma unroll
      for (int tt = 0; tt < (GLU ? NT / 2 : NT); ++tt)
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int64_t rr = r0 + 16 * i + 4 * q + v;
            const int col = n0 + 16 * tt + r;
            if (rr < rows_total && col < N) store(rr, col, Y[tt][i][v], GLU ? Y[tt + NT / 2][i][v] : 0.f);
          }
    } else {
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int v = 0; v < 4; ++v) red[((wave * NT + tt) * 2 + i) * 256 + (4 * q + v) * 16 + r] = Y[tt][i][v];
      __syncthreads();
      for (int idx = t; idx < 16 * MT * NC; idx += 64 * S) {
        const int m = idx / NC, nn = idx % NC;
        const int i = m >> 4, mr = m & 15;
        const int64_t rr = r0 + m;
        if (rr >= rows_total || n0 + nn >= N) continue;
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int h = 0; h < (GLU ? 2 : 1); ++h) {
          const int tt = GLU ? h * (NT / 2) + (nn >> 4) : (nn >> 4);
#pragma unroll
          for (int w2 = 0; w2 < S; ++w2) acc[h] += red[((w2 * NT + tt) * 2 + i) * 256 + mr * 16 + (nn & 15)];
        }
        store(rr, n0 + nn, acc[0], acc[1]);
      }
      __syncthreads();
    }
  };
  for (int64_t r0 = 0; r0 < rows_total; r0 += 32) {
    if (rows_total - r0 > 16) pass(std::integral_constant<int, 2>{}, r0);
    else pass(std::integral_constant<int, 1>{}, r0);
  }
}

struct GatCfg {
  int nt, s, d, kb;
};

// grouped configurations (measured, 256 experts, top 8, q4 gs 64): K = 2048
// (gate / up) four waves of four blocks; K = 512 (down) two waves of two
GatCfg gather_choose(const QmmArgs& a) {
  const int P = a.K >> 7;
  if (P % 4 == 0 && P / 4 <= 8) return GatCfg{4, 4, 2, P / 4};
  if (P % 2 == 0 && P / 2 <= 8) return GatCfg{4, 2, 2, P / 2};
  return GatCfg{0, 0, 0, 0};
}

template <int XT, int GB, bool GLU>
hipError_t gather_dec_go(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  const GatCfg c = gather_choose(a);
  constexpr int NT = 4;
  constexpr int NC = GLU ? 8 * NT : 16 * NT;
  const dim3 grid(static_cast<unsigned>((a.N + NC - 1) / NC), static_cast<unsigned>(E + 1));
#define IQMM_GDEC(S_, D_, KB_)                                                                                     \
  if (c.s == S_ && c.d == D_ && c.kb == KB_) {                                                                     \
    hipLaunchKernelGGL((gather_decode_kernel<XT, NT, GB, S_, D_, KB_, GLU>), grid, dim3(64 * S_), 0, a.stream, a, \
                       nflat, off);                                                                                \
    return hipGetLastError();                                                                                      \
  }
  IQMM_GDEC(4, 2, 4)
  IQMM_GDEC(4, 2, 2)
  IQMM_GDEC(4, 2, 8)
  IQMM_GDEC(2, 2, 2)
  IQMM_GDEC(2, 2, 4)
  IQMM_GDEC(2, 2, 8)
  IQMM_GDEC(4, 2, 1)
  IQMM_GDEC(2, 2, 1)
#undef IQMM_GDEC
  return hipErrorInvalidValue;
}

template <int XT, bool GLU>
hipError_t gather_dec_gs(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  switch (a.gs) {
    case 32: return gather_dec_go<XT, 4, GLU>(a, nflat, E, off);
    case 64: return gather_dec_go<XT, 2, GLU>(a, nflat, E, off);
    default: return gather_dec_go<XT, 1, GLU>(a, nflat, E, off);
  }
}

}  // namespace

bool gather_decode_supported(const QmmArgs& a) {
  if (!(a.transpose && a.mode == AFFINE && a.bits == 4 && (a.xdt == BF16 || a.xdt == F16) && a.K % 128 == 0 &&
        a.N >= 1 && a.bm.rhs != nullptr))
    return false;
  if (a.gs != 32 && a.gs != 64 && a.gs != 128) return false;
  const GatCfg c = gather_choose(a);
  if (c.kb == 0) return false;
  if (a.gs == 128 && c.kb % 2 != 0) return false;
  return (reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 4 == 0 && ((a.K / a.gs) * 2) % 4 == 0;
}

hipError_t launch_gather_decode(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  if (a.glu) return a.xdt == BF16 ? gather_dec_gs<BF16, true>(a, nflat, E, off) : gather_dec_gs<F16, true>(a, nflat, E, off);
  return a.xdt == BF16 ? gather_dec_gs<BF16, false>(a, nflat, E, off) : gather_dec_gs<F16, false>(a, nflat, E, off);
}

}  // namespace iqmm
