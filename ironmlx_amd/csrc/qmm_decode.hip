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
// group for gs >= 32) and lane (r, q) its 8-code piece q; each lane reads one
// 16-byte weight chunk and a 4 x 4 dword transpose across the lanes q
// (v_permlane32_swap, then v_permlane16_swap) hands it out.
//
// A workgroup owns NT 16-row tiles (NC = 16 NT output columns) and its S waves
// split K into ranges of KB blocks (a template argument: the K loop is fully
// unrolled).  Each wave streams its range in stages of two blocks through a
// ring of D stages in its own slice of LDS, filled by LDS DMA
// (global_load_lds_dwordx4): weights as 8 rows x 128 B per instruction (whole
// cache lines; 16 rows x 64 B straight into the MFMA layout measured 30%
// slower on the read alone) and, with XL, x as 2 rows x 512 B, each row's
// 16-byte pieces XOR-swizzled by the row so the MFMA-layout ds_read_b128 are
// conflict-free.  Without XL, x fragments are loaded straight into registers
// (16 rows x 64 B; cheaper where four tiles share each fragment).  Every
// global load of the K loop is inline assembly with explicit vmcnt waits
// (straight-line code, so each wait is exact).  Scale / bias words of the
// wave's K range are read once per tile.  Rows past M read the last x row and
// produce output rows that are never stored.  GLU: the weight holds 2N rows
// (gate [0, N), up [N, 2N)); tiles [0, NT/2) take gate rows and [NT/2, NT) the
// matching up rows, and the epilogue writes silu(gate) * up (NC = 8 NT).
//
// Measured (bf16, gs 64, rotating weight pool): K = 4096, N = 14336, M = 4 / 16
// / 32: 11.2 / 12.4 / 17.3 us; N = 4096, K = 14336, M = 4 / 16 / 32: 11.6 /
// 14.0 / 20.5 us (the round-1 kernel: 17.9 / 20.2 / 23.5 and 21.4 / 27.7 /
// 39.8 us).
#include <type_traits>

#include "launch.h"
#include "mfma_common.h"
#include "decode_common.h"

namespace iqmm {
namespace {

template <int NT, int MT, int S, int D, bool XL, int KB>
constexpr int dec_lds_bytes() {
  constexpr int ring = D < KB / 2 ? D : KB / 2;  // stages allocated
  constexpr int wave = ring * (NT * 2048 + (XL ? MT * 8192 : 0));
  constexpr int red = S > 1 ? S * NT * MT * 1024 : 0;
  return S * wave > red ? S * wave : red;
}

// a configuration fits: LDS within 160 KiB, the loads of the stages in flight
// behind the oldest within vmcnt's 6 bits
template <int NT, int MT, int S, int D, bool XL, int KB>
constexpr bool dec_fits() {
  constexpr int per = 2 * NT + 8 * MT;
  return dec_lds_bytes<NT, MT, S, D, XL, KB>() <= 160 * 1024 && D <= 3 && (D - 1) * per < 64;
}

template <int XT, int NT, int MT, int GB, int S, int D, int KB, bool XL, bool GLU, bool MAPPED>
__global__ __launch_bounds__(64 * S) void qmm_decode_kernel(QmmArgs a) {
  static_assert(!GLU || NT % 2 == 0, "GLU pairs gate tiles with up tiles");
  static_assert(KB % 2 == 0, "stages of two blocks");
  constexpr int NC = GLU ? 8 * NT : 16 * NT;  // output columns per workgroup
  using XS = uint16_t;
  constexpr int SW = (KB * GB + 1) / 2; // 32-bit scale words of the wave's K range
  constexpr int NS = KB / 2;            // stages per wave
  constexpr int WSTAGE = NT * 16 * 128; // weight bytes per stage
  constexpr int XSTAGE = XL ? MT * 16 * 512 : 0;
  constexpr int SSTAGE = WSTAGE + XSTAGE;
  constexpr int WAVE_LDS = (D < NS ? D : NS) * SSTAGE;
  constexpr int LDS = dec_lds_bytes<NT, MT, S, D, XL, KB>();
  static_assert(LDS <= 160 * 1024, "LDS budget");
  constexpr int NDW = 2 * NT;            // weight DMA instructions per stage (8 rows x 128 B)
  constexpr int NDX = XL ? 8 * MT : 0;   // x DMA instructions per stage (2 rows x 512 B)
  constexpr int NRX = XL ? 0 : 8 * MT;   // x register loads per stage (16 rows x 64 B)
  constexpr int PER = NDW + NDX + NRX;   // vector-memory instructions per stage
  __shared__ __attribute__((aligned(1024))) char lds[LDS];
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
  const char* w = reinterpret_cast<const char*>(a.w + wb * a.w_mat);
  const char* sp = reinterpret_cast<const char*>(static_cast<const XS*>(a.s) + wb * a.s_mat);
  const char* bp = reinterpret_cast<const char*>(static_cast<const XS*>(a.b) + wb * a.s_mat);
  auto wrow_of = [&](int row) {  // tile row (0 .. 16 NT - 1) -> weight row
    const int tt = row >> 4, rr = row & 15;
    return GLU ? static_cast<int64_t>(tt / (NT / 2)) * N + min(n0 + 16 * (tt % (NT / 2)) + rr, N - 1)
               : static_cast<int64_t>(min(n0 + row, N - 1));
  };
  // weight DMA u: tile rows 8u .. 8u + 7, lane -> row 8u + lane / 8, 16-byte
  // position lane % 8 holding piece (lane % 8) ^ (row & 7) of the stage's 128 B
  const char* wsrc[NDW];
#pragma unroll
  for (int u = 0; u < NDW; ++u) {
    const int row = 8 * u + (lane >> 3);
    wsrc[u] = w + wrow_of(row) * wrow + pb * 64 + 16 * ((lane & 7) ^ (row & 7));
  }
  // x DMA u (XL): rows 2u, 2u + 1, position lane % 32 holding piece
  // (lane % 32) ^ (row & 15) of the row's 512-byte stage segment
  const char* xsrc[XL ? NDX : 1];
  const char* xr[XL ? 1 : MT];
  if constexpr (XL) {
#pragma unroll
    for (int u = 0; u < NDX; ++u) {
      const int row = 2 * u + (lane >> 5);
      xsrc[u] = xbase + min(row, M - 1) * xrow + pb * 256 + 16 * ((lane & 31) ^ (row & 15));
    }
  } else {
#pragma unroll
    for (int i = 0; i < MT; ++i) xr[i] = xbase + min(i * 16 + r, M - 1) * xrow + pb * 256 + 16 * q;
  }
  uint32_t sw[NT][SW], bw[NT][SW];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int64_t n = wrow_of(16 * tt + r);
    // the scale halves of [pb, pb + KB) start at half pb * GB (even: KB is even)
    const char* s0 = sp + n * srow + pb * GB * 2;
    const char* b0 = bp + n * srow + pb * GB * 2;
#pragma unroll
    for (int h = 0; h < SW; ++h) {
      sw[tt][h] = *reinterpret_cast<const uint32_t*>(s0 + 4 * h);
      bw[tt][h] = *reinterpret_cast<const uint32_t*>(b0 + 4 * h);
    }
  }
  // the compiler sees this wait: nothing of its own is outstanding in the K loop
  __builtin_amdgcn_s_waitcnt(0);
  const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds_u32(lds)) + wave * WAVE_LDS;
  const char* lds_w = lds + wave * WAVE_LDS;
  g_u32x4_t xreg[XL ? 1 : D][2][MT][4];
  auto issue = [&](int st, int slot) {  // stage st (blocks 2 st, 2 st + 1) into ring slot
#pragma unroll
    for (int u = 0; u < NDW; ++u) dma16(wsrc[u] + st * 128, lds_wave + slot * SSTAGE + u * 1024);
    if constexpr (XL) {
#pragma unroll
      for (int u = 0; u < NDX; ++u) dma16(xsrc[u] + st * 512, lds_wave + slot * SSTAGE + WSTAGE + u * 1024);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) xreg[slot][h][i][j] = gload16(xr[i] + (2 * st + h) * 256 + 64 * j);
    }
  };
  f32x4d_t Y[NT][MT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int i = 0; i < MT; ++i) Y[tt][i] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int slot, int h, int b) {  // block b (half h of the stage in `slot`)
    g_u32x4_t A[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (XL) {
          const int m = 16 * i + r, p = 16 * h + 4 * j + q;  // 16-byte piece of the row's stage segment
          A[i][j] = x_pairs(
              *reinterpret_cast<const g_u32x4_t*>(lds_w + slot * SSTAGE + WSTAGE + m * 512 + 16 * (p ^ (m & 15))));
        } else {
          A[i][j] = x_pairs(xreg[slot][h][i][j]);
        }
      }
    fac_block<XT, NT, MT, GB, SW>(Y, A, lds_w + slot * SSTAGE, h, b * GB, sw, bw, r, q);
  };
#pragma unroll
  for (int st = 0; st < D && st < NS; ++st) issue(st, st);
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int slot = st % D;
    // stage st complete; the later stages issued so far (PER instructions
    // each) may stay in flight
    const int later = st + D <= NS ? D - 1 : NS - 1 - st;
    static_assert(D <= 3 && (D - 1) * PER < 64, "vmcnt holds at most 63 outstanding loads");
    if (later == 2) vm_wait<(D >= 3 ? 2 * PER : 0)>();
    else if (later == 1) vm_wait<PER>();
    else vm_wait<0>();
    if constexpr (!XL) {
      // the stage's x registers are written by the loads the wait covered
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(xreg[slot][h][i][j])::"memory");
    }
    compute(slot, 0, 2 * st);
    compute(slot, 1, 2 * st + 1);
    if (st + D < NS) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's LDS reads are done
      issue(st + D, slot);
    }
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
  __syncthreads();  // every wave's ring reads are done before the partials overwrite LDS
  float* red = reinterpret_cast<float*>(lds);
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
      for (int hh = 0; hh < 2; ++hh) {
        const int tt = hh * (NT / 2) + (nn >> 4);
#pragma unroll
        for (int w2 = 0; w2 < S; ++w2) acc[hh] += red[((w2 * NT + tt) * MT + i) * 256 + mr * 16 + (nn & 15)];
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

// One configuration: NT tiles per workgroup, S waves, D stages in flight, KB
// blocks per wave (K = 128 KB S), XL: x through the LDS ring.
struct DecCfg {
  int nt, s, d, kb;
  bool xl;
};

// Choice per shape, measured on MI355X (bf16, gs 64, M in {4, 8, 16, 32},
// rotating weight pool): K = 4096 with >= 8192 rows: four tiles, eight waves,
// x in registers (four tiles share each x fragment); 6144 rows: two tiles, x
// in registers up to M = 8, through LDS above; narrower matrices and K = 14336:
// one tile, four waves, x through LDS (down projection M = 16: 19.2 -> 14.0 us).
DecCfg choose(const QmmArgs& a, int64_t rows) {
  const int P = a.K >> 7;
  const bool two_mt = a.M > 16;
  DecCfg c{0, 0, 0, 0, false};
  if (P == 32 && rows >= 8192) c = DecCfg{4, 8, 2, 4, false};
  else if (P == 32 && rows >= 6144) c = a.M <= 8 ? DecCfg{2, 8, 2, 4, false} : DecCfg{2, 4, 2, 8, true};
  else if (P == 8 || P == 16 || P == 32 || P == 64 || P == 112) c = DecCfg{1, 4, two_mt ? 2 : 3, P / 4, true};
  // gs 32 at two m tiles: four tiles' scale words do not fit in registers
  // next to the x ring
  if (a.gs == 32 && two_mt && c.nt == 4 && !c.xl) c.nt = 2;
  if (a.glu && c.nt == 1) {
    c.nt = 2;
    c.d = 2;  // two tiles of x + weights in the LDS budget
  }
  return c;
}

template <int XT, int NT, int MT, int GB, int S, int D, int KB, bool XL, bool GLU>
hipError_t dec_go(const QmmArgs& a, dim3 grid) {
  if constexpr ((GLU && NT % 2 != 0) || !dec_fits<NT, MT, S, D, XL, KB>() || (!XL && GB == 4 && NT == 4 && MT == 2)) {
    return hipErrorInvalidValue;  // not produced by choose()
  } else {
    const bool mapped = a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr;
    if (mapped)
      hipLaunchKernelGGL((qmm_decode_kernel<XT, NT, MT, GB, S, D, KB, XL, GLU, true>), grid, dim3(64 * S), 0,
                         a.stream, a);
    else
      hipLaunchKernelGGL((qmm_decode_kernel<XT, NT, MT, GB, S, D, KB, XL, GLU, false>), grid, dim3(64 * S), 0,
                         a.stream, a);
    return hipGetLastError();
  }
}

// the configurations choose() produces
#define IQMM_DEC_CONFIGS(X)                                                                           \
  X(4, 8, 2, 4, false) X(2, 8, 2, 4, false) X(2, 4, 2, 8, true) X(1, 4, 3, 2, true) X(1, 4, 2, 2, true) \
  X(1, 4, 3, 4, true) X(1, 4, 2, 4, true) X(1, 4, 3, 8, true) X(1, 4, 2, 8, true) X(1, 4, 3, 16, true) \
  X(1, 4, 2, 16, true) X(1, 4, 3, 28, true) X(1, 4, 2, 28, true) X(2, 4, 2, 2, true)                  \
  X(2, 4, 2, 4, true) X(2, 4, 2, 16, true) X(2, 4, 2, 28, true)

template <int XT, int MT, int GB, bool GLU>
hipError_t dec_cfg(const QmmArgs& a, const DecCfg& c, dim3 grid) {
#define IQMM_DEC(NT_, S_, D_, KB_, XL_)                                              \
  if (c.nt == NT_ && c.s == S_ && c.d == D_ && c.kb == KB_ && c.xl == XL_)          \
    return dec_go<XT, NT_, MT, GB, S_, D_, KB_, XL_, GLU>(a, grid);
  IQMM_DEC_CONFIGS(IQMM_DEC)
#undef IQMM_DEC
  return hipErrorInvalidValue;
}

bool cfg_instantiated(const DecCfg& c, int mt) {
  bool ok = false;
#define IQMM_DEC_K(NT_, S_, D_, KB_, XL_)                                                              \
  ok = ok || (c.nt == NT_ && c.s == S_ && c.d == D_ && c.kb == KB_ && c.xl == XL_ &&                    \
              (mt == 1 ? dec_fits<NT_, 1, S_, D_, XL_, KB_>() : dec_fits<NT_, 2, S_, D_, XL_, KB_>()));
  IQMM_DEC_CONFIGS(IQMM_DEC_K)
#undef IQMM_DEC_K
  return ok;
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
  if (c.kb == 0 || c.kb * c.s * 128 != a.K || !cfg_instantiated(c, a.M > 16 ? 2 : 1)) return false;
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
