// qmm_skinny.hip — decode-width quantized matmul (transpose=true, 2 <= M <= 64)
// on CDNA4 matrix cores.
//
// The batched-decode widths (M in {4, 8, 16, 32} for continuous batching) are
// still HBM-bound on the weights, but far too much arithmetic for the
// vector-ALU GEMV.  A workgroup owns 32 weight rows; its S waves split K.
// Per 64-code block p, lane l = (n = l % 32, h = l / 32) streams the 16-byte
// chunk 2p + h of row n (one coalesced 32-byte run per row per wave), reads
// that chunk's scale/bias, dequantizes the 32 codes in registers (the
// `dequantize` arithmetic, so every group size and mode works) and feeds
// them as the B operand of four v_mfma_f32_32x32x16 (code 8j..8j+7 to MFMA
// j).  The A operand is x rows m = l % 32 (16-byte loads of the matching k
// positions; rows >= M read as zero).  Each wave leaves a 32 x 32 fp32
// partial; the S partials are summed through LDS and rows < M are stored.
// Reference op: mlx/src/ops.rs:695-727 with x = [B, 1, K] (one decode step
// for B sequences, which mlx/src/generate/batch.rs:313-339 runs as B
// separate M = 1 calls today).
#include <type_traits>

#include "launch.h"
#include "mfma_common.h"

namespace iqmm {

constexpr int SK_ROWS = 32;

template <int XT, int MODE, int BITS, int S, int U>
__global__ __launch_bounds__(64 * S) void qmm_skinny_kernel(QmmArgs a, int nmt) {
  using XS = uint16_t;
  constexpr bool AFF = MODE == AFFINE;
  __shared__ float red[S * 32 * 33];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int M = a.M, N = a.N, K = a.K;
  const int n0 = blockIdx.x * SK_ROWS;
  const int mt = blockIdx.y % nmt;
  const int64_t bb = blockIdx.y / nmt;
  const int m0 = mt * 32;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;

  int64_t xb = 0, wb = 0;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      for (int i = t; i < 32 * SK_ROWS; i += 64 * S) {
        const int r = m0 + i / SK_ROWS, c = n0 + i % SK_ROWS;
        if (r < M && c < N) out[static_cast<int64_t>(r) * N + c] = from_f<XT>(__builtin_nanf(""));
      }
      return;
    }
  }
  const XS* x = static_cast<const XS*>(a.x) + xb * a.x_mat;
  const uint32_t* w = a.w + wb * a.w_mat;
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const int G = K / gs;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = AFF ? static_cast<const XS*>(a.b) + wb * a.s_mat : nullptr;
  const uint8_t* s8 = static_cast<const uint8_t*>(a.s) + wb * a.s_mat;
  const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;

  const int nl = lane & 31, h = lane >> 5;
  const int row = min(n0 + nl, N - 1);
  const uint32_t* wrow = w + static_cast<int64_t>(row) * wpr;
  const int xm = m0 + nl;                      // this lane's x row (A operand)
  const bool xvalid = xm < M;
  const XS* xrow = x + static_cast<int64_t>(xvalid ? xm : 0) * K;

  // K blocks of 64 codes split evenly over the S waves
  const int P = K >> 6;
  const int pb = (P * wave) / S, pe = (P * (wave + 1)) / S;

  f32x16_t acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.f;

  // U blocks per batch: all loads of the batch are issued before any
  // dequantization, so U x (16 B of W + 64 B of x) per lane are in flight
  struct Blk {
    uint32_t wd[BITS];
    float s, b, s2;
    g_u32x4_t xa[4];
  };
  auto load = [&](int p, Blk& B) {
    const int c = 2 * min(p, pe - 1) + h;
    load_chunk<BITS>(B.wd, wrow + c * BITS);
    const int gi = (c * 32) / gs;
    if constexpr (AFF) {
      B.s = to_f<XT>(sp[static_cast<int64_t>(row) * G + gi]);
      B.b = to_f<XT>(bp[static_cast<int64_t>(row) * G + gi]);
      B.s2 = B.s;
    } else {
      B.s = fp_scale<MODE>(s8[static_cast<int64_t>(row) * G + gi]);
      B.b = 0.f;
      B.s2 = MODE == NVFP4 ? fp_scale<MODE>(s8[static_cast<int64_t>(row) * G + gi + 1]) : B.s;
    }
    const g_u32x4_t* xp = reinterpret_cast<const g_u32x4_t*>(xrow + c * 32);
    const bool live = xvalid && p < pe;
#pragma unroll
    for (int j = 0; j < 4; ++j) B.xa[j] = live ? xp[j] : g_u32x4_t{0, 0, 0, 0};
  };
  auto compute = [&](const Blk& B) {
    uint32_t o[16];
    dequant32<XT, MODE, BITS>(B.wd, B.s, B.b, B.s2, o);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = mfma32<XT>(B.xa[j], g_u32x4_t{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]}, acc);
  };
  for (int p = pb; p < pe; p += U) {
    Blk B[U];
#pragma unroll
    for (int u = 0; u < U; ++u) load(p + u, B[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) compute(B[u]);   // blocks past pe carry x = 0
  }

  // lane holds C[m = 8(v/4) + 4h + v%4][n = nl]
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int m = 8 * (v >> 2) + 4 * h + (v & 3);
    red[(wave * 32 + m) * 33 + nl] = acc[v];
  }
  __syncthreads();
  for (int i = t; i < 32 * SK_ROWS; i += 64 * S) {
    const int m = i / SK_ROWS, n = i % SK_ROWS;
    float v = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < S; ++w2) v += red[(w2 * 32 + m) * 33 + n];
    if (m0 + m < M && n0 + n < N) out[static_cast<int64_t>(m0 + m) * N + n0 + n] = from_f<XT>(v);
  }
}

// ---------------------------------------------------------------------------
// 16x16x32 variant: lane l = (n = l % 16, q = l / 16) streams chunk 4p + q of
// row n, so each wave instruction reads 16 rows x 64 contiguous bytes (the
// 32x32 layout's 32-byte runs leave half-used 128-byte lines behind).  The 32
// codes are dequantized in registers and feed four v_mfma_f32_16x16x32 per
// 16-row x-tile (word j -> MFMA j; x positions 128p + 32q + 8j .. +8).
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

template <int XT>
__device__ __forceinline__ f32x4_t mfma16x(const g_u32x4_t& a, const g_u32x4_t& b, const f32x4_t& c) {
  if constexpr (XT == BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, a),
                                                   __builtin_bit_cast(g_bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(g_f16x8_t, a),
                                                  __builtin_bit_cast(g_f16x8_t, b), c, 0, 0, 0);
}

// affine 4-bit chunk -> 16 packed pairs in natural order
template <int XT>
__device__ __forceinline__ void deq4_fast(const g_u32x4_t& wv, float s, float b, uint32_t (&o)[16]) {
  const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t lo = wd[q] & 0x0F0F0F0Fu, hi = (wd[q] >> 4) & 0x0F0F0F0Fu;
    o[4 * q + 0] = pack2<XT>(fmaf(s, ubyte_f<0>(lo), b), fmaf(s, ubyte_f<0>(hi), b));
    o[4 * q + 1] = pack2<XT>(fmaf(s, ubyte_f<1>(lo), b), fmaf(s, ubyte_f<1>(hi), b));
    o[4 * q + 2] = pack2<XT>(fmaf(s, ubyte_f<2>(lo), b), fmaf(s, ubyte_f<2>(hi), b));
    o[4 * q + 3] = pack2<XT>(fmaf(s, ubyte_f<3>(lo), b), fmaf(s, ubyte_f<3>(hi), b));
  }
}

// GBT > 0 (affine 4-bit, GBT = 128 / gs): chunk-major k slots -- MFMA j of a
// block takes chunk 4p + j, lane (n, q) its 8-code piece q, so x loads are 64
// contiguous bytes per row; the weight dwords are transposed across the lanes
// q and dword j is dequantized with chunk 4p + j's scale and bias.
template <int XT, int MODE, int BITS, int S, int MT, int U, int GBT = 0>
__global__ __launch_bounds__(64 * S) void qmm_skinny16_kernel(QmmArgs a, int nmt) {
  using XS = uint16_t;
  constexpr bool AFF = MODE == AFFINE;
  constexpr bool TRX = GBT > 0;
  static_assert(!TRX || (AFF && BITS == 4), "chunk-major slots: affine 4-bit");
  using SG = typename std::conditional<GBT == 4, uint64_t, typename std::conditional<GBT == 2, uint32_t, XS>::type>::type;
  __shared__ float red[S * 32 * 17];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int M = a.M, N = a.N, K = a.K;
  const int n0 = blockIdx.x * 16;
  const int mt = blockIdx.y % nmt;
  const int64_t bb = blockIdx.y / nmt;
  const int m0 = mt * 32;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;
  int64_t xb = 0, wb = 0;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      for (int i = t; i < 32 * 16; i += 64 * S) {
        const int r = m0 + i / 16, c = n0 + i % 16;
        if (r < M && c < N) out[static_cast<int64_t>(r) * N + c] = from_f<XT>(__builtin_nanf(""));
      }
      return;
    }
  }
  const XS* x = static_cast<const XS*>(a.x) + xb * a.x_mat;
  const uint32_t* w = a.w + wb * a.w_mat;
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const int G = K / gs;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = AFF ? static_cast<const XS*>(a.b) + wb * a.s_mat : nullptr;
  const uint8_t* s8 = static_cast<const uint8_t*>(a.s) + wb * a.s_mat;
  const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
  const int nl = lane & 15, q = lane >> 4;
  const int row = min(n0 + nl, N - 1);
  const uint32_t* wrow = w + static_cast<int64_t>(row) * wpr;
  // x rows for the MT 16-row tiles: lane feeds row m0 + 16 i + nl
  const XS* xrows[MT];
  bool xv[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int xm = m0 + 16 * i + nl;
    xv[i] = xm < M;
    xrows[i] = x + static_cast<int64_t>(xv[i] ? xm : 0) * K;
  }
  const int P = K >> 7;   // 128-code blocks
  const int pb = (P * wave) / S, pe = (P * (wave + 1)) / S;
  f32x4_t acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  struct Blk {
    uint32_t wd[BITS];
    float s, b, s2;
    SG sg, bg;
    g_u32x4_t xa[MT][4];
  };
  auto load = [&](int p, Blk& B) {
    const int pc = min(p, pe - 1);
    const int c = 4 * pc + q;
    load_chunk<BITS>(B.wd, wrow + c * BITS);
    const int gi = (c * 32) / gs;
    if constexpr (TRX) {
      const int64_t g0 = static_cast<int64_t>(row) * G + pc * GBT;
      B.sg = *reinterpret_cast<const SG*>(sp + g0);
      B.bg = *reinterpret_cast<const SG*>(bp + g0);
      B.s = B.b = B.s2 = 0.f;
    } else if constexpr (AFF) {
      B.s = to_f<XT>(sp[static_cast<int64_t>(row) * G + gi]);
      B.b = to_f<XT>(bp[static_cast<int64_t>(row) * G + gi]);
      B.s2 = B.s;
    } else {
      B.s = fp_scale<MODE>(s8[static_cast<int64_t>(row) * G + gi]);
      B.b = 0.f;
      B.s2 = MODE == NVFP4 ? fp_scale<MODE>(s8[static_cast<int64_t>(row) * G + gi + 1]) : B.s;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const bool live = xv[i] && p < pe;
      if constexpr (TRX) {
        const XS* xg = xrows[i] + 4 * pc * 32 + 8 * q;   // piece q of chunks 4 pc + j
#pragma unroll
        for (int j = 0; j < 4; ++j)
          B.xa[i][j] = live ? *reinterpret_cast<const g_u32x4_t*>(xg + 32 * j) : g_u32x4_t{0, 0, 0, 0};
      } else {
        const g_u32x4_t* xp = reinterpret_cast<const g_u32x4_t*>(xrows[i] + c * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) B.xa[i][j] = live ? xp[j] : g_u32x4_t{0, 0, 0, 0};
      }
    }
  };
  auto compute = [&](const Blk& B) {
    uint32_t o[16];
    if constexpr (TRX) {
      // 4 x 4 dword transpose over the lanes q: dword j <- dword q of chunk 4p + j
      auto s02 = __builtin_amdgcn_permlane32_swap(B.wd[0], B.wd[2], false, false);
      auto s13 = __builtin_amdgcn_permlane32_swap(B.wd[1], B.wd[3], false, false);
      auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
      auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
      const uint32_t wt[4] = {s01[0], s01[1], s23[0], s23[1]};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int sh = 16 * ((j * GBT) >> 2);
        const float s = to_f<XT>(static_cast<XS>(B.sg >> sh));
        const float b = to_f<XT>(static_cast<XS>(B.bg >> sh));
        const uint32_t lo = wt[j] & 0x0F0F0F0Fu, hi = (wt[j] >> 4) & 0x0F0F0F0Fu;
        o[4 * j + 0] = pack2<XT>(fmaf(s, ubyte_f<0>(lo), b), fmaf(s, ubyte_f<0>(hi), b));
        o[4 * j + 1] = pack2<XT>(fmaf(s, ubyte_f<1>(lo), b), fmaf(s, ubyte_f<1>(hi), b));
        o[4 * j + 2] = pack2<XT>(fmaf(s, ubyte_f<2>(lo), b), fmaf(s, ubyte_f<2>(hi), b));
        o[4 * j + 3] = pack2<XT>(fmaf(s, ubyte_f<3>(lo), b), fmaf(s, ubyte_f<3>(hi), b));
      }
    } else if constexpr (AFF && BITS == 4)
      deq4_fast<XT>(g_u32x4_t{B.wd[0], B.wd[1], B.wd[2], B.wd[3]}, B.s, B.b, o);
    else
      dequant32<XT, MODE, BITS>(B.wd, B.s, B.b, B.s2, o);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const g_u32x4_t wb4 = {o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]};
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[i] = mfma16x<XT>(B.xa[i][j], wb4, acc[i]);
    }
  };
  for (int p = pb; p < pe; p += U) {
    Blk B[U];
#pragma unroll
    for (int u = 0; u < U; ++u) load(p + u, B[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) compute(B[u]);   // blocks past pe carry x = 0
  }
  // lane holds C[4 q + r][nl] of each 16 x 16 tile i
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * 32 + 16 * i + 4 * q + r) * 17 + nl] = acc[i][r];
  __syncthreads();
  for (int i = t; i < 16 * MT * 16; i += 64 * S) {
    const int m = i / 16, n = i % 16;
    float v = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < S; ++w2) v += red[(w2 * 32 + m) * 17 + n];
    if (m0 + m < M && n0 + n < N) out[static_cast<int64_t>(m0 + m) * N + n0 + n] = from_f<XT>(v);
  }
}

// ---------------------------------------------------------------------------
// Factored affine 4-bit kernel for decode widths (transpose, K % 128 == 0).
// The weights enter the MFMA undequantized: v_perm_b32 turns each nibble n
// into the 16-bit value C + n (C = 128 bf16 / 1024 fp16, unit spacing) in the
// pair order (n0,n4) (n2,n6) (n1,n5) (n3,n7), and x is permuted the same way.
// With D = sum x (C + q) and X = sum x over one quantization group,
//   sum x (s q + b) = s D + (b - C s) X,
// so per 128-code block a lane spends 7 VALU per 8 codes on unpacking and two
// FMAs per accumulator on the group scale, instead of a full dequantization.
// Every MFMA's sum must stay inside one group.  Without TR (used at gs 128,
// one group per block) lane q's k slot is chunk 4p + q, and for GB = 128 / gs
// groups per block the 16 A rows would be (x row, group-in-block) pairs with
// RPT = 16 / GB x rows per m tile, the rows of the other group zero in each
// k slot.  TR (gs 32 / 64) avoids those zero rows.  X comes from the same MFMA with
// an all-ones B.  A wave covers NT 16-row weight tiles (x pairs and X are
// shared by them) for the blocks [pb, pe) of K; the S waves of a workgroup
// split K and their partial sums meet in LDS.
// GLU (NT even): the weight holds 2N rows (gate [0, N), up [N, 2N)); tiles
// [0, NT/2) of a workgroup are gate rows n0.. and tiles [NT/2, NT) the
// matching up rows, and the epilogue writes silu(gate) * up for 8 NT columns.
//
// TR (chunk-major k slots): MFMA j of a block takes chunk 4p + j (32 codes,
// one quantization group for gs >= 32) and lane (r, q) supplies its 8-code
// piece q.  Every A row is then a live x row (RPT = 16), and the x pieces of
// one load are 64 contiguous bytes per row.  The weights still arrive as one
// 16-byte chunk per lane (lane q: chunk 4p + q) and a 4 x 4 dword transpose
// across the lanes q (v_permlane32_swap, then v_permlane16_swap) turns them
// into piece q of chunks 4p + 0..3.  The group scale then applies per MFMA
// group: Y += s_g D_g + (b_g - C s_g) X_g.
template <int XT, int NT, int MT, int GB, int S, int NB = 2, bool GLU = false, bool TR = false>
__global__ __launch_bounds__(64 * S) void qmm_skinny_fac_kernel(QmmArgs a) {
  static_assert(!GLU || NT % 2 == 0, "GLU pairs gate tiles with up tiles");
  constexpr int NC = GLU ? 8 * NT : 16 * NT;  // output columns per workgroup
  using XS = uint16_t;
  constexpr int RPT = TR ? 16 : 16 / GB;
  constexpr int GR = TR ? 1 : GB;  // groups summed in the epilogue
  constexpr float CM = XT == BF16 ? 128.f : 1024.f;
  constexpr uint32_t EB = XT == BF16 ? 0x43434343u : 0x64646464u;
  constexpr uint32_t ONE2 = XT == BF16 ? 0x3f803f80u : 0x3c003c00u;
  __shared__ float red[S * NT * MT * 256];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int M = a.M, N = a.N, K = a.K;
  const int n0 = blockIdx.x * NC;
  const int64_t bb = blockIdx.y;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;
  int64_t xb = 0, wb = 0;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      for (int i = t; i < M * NC; i += 64 * S) {
        const int m = i / NC, n = n0 + i % NC;
        if (n < N) out[static_cast<int64_t>(m) * N + n] = from_f<XT>(__builtin_nanf(""));
      }
      return;
    }
  }
  const char* x = reinterpret_cast<const char*>(static_cast<const XS*>(a.x) + xb * a.x_mat);
  const char* w = reinterpret_cast<const char*>(a.w + wb * a.w_mat);
  const char* sp = reinterpret_cast<const char*>(static_cast<const XS*>(a.s) + wb * a.s_mat);
  const char* bp = reinterpret_cast<const char*>(static_cast<const XS*>(a.b) + wb * a.s_mat);
  const int gshift = __builtin_ctz(a.gs);
  const int64_t wrow = K / 2, srow = (K >> gshift) * 2, xrow = static_cast<int64_t>(K) * 2;
  const int r = lane & 15, q = lane >> 4;
  const int gq = (q * GB) >> 2;   // group (within the block) of this lane's k slot
  // A rows: m tile i, row r -> x row i RPT + r % RPT, group r / RPT
  const char* xr[MT];
  bool xlive[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int m = i * RPT + r % RPT;
    xlive[i] = TR ? m < M : (r / RPT == gq) && m < M;
    xr[i] = x + (xlive[i] ? m : 0) * xrow;
  }
  const char* wr[NT];
  const char* sr[NT];
  const char* br[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int64_t n = GLU ? static_cast<int64_t>(tt / (NT / 2)) * N + min(n0 + 16 * (tt % (NT / 2)) + r, N - 1)
                          : min(n0 + 16 * tt + r, N - 1);
    wr[tt] = w + n * wrow;
    sr[tt] = sp + n * srow;
    br[tt] = bp + n * srow;
  }
  const int P = K >> 7;
  const int pb = (P * wave) / S, pe = (P * (wave + 1)) / S;

  // TR: the GB group scales / biases of a block, one load each
  using SG = typename std::conditional<!TR || GB == 1, XS, typename std::conditional<GB == 2, uint32_t, uint64_t>::type>::type;
  struct Blk {
    g_u32x4_t xa[MT][4];
    g_u32x4_t wv[NT];
    SG sv[NT], bv[NT];
  };
  auto load = [&](int p, Blk& B) {
    const int pc = min(p, pe - 1);
    const int c = 4 * pc + q;   // chunk of this lane's weight load (and, without TR, its k slot)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        B.xa[i][j] = TR ? *reinterpret_cast<const g_u32x4_t*>(xr[i] + (4 * pc + j) * 64 + 16 * q)
                        : *reinterpret_cast<const g_u32x4_t*>(xr[i] + c * 64 + 16 * j);
    const int go = TR ? ((pc * 128) >> gshift) * 2 : ((c * 32) >> gshift) * 2;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      B.wv[tt] = __builtin_nontemporal_load(reinterpret_cast<const g_u32x4_t*>(wr[tt] + c * 16));
      B.sv[tt] = *reinterpret_cast<const SG*>(sr[tt] + go);
      B.bv[tt] = *reinterpret_cast<const SG*>(br[tt] + go);
    }
  };
  f32x4_t Y[NT][MT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int i = 0; i < MT; ++i) Y[tt][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const g_u32x4_t ones = {ONE2, ONE2, ONE2, ONE2};
  auto compute = [&](const Blk& B) {
    g_u32x4_t A[MT][4];
    f32x4_t X[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // (x0,x1) (x2,x3) (x4,x5) (x6,x7); rows of the other group (or past M)
        // are zeroed here rather than by a predicated load, which would split
        // the load stream into branches and serialize the waits
        const g_u32x4_t v = xlive[i] ? B.xa[i][j] : g_u32x4_t{0, 0, 0, 0};
        A[i][j] = g_u32x4_t{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                            __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
      }
      if constexpr (!TR) {
        X[i] = mfma16x<XT>(A[i][0], ones, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int j = 1; j < 4; ++j) X[i] = mfma16x<XT>(A[i][j], ones, X[i]);
      }
    }
    constexpr int JG = 4 / GB;  // TR: MFMAs per group
    f32x4_t XG[TR ? MT : 1][TR ? GB : 1];
    if constexpr (TR) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          XG[i][g] = mfma16x<XT>(A[i][g * JG], ones, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int j = 1; j < JG; ++j) XG[i][g] = mfma16x<XT>(A[i][g * JG + j], ones, XG[i][g]);
        }
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      uint32_t wd[4] = {B.wv[tt].x, B.wv[tt].y, B.wv[tt].z, B.wv[tt].w};
      if constexpr (TR) {
        // 4 x 4 transpose over the lanes q = lane / 16: afterwards wd[j] of
        // lane q is dword q of the chunk that lane j loaded (chunk 4p + j)
        auto s02 = __builtin_amdgcn_permlane32_swap(wd[0], wd[2], false, false);
        auto s13 = __builtin_amdgcn_permlane32_swap(wd[1], wd[3], false, false);
        auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
        auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
        wd[0] = s01[0]; wd[1] = s01[1]; wd[2] = s23[0]; wd[3] = s23[1];
      }
      g_u32x4_t Wp[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = wd[j] & 0x0F0F0F0Fu, hi = (wd[j] >> 4) & 0x0F0F0F0Fu;
        // pair order (n0,n4) (n1,n5) (n2,n6) (n3,n7), matching A above
        Wp[j] = g_u32x4_t{__builtin_amdgcn_perm(EB, lo, 0x04020400u), __builtin_amdgcn_perm(EB, hi, 0x04020400u),
                          __builtin_amdgcn_perm(EB, lo, 0x04030401u), __builtin_amdgcn_perm(EB, hi, 0x04030401u)};
      }
      if constexpr (TR) {
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          const float s = to_f<XT>(static_cast<XS>(B.sv[tt] >> (16 * g)));
          const float b = to_f<XT>(static_cast<XS>(B.bv[tt] >> (16 * g)));
          const float cb = fmaf(-CM, s, b);
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            f32x4_t D = mfma16x<XT>(A[i][g * JG], Wp[g * JG], f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int j = 1; j < JG; ++j) D = mfma16x<XT>(A[i][g * JG + j], Wp[g * JG + j], D);
#pragma unroll
            for (int v = 0; v < 4; ++v) Y[tt][i][v] = fmaf(s, D[v], fmaf(cb, XG[i][g][v], Y[tt][i][v]));
          }
        }
        continue;
      }
      const float s = to_f<XT>(static_cast<XS>(B.sv[tt])), b = to_f<XT>(static_cast<XS>(B.bv[tt]));
      const float cb = fmaf(-CM, s, b);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        f32x4_t D = mfma16x<XT>(A[i][0], Wp[0], f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int j = 1; j < 4; ++j) D = mfma16x<XT>(A[i][j], Wp[j], D);
#pragma unroll
        for (int v = 0; v < 4; ++v) Y[tt][i][v] = fmaf(s, D[v], fmaf(cb, X[i][v], Y[tt][i][v]));
      }
    }
  };
  // NB blocks per round: all their loads are issued before any arithmetic
  // (straight-line code, so each wait is exact); blocks past pe reload block
  // pe - 1 with zero scale and bias and add nothing
  for (int p0 = pb; p0 < pe; p0 += NB) {
    Blk B[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) load(p0 + u, B[u]);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (p0 + u >= pe) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) B[u].sv[tt] = B[u].bv[tt] = 0;
      }
      compute(B[u]);
    }
  }
  // lane holds Y[(m, group) = 4 q + v][n = r] of each (n tile, m tile)
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[((wave * NT + tt) * MT + i) * 256 + (4 * q + v) * 16 + r] = Y[tt][i][v];
  __syncthreads();
  if constexpr (GLU) {
    for (int idx = t; idx < M * NC; idx += 64 * S) {
      const int m = idx / NC, nn = idx % NC, i = m / RPT, mr = m % RPT;
      const int sub = nn >> 4;
      float acc[2] = {0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int tt = h * (NT / 2) + sub;
#pragma unroll
        for (int w2 = 0; w2 < S; ++w2)
#pragma unroll
          for (int g = 0; g < GR; ++g) acc[h] += red[((w2 * NT + tt) * MT + i) * 256 + (mr + RPT * g) * 16 + (nn & 15)];
      }
      if (n0 + nn < N) out[static_cast<int64_t>(m) * N + n0 + nn] = swiglu_out<XT>(acc[0], acc[1]);
    }
    return;
  }
  for (int idx = t; idx < M * 16 * NT; idx += 64 * S) {
    const int m = idx / (16 * NT), nn = idx % (16 * NT);
    const int tt = nn >> 4, i = m / RPT, mr = m % RPT;
    float acc = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < S; ++w2)
#pragma unroll
      for (int g = 0; g < GR; ++g) acc += red[((w2 * NT + tt) * MT + i) * 256 + (mr + RPT * g) * 16 + (nn & 15)];
    if (n0 + nn < N) out[static_cast<int64_t>(m) * N + n0 + nn] = from_f<XT>(acc);
  }
}

namespace {
template <int XT, int NT, int MT, int GB, bool GLU, int NB, bool TR>
hipError_t fac_launch_nb(const QmmArgs& a, dim3 grid, int S) {
  switch (S) {
    case 8: hipLaunchKernelGGL((qmm_skinny_fac_kernel<XT, NT, MT, GB, 8, NB, GLU, TR>), grid, dim3(512), 0, a.stream, a); break;
    case 4: hipLaunchKernelGGL((qmm_skinny_fac_kernel<XT, NT, MT, GB, 4, NB, GLU, TR>), grid, dim3(256), 0, a.stream, a); break;
    case 2: hipLaunchKernelGGL((qmm_skinny_fac_kernel<XT, NT, MT, GB, 2, NB, GLU, TR>), grid, dim3(128), 0, a.stream, a); break;
    default: hipLaunchKernelGGL((qmm_skinny_fac_kernel<XT, NT, MT, GB, 1, NB, GLU, TR>), grid, dim3(64), 0, a.stream, a); break;
  }
  return hipGetLastError();
}
template <int XT, int NT, int MT, int GB, bool GLU, bool TR>
hipError_t fac_launch_s(const QmmArgs& a, dim3 grid, int S) {
  return fac_launch_nb<XT, NT, MT, GB, GLU, 2, TR>(a, grid, S);
}
template <int XT, int GB, bool GLU, int NT, int MT, bool TR = false>
hipError_t fac_launch_gbn(const QmmArgs& a) {
  constexpr int NC = GLU ? 8 * NT : 16 * NT;  // output columns per workgroup
  const int64_t nwg = (a.N + NC - 1) / NC;
  if (nwg <= 0 || a.nbatch <= 0) return hipSuccess;
  if (nwg > 0x7fffffffLL || a.nbatch > 65535) return hipErrorInvalidConfiguration;
  const int P = a.K >> 7;
  int S = 1;
  while (S < 8 && P / (2 * S) >= 2 && nwg * a.nbatch * S < 4096) S *= 2;
  // the LDS partial tiles (S NT MT KiB) stay within 64 KiB so two workgroups fit a CU
  while (S > 1 && S * NT * MT > 64) S >>= 1;
  const dim3 grid(static_cast<unsigned>(nwg), static_cast<unsigned>(a.nbatch));
  return fac_launch_s<XT, NT, MT, GB, GLU, TR>(a, grid, S);
}
template <int XT, int GB, bool GLU>
hipError_t fac_launch_gb(const QmmArgs& a) {
  // gs 32 / 64 (two or four groups per 128-code block): chunk-major k slots,
  // every A row a live x row; four weight tiles per wave share each x
  // fragment (measured at N = 14336, K = 4096, gs 64: M = 16 21.8 -> 20.5 us,
  // M = 24 31.1 -> 23.0 us, M = 32 32.7 -> 24.1 us against the group-split
  // rows; gs 32, M = 16: 30.1 -> 20.5 us).  Two tiles at gs 64 up to M = 8
  // (M = 4: 17.8 against 18.7 us with four; gs 32 prefers four, 18.5 against
  // 19.1 us) and for two m tiles at gs 32, whose four group accumulators would
  // otherwise spill.
  const bool wide = static_cast<int64_t>(a.N) * a.nbatch * (a.glu ? 2 : 1) >= 8192;
  if constexpr (GB > 1) {
    if (GB == 2 && a.M <= 8) return fac_launch_gbn<XT, GB, GLU, 2, 1, true>(a);
    // four tiles halve the workgroups: only on matrices of >= 8192 rows
    if (a.M <= 16 && wide) return fac_launch_gbn<XT, GB, GLU, 4, 1, true>(a);
    if (a.M <= 16) return fac_launch_gbn<XT, GB, GLU, 2, 1, true>(a);
    // two m tiles: two weight tiles below 8192 rows (N = 6144, M = 32: 22.7 ->
    // 16.4 us), four from 8192 (N = 14336, M = 32: 31.2 -> 24.4 us)
    if constexpr (GB == 4) return fac_launch_gbn<XT, GB, GLU, 2, 2, true>(a);
    else if (!wide) return fac_launch_gbn<XT, GB, GLU, 2, 2, true>(a);
    else return fac_launch_gbn<XT, GB, GLU, 4, 2, true>(a);
  } else {
    // gs 128: one group per block, so every A row is already live
    if (a.M <= 16) return fac_launch_gbn<XT, GB, GLU, 2, 1>(a);
    return fac_launch_gbn<XT, GB, GLU, 4, 2>(a);
  }
}
template <int XT, bool GLU>
hipError_t fac_launch(const QmmArgs& a) {
  switch (a.gs) {
    case 32: return fac_launch_gb<XT, 4, GLU>(a);
    case 64: return fac_launch_gb<XT, 2, GLU>(a);
    default: return fac_launch_gb<XT, 1, GLU>(a);
  }
}
}  // namespace

bool qmm_skinny_fac_supported(const QmmArgs& a) {
  if (!(a.transpose && a.mode == AFFINE && a.bits == 4 && (a.xdt == BF16 || a.xdt == F16) &&
        a.K % 128 == 0 && a.K >= 128))
    return false;
  // with fewer than 1536 waves (8 per 32-row tile pair) the split-K skinny
  // kernel keeps more loads in flight (measured at K = 4096: N = 6144 runs
  // faster here, 12.1 -> 10.1 us at M = 4, N = 4096 slower)
  // (GLU: 2N weight rows, 16 output columns per workgroup)
  const int64_t waves = (a.N + 31) / 32 * 8 * a.nbatch * (a.glu ? 2 : 1);
  // chunk-major slots load the 2 / 4 group scales and biases of a block as one
  // 4- / 8-byte word
  const bool aligned = (reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 8 == 0;
  return a.M >= 1 && a.M <= 32 && waves >= 1536 && (a.gs == 128 || aligned);
}

hipError_t launch_qmm_skinny_fac(const QmmArgs& a) {
  if (a.glu) return a.xdt == BF16 ? fac_launch<BF16, true>(a) : fac_launch<F16, true>(a);
  return a.xdt == BF16 ? fac_launch<BF16, false>(a) : fac_launch<F16, false>(a);
}

// ---------------------------------------------------------------------------
// Grouped gather_qmm for sorted expert indices (mlx-c gather_qmm with
// sorted_indices = true; the MoE layer of mlx/src/nn/moe.rs:84-170 over the
// stacked [E, N, K/pack] expert tensors of mlx/src/model/qwen35.rs:653-775).
// A pre-pass turns the sorted flat rhs index array into segment offsets
// off[e] = first row whose expert is >= e (off[E] = end of the valid rows), so
// every workgroup finds its row segment with two loads.  blockIdx.y = expert
// e; each wave owns 16 output columns over the whole K, so the expert's
// weight rows are read once for all of the tokens routed to it (in 32-row m
// tiles).  Segment row r is batch element b = lo + r / Mx, matrix row r % Mx,
// x matrix lhs[b].  Rows whose expert index is outside [0, E) sort before
// off[0] or from off[E] on and get NaN rows (blockIdx.y = E).
__global__ __launch_bounds__(256) void segment_offsets_kernel(const void* rhs, int rhs_dt, int64_t nflat,
                                                              int64_t E, int64_t* off) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i > nflat) return;
  auto key = [&](int64_t j) {
    const int64_t v = load_index(rhs, rhs_dt, j);
    return v < 0 ? int64_t{-1} : v > E ? E : v;
  };
  const int64_t kp = i > 0 ? key(i - 1) : -1;
  const int64_t kc = i < nflat ? key(i) : E + 1;
  for (int64_t e = kp + 1; e <= min(kc, E); ++e) off[e] = i;
}

// Workgroup = S <= 8 waves over CS 16-column strips of one expert; wave w
// takes chunk groups [w IT, (w + 1) IT) of K (a chunk group is 128 k: 4 lane
// quarters x 32 codes) for all CS strips and issues every weight / scale load
// before its first MFMA (CS x IT x 1 KiB of weights in flight per wave); each
// x fragment (an L2-resident operand, loaded one group at a time) feeds the CS
// strips' MFMAs.  The S partial tiles are summed through LDS.
// GBT > 0 (affine 4-bit, GBT = 128 / gs groups per chunk group): chunk-major
// k slots as in qmm_skinny_fac_kernel -- MFMA j of a chunk group takes chunk
// 4p + j and lane (r, q) its 8-code piece q, so each x load is 64 contiguous
// bytes per row; the weight dwords are transposed across the lanes q and each
// dword j is dequantized with the scale / bias of chunk 4p + j.
// GLU (CS even): each expert holds 2N rows (gate [0, N), up [N, 2N)); strips
// [0, CS/2) are gate columns n0.. and [CS/2, CS) the matching up columns, and
// the epilogue writes silu(gate) * up for 8 CS columns.
template <int XT, int MODE, int BITS, int IT, int CS, int GBT = 0, bool GLU = false>
__global__ __launch_bounds__(512) void gather_sorted_kernel(QmmArgs a, int64_t nflat, const int64_t* off) {
  using XS = uint16_t;
  constexpr bool AFF = MODE == AFFINE;
  constexpr bool TRX = GBT > 0;
  static_assert(!TRX || (AFF && BITS == 4), "chunk-major slots: affine 4-bit");
  using SG = typename std::conditional<GBT == 4, uint64_t, typename std::conditional<GBT == 2, uint32_t, XS>::type>::type;
  __shared__ float red[8][CS][16 * 17];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int S = blockDim.x >> 6;
  const int Mx = a.M, N = a.N, K = a.K;
  static_assert(!GLU || CS % 2 == 0, "GLU pairs gate strips with up strips");
  constexpr int NC = GLU ? 8 * CS : 16 * CS;  // output columns per workgroup
  const int n0 = blockIdx.x * NC;
  const int64_t e = blockIdx.y;
  if (e == a.bm.nw) {
    // offsets are clamped into [0, nflat]: indices that are not sorted as
    // promised give wrong rows, never out-of-range accesses
    const int64_t first_valid = min(max(off[0], int64_t{0}), nflat);
    const int64_t end_valid = min(max(off[e], first_valid), nflat);
    XS* o = static_cast<XS*>(a.out);
    const int64_t nbad = first_valid + (nflat - end_valid);
    for (int64_t i = t; i < nbad * Mx * NC; i += blockDim.x) {
      const int64_t rr = i / NC, n = i % NC;
      const int64_t bi = rr / Mx, mrow = rr % Mx;
      const int64_t b = bi < first_valid ? bi : end_valid + (bi - first_valid);
      if (n0 + n < N) o[(b * Mx + mrow) * N + n0 + n] = from_f<XT>(__builtin_nanf(""));
    }
    return;
  }
  const int64_t blo = min(max(off[e], int64_t{0}), nflat);
  const int64_t bhi = min(max(off[e + 1], blo), nflat);
  if (blo >= bhi) return;  // workgroup-uniform
  const int64_t rows_total = (bhi - blo) * Mx;
  XS* out = static_cast<XS*>(a.out);
  const XS* x = static_cast<const XS*>(a.x);
  const uint32_t* w = a.w + e * a.w_mat;
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const int G = K / gs;
  const XS* sp = static_cast<const XS*>(a.s) + e * a.s_mat;
  const XS* bp = AFF ? static_cast<const XS*>(a.b) + e * a.s_mat : nullptr;
  const uint8_t* s8 = static_cast<const uint8_t*>(a.s) + e * a.s_mat;
  const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
  const int nl = lane & 15, q = lane >> 4;
  const int p0 = wave * IT;

  // weights and scales of this wave's chunks for every strip: loaded once,
  // reused by every m tile
  uint32_t wd[CS][IT][BITS];
  float sv[CS][IT], bv[CS][IT], s2[CS][IT];
  SG sg[TRX ? CS : 1][TRX ? IT : 1], bg[TRX ? CS : 1][TRX ? IT : 1];
#pragma unroll
  for (int cs = 0; cs < CS; ++cs) {
    const int row = GLU ? (cs / (CS / 2)) * N + min(n0 + 16 * (cs % (CS / 2)) + nl, N - 1)
                        : min(n0 + 16 * cs + nl, N - 1);
    const uint32_t* wrow = w + static_cast<int64_t>(row) * wpr;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int c = 4 * (p0 + it) + q;
      load_chunk<BITS>(wd[cs][it], wrow + c * BITS);
      const int gi = (c * 32) / gs;
      if constexpr (TRX) {
        // the GBT scales / biases of chunk group p0 + it, one load each
        const int64_t g0 = static_cast<int64_t>(row) * G + (p0 + it) * GBT;
        sg[cs][it] = *reinterpret_cast<const SG*>(sp + g0);
        bg[cs][it] = *reinterpret_cast<const SG*>(bp + g0);
        sv[cs][it] = bv[cs][it] = s2[cs][it] = 0.f;
      } else if constexpr (AFF) {
        sv[cs][it] = to_f<XT>(sp[static_cast<int64_t>(row) * G + gi]);
        bv[cs][it] = to_f<XT>(bp[static_cast<int64_t>(row) * G + gi]);
        s2[cs][it] = sv[cs][it];
      } else {
        sv[cs][it] = fp_scale<MODE>(s8[static_cast<int64_t>(row) * G + gi]);
        s2[cs][it] = MODE == NVFP4 ? fp_scale<MODE>(s8[static_cast<int64_t>(row) * G + gi + 1]) : sv[cs][it];
        bv[cs][it] = 0.f;
      }
    }
  }

  if constexpr (TRX) {
    // 4 x 4 dword transpose over the lanes q: wd[j] of lane q becomes dword q
    // of chunk 4p + j (the chunk lane j loaded)
#pragma unroll
    for (int cs = 0; cs < CS; ++cs)
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        uint32_t (&v)[BITS] = wd[cs][it];
        auto s02 = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
        auto s13 = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
        auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
        auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
        v[0] = s01[0]; v[1] = s01[1]; v[2] = s23[0]; v[3] = s23[1];
      }
  }
  for (int64_t r0 = 0; r0 < rows_total; r0 += 16) {
    // this lane's x row (A operand) of the 16-row tile
    const int64_t r = r0 + nl;
    bool xv = r < rows_total;
    const int64_t b = blo + (xv ? r : 0) / Mx;
    const int64_t mrow = (xv ? r : 0) % Mx;
    const int64_t xm = a.bm.lhs ? load_index(a.bm.lhs, a.bm.lhs_dt, b) : b;
    const bool inb = xm >= 0 && xm < a.bm.nx;
    xv = xv && inb;
    const XS* xrow = x + (inb ? xm : 0) * a.x_mat + mrow * K;
    f32x4_t acc[CS];
#pragma unroll
    for (int cs = 0; cs < CS; ++cs) acc[cs] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      g_u32x4_t xa[4];
      if constexpr (TRX) {
        // piece q of chunks 4 (p0 + it) + j
        const XS* xg = xrow + 4 * (p0 + it) * 32 + 8 * q;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xa[j] = xv ? *reinterpret_cast<const g_u32x4_t*>(xg + 32 * j) : g_u32x4_t{0, 0, 0, 0};
      } else {
        const g_u32x4_t* xp = reinterpret_cast<const g_u32x4_t*>(xrow + (4 * (p0 + it) + q) * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) xa[j] = xv ? xp[j] : g_u32x4_t{0, 0, 0, 0};
      }
#pragma unroll
      for (int cs = 0; cs < CS; ++cs) {
        uint32_t o[16];
        if constexpr (TRX) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int sh = 16 * ((j * GBT) >> 2);
            const float s = to_f<XT>(static_cast<XS>(sg[cs][it] >> sh));
            const float b = to_f<XT>(static_cast<XS>(bg[cs][it] >> sh));
            const uint32_t lo = wd[cs][it][j] & 0x0F0F0F0Fu, hi = (wd[cs][it][j] >> 4) & 0x0F0F0F0Fu;
            o[4 * j + 0] = pack2<XT>(fmaf(s, ubyte_f<0>(lo), b), fmaf(s, ubyte_f<0>(hi), b));
            o[4 * j + 1] = pack2<XT>(fmaf(s, ubyte_f<1>(lo), b), fmaf(s, ubyte_f<1>(hi), b));
            o[4 * j + 2] = pack2<XT>(fmaf(s, ubyte_f<2>(lo), b), fmaf(s, ubyte_f<2>(hi), b));
            o[4 * j + 3] = pack2<XT>(fmaf(s, ubyte_f<3>(lo), b), fmaf(s, ubyte_f<3>(hi), b));
          }
        } else if constexpr (AFF && BITS == 4)
          deq4_fast<XT>(g_u32x4_t{wd[cs][it][0], wd[cs][it][1], wd[cs][it][2], wd[cs][it][3]}, sv[cs][it],
                        bv[cs][it], o);
        else
          dequant32<XT, MODE, BITS>(wd[cs][it], sv[cs][it], bv[cs][it], s2[cs][it], o);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[cs] = mfma16x<XT>(xa[j], g_u32x4_t{o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]}, acc[cs]);
      }
    }
    // D[m][n]: m = 4 q + rr, n = nl
#pragma unroll
    for (int cs = 0; cs < CS; ++cs)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) red[wave][cs][(4 * q + rr) * 17 + nl] = acc[cs][rr];
    __syncthreads();
    if constexpr (GLU) {
      for (int i = t; i < (CS / 2) * 16 * 16; i += blockDim.x) {
        const int cs = i / 256, m = (i / 16) % 16, n = i % 16;
        const int64_t rm = r0 + m;
        const int col = n0 + 16 * cs + n;
        if (rm < rows_total && col < N) {
          float g = 0.f, u = 0.f;
          for (int w2 = 0; w2 < S; ++w2) g += red[w2][cs][m * 17 + n];
          for (int w2 = 0; w2 < S; ++w2) u += red[w2][cs + CS / 2][m * 17 + n];
          const int64_t bb = blo + rm / Mx, mr = rm % Mx;
          const int64_t xi = a.bm.lhs ? load_index(a.bm.lhs, a.bm.lhs_dt, bb) : bb;
          const bool ok = xi >= 0 && xi < a.bm.nx;
          out[(bb * Mx + mr) * N + col] = ok ? swiglu_out<XT>(g, u) : from_f<XT>(__builtin_nanf(""));
        }
      }
      __syncthreads();
      continue;
    }
    for (int i = t; i < CS * 16 * 16; i += blockDim.x) {
      const int cs = i / 256, m = (i / 16) % 16, n = i % 16;
      const int64_t rm = r0 + m;
      const int col = n0 + 16 * cs + n;
      if (rm < rows_total && col < N) {
        float v = 0.f;
        for (int w2 = 0; w2 < S; ++w2) v += red[w2][cs][m * 17 + n];
        const int64_t bb = blo + rm / Mx, mr = rm % Mx;
        const int64_t xi = a.bm.lhs ? load_index(a.bm.lhs, a.bm.lhs_dt, bb) : bb;
        const bool ok = xi >= 0 && xi < a.bm.nx;
        out[(bb * Mx + mr) * N + col] = from_f<XT>(ok ? v : __builtin_nanf(""));
      }
    }
    __syncthreads();
  }
}

// chunk groups per wave of the grouped gather (P = K / 128 groups): the
// smallest of 1 / 2 / 4 (<= itmax) that splits K over at most 4 waves
// (measured best: K = 512 -> 1 group x 4 waves, K = 2048 -> 4 x 4), else the
// largest that keeps the workgroup at <= 8 waves; 0 if none fits
int gather_groups_per_wave(int K, int itmax) {
  const int P = K >> 7;
  for (int it = 1; it <= itmax; it <<= 1)
    if (P % it == 0 && P / it <= 4) return it;
  for (int it = itmax; it >= 1; it >>= 1)
    if (P % it == 0 && P / it <= 8) return it;
  return 0;
}

// the SwiGLU epilogue: affine 4-bit with 8-byte aligned scales / biases
bool gather_sorted_glu_supported(const QmmArgs& a) {
  return a.mode == AFFINE && a.bits == 4 &&
         (reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 8 == 0;
}

bool gather_sorted_supported(const QmmArgs& a) {
  return a.transpose && (a.xdt == BF16 || a.xdt == F16) && a.K % 128 == 0 && a.K >= 128 &&
         gather_groups_per_wave(a.K, 4) > 0 && a.bm.rhs != nullptr;
}

bool qmm_skinny_supported(const QmmArgs& a) {
  return a.transpose && (a.xdt == BF16 || a.xdt == F16) && a.K % 64 == 0 && a.M <= 64;
}

namespace {
template <int XT, int MODE, int BITS>
hipError_t skinny_launch_t(const QmmArgs& a) {
  const int64_t ntiles = (a.N + SK_ROWS - 1) / SK_ROWS;
  const int nmt = (a.M + 31) / 32;
  const int64_t ny = static_cast<int64_t>(nmt) * a.nbatch;
  if (ntiles <= 0 || ny <= 0) return hipSuccess;
  if (ntiles > 0x7fffffffLL || ny > 65535) return hipErrorInvalidConfiguration;
  // split K over S waves so that about 2048+ waves are in flight
  const int P = a.K >> 6;
  const int64_t tiles = ntiles * ny;
  int S = 4;
  if (tiles * 4 < 4096 && P >= 32) S = 8;
  if (tiles * 8 < 4096 && P >= 64) S = 16;
  const dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(ny));
#define IQMM_SK(SS) hipLaunchKernelGGL((qmm_skinny_kernel<XT, MODE, BITS, SS, 2>), grid, dim3(64 * SS), 0, a.stream, a, nmt)
  switch (S) { case 16: IQMM_SK(16); break; case 8: IQMM_SK(8); break; default: IQMM_SK(4); break; }
#undef IQMM_SK
  return hipGetLastError();
}

template <int XT, int MODE, int BITS, int S, int GBT>
void s16_launch_g(const QmmArgs& a, dim3 grid, int nmt) {
  const int rows = a.M >= 32 ? 32 : a.M;
  if (rows <= 16) hipLaunchKernelGGL((qmm_skinny16_kernel<XT, MODE, BITS, S, 1, 4, GBT>), grid, dim3(64 * S), 0, a.stream, a, nmt);
  else hipLaunchKernelGGL((qmm_skinny16_kernel<XT, MODE, BITS, S, 2, 4, GBT>), grid, dim3(64 * S), 0, a.stream, a, nmt);
}

template <int XT, int MODE, int BITS, int S>
hipError_t s16_launch_s(const QmmArgs& a, dim3 grid, int nmt) {
  // affine 4-bit: chunk-major k slots (measured 3-7% faster at M = 4 ... 32 for
  // N x K = 4096 x 14336, 4096 x 4096 and 1024 x 4096, e.g. 29.7 -> 27.8 us
  // at M = 16, N = 4096, K = 14336); needs 8-byte aligned scales / biases
  if constexpr (MODE == AFFINE && BITS == 4) {
    if ((reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 8 == 0) {
      switch (a.gs) {
        case 32: s16_launch_g<XT, MODE, BITS, S, 4>(a, grid, nmt); break;
        case 64: s16_launch_g<XT, MODE, BITS, S, 2>(a, grid, nmt); break;
        default: s16_launch_g<XT, MODE, BITS, S, 1>(a, grid, nmt); break;
      }
      return hipGetLastError();
    }
  }
  s16_launch_g<XT, MODE, BITS, S, 0>(a, grid, nmt);
  return hipGetLastError();
}

template <int XT, int MODE, int BITS>
hipError_t s16_launch(const QmmArgs& a) {
  const int64_t ntiles = (a.N + 15) / 16;
  const int nmt = (a.M + 31) / 32;
  const int64_t ny = static_cast<int64_t>(nmt) * a.nbatch;
  if (ntiles <= 0 || ny <= 0) return hipSuccess;
  if (ntiles > 0x7fffffffLL || ny > 65535) return hipErrorInvalidConfiguration;
  const int P = a.K >> 7;
  const int64_t tiles = ntiles * ny;
  int S = 2;
  if (tiles * 2 < 4096 && P >= 16) S = 4;
  if (tiles * 4 < 4096 && P >= 32) S = 8;
  const dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(ny));
  switch (S) {
    case 8: return s16_launch_s<XT, MODE, BITS, 8>(a, grid, nmt);
    case 4: return s16_launch_s<XT, MODE, BITS, 4>(a, grid, nmt);
    default: return s16_launch_s<XT, MODE, BITS, 2>(a, grid, nmt);
  }
}

template <int XT>
hipError_t skinny_by_mode(const QmmArgs& a) {
  // 16x16x32 layout (64-byte row runs) when K is a multiple of 128
  if (a.K % 128 == 0) {
    switch (a.mode) {
      case AFFINE:
        switch (a.bits) {
          case 2: return s16_launch<XT, AFFINE, 2>(a);
          case 3: return s16_launch<XT, AFFINE, 3>(a);
          case 4: return s16_launch<XT, AFFINE, 4>(a);
          case 5: return s16_launch<XT, AFFINE, 5>(a);
          case 6: return s16_launch<XT, AFFINE, 6>(a);
          case 8: return s16_launch<XT, AFFINE, 8>(a);
        }
        break;
      case MXFP4: return s16_launch<XT, MXFP4, 4>(a);
      case MXFP8: return s16_launch<XT, MXFP8, 8>(a);
      case NVFP4: return s16_launch<XT, NVFP4, 4>(a);
    }
  }
  switch (a.mode) {
    case AFFINE:
      switch (a.bits) {
        case 2: return skinny_launch_t<XT, AFFINE, 2>(a);
        case 3: return skinny_launch_t<XT, AFFINE, 3>(a);
        case 4: return skinny_launch_t<XT, AFFINE, 4>(a);
        case 5: return skinny_launch_t<XT, AFFINE, 5>(a);
        case 6: return skinny_launch_t<XT, AFFINE, 6>(a);
        case 8: return skinny_launch_t<XT, AFFINE, 8>(a);
      }
      break;
    case MXFP4: return skinny_launch_t<XT, MXFP4, 4>(a);
    case MXFP8: return skinny_launch_t<XT, MXFP8, 8>(a);
    case NVFP4: return skinny_launch_t<XT, NVFP4, 4>(a);
  }
  return hipErrorInvalidValue;
}
}  // namespace

namespace {
template <int XT, int MODE, int BITS, int CS, int GBT = 0, bool GLU = false>
hipError_t gather_launch_cs(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  constexpr int NC = GLU ? 8 * CS : 16 * CS;
  const int64_t ntiles = (a.N + NC - 1) / NC;
  if (ntiles > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(E + 1));
  // IT chunk groups (128 k each, P = K / 128) per wave, P / IT <= 8 waves.
  // Register budget with CS strips held at once: 4-bit affine (fast byte
  // dequant) holds 4 groups, other widths 2, 8-bit codes 1 (CS = 1: 4 for all)
  constexpr int ITMAX = CS == 1 ? 4 : MODE == AFFINE && BITS == 4 ? 4 : BITS == 8 ? 1 : 2;
  const int it = gather_groups_per_wave(a.K, ITMAX);
  const dim3 block(static_cast<unsigned>(64 * ((a.K >> 7) / it)));
  switch (it) {
    case 4:
      if constexpr (ITMAX >= 4)
        hipLaunchKernelGGL((gather_sorted_kernel<XT, MODE, BITS, 4, CS, GBT, GLU>), grid, block, 0, a.stream, a, nflat, off);
      break;
    case 2:
      if constexpr (ITMAX >= 2)
        hipLaunchKernelGGL((gather_sorted_kernel<XT, MODE, BITS, 2, CS, GBT, GLU>), grid, block, 0, a.stream, a, nflat, off);
      break;
    case 1: hipLaunchKernelGGL((gather_sorted_kernel<XT, MODE, BITS, 1, CS, GBT, GLU>), grid, block, 0, a.stream, a, nflat, off); break;
    default: return hipErrorInvalidConfiguration;
  }
  return hipGetLastError();
}

template <int XT, int MODE, int BITS>
hipError_t gather_launch_t(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  // four strips per wave: 4x the weight bytes in flight per wave and each x
  // fragment shared by four MFMAs (measured faster than one strip at 2 and
  // 16 rows per expert for both MoE projections)
  // affine 4-bit: chunk-major k slots (measured at 256 experts, top 8, K =
  // 2048: T = 512 gate 106.6 -> 85 us, T = 64 down 57.5 -> 56.2 us, others
  // equal); the group scales / biases of a chunk group are one word
  if constexpr (MODE == AFFINE && BITS == 4) {
    if ((reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 8 == 0) {
      if (a.glu) {
        switch (a.gs) {
          case 32: return gather_launch_cs<XT, MODE, BITS, 4, 4, true>(a, nflat, E, off);
          case 64: return gather_launch_cs<XT, MODE, BITS, 4, 2, true>(a, nflat, E, off);
          default: return gather_launch_cs<XT, MODE, BITS, 4, 1, true>(a, nflat, E, off);
        }
      }
      switch (a.gs) {
        case 32: return gather_launch_cs<XT, MODE, BITS, 4, 4>(a, nflat, E, off);
        case 64: return gather_launch_cs<XT, MODE, BITS, 4, 2>(a, nflat, E, off);
        default: return gather_launch_cs<XT, MODE, BITS, 4, 1>(a, nflat, E, off);
      }
    }
  }
  if (a.glu) return hipErrorInvalidValue;  // callers check gather_sorted_glu_supported
  return gather_launch_cs<XT, MODE, BITS, 4>(a, nflat, E, off);
}

template <int XT>
hipError_t gather_by_mode(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  switch (a.mode) {
    case AFFINE:
      switch (a.bits) {
        case 2: return gather_launch_t<XT, AFFINE, 2>(a, nflat, E, off);
        case 3: return gather_launch_t<XT, AFFINE, 3>(a, nflat, E, off);
        case 4: return gather_launch_t<XT, AFFINE, 4>(a, nflat, E, off);
        case 5: return gather_launch_t<XT, AFFINE, 5>(a, nflat, E, off);
        case 6: return gather_launch_t<XT, AFFINE, 6>(a, nflat, E, off);
        case 8: return gather_launch_t<XT, AFFINE, 8>(a, nflat, E, off);
      }
      break;
    case MXFP4: return gather_launch_t<XT, MXFP4, 4>(a, nflat, E, off);
    case MXFP8: return gather_launch_t<XT, MXFP8, 8>(a, nflat, E, off);
    case NVFP4: return gather_launch_t<XT, NVFP4, 4>(a, nflat, E, off);
  }
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_gather_sorted(const QmmArgs& a, int64_t nflat, int64_t E) {
  if (a.xdt != BF16 && a.xdt != F16) return hipErrorInvalidValue;
  if (a.N <= 0 || E <= 0 || nflat <= 0) return hipSuccess;
  if (E + 1 > 65535) return hipErrorInvalidConfiguration;
  // K of 1024 or more (affine 4-bit, gs 64), or few rows per expert (at most
  // 8 on average): the per-expert streaming kernel, which fetches and converts
  // each pass's x rows once and streams the expert's weights past them,
  // finding its row segment in the sorted rhs itself (no offsets pre-pass).
  // 256 experts, top 8: T = 64 gate 2048 -> 512 39.5 -> 32.8 us, down
  // 512 -> 2048 38.3 -> 35.3 us; T = 512 gate 62-63 -> 60.1 us; fused gate_up
  // expert block T = 64 / 512: 138 / 213 -> 119 / 199 us.  The T = 512 down
  // projection (K = 512, 16 rows per expert) keeps the column-block kernel
  // (streamed: 62 -> 68 us), whose many short workgroups read the pre-pass's
  // offsets (an in-kernel search there: 63 -> 69 us).
  if (gather_stream_supported(a) && (a.K >= 1024 || nflat * a.M <= 8 * E)) return launch_gather_stream(a, nflat, E);
  // segment offsets in the stream's offsets workspace (workspace.hip)
  void* ws = nullptr;
  hipError_t e = workspace_get(a.stream, WS_OFFSETS, static_cast<size_t>(E + 1) * sizeof(int64_t), &ws);
  if (e != hipSuccess) return e;
  int64_t* off = static_cast<int64_t*>(ws);
  const int64_t nb = (nflat + 1 + 255) / 256;
  hipLaunchKernelGGL(segment_offsets_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, a.stream, a.bm.rhs,
                     a.bm.rhs_dt, nflat, E, off);
  e = hipGetLastError();
  if (e == hipSuccess) {
    if (gather_decode_supported(a)) e = launch_gather_decode(a, nflat, E, off);
    else e = a.xdt == BF16 ? gather_by_mode<BF16>(a, nflat, E, off) : gather_by_mode<F16>(a, nflat, E, off);
  }
  return e;
}

hipError_t launch_qmm_skinny(const QmmArgs& a) {
  if (a.xdt == BF16) return skinny_by_mode<BF16>(a);
  if (a.xdt == F16) return skinny_by_mode<F16>(a);
  return hipErrorInvalidValue;
}

}  // namespace iqmm
