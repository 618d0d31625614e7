// qmv_q4.hip — the decode GEMV fast path: affine 4-bit, transpose=true,
// M = 1..3 rows of bf16 or fp16 activations (the shape every ironmlx decode
// step runs, mlx/src/nn/linear.rs:51-63 with x = [1, 1, K]).
//
// One wave per workgroup owns RB (1, 2 or 4) consecutive weight rows (for
// K >= 10240, four waves split each of a workgroup's four rows, KS below).  Lane
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
#include "mfma_common.h"
#include "gemv_common.h"

namespace iqmm {

// fp4 (e2m1) chunk -> 16 pairs in the same (n0,n4) (n2,n6) (n1,n5) (n3,n7)
// order.  The 3-bit magnitude indexes an 8-byte table with v_perm_b32 (high
// and low bytes of the 16-bit value {0, .5, 1, 1.5, 2, 3, 4, 6}); the sign bit
// moves to bit 7 of the high byte.  Every value is exact in bf16 and fp16.
template <int XT>
__device__ __forceinline__ void fp4_pairs(const u32x4_t& wv, uint32_t (&W)[16]) {
  // high bytes: bf16 00 3f 3f 3f 40 40 40 40, fp16 00 38 3c 3e 40 42 44 46
  constexpr uint32_t H0 = XT == BF16 ? 0x3f3f3f00u : 0x3e3c3800u;
  constexpr uint32_t H1 = XT == BF16 ? 0x40404040u : 0x46444240u;
  // low bytes (bf16 only): 00 00 80 c0 00 40 80 c0
  constexpr uint32_t L0 = 0xc0800000u, L1 = 0xc0804000u;
  const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t c = (half ? wd[q] >> 4 : wd[q]) & 0x0F0F0F0Fu;   // codes n(2i+half)
      const uint32_t m = c & 0x07070707u;
      const uint32_t hb = __builtin_amdgcn_perm(H1, H0, m) | ((c << 4) & 0x80808080u);
      if constexpr (XT == BF16) {
        const uint32_t lb = __builtin_amdgcn_perm(L1, L0, m);
        W[4 * q + 2 * half + 0] = __builtin_amdgcn_perm(hb, lb, 0x06020400u);
        W[4 * q + 2 * half + 1] = __builtin_amdgcn_perm(hb, lb, 0x07030501u);
      } else {
        W[4 * q + 2 * half + 0] = __builtin_amdgcn_perm(hb, hb, 0x060c040cu);
        W[4 * q + 2 * half + 1] = __builtin_amdgcn_perm(hb, hb, 0x070c050cu);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Single-pass kernel.  One wave per workgroup owns RB rows; lane l owns
// chunks l, l+64, ... (CPL per row).  Every load is issued before any
// arithmetic -- x first (cache-resident), then for each row its weight chunks
// followed by its scales and biases -- and a scheduling barrier keeps the
// compiler from sinking loads behind the first wait, so with in-order vmcnt
// accounting row r's arithmetic and DPP reduction run while the loads of rows
// r+1.. are still in flight.  The arguments are a compact block (one scalar
// load); the general batch map is read only by the MAPPED instantiation.
struct Q4Args {
  const char* x;
  const char* w;
  const char* s;
  const char* b;
  char* out;
  int N, K, gshift, pad;
  int64_t x_mat, w_mat, s_mat;  // byte strides between batch elements
};

//
// GLU: the weight holds 2N rows (gate rows [0, N), up rows [N, 2N), the fused
// gate_up layout); a wave reduces RB / 2 gate rows and the matching up rows
// and writes RB / 2 SwiGLU outputs.
//
// KS > 1 (long K): the workgroup's KS waves split each row's chunks -- lane l
// of wave w owns chunks l + 64 (w + KS j) -- and their row sums meet in LDS,
// added in wave order.
//
// WG > 1 (M = 1, KS = 1): WG waves per workgroup, each with its own RB rows,
// share one copy of x through LDS.  Every wave needs all of x (lane l reads
// the x of chunks l, l + 64, ...), so with one wave per workgroup the x
// reloads (K * 2 bytes per wave) outweigh the wave's weight bytes (RB * K / 2)
// in each CU's vector-memory pipeline; here the workgroup loads x once
// (issued first, before the weight loads), stores it piece-major in LDS
// (piece i of chunk c at [i][c], so the lanes' reads are contiguous) and the
// waves read their x chunks from LDS after one barrier.
template <int XT, int RB, int CPL, bool MAPPED, int MR, int MODE = AFFINE, bool GLU = false, int KS = 1, int WG = 1>
__global__ __launch_bounds__(64 * KS * WG)
__attribute__((amdgpu_waves_per_eu(MR == 1 && RB == 2 && CPL == 2 && KS == 1 ? 7 : 1))) void qmv_q4_kernel(
    Q4Args p, BatchMap bm, int64_t batch0) {
  static_assert(!GLU || (MR == 1 && RB % 2 == 0), "GLU pairs gate / up rows at M = 1");
  static_assert(WG == 1 || (KS == 1 && MR == 1 && (4 * CPL) % WG == 0), "shared x: one row of x, no K split");
  constexpr int RO = GLU ? RB / 2 : RB;  // outputs per wave
  using XS = uint16_t;
  const int lane = threadIdx.x & 63;
  const int kw = KS > 1 ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)) : 0;
  const int64_t bb = batch0 + blockIdx.y;
  const int N = p.N, K = p.K, C = K >> 5;
  XS* out = reinterpret_cast<XS*>(p.out) + bb * static_cast<int64_t>(N) * MR;
  const int wv_id = WG > 1 ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)) : 0;
  const int row0 = (blockIdx.x * WG + wv_id) * RO;

  int64_t xi = bb, wi = bb;
  if constexpr (MAPPED) {
    if (!map_batch(bm, bb, xi, wi)) {
      if (kw == 0 && lane < RO * MR && row0 + lane % RO < N)
        out[static_cast<int64_t>(lane / RO) * N + row0 + lane % RO] = from_f<XT>(__builtin_nanf(""));
      return;
    }
  }
  const char* xbase = p.x + xi * p.x_mat;
  const char* w = p.w + wi * p.w_mat;
  const char* sp = p.s + wi * p.s_mat;
  const char* bp = p.b + wi * p.s_mat;
  // bytes per row; one matrix's packed codes and scales stay below 4 GiB
  // (checked by the launcher), so row offsets are 32-bit scalar products
  const uint32_t wrow = static_cast<uint32_t>(K) >> 1;
  const uint32_t srow = MODE == AFFINE ? (static_cast<uint32_t>(K) >> p.gshift) * 2
                                       : static_cast<uint32_t>(K) >> (MODE == MXFP4 ? 5 : 4);
  const uint32_t xrow = static_cast<uint32_t>(K) * 2;

  // per-lane byte offsets (32-bit) of each slot's chunk, x chunk and group
  uint32_t cw[CPL], cx[CPL], cg[CPL];
  int cl[CPL];  // logical chunk of each slot (masked when >= C)
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    cl[j] = lane + 64 * (kw + KS * j);
    const uint32_t cidx = static_cast<uint32_t>(min(cl[j], C - 1));
    cw[j] = cidx << 4;
    cx[j] = cidx << 6;
    // scale byte offset: affine 16-bit per group, MX one byte per chunk,
    // NV two bytes (groups 2c, 2c+1) per chunk
    cg[j] = MODE == AFFINE ? ((cidx << 5) >> p.gshift) * 2 : MODE == MXFP4 ? cidx : 2 * cidx;
  }

  // 1. x chunks (cache-resident) first: each lane's own, or (WG > 1) this
  //    thread's share of the workgroup's one copy
  u32x4_t xv[MR][CPL][4];
  constexpr int XSH = WG > 1 ? 4 * CPL / WG : 1;  // 16-byte x pieces per thread
  u32x4_t xsh[XSH];
  if constexpr (WG > 1) {
#pragma unroll
    for (int u = 0; u < XSH; ++u) {
      const int v = static_cast<int>(threadIdx.x) + 64 * WG * u;  // piece v % 4 of chunk v / 4
      xsh[u] = *reinterpret_cast<const u32x4_t*>(xbase + min(v, 4 * C - 1) * 16);
    }
  } else {
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          xv[m][j][i] = *reinterpret_cast<const u32x4_t*>(xbase + m * xrow + cx[j] + 16 * i);
  }
  // 2. per row: weight chunks, then that row's scales / biases (row bases are
  //    wave-uniform, so every load is scalar base + 32-bit lane offset)
  u32x4_t wv[RB][CPL];
  XS sr[RB][CPL], br[RB][CPL];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int wrow_i = GLU ? (r < RO ? min(row0 + r, N - 1) : N + min(row0 + r - RO, N - 1))
                           : min(row0 + r, N - 1);
    const uint32_t row = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(wrow_i));
    const char* wr = w + row * wrow;
    const char* sr_ = sp + row * srow;
    const char* br_ = bp + row * srow;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      wv[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wr + cw[j]));
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if constexpr (MODE == AFFINE) {
        sr[r][j] = *reinterpret_cast<const XS*>(sr_ + cg[j]);
        br[r][j] = *reinterpret_cast<const XS*>(br_ + cg[j]);
      } else if constexpr (MODE == MXFP4) {
        sr[r][j] = *reinterpret_cast<const uint8_t*>(sr_ + cg[j]);
      } else {
        sr[r][j] = *reinterpret_cast<const XS*>(sr_ + cg[j]);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (WG > 1) {
    __shared__ u32x4_t xl[4][64 * CPL];
#pragma unroll
    for (int u = 0; u < XSH; ++u) {
      const int v = static_cast<int>(threadIdx.x) + 64 * WG * u;
      xl[v & 3][v >> 2] = xsh[u];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[0][j][i] = xl[i][cx[j] >> 6];
  }
  // 3. x pairs and chunk sums (overlaps the weight loads)
  uint32_t P[MR][CPL][16];
  float xs[MR][CPL];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      uint32_t X[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        X[4 * i] = xv[m][j][i].x; X[4 * i + 1] = xv[m][j][i].y;
        X[4 * i + 2] = xv[m][j][i].z; X[4 * i + 3] = xv[m][j][i].w;
      }
      if constexpr (MODE == AFFINE) {
        make_pairs<XT>(X, P[m][j], xs[m][j]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t A0 = X[4 * q], A1 = X[4 * q + 1], B0 = X[4 * q + 2], B1 = X[4 * q + 3];
          P[m][j][4 * q + 0] = __builtin_amdgcn_perm(B0, A0, 0x05040100u);
          P[m][j][4 * q + 1] = __builtin_amdgcn_perm(B1, A1, 0x05040100u);
          P[m][j][4 * q + 2] = __builtin_amdgcn_perm(B0, A0, 0x07060302u);
          P[m][j][4 * q + 3] = __builtin_amdgcn_perm(B1, A1, 0x07060302u);
        }
        xs[m][j] = 0.f;
      }
      if (cl[j] >= C) xs[m][j] = 0.f;  // masked slot contributes nothing
    }
  // 4. rows in load order
  float red[RB];  // GLU: reduced sums, valid in lane 63
  float rsum[KS > 1 ? RB * MR : 1];  // KS > 1: this wave's row sums, lane 63
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const bool live = cl[j] < C;
      if constexpr (MODE != AFFINE) {
        uint32_t Wp[16];
        fp4_pairs<XT>(wv[r][j], Wp);
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d0 = dot2<XT>(Wp[i], P[0][j][i], d0);
#pragma unroll
        for (int i = 8; i < 16; ++i) d1 = dot2<XT>(Wp[i], P[0][j][i], d1);
        if (!live) d0 = d1 = 0.f;
        if constexpr (MODE == MXFP4) {
          acc[0] = fmaf(fp_scale<MODE>(sr[r][j]), d0 + d1, acc[0]);
        } else {
          acc[0] = fmaf(fp_scale<MODE>(sr[r][j] & 0xffu), d0, acc[0]);
          acc[0] = fmaf(fp_scale<MODE>(sr[r][j] >> 8), d1, acc[0]);
        }
        continue;
      }
      const float s = to_f<XT>(sr[r][j]), b = to_f<XT>(br[r][j]);
      if constexpr (MR == 1) {
        float d = chunk_dot<XT>(wv[r][j], P[0][j]);
        if (!live) d = 0.f;
        acc[0] = fmaf(s, fmaf(-Magic<XT>::c, xs[0][j], d), fmaf(b, xs[0][j], acc[0]));
      } else {
        uint32_t Wp[16];
        chunk_pairs<XT>(wv[r][j], Wp);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) d = dot2<XT>(Wp[i], P[m][j][i], d);
          if (!live) d = 0.f;
          acc[m] = fmaf(s, fmaf(-Magic<XT>::c, xs[m][j], d), fmaf(b, xs[m][j], acc[m]));
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float v = dpp_sum_to_lane63(acc[m]);
      if constexpr (GLU) red[r] = v;
      else if constexpr (KS > 1) rsum[r * MR + m] = v;
      else if (lane == 63 && row0 + r < N) out[static_cast<int64_t>(m) * N + row0 + r] = from_f<XT>(v);
    }
  }
  if constexpr (KS > 1) {
    constexpr int NV = GLU ? RB : RB * MR;
    __shared__ float ps[KS][NV];
    if (lane == 63) {
#pragma unroll
      for (int i = 0; i < NV; ++i) ps[kw][i] = GLU ? red[i] : rsum[i];
    }
    __syncthreads();
    if (kw != 0) return;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float v = ps[0][i];
#pragma unroll
      for (int k = 1; k < KS; ++k) v += ps[k][i];
      if constexpr (GLU) red[i] = v;
      else rsum[i] = v;
    }
    if constexpr (!GLU) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m)
          if (lane == 63 && row0 + r < N) out[static_cast<int64_t>(m) * N + row0 + r] = from_f<XT>(rsum[r * MR + m]);
    }
  }
  if constexpr (GLU) {
#pragma unroll
    for (int o = 0; o < RO; ++o)
      if (lane == 63 && row0 + o < N) out[row0 + o] = swiglu_out<XT>(red[o], red[RO + o]);
  }
}


// ---------------------------------------------------------------------------
// M = 1 GEMV for affine 2-, 3- and 6-bit codes (transpose, one matrix).  Same
// structure as qmv_q4_kernel: one wave per RB rows, lane l owns the 32-code
// chunks l, l + 64, ... (BITS words each, LSB-first code stream), x chunk
// loaded once for all rows, scale / bias per group, factored rescale
// s (d - C xs) + b xs.  Codes become C + q halves without conversions:
// 2-bit codes are spread one per byte by masks and placed by v_perm_b32
// against the exponent bytes (as the 4-bit kernel does with nibbles), pairing
// codes (k, 8 + k) and (4 + k, 12 + k) of each word with x permuted alike;
// 3- and 6-bit codes (which straddle bytes and words) are cut with bitfield
// extracts into natural pairs (2t, 2t + 1), which take the raw x dwords.
template <int XT, int BITS, int RB, int CPL>
__global__ __launch_bounds__(64) void qmv_lb_kernel(Q4Args p) {
  static_assert(BITS == 2 || BITS == 3 || BITS == 6, "low-bit kernel");
  using XS = uint16_t;
  const int lane = threadIdx.x;
  const int N = p.N, K = p.K, C = K >> 5;
  XS* out = reinterpret_cast<XS*>(p.out);
  const int row0 = blockIdx.x * RB;
  const uint32_t wrow = static_cast<uint32_t>(K) / 8 * BITS;
  const uint32_t srow = (static_cast<uint32_t>(K) >> p.gshift) * 2;
  const uint32_t E = Magic<XT>::ebytes;
  int cl[CPL];
  uint32_t cidx[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    cl[j] = lane + 64 * j;
    cidx[j] = static_cast<uint32_t>(min(cl[j], C - 1));
  }
  // x of each chunk: raw dwords (natural pairs) or the 2-bit pair order
  uint32_t P[CPL][16];
  float xs[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const u32x4_t* xc = reinterpret_cast<const u32x4_t*>(p.x + cidx[j] * 64);
    uint32_t X[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t v = xc[i];
      X[4 * i] = v.x; X[4 * i + 1] = v.y; X[4 * i + 2] = v.z; X[4 * i + 3] = v.w;
    }
    xs[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) xs[j] = dot2<XT>(X[i], Magic<XT>::one2, xs[j]);
    if (cl[j] >= C) xs[j] = 0.f;
    if constexpr (BITS == 2) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t sel = (k & 1) ? 0x07060302u : 0x05040100u;
          // pairs (16u + k, 16u + 8 + k) and (16u + 4 + k, 16u + 12 + k)
          P[j][8 * u + 2 * k] = __builtin_amdgcn_perm(X[(16 * u + 8 + k) / 2], X[(16 * u + k) / 2], sel);
          P[j][8 * u + 2 * k + 1] = __builtin_amdgcn_perm(X[(16 * u + 12 + k) / 2], X[(16 * u + 4 + k) / 2], sel);
        }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) P[j][i] = X[i];
    }
  }
  float red[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint32_t row = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(min(row0 + r, N - 1)));
    const char* wr = p.w + row * wrow;
    const char* sr_ = p.s + row * srow;
    const char* br_ = p.b + row * srow;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      uint32_t w[BITS];
      const uint32_t* wc = reinterpret_cast<const uint32_t*>(wr + cidx[j] * (4 * BITS));
#pragma unroll
      for (int i = 0; i < BITS; ++i) w[i] = __builtin_nontemporal_load(wc + i);
      const uint32_t g = ((cidx[j] << 5) >> p.gshift) * 2;
      const float s = to_f<XT>(*reinterpret_cast<const XS*>(sr_ + g));
      const float b = to_f<XT>(*reinterpret_cast<const XS*>(br_ + g));
      float d = 0.f;
      if constexpr (BITS == 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t m = (w[u] >> (2 * k)) & 0x03030303u;  // codes 4 byte + k, one per byte
            d = dot2<XT>(__builtin_amdgcn_perm(E, m, SEL_B0B2), P[j][8 * u + 2 * k], d);
            d = dot2<XT>(__builtin_amdgcn_perm(E, m, SEL_B1B3), P[j][8 * u + 2 * k + 1], d);
          }
      } else {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          uint32_t c[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int pos = BITS * (2 * t + h), wi = pos >> 5, bit = pos & 31;
            c[h] = bit + BITS <= 32 ? __builtin_amdgcn_ubfe(w[wi], bit, BITS)
                                    : __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(w[wi + 1], w[wi], bit), 0, BITS);
          }
          d = dot2<XT>((c[1] << 16) | c[0] | (E & 0xFF00FF00u), P[j][t], d);
        }
      }
      if (cl[j] >= C) d = 0.f;
      acc = fmaf(s, fmaf(-Magic<XT>::c, xs[j], d), fmaf(b, xs[j], acc));
    }
    red[r] = dpp_sum_to_lane63(acc);
  }
  if (lane == 63) {
#pragma unroll
    for (int r = 0; r < RB; ++r)
      if (row0 + r < N) out[row0 + r] = from_f<XT>(red[r]);
  }
}

bool qmv_q4_m1_supported(const QmmArgs& a) {
  // K in [1024, 16384]: one to eight 32-code chunks per lane per row
  // one matrix's codes below 4 GiB: row offsets are 32-bit
  // M x rows share each unpacked weight chunk; their x pairs stay in
  // registers, so M * chunks-per-lane is kept to 8.  Each extra row costs
  // 16 dot2 per chunk, so from M = 4 the MFMA skinny kernel is faster.
  const int cpl = ((a.K >> 5) + 63) / 64;
  // mxfp4 / nvfp4 (e2m1 codes, one or two byte scales per chunk) at M = 1
  const bool mode_ok = a.mode == AFFINE ? a.bits == 4 : (a.mode == MXFP4 || a.mode == NVFP4) && a.M == 1;
  // GLU (fused gate / up rows, 2N weight rows) at M = 1 only
  const int64_t wrows = a.glu ? 2 * static_cast<int64_t>(a.N) : a.N;
  return a.transpose && a.M >= 1 && a.M <= 3 && a.M * cpl <= 8 && mode_ok && (!a.glu || a.M == 1) &&
         (a.xdt == BF16 || a.xdt == F16) && a.K >= 1024 && a.K <= 16384 &&
         wrows * (a.K / 2) < (int64_t{1} << 32);
}

namespace {
template <int XT, int RB, int CPL, int MR, int MODE = AFFINE, bool GLU = false, int KS = 1, int WG = 1>
void launch_mr(dim3 grid, const QmmArgs& a, const Q4Args& p, bool mapped, int64_t b0) {
  if constexpr (MR * CPL * KS > 8 || (GLU && (MR != 1 || RB % 2 != 0))) return;  // excluded by the callers
  else if (mapped)
    hipLaunchKernelGGL((qmv_q4_kernel<XT, RB, CPL, true, MR, MODE, GLU, KS>), grid, dim3(64 * KS), 0, a.stream, p,
                       a.bm, b0);
  else
    hipLaunchKernelGGL((qmv_q4_kernel<XT, RB, CPL, false, MR, MODE, GLU, KS, WG>), dim3((grid.x + WG - 1) / WG, grid.y),
                       dim3(64 * KS * WG), 0, a.stream, p, a.bm, b0);
}

template <int XT, int RB, int CPL, int KS = 1>
hipError_t launch_ord(const QmmArgs& a) {
  const int ro = a.glu ? RB / 2 : RB;  // outputs per wave
  const int64_t nrb = (a.N + ro - 1) / ro;
  if (nrb <= 0 || a.nbatch <= 0) return hipSuccess;
  Q4Args p;
  p.x = static_cast<const char*>(a.x);
  p.w = reinterpret_cast<const char*>(a.w);
  p.s = static_cast<const char*>(a.s);
  p.b = static_cast<const char*>(a.b);
  p.out = static_cast<char*>(a.out);
  p.N = a.N;
  p.K = a.K;
  p.gshift = a.mode == AFFINE ? __builtin_ctz(a.gs) : 0;
  p.pad = 0;
  p.x_mat = a.x_mat * 2;
  p.w_mat = a.w_mat * 4;
  p.s_mat = a.s_mat * 2;
  const bool mapped = a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr;
  for (int64_t b0 = 0; b0 < a.nbatch; b0 += 65535) {
    const int64_t nb = a.nbatch - b0 < 65535 ? a.nbatch - b0 : 65535;
    const dim3 grid(static_cast<unsigned>(nrb), static_cast<unsigned>(nb));
    if (a.glu) {
      // gate / up row pairs sharing x the same way from 10240 rows (2 I =
      // 12288: 8.6 -> 8.2 us; even at 28672 rows, which keep four rows per wave)
      if constexpr (KS == 1 && RB == 2) {
        if (a.mode == AFFINE && !mapped && 2 * static_cast<int64_t>(a.N) >= 10240) {
          launch_mr<XT, RB, CPL, 1, AFFINE, true, KS, 4>(grid, a, p, mapped, b0);
          continue;
        }
      }
      if (a.mode == MXFP4) launch_mr<XT, RB, CPL, 1, MXFP4, true, KS>(grid, a, p, mapped, b0);
      else if (a.mode == NVFP4) launch_mr<XT, RB, CPL, 1, NVFP4, true, KS>(grid, a, p, mapped, b0);
      else launch_mr<XT, RB, CPL, 1, AFFINE, true, KS>(grid, a, p, mapped, b0);
      continue;
    }
    if (a.mode == MXFP4) { launch_mr<XT, RB, CPL, 1, MXFP4, false, KS>(grid, a, p, mapped, b0); continue; }
    if (a.mode == NVFP4) { launch_mr<XT, RB, CPL, 1, NVFP4, false, KS>(grid, a, p, mapped, b0); continue; }
    // four waves sharing x through LDS (measured, two rows per wave: K = 4096,
    // N = 11008 / 14336 / 20480: 7.5 / 8.9 / 11.8 -> 7.2 / 8.3 / 10.5 us;
    // K = 2048 / 6144 / 8192: 3-9% faster; even at 8192 rows, behind at 6144
    // for the SwiGLU rows at four rows per wave)
    if constexpr (KS == 1 && RB == 2) {
      if (a.M == 1 && !mapped && a.N >= 10240) {
        launch_mr<XT, RB, CPL, 1, AFFINE, false, KS, 4>(grid, a, p, mapped, b0);
        continue;
      }
    }
    switch (a.M) {
      case 1: launch_mr<XT, RB, CPL, 1, AFFINE, false, KS>(grid, a, p, mapped, b0); break;
      case 2: launch_mr<XT, RB, CPL, 2, AFFINE, false, KS>(grid, a, p, mapped, b0); break;
      default: launch_mr<XT, RB, CPL, 3, AFFINE, false, KS>(grid, a, p, mapped, b0); break;
    }
  }
  return hipGetLastError();
}

template <int XT, int CPL>
hipError_t launch_ord_cpl(const QmmArgs& a) {
  // rows per wave (measured on MI355X): 2 from 4096 rows, 4 from 24576 rows
  // (x and the per-chunk setup amortize over more rows once the grid is
  // large), 1 below 4096 rows so small matrices still spread over the CUs.
  // One plain matrix at M = 1 whose two-row waves share x through LDS (from
  // 10240 rows, launch_ord) keeps two rows up to 65536 rows (N = 28672:
  // 14.1 -> 13.1-13.7 us).
  const int64_t rows = static_cast<int64_t>(a.glu ? 2 * a.N : a.N) * a.nbatch;
  const bool mapped = a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr;
  const bool shared_x = !a.glu && a.M == 1 && a.nbatch == 1 && !mapped && a.mode == AFFINE;
  int rb = rows >= (shared_x ? 65536 : 24576) ? 4 : rows >= 4096 ? 2 : 1;
  if (CPL >= 4 && rb > 2) rb = 2;
  if (a.glu && rb < 2) rb = 2;  // a gate row and its up row per output
  switch (rb) {
    case 4: return launch_ord<XT, 4, CPL>(a);
    case 2: return launch_ord<XT, 2, CPL>(a);
    default: return launch_ord<XT, 1, CPL>(a);
  }
}

// K >= 10240 (more than four chunks per lane): four waves split each row
// and every workgroup takes four rows (N = 4096, K = 14336: 11.3 -> 9.7 us;
// N = 2048, K = 16384: 8.9 -> 6.7 us), so the rows' loads are spread over
// 4x more waves and each wave keeps one or two chunks per row
template <int XT>
hipError_t launch_ks(const QmmArgs& a) {
  return ((a.K >> 5) + 255) / 256 == 1 ? launch_ord<XT, 4, 1, 4>(a) : launch_ord<XT, 4, 2, 4>(a);
}

template <int XT>
hipError_t launch_xt(const QmmArgs& a) {
  if (((a.K >> 5) + 63) / 64 >= 5) return launch_ks<XT>(a);
  switch (((a.K >> 5) + 63) / 64) {
    case 1: return launch_ord_cpl<XT, 1>(a);
    case 2: return launch_ord_cpl<XT, 2>(a);
    case 3: return launch_ord_cpl<XT, 3>(a);
    default: return launch_ord_cpl<XT, 4>(a);
  }
}
}  // namespace

hipError_t launch_qmv_q4_m1(const QmmArgs& a) {
  return a.xdt == BF16 ? launch_xt<BF16>(a) : launch_xt<F16>(a);
}

}  // namespace iqmm

// ---------------------------------------------------------------------------
// M = 1 GEMV for 8-bit codes: affine 8-bit and mxfp8 (transpose).  Same load
// plan as the 4-bit kernel, in 16-code half chunks: lane l owns half chunks
// l, l + 64, ... of every row, so each weight load is a contiguous 1 KiB per
// wave, and every load is issued before any arithmetic.  x (cache-resident)
// is converted to fp32 once per lane and shared by the RB rows; a code becomes
// fp32 with one v_cvt_f32_ubyte (affine) or a 16-bit e4m3 -> fp16 bit move and
// v_cvt_f32_f16 (mxfp8: e4m3 / 256 exactly; the 256 is folded into the group
// scale).  Affine groups are rescaled per half chunk as s . sum x q + b . sum x.
namespace iqmm {

template <int XT, int RB, int HPL, int MODE>
__global__ __launch_bounds__(64) void qmv_q8_kernel(Q4Args p) {
  using XS = uint16_t;
  constexpr bool AFF = MODE == AFFINE;
  const int lane = threadIdx.x;
  const int N = p.N, K = p.K, H = K >> 4;
  XS* out = reinterpret_cast<XS*>(p.out);
  const int row0 = blockIdx.x * RB;
  const uint32_t wrow = static_cast<uint32_t>(K);
  const uint32_t srow = AFF ? (static_cast<uint32_t>(K) >> p.gshift) * 2 : static_cast<uint32_t>(K) >> 5;

  uint32_t hw[HPL], hx[HPL], hg[HPL];
#pragma unroll
  for (int j = 0; j < HPL; ++j) {
    const uint32_t h = static_cast<uint32_t>(min(lane + 64 * j, H - 1));
    hw[j] = h << 4;
    hx[j] = h << 5;
    hg[j] = AFF ? ((h << 4) >> p.gshift) * 2 : (h >> 1);
  }
  // 1. x half chunks (16 values, 32 bytes) first
  u32x4_t xv[HPL][2];
#pragma unroll
  for (int j = 0; j < HPL; ++j)
#pragma unroll
    for (int i = 0; i < 2; ++i) xv[j][i] = *reinterpret_cast<const u32x4_t*>(p.x + hx[j] + 16 * i);
  // 2. per row: weight half chunks, then scales / biases
  u32x4_t wv[RB][HPL];
  XS sr[RB][HPL], br[RB][HPL];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint32_t row = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(min(row0 + r, N - 1)));
    const char* wr = p.w + row * wrow;
#pragma unroll
    for (int j = 0; j < HPL; ++j) wv[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wr + hw[j]));
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
      if constexpr (AFF) {
        sr[r][j] = *reinterpret_cast<const XS*>(p.s + row * srow + hg[j]);
        br[r][j] = *reinterpret_cast<const XS*>(p.b + row * srow + hg[j]);
      } else {
        sr[r][j] = *reinterpret_cast<const uint8_t*>(p.s + row * srow + hg[j]);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // 3. x to fp32 (and its half-chunk sums for the affine bias term)
  float xf[HPL][16], xsum[HPL];
#pragma unroll
  for (int j = 0; j < HPL; ++j) {
    const uint32_t w8[8] = {xv[j][0].x, xv[j][0].y, xv[j][0].z, xv[j][0].w,
                            xv[j][1].x, xv[j][1].y, xv[j][1].z, xv[j][1].w};
    float sacc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xf[j][2 * i] = to_f<XT>(static_cast<XS>(w8[i] & 0xffffu));
      xf[j][2 * i + 1] = to_f<XT>(static_cast<XS>(w8[i] >> 16));
      sacc += xf[j][2 * i] + xf[j][2 * i + 1];
    }
    xsum[j] = lane + 64 * j < H ? sacc : 0.f;
  }
  // 4. rows in load order
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
      const uint32_t wd[4] = {wv[r][j].x, wv[r][j].y, wv[r][j].z, wv[r][j].w};
      float d = 0.f;
      bool nan = false;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (AFF) {
          d = fmaf(xf[j][4 * q + 0], ubyte_f<0>(wd[q]), d);
          d = fmaf(xf[j][4 * q + 1], ubyte_f<1>(wd[q]), d);
          d = fmaf(xf[j][4 * q + 2], ubyte_f<2>(wd[q]), d);
          d = fmaf(xf[j][4 * q + 3], ubyte_f<3>(wd[q]), d);
        } else {
          // bytes 0, 2 and 1, 3 spread to 16-bit lanes: e4m3 -> fp16 bits of e4m3 / 256
          const uint32_t even = wd[q] & 0x00ff00ffu, odd = (wd[q] >> 8) & 0x00ff00ffu;
          const uint32_t he = ((even & 0x007f007fu) << 7) | ((even & 0x00800080u) << 8);
          const uint32_t ho = ((odd & 0x007f007fu) << 7) | ((odd & 0x00800080u) << 8);
          d = fmaf(xf[j][4 * q + 0], h_to_f(static_cast<uint16_t>(he)), d);
          d = fmaf(xf[j][4 * q + 1], h_to_f(static_cast<uint16_t>(ho)), d);
          d = fmaf(xf[j][4 * q + 2], h_to_f(static_cast<uint16_t>(he >> 16)), d);
          d = fmaf(xf[j][4 * q + 3], h_to_f(static_cast<uint16_t>(ho >> 16)), d);
          // S.1111.111 codes are NaN
          nan = nan || ((((wd[q] & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u) != 0u);
        }
      }
      if (lane + 64 * j >= H) d = 0.f;
      if constexpr (AFF) {
        acc = fmaf(to_f<XT>(sr[r][j]), d, fmaf(to_f<XT>(br[r][j]), xsum[j], acc));
      } else {
        const float sc = fp_scale<MODE>(sr[r][j]) * 256.0f;
        acc = fmaf(sc, nan && lane + 64 * j < H ? __builtin_nanf("") : d, acc);
      }
    }
    const float v = dpp_sum_to_lane63(acc);
    if (lane == 63 && row0 + r < N) out[row0 + r] = from_f<XT>(v);
  }
}


bool qmv_lb_m1_supported(const QmmArgs& a) {
  // M = 1, affine 2 / 3 / 6-bit, K in [1024, 16384] (one to eight chunks per
  // lane), one matrix below 4 GiB of codes
  return a.transpose && a.M == 1 && !a.glu && a.mode == AFFINE && (a.bits == 2 || a.bits == 3 || a.bits == 6) &&
         (a.xdt == BF16 || a.xdt == F16) && a.nbatch == 1 && a.bm.ndim == 0 && a.bm.lhs == nullptr &&
         a.bm.rhs == nullptr && a.K % 32 == 0 && a.K >= 1024 && a.K <= 16384 &&
         static_cast<int64_t>(a.N) * a.K / 8 * a.bits < (int64_t{1} << 32);
}

namespace {
template <int XT, int BITS, int CPL>
hipError_t lb_launch(const QmmArgs& a, const Q4Args& p) {
  // two rows per wave from 4096 rows (as the 4-bit kernel), one below
  if (a.N >= 4096) {
    hipLaunchKernelGGL((qmv_lb_kernel<XT, BITS, 2, CPL>), dim3(static_cast<unsigned>((a.N + 1) / 2)), dim3(64), 0,
                       a.stream, p);
  } else {
    hipLaunchKernelGGL((qmv_lb_kernel<XT, BITS, 1, CPL>), dim3(static_cast<unsigned>(a.N)), dim3(64), 0, a.stream, p);
  }
  return hipGetLastError();
}
template <int XT, int BITS>
hipError_t lb_cpl(const QmmArgs& a, const Q4Args& p) {
  switch (((a.K >> 5) + 63) / 64) {
    case 1: return lb_launch<XT, BITS, 1>(a, p);
    case 2: return lb_launch<XT, BITS, 2>(a, p);
    case 3: return lb_launch<XT, BITS, 3>(a, p);
    case 4: return lb_launch<XT, BITS, 4>(a, p);
    case 5: case 6: return lb_launch<XT, BITS, 6>(a, p);
    default: return lb_launch<XT, BITS, 8>(a, p);
  }
}
template <int XT>
hipError_t lb_bits(const QmmArgs& a, const Q4Args& p) {
  if (a.bits == 2) return lb_cpl<XT, 2>(a, p);
  if (a.bits == 3) return lb_cpl<XT, 3>(a, p);
  return lb_cpl<XT, 6>(a, p);
}
}  // namespace

hipError_t launch_qmv_lb_m1(const QmmArgs& a) {
  if (a.N <= 0) return hipSuccess;
  Q4Args p;
  p.x = static_cast<const char*>(a.x);
  p.w = reinterpret_cast<const char*>(a.w);
  p.s = static_cast<const char*>(a.s);
  p.b = static_cast<const char*>(a.b);
  p.out = static_cast<char*>(a.out);
  p.N = a.N;
  p.K = a.K;
  p.gshift = __builtin_ctz(a.gs);
  p.pad = 0;
  p.x_mat = p.w_mat = p.s_mat = 0;
  return a.xdt == BF16 ? lb_bits<BF16>(a, p) : lb_bits<F16>(a, p);
}

bool qmv_q8_m1_supported(const QmmArgs& a) {
  // 1..8 half chunks per lane (K in [1024, 8192], K % 16 == 0); one matrix below 4 GiB
  const bool mode_ok = (a.mode == AFFINE && a.bits == 8) || a.mode == MXFP8;
  return a.transpose && a.M == 1 && !a.glu && mode_ok && (a.xdt == BF16 || a.xdt == F16) && a.nbatch == 1 &&
         a.bm.ndim == 0 && a.bm.lhs == nullptr && a.bm.rhs == nullptr && a.K % 16 == 0 && a.K >= 1024 &&
         a.K <= 8192 && static_cast<int64_t>(a.N) * a.K < (int64_t{1} << 32);
}

namespace {
template <int XT, int RB, int HPL>
hipError_t q8_launch(const QmmArgs& a, const Q4Args& p) {
  const dim3 grid(static_cast<unsigned>((a.N + RB - 1) / RB));
  if (a.mode == MXFP8) hipLaunchKernelGGL((qmv_q8_kernel<XT, RB, HPL, MXFP8>), grid, dim3(64), 0, a.stream, p);
  else hipLaunchKernelGGL((qmv_q8_kernel<XT, RB, HPL, AFFINE>), grid, dim3(64), 0, a.stream, p);
  return hipGetLastError();
}
template <int XT>
hipError_t q8_launch_x(const QmmArgs& a, const Q4Args& p) {
  // rows per wave as the 4-bit kernel: 2 from 4096 rows, 1 below
  const bool two = a.N >= 4096;
  switch ((((a.K >> 4) + 63) / 64 + 1) / 2 * 2) {  // half chunks per lane, rounded up to even
    case 2: return two ? q8_launch<XT, 2, 2>(a, p) : q8_launch<XT, 1, 2>(a, p);
    case 4: return two ? q8_launch<XT, 2, 4>(a, p) : q8_launch<XT, 1, 4>(a, p);
    case 6: return two ? q8_launch<XT, 2, 6>(a, p) : q8_launch<XT, 1, 6>(a, p);
    default: return two ? q8_launch<XT, 2, 8>(a, p) : q8_launch<XT, 1, 8>(a, p);
  }
}
}  // namespace

hipError_t launch_qmv_q8_m1(const QmmArgs& a) {
  if (a.N <= 0) return hipSuccess;
  Q4Args p{};
  p.x = static_cast<const char*>(a.x);
  p.w = reinterpret_cast<const char*>(a.w);
  p.s = static_cast<const char*>(a.s);
  p.b = static_cast<const char*>(a.b);
  p.out = static_cast<char*>(a.out);
  p.N = a.N;
  p.K = a.K;
  p.gshift = a.mode == AFFINE ? __builtin_ctz(a.gs) : 0;
  return a.xdt == BF16 ? q8_launch_x<BF16>(a, p) : q8_launch_x<F16>(a, p);
}

}  // namespace iqmm
