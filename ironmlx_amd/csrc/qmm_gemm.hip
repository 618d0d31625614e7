// qmm_gemm.hip — prefill-shaped quantized matmul on CDNA4 matrix cores.
//
// out[M, N] = x[M, K] . deq(W)^T  (transpose)  or  x . deq(W)  (!transpose),
// x bf16 or fp16, fp32 accumulation.  Reference op: mlx/src/ops.rs:695-727
// at prefill (x = [1, L, K], mlx/src/generate/mod.rs:76-80).
//
// Three kernels, all with 256 x 256 output tiles and fp32 accumulation in
// v_mfma_f32_32x32x16_{bf16,f16}:
//   - register-B kernel (transpose, 4- and 8-bit codes, K % 128 == 0 and the
//     group count a multiple of one scale chunk): the prefill path;
//   - eight-wave DMA kernel (other transposed shapes): dequantized W shared
//     through an LDS ring;
//   - register-staged kernel (transpose = false).
// Affine 2 / 3 / 5 / 6-bit codes of one weight matrix are first widened to 4 /
// 8-bit codes (widen_codes_kernel) and take the register-B kernel.
// Dequantization uses the arithmetic of `dequantize` (s * q + b, or the fp
// element times its scale) rounded once to x's 16-bit type.

#include <stdlib.h>

#include <algorithm>
#include <atomic>

#include <type_traits>

#include "launch.h"
#include "mfma_common.h"

namespace iqmm {

namespace {
constexpr int GBM = 256, GBN = 256, GBK = 64;

}  // namespace

// ---------------------------------------------------------------------------
// Register-staged kernel (transpose=false, and shapes the DMA kernel does not
// take): the next step's x tile and packed W tile are fetched into registers
// during the current step's MFMAs, then written (W dequantized) into the other
// of two padded LDS stages.
constexpr int RLD = GBK + 8;  // padded row pitch (elements)
constexpr size_t REG_LDS_BYTES = 2ull * 2 * GBM * RLD * sizeof(uint16_t);

template <int XT, int MODE, int BITS, bool TRANS>
__global__ __launch_bounds__(256, 1) void qmm_gemm_reg_kernel(QmmArgs a, int ntm, int ntn) {
  using XS = uint16_t;
  constexpr bool AFF = MODE == AFFINE;
  extern __shared__ __attribute__((aligned(16))) uint16_t glds[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int M = a.M, N = a.N, K = a.K;
  const int nblk = ntm * ntn;
  int bid = blockIdx.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int tm = bid % ntm, tn = bid / ntm;
  const int m0 = tm * GBM, n0 = tn * GBN;
  const int64_t bb = blockIdx.y;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;
  int64_t xb = 0, wb = 0;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      for (int i = t; i < GBM * GBN; i += 256) {
        const int r = m0 + i / GBN, c = n0 + i % GBN;
        if (r < M && c < N) out[static_cast<int64_t>(r) * N + c] = from_f<XT>(__builtin_nanf(""));
      }
      return;
    }
  }
  const XS* x = static_cast<const XS*>(a.x) + xb * a.x_mat;
  const uint32_t* w = a.w + wb * a.w_mat;
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const XS* sp = static_cast<const XS*>(a.s) + wb * a.s_mat;
  const XS* bp = AFF ? static_cast<const XS*>(a.b) + wb * a.s_mat : nullptr;
  const uint8_t* s8 = static_cast<const uint8_t*>(a.s) + wb * a.s_mat;
  auto As = [&](int st) { return glds + st * (GBM + GBN) * RLD; };
  auto Bs = [&](int st) { return glds + st * (GBM + GBN) * RLD + GBM * RLD; };

  g_u32x4_t ar[8];
  uint32_t wr[2][BITS];
  float sr[2], br[2], sr2[2];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = t + 256 * i, r = idx >> 3, cv = (idx & 7) * 8;
      const int gm = m0 + r, gk = k0 + cv;
      ar[i] = (gm < M && gk < K)
                  ? *reinterpret_cast<const g_u32x4_t*>(x + static_cast<int64_t>(gm) * K + gk)
                  : g_u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      int gn, gk;
      if constexpr (TRANS) {
        gn = n0 + 128 * p + (t >> 1);
        gk = k0 + 32 * (t & 1);
      } else {
        const int idx = t + 256 * p;
        gk = k0 + (idx >> 3);
        gn = n0 + 32 * (idx & 7);
      }
      if (gn < N && gk < K) {
        const int64_t wpr = TRANS ? static_cast<int64_t>(K) * BITS / 32 : static_cast<int64_t>(N) * BITS / 32;
        const int64_t row = TRANS ? gn : gk;
        const int col = TRANS ? gk : gn;
        load_chunk<BITS>(wr[p], w + row * wpr + (col >> 5) * BITS);
        const int G = (TRANS ? K : N) / gs;
        const int64_t gi = row * G + col / gs;
        if constexpr (AFF) {
          sr[p] = to_f<XT>(sp[gi]);
          br[p] = to_f<XT>(bp[gi]);
          sr2[p] = sr[p];
        } else {
          sr[p] = fp_scale<MODE>(s8[gi]);
          br[p] = 0.f;
          sr2[p] = MODE == NVFP4 ? fp_scale<MODE>(s8[gi + 1]) : sr[p];
        }
      } else {
#pragma unroll
        for (int i = 0; i < BITS; ++i) wr[p][i] = 0u;
        sr[p] = 0.f; br[p] = 0.f; sr2[p] = 0.f;
      }
    }
  };
  auto stash = [&](int st) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = t + 256 * i, r = idx >> 3, cv = (idx & 7) * 8;
      *reinterpret_cast<g_u32x4_t*>(&As(st)[r * RLD + cv]) = ar[i];
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      uint32_t o[16];
      dequant32<XT, MODE, BITS>(wr[p], sr[p], br[p], sr2[p], o);
      if constexpr (TRANS) {
        const int n = 128 * p + (t >> 1), kc = 32 * (t & 1);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<g_u32x4_t*>(&Bs(st)[n * RLD + kc + 8 * i]) =
              g_u32x4_t{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
      } else {
        const int idx = t + 256 * p, kk = idx >> 3, nc = 32 * (idx & 7);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          Bs(st)[(nc + 2 * i) * RLD + kk] = static_cast<uint16_t>(o[i] & 0xffffu);
          Bs(st)[(nc + 2 * i + 1) * RLD + kk] = static_cast<uint16_t>(o[i] >> 16);
        }
      }
    }
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  const int nk = (K + GBK - 1) / GBK;
  fetch(0);
  stash(0);
  __syncthreads();
  for (int ks = 0; ks < nk; ++ks) {
    const int st = ks & 1;
    const bool more = ks + 1 < nk;
    if (more) fetch((ks + 1) * GBK);
    const uint16_t* Ast = As(st);
    const uint16_t* Bst = Bs(st);
#pragma unroll
    for (int kk = 0; kk < GBK / 16; ++kk) {
      const int koff = kk * 16 + 8 * (lane >> 5);
      g_u32x4_t af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const g_u32x4_t*>(&Ast[(wm * 128 + i * 32 + (lane & 31)) * RLD + koff]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = *reinterpret_cast<const g_u32x4_t*>(&Bst[(wn * 128 + j * 32 + (lane & 31)) * RLD + koff]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32<XT>(af[i], bf[j], acc[i][j]);
    }
    if (more) stash(st ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M && col < N) out[static_cast<int64_t>(row) * N + col] = from_f<XT>(acc[i][j][v]);
      }
    }
}

// ---------------------------------------------------------------------------
// Shared pieces of the DMA kernels.  Every global read of x, packed W, scales
// and biases is an LDS DMA (global_load_lds_dword[x4]) issued several K steps
// ahead into rings, so no global data passes through registers and the only
// waits are explicit s_waitcnt vmcnt before each step's barrier.  K step
// (BK) = 32; x rows are 64 bytes (4 granules of 16 B), XOR-swizzled so the
// fragment reads of 32 consecutive rows hit distinct banks.
constexpr int DBK = 32, DEPTH = 4;
constexpr int DA_STAGE = GBM * DBK;  // elements (16 KiB)
constexpr int DB_STAGE = GBN * DBK;  // elements (16 KiB)

// granule swizzle f(row) = (row ^ (row >> 2)) & 3, chosen by measuring the
// fragment-read pattern of v_mfma_f32_32x32x16 on gfx950 (best of the XOR
// swizzles tried; unswizzled 64-byte rows run at about a third of its rate)
__device__ __forceinline__ int dswzf(int row) { return (row ^ (row >> 2)) & 3; }
__device__ __forceinline__ int dswz(int row, int k) {
  return row * DBK + ((((k >> 3) ^ dswzf(row)) & 3) << 3) + (k & 7);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) char*)(p)));
}
// lds: wave-uniform LDS byte address (forced into an SGPR for M0)
__device__ __forceinline__ void dma_x4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
__device__ __forceinline__ void dma_x1(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}

// DMA with a wave-uniform 64-bit base (SGPRs) and a 32-bit per-lane offset
__device__ __forceinline__ void dma_x4s(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}

template <int BITS, int MODE>
struct DmaCounts {
  static constexpr int WBYTES = GBN * 4 * BITS;            // packed W bytes per step
};

// ---------------------------------------------------------------------------
// Eight-wave DMA kernel: 512 threads, two waves per SIMD, each wave owning a
// 64 x 128 sub-tile (2 x 4 blocks of 32 x 32).  Per step one thread
// dequantizes 16 codes of one W row from the packed ring into a 2-stage bf16 /
// fp16 ring that all waves read; step k's MFMAs run interleaved
// (sched_group_barrier) with the dequantization of step k+1, whose packed W
// was made resident by the wait ending step k-1.  DMA instructions are spread
// round-robin over the waves; each wave waits on its own issue count.
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
    case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
    case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
    case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
    case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
    case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    case 25: asm volatile("s_waitcnt vmcnt(25)" ::: "memory"); break;
    case 26: asm volatile("s_waitcnt vmcnt(26)" ::: "memory"); break;
    case 27: asm volatile("s_waitcnt vmcnt(27)" ::: "memory"); break;
    case 28: asm volatile("s_waitcnt vmcnt(28)" ::: "memory"); break;
    case 29: asm volatile("s_waitcnt vmcnt(29)" ::: "memory"); break;
    case 30: asm volatile("s_waitcnt vmcnt(30)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
  }
}

template <int N>
__device__ __forceinline__ void wait_vmc() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <int XT, int MODE, int BITS>
__global__ __launch_bounds__(512, 1) void qmm_gemm_dma8_kernel(QmmArgs a, int ntm, int ntn, float* part) {
  using XS = uint16_t;
  using DC = DmaCounts<BITS, MODE>;
  constexpr bool AFF = MODE == AFFINE;
  constexpr int NW = 8;
  constexpr int WINSTR = 4 * BITS;   // dword DMA instructions for the packed W stage
  extern __shared__ __attribute__((aligned(16))) uint16_t glds[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave >> 1, wn = wave & 1;
  const int M = a.M, N = a.N, K = a.K;
  const int nblk = ntm * ntn;
  int bid = blockIdx.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int tm = bid % ntm, tn = bid / ntm;
  const int m0 = tm * GBM, n0 = tn * GBN;
  const int64_t bb = blockIdx.y;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;
  // split K as in the register-B kernel: [kbeg, kbeg + klen), fp32 partials
  const int KSPL = gridDim.z, kz = blockIdx.z;
  const int klen = K / KSPL, kbeg = kz * klen;
  float* pt = part + (static_cast<int64_t>(kz) * gridDim.y + bb) * M * N;
  int64_t xb = 0, wb = 0;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      for (int i = t; i < GBM * GBN; i += 512) {
        const int r = m0 + i / GBN, c = n0 + i % GBN;
        if (r < M && c < N) {
          if (KSPL == 1) out[static_cast<int64_t>(r) * N + c] = from_f<XT>(__builtin_nanf(""));
          else pt[static_cast<int64_t>(r) * N + c] = __builtin_nanf("");
        }
      }
      return;
    }
  }
  const XS* x = static_cast<const XS*>(a.x) + xb * a.x_mat;
  const uint32_t* w = a.w + wb * a.w_mat;
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const int G = K / gs;
  const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
  const char* sbase = static_cast<const char*>(a.s) + wb * a.s_mat * (AFF ? 2 : 1);
  const char* bbase = AFF ? static_cast<const char*>(a.b) + wb * a.s_mat * 2 : nullptr;

  // LDS map (bytes from glds): x ring | W-packed ring | scale ring | bias ring | deq-W ring
  constexpr int XR = 0;
  constexpr int WR = XR + DEPTH * DA_STAGE * 2;
  constexpr int SR = WR + DEPTH * DC::WBYTES;
  constexpr int BR = SR + DEPTH * GBN * 4;
  constexpr int DQ = BR + DEPTH * GBN * 4;
  char* lb = reinterpret_cast<char*>(glds);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lb));

  // ---- per-lane DMA sources at k0 = 0 (advanced by k0 each step)
  const XS* xsrc[2];
  uint32_t xdst[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rbase = (wave + NW * i) * 16;
    const int row = rbase + (lane >> 2);
    const int g = ((lane & 3) ^ dswzf(row)) & 3;
    xsrc[i] = x + static_cast<int64_t>(min(m0 + row, M - 1)) * K + kbeg + g * 8;
    xdst[i] = rbase * DBK * 2;
  }
  const int my_w = (WINSTR - wave + NW - 1) / NW;
  const int my_s = AFF ? 1 : (wave < 4 ? 1 : 0);
  const int per_step = 2 + my_w + my_s;
  const int gshift = __builtin_ctz(gs);
  // wave-uniform LDS destinations (SGPRs) and per-lane sources at k0 = 0
  uint32_t xdst_s[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) xdst_s[i] = __builtin_amdgcn_readfirstlane(lds0 + XR + xdst[i]);
  constexpr int MAXW = (WINSTR + NW - 1) / NW;
  const uint32_t* wsrc[MAXW];
  uint32_t wdst_s[MAXW];
#pragma unroll
  for (int jj = 0; jj < MAXW; ++jj) {
    const int j = min(wave + NW * jj, WINSTR - 1);
    const int idx = j * 64 + lane;
    const int row = idx / BITS, word = idx - row * BITS;
    wsrc[jj] = w + min(n0 + row, N - 1) * wpr + static_cast<int64_t>(kbeg) * BITS / 32 + word;
    wdst_s[jj] = __builtin_amdgcn_readfirstlane(lds0 + WR + j * 256);
  }
  const int srow = min(n0 + (wave & 3) * 64 + lane, N - 1);
  const char* ssrc = ((AFF && wave >= 4) ? bbase : sbase) +
                     (static_cast<int64_t>(srow) * G + (kbeg >> gshift)) * (AFF ? 2 : 1);
  const uint32_t sdst_s = __builtin_amdgcn_readfirstlane(lds0 + (AFF && wave >= 4 ? BR : SR) + (wave & 3) * 256);

  auto issue = [&](int ks, auto slot_c) {
    constexpr int SL = decltype(slot_c)::value;
    const int k0 = ks * DBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) dma_x4(xsrc[i] + k0, xdst_s[i] + SL * DA_STAGE * 2);
#pragma unroll
    for (int jj = 0; jj < MAXW; ++jj)
      if (jj < my_w) dma_x1(wsrc[jj] + (k0 >> 5) * BITS, wdst_s[jj] + SL * DC::WBYTES);
    if (my_s) {
      const int g = k0 >> gshift;
      const int ge = AFF ? (g & ~1) : (g & ~3);
      dma_x1(ssrc + ge * (AFF ? 2 : 1), sdst_s + SL * GBN * 4);
    }
  };

  // thread t dequantizes codes [16 h, 16 h + 16) of W row t / 2 (h = t & 1)
  const int dn = t >> 1, dh = t & 1;
  int dqoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) dqoff[i] = dswz(dn, 16 * dh + 8 * i) * 2;
  auto dequant = [&](int ks, auto slot_c, auto dst_c) {
    constexpr int SL = decltype(slot_c)::value, DS = decltype(dst_c)::value;
    const int k0 = ks * DBK;
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(lb + WR + SL * DC::WBYTES) + dn * BITS;
    const int g = k0 >> gshift;
    const uint32_t sw = reinterpret_cast<const uint32_t*>(lb + SR + SL * GBN * 4)[dn];
    float sv, bv = 0.f;
    if constexpr (AFF) {
      const uint32_t bw = reinterpret_cast<const uint32_t*>(lb + BR + SL * GBN * 4)[dn];
      sv = to_f<XT>(static_cast<uint16_t>((g & 1) ? (sw >> 16) : (sw & 0xffffu)));
      bv = to_f<XT>(static_cast<uint16_t>((g & 1) ? (bw >> 16) : (bw & 0xffffu)));
    } else {
      const int gg = MODE == NVFP4 ? g + dh : g;
      sv = fp_scale<MODE>((sw >> (8 * (gg & 3))) & 0xffu);
    }
    uint32_t o[8];
    if constexpr (AFF && BITS == 4) {
      const uint2 wd2 = *reinterpret_cast<const uint2*>(wp + 2 * dh);
      const uint32_t wdq[2] = {wd2.x, wd2.y};
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t lo = wdq[q] & 0x0F0F0F0Fu, hi = (wdq[q] >> 4) & 0x0F0F0F0Fu;
        o[4 * q + 0] = pack2<XT>(fmaf(sv, ubyte_f<0>(lo), bv), fmaf(sv, ubyte_f<0>(hi), bv));
        o[4 * q + 1] = pack2<XT>(fmaf(sv, ubyte_f<1>(lo), bv), fmaf(sv, ubyte_f<1>(hi), bv));
        o[4 * q + 2] = pack2<XT>(fmaf(sv, ubyte_f<2>(lo), bv), fmaf(sv, ubyte_f<2>(hi), bv));
        o[4 * q + 3] = pack2<XT>(fmaf(sv, ubyte_f<3>(lo), bv), fmaf(sv, ubyte_f<3>(hi), bv));
      }
    } else {
      uint32_t wd[BITS];
#pragma unroll
      for (int i = 0; i < BITS; ++i) wd[i] = wp[i];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v[2];
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
          const uint32_t qc = chunk_code<BITS>(wd, 16 * dh + 2 * i + e2);
          if constexpr (AFF) v[e2] = fmaf(sv, static_cast<float>(qc), bv);
          else v[e2] = fp_elem<MODE>(qc) * sv;
        }
        o[i] = pack2<XT>(v[0], v[1]);
      }
    }
    char* B = lb + DQ + DS * DB_STAGE * 2;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<g_u32x4_t*>(B + dqoff[i]) = g_u32x4_t{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
  };

  // fragment offsets (bytes within a stage) for both 16-k halves of a step
  int offA[2][2], offB[2][4];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int kq = kk * 16 + 8 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < 2; ++i) offA[kk][i] = dswz(wm * 64 + i * 32 + (lane & 31), kq) * 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) offB[kk][j] = dswz(wn * 128 + j * 32 + (lane & 31), kq) * 2;
  }

  f32x16_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  auto mfma_step = [&](auto sa_c, auto sb_c) {
    constexpr int SA = decltype(sa_c)::value, SB = decltype(sb_c)::value;
    const char* Ast = lb + XR + SA * DA_STAGE * 2;
    const char* Bst = lb + DQ + SB * DB_STAGE * 2;
    g_u32x4_t af[2][2], bf[2][4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int i = 0; i < 2; ++i) af[kk][i] = *reinterpret_cast<const g_u32x4_t*>(Ast + offA[kk][i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[kk][j] = *reinterpret_cast<const g_u32x4_t*>(Bst + offB[kk][j]);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32<XT>(af[kk][i], bf[kk][j], acc[i][j]);
  };

  const int nk = klen / DBK;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  if (nk > 0) issue(0, I0{});
  if (nk > 1) issue(1, I1{});
  if (nk > 2) issue(2, I2{});
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  dequant(0, I0{}, I0{});
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // one K step: DMA step ks+3 into slot (ks+3)%4, MFMA on slot ks%4 / deq ks%2,
  // dequantize step ks+1 (slot (ks+1)%4) into deq (ks+1)%2
  auto step = [&](int ks, auto sa_c, auto sdq_c, auto snext_c, auto sissue_c) {
    const bool pre = ks + DEPTH - 1 < nk;
    if (pre) issue(ks + DEPTH - 1, sissue_c);
    mfma_step(sa_c, sdq_c);
    if (ks + 1 < nk) dequant(ks + 1, snext_c, std::integral_constant<int, 1 - decltype(sdq_c)::value>{});
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      if (g % 4 == 3) __builtin_amdgcn_sched_group_barrier(0x300, 2, 0);
    }
    if (ks + 2 < nk && pre) wait_vm(per_step);
    else wait_vm(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  for (int ks = 0; ks < nk; ks += 4) {
    step(ks, I0{}, I0{}, I1{}, I3{});
    if (ks + 1 < nk) step(ks + 1, I1{}, I1{}, I2{}, I0{});
    if (ks + 2 < nk) step(ks + 2, I2{}, I0{}, I3{}, I1{});
    if (ks + 3 < nk) step(ks + 3, I3{}, I1{}, I0{}, I2{});
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M && col < N) {
          if (KSPL == 1) out[static_cast<int64_t>(row) * N + col] = from_f<XT>(acc[i][j][v]);
          else pt[static_cast<int64_t>(row) * N + col] = acc[i][j][v];
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Register-B kernel (4- and 8-bit codes).  Wave w owns the 256 x 32 column
// strip [32 w, 32 w + 32) of the tile, so its B operand is private: each lane
// dequantizes its two 32x32x16 B fragments straight from the packed ring into
// registers one step ahead of the MFMAs, and x is the only operand read from
// LDS per MFMA.
//
// Loads are sized by cache-line requests, which bound the DMA rate: x comes
// per step (256 rows x 64 B), packed W in chunks of WC steps (64 B per row:
// 4 steps at 4 bits, 2 at 8 bits) and scales / biases in chunks of 16 bytes
// per row (8 bf16/fp16 groups, or 16 one-byte MX / NV groups), all as
// 16-byte-per-lane DMAs.  The k order inside a step is permuted identically
// for both operands: lane half h of fragment kk covers k = 16 h + 8 kk .. +8,
// which is packed word 2 h + kk at 4 bits, so a lane's B codes are one
// contiguous 8- or 16-byte read.
template <int BITS>
struct WrCfg {
  static constexpr int STEP_B = 4 * BITS;          // packed bytes per row per step
  static constexpr int WC = 64 / STEP_B;           // steps per W chunk
  static constexpr int WSLOT = GBN * 64;           // bytes per W chunk slot
  // chunk slots: a slot is refilled WD-1 = 5 steps before its chunk starts,
  // which must come after the last read of the chunk it held: (WSL-1) WC > 3
  static constexpr int WSL = BITS == 4 ? 2 : 3;
};

// Tile order: workgroup ids are first made contiguous per XCD (the hardware
// deals consecutive ids round-robin over the 8 XCDs), then walked in groups of
// GM row tiles, m fastest, so each XCD's L2 holds a GM-tile strip of x and the
// W column tiles in flight.
template <int GM>
__device__ __forceinline__ void tile_of(int bid, int ntm, int ntn, int& tm, int& tn) {
  const int nblk = ntm * ntn;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int per = GM * ntn;
  const int grp = bid / per, first = grp * GM;
  const int gsz = min(ntm - first, GM);
  const int r = bid - grp * per;
  tm = first + r % gsz;
  tn = r / gsz;
}

template <int XT, int MODE, int BITS, int WD, int TM, int TN>
__global__ __launch_bounds__(2 * TN, 1) void qmm_gemm_wr_kernel(QmmArgs a, int ntm, int ntn, float* part) {
  static_assert(BITS == 4 || BITS == 8, "register-B kernel takes 4- and 8-bit codes");
  static_assert(WD % 2 == 0 && WD >= 4, "B double buffer alternates with the x slot");
  using XS = uint16_t;
  using CF = WrCfg<BITS>;
  constexpr bool AFF = MODE == AFFINE;
  // tile TM x TN; wave w owns the TM x 32 column strip [32 w, 32 w + 32)
  constexpr int NW = TN / 32, NT = 64 * NW, RB = TM / 32, NCB = 1;
  constexpr int XI = TM / 16 / NW;      // x DMA instructions per wave (16 rows each)
  constexpr int WI = 2;                 // W-chunk DMA instructions per wave (TN / 16 over NW)
  constexpr int SQ = (TN / 64) * (AFF ? 2 : 1);  // scale(+bias)-chunk instructions
  constexpr int SW = SQ < NW ? SQ : NW;          // waves issuing them, SI each
  constexpr int SI = SQ / SW;
  static_assert(XI >= 1 && XI * 16 * NW == TM && SI * SW == SQ, "tile / wave split");
  constexpr int GPC = AFF ? 8 : 16;  // groups per 16-byte scale chunk row
  constexpr int XSTAGE = TM * DBK * 2;  // bytes of one x stage
  constexpr int WSLOT = TN * 64;        // bytes of one W chunk slot
  extern __shared__ __attribute__((aligned(16))) uint16_t glds[];
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: keeps DMA counts scalar
  const int wn = wave, wm = 0;
  const int M = a.M, N = a.N, K = a.K;
  int tm, tn;
  tile_of<4>(blockIdx.x, ntm, ntn, tm, tn);
  const int m0 = tm * TM, n0 = tn * TN;
  // split K: this workgroup takes [kbeg, kbeg + klen); with more than one
  // split the fp32 partial tile goes to part[z] and a second pass sums them
  const int KSPL = gridDim.z, kz = blockIdx.z;
  const int klen = K / KSPL, kbeg = kz * klen;
  const int64_t bb = blockIdx.y;
  XS* out = static_cast<XS*>(a.out) + bb * static_cast<int64_t>(M) * N;
  int64_t xb = 0, wb = 0;
  if (a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr) {
    if (!map_batch(a.bm, bb, xb, wb)) {
      for (int i = t; i < TM * TN; i += NT) {
        const int r = m0 + i / TN, c = n0 + i % TN;
        if (r < M && c < N) {
          if (KSPL == 1) out[static_cast<int64_t>(r) * N + c] = from_f<XT>(__builtin_nanf(""));
          else part[((static_cast<int64_t>(kz) * gridDim.y + bb) * M + r) * N + c] = __builtin_nanf("");
        }
      }
      return;
    }
  }
  const XS* x = static_cast<const XS*>(a.x) + xb * a.x_mat;
  const char* w = reinterpret_cast<const char*>(a.w + wb * a.w_mat);
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const int G = K / gs;
  const int64_t wrow = static_cast<int64_t>(K) * BITS / 8;   // packed bytes per W row
  const int ssz = AFF ? 2 : 1;                               // bytes per scale
  const char* sbase = static_cast<const char*>(a.s) + wb * a.s_mat * ssz;
  const char* bbase = AFF ? static_cast<const char*>(a.b) + wb * a.s_mat * 2 : nullptr;

  // LDS map (bytes from glds): x ring (WD) | W chunk ring (WSL) | scale ring (2) | bias ring (2)
  constexpr int XR = 0;
  constexpr int WR = XR + WD * XSTAGE;
  constexpr int SR = WR + CF::WSL * WSLOT;
  constexpr int SSLOT = TN * 16;
  constexpr int BR = SR + 2 * SSLOT;
  char* lb = reinterpret_cast<char*>(glds);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lb));

  // ---- DMA: wave-uniform bases (SGPRs, advanced per step) + per-lane 32-bit
  // offsets within the tile, and wave-uniform LDS destinations
  const char* xtile = reinterpret_cast<const char*>(x + static_cast<int64_t>(m0) * K + kbeg);
  uint32_t xoff[XI], xdst_s[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int rbase = (wave + NW * i) * 16;
    const int row = rbase + (lane >> 2);
    const int g = ((lane & 3) ^ dswzf(row)) & 3;
    xoff[i] = static_cast<uint32_t>((min(m0 + row, M - 1) - m0) * K * 2 + g * 16);
    xdst_s[i] = __builtin_amdgcn_readfirstlane(lds0 + XR + rbase * DBK * 2);
  }
  // W chunk: TN rows x 4 granules = TN / 16 instructions; stored granule p
  // of row r holds logical granule p ^ f(r)
  const char* wtile = w + static_cast<int64_t>(n0) * wrow + static_cast<int64_t>(kbeg) * BITS / 8;
  uint32_t woff[WI], wdst_s[WI];
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int j = wave + NW * i;
    const int row = j * 16 + (lane >> 2);
    const int g = ((lane & 3) ^ dswzf(row)) & 3;
    woff[i] = static_cast<uint32_t>((min(n0 + row, N - 1) - n0) * wrow + g * 16);
    wdst_s[i] = __builtin_amdgcn_readfirstlane(lds0 + WR + j * 1024);
  }
  // scale chunk: 64 rows x 16 B per instruction; TN / 64 instructions of
  // scales (+ as many of biases), instruction q = wave + NW i on waves < SW
  constexpr int SQR = TN / 64;
  const int my_s = wave < SW ? SI : 0;
  const int gshift = __builtin_ctz(gs);
  const char* stile[SI];
  uint32_t soff[SI], sdst_s[SI];
#pragma unroll
  for (int i = 0; i < SI; ++i) {
    const int q = min(wave + NW * i, SQ - 1);
    const bool isb = AFF && q >= SQR;
    const int qr = isb ? q - SQR : q;
    const int srow = min(n0 + qr * 64 + lane, N - 1);
    stile[i] = (isb ? bbase : sbase) + (static_cast<int64_t>(n0) * G + (kbeg >> gshift)) * ssz;
    soff[i] = static_cast<uint32_t>((srow - n0) * G * ssz);
    sdst_s[i] = __builtin_amdgcn_readfirstlane(lds0 + (isb ? BR : SR) + qr * 1024);
  }
  // steps per scale chunk (P = GPC * gs / 32 >= 8)
  const int pshift = __builtin_ctz(GPC) + gshift - 5;
  constexpr int WCS = BITS == 4 ? 2 : 1;  // log2(WC)

  // DMAs for step j into x slot SL; W chunk when j % WC == 0 (compile-time
  // in the unrolled loop), scale chunk when j % P == 0
  auto issue = [&](int j, auto slot_c, auto wchunk_c) {
    constexpr int SL = decltype(slot_c)::value;
    constexpr bool WCH = decltype(wchunk_c)::value;
    const int k0 = j * DBK;
    const char* xk = xtile + k0 * 2;
#pragma unroll
    for (int i = 0; i < XI; ++i) dma_x4s(xoff[i], xk, xdst_s[i] + SL * XSTAGE);
    if constexpr (WCH) {
      const uint32_t wsl = ((j >> WCS) % CF::WSL) * WSLOT;
      const char* wk = wtile + (k0 >> 5) * CF::STEP_B;
#pragma unroll
      for (int i = 0; i < WI; ++i) dma_x4s(woff[i], wk, wdst_s[i] + wsl);
    }
    if ((j & ((1 << pshift) - 1)) == 0 && my_s) {
      const int g0 = k0 >> gshift;
#pragma unroll
      for (int i = 0; i < SI; ++i) dma_x4s(soff[i], stile[i] + g0 * ssz, sdst_s[i] + ((j >> pshift) & 1) * SSLOT);
    }
  };

  // ---- B fragments of step ks for column cn of the tile
  auto deq_b = [&](int ks, int cb, g_u32x4_t (&bo)[2]) {
    const int cn = 32 * (NCB * wn + cb) + (lane & 31);
    const int wsw = dswzf(cn);
    const int g = (ks * DBK) >> gshift;
    const char* ch = lb + WR + ((ks >> WCS) % CF::WSL) * WSLOT;
    const char* sc = lb + ((ks >> pshift) & 1) * SSLOT + cn * 16;
    const int gi = g & (GPC - 1);
    float sv[2], bv = 0.f;
    if constexpr (AFF) {
      sv[0] = sv[1] = to_f<XT>(*reinterpret_cast<const uint16_t*>(sc + SR + gi * 2));
      bv = to_f<XT>(*reinterpret_cast<const uint16_t*>(sc + BR + gi * 2));
    } else {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        // nvfp4: 16-wide groups; fragment kk of half h covers k 16 h + 8 kk
        const int gg = MODE == NVFP4 ? gi + h : gi;
        sv[kk] = fp_scale<MODE>(*reinterpret_cast<const uint8_t*>(sc + SR + gg));
      }
    }
    uint32_t wv[4];
    if constexpr (BITS == 4) {
      const int gr = (ks & 3) ^ wsw;
      const uint2 d = *reinterpret_cast<const uint2*>(ch + cn * 64 + gr * 16 + 8 * h);
      wv[0] = d.x; wv[1] = d.y;
    } else {
      const int gr = ((2 * (ks & 1) + h) ^ wsw) & 3;
      const g_u32x4_t d = *reinterpret_cast<const g_u32x4_t*>(ch + cn * 64 + gr * 16);
      wv[0] = d[0]; wv[1] = d[1]; wv[2] = d[2]; wv[3] = d[3];
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      uint32_t o[4];
      if constexpr (BITS == 4) {
        const uint32_t lo = wv[kk] & 0x0F0F0F0Fu, hi = (wv[kk] >> 4) & 0x0F0F0F0Fu;
        if constexpr (AFF) {
          o[0] = pack2<XT>(fmaf(sv[kk], ubyte_f<0>(lo), bv), fmaf(sv[kk], ubyte_f<0>(hi), bv));
          o[1] = pack2<XT>(fmaf(sv[kk], ubyte_f<1>(lo), bv), fmaf(sv[kk], ubyte_f<1>(hi), bv));
          o[2] = pack2<XT>(fmaf(sv[kk], ubyte_f<2>(lo), bv), fmaf(sv[kk], ubyte_f<2>(hi), bv));
          o[3] = pack2<XT>(fmaf(sv[kk], ubyte_f<3>(lo), bv), fmaf(sv[kk], ubyte_f<3>(hi), bv));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = pack2<XT>(fp_elem<MODE>((lo >> (8 * e)) & 0xfu) * sv[kk],
                             fp_elem<MODE>((hi >> (8 * e)) & 0xfu) * sv[kk]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t d = wv[2 * kk + (e >> 1)] >> (16 * (e & 1));
          if constexpr (AFF)
            o[e] = pack2<XT>(fmaf(sv[kk], static_cast<float>(d & 0xffu), bv),
                             fmaf(sv[kk], static_cast<float>((d >> 8) & 0xffu), bv));
          else
            o[e] = pack2<XT>(fp_elem<MODE>(d & 0xffu) * sv[kk], fp_elem<MODE>((d >> 8) & 0xffu) * sv[kk]);
        }
      }
      bo[kk] = g_u32x4_t{o[0], o[1], o[2], o[3]};
    }
  };

  // A fragment (kk, block i): rows 32 i + lane % 32, k = 16 h + 8 kk; the
  // swizzle depends on row % 32 only, so block i is +i * 32 rows.
  int offA[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) offA[kk] = dswz(lane & 31, 16 * h + 8 * kk) * 2 + wm * RB * 32 * DBK * 2;

  f32x16_t acc[RB][NCB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int c = 0; c < NCB; ++c)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][c][v] = 0.f;

  // MFMAs of one step; each A fragment register is refilled with the next
  // step's fragment (slot sn, resident since the previous barrier) right after
  // its last use, so the next step starts with its operands in flight.
  auto mfma_step = [&](const g_u32x4_t (&bf)[NCB][2], g_u32x4_t (&af)[2][RB], auto sn_c) {
    constexpr int SN = decltype(sn_c)::value;
    const char* An = lb + XR + SN * XSTAGE;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < RB; ++i) {
#pragma unroll
        for (int c = 0; c < NCB; ++c) acc[i][c] = mfma32<XT>(af[kk][i], bf[c][kk], acc[i][c]);
        af[kk][i] = *reinterpret_cast<const g_u32x4_t*>(An + offA[kk] + i * 32 * DBK * 2);
      }
  };

  // x ring of WD stages: step ks lives in slot ks % WD; DMAs run WD-1 steps
  // ahead.  Step ks dequantizes step ks+1's B and reads step ks+1's A, so the
  // wait closing step ks must leave steps ks+1 and ks+2 resident: only the
  // DMAs of steps ks+3 .. ks+WD-1 may still be in flight.  W / scale chunk
  // slots are refilled only after every reader of their previous chunk has
  // passed a barrier ((WSL - 1) WC > WD - 3 and P > WD - 3 steps).
  const int nk = klen / DBK;
  g_u32x4_t bq[2][NCB][2], af[2][RB];
  static_for<0, WD - 1>([&](auto s_c) {
    constexpr int J = decltype(s_c)::value;
    if (J < nk) issue(J, s_c, std::integral_constant<bool, J % CF::WC == 0>{});
  });
  // steps 0 and 1 resident: DMAs of steps 2 .. WD-2 may stay in flight
  {
    if (nk >= WD - 1) {
      constexpr int nx = [] {
        int n = 0;
        for (int j = 2; j <= WD - 2; ++j) n += XI + (j % CF::WC == 0 ? WI : 0);
        return n;
      }();
      wait_vmc<nx>();   // scale chunks are issued at j = 0 only within 0 .. WD-2 (P >= 8)
    } else {
      wait_vmc<0>();
    }
  }
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int c = 0; c < NCB; ++c) deq_b(0, c, bq[0][c]);
  {
    const char* Ast = lb + XR;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < RB; ++i)
        af[kk][i] = *reinterpret_cast<const g_u32x4_t*>(Ast + offA[kk] + i * 32 * DBK * 2);
  }

  // unrolled by U = lcm(WD, WC) so the x slot, the B buffer and the W-chunk
  // issue pattern are compile-time; steady-state waits are immediates.
  constexpr int U = WD % CF::WC == 0 ? WD : WD * CF::WC / (WD % CF::WC == 2 ? 2 : 1);
  static_assert(U % WD == 0 && U % CF::WC == 0, "unroll must cover both periods");
  const int pmask = (1 << pshift) - 1;
  for (int ks0 = 0; ks0 < nk; ks0 += U) {
    static_for<0, U>([&](auto s_c) {
      constexpr int S = decltype(s_c)::value;
      const int ks = ks0 + S;
      if (ks < nk) {
        const bool steady = ks + WD - 1 < nk;
        if (steady)
          issue(ks + WD - 1, std::integral_constant<int, (S + WD - 1) % WD>{},
                std::integral_constant<bool, (S + WD - 1) % CF::WC == 0>{});
#pragma unroll
        for (int c = 0; c < NCB; ++c) deq_b(ks + 1, c, bq[(S + 1) & 1][c]);
        mfma_step(bq[S & 1], af, std::integral_constant<int, (S + 1) % WD>{});
        // 256-row tiles: interleave each MFMA with one LDS read and the
        // dequantization VALU work, so the matrix pipe is fed while the next
        // step's operands are prepared (measured ~5% at M = 2048, K = 4096,
        // N = 14336; slower on 128-row tiles, which keep the compiler's order)
        if constexpr (TM == 256)
          static_for<0, 2 * RB * NCB>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
          });
        {
          if (steady) {
            // DMAs of steps ks+3 .. ks+WD-1 may stay in flight
            constexpr int nx = [] {
              int n = 0;
              for (int j = S + 3; j <= S + WD - 1; ++j) n += XI + (j % CF::WC == 0 ? WI : 0);
              return n;
            }();
            if (my_s && ((ks + WD - 1) & pmask) <= WD - 4) wait_vmc<nx + SI>();
            else wait_vmc<nx>();
          } else {
            wait_vmc<0>();  // last WD-1 steps: nothing further is issued
          }
        }
        // the A reads still in flight target slot ks+1, which no DMA issued
        // before the next barrier touches, so the barrier need not drain them
        asm volatile("s_barrier" ::: "memory");
      }
    });
  }

  if (KSPL > 1) {
    float* pt = part + (static_cast<int64_t>(kz) * gridDim.y + bb) * M * N;
    const int col = n0 + 32 * wn + (lane & 31);
    if (col < N) {
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
          if (row < M) pt[static_cast<int64_t>(row) * N + col] = acc[i][0][v];
        }
    }
    return;
  }
  if (m0 + 32 * RB * (wm + 1) <= M) {
    // full row tile: wave-uniform row bases (SGPRs) + one 32-bit lane offset
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
      const int col = n0 + 32 * (NCB * wn + c) + (lane & 31);
      const uint32_t voff = static_cast<uint32_t>((4 * h * N + col) * 2);
      if (col < N) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const XS* ub = out + static_cast<int64_t>(m0 + (RB * wm + i) * 32 + 8 * (v >> 2) + (v & 3)) * N;
            const uint32_t d = from_f<XT>(acc[i][c][v]);
            asm volatile("global_store_short %0, %1, %2" ::"v"(voff), "v"(d), "s"(ub) : "memory");
          }
      }
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < NCB; ++c) {
    const int col = n0 + 32 * (NCB * wn + c) + (lane & 31);
    if (col < N) {
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = m0 + (RB * wm + i) * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
          if (row < M) out[static_cast<int64_t>(row) * N + col] = from_f<XT>(acc[i][c][v]);
        }
    }
  }
}

template <int BITS>
constexpr size_t wr_lds_bytes(int wd, int tm, int tn) {
  return static_cast<size_t>(wd) * tm * DBK * 2 + WrCfg<BITS>::WSL * tn * 64 + 4 * tn * 16;
}

// sum of the split-K fp32 partials -> x's 16-bit type
template <int XT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, uint16_t* out, int64_t n,
                                                            int ks) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  if (i + 4 <= n) {
    float4 acc = *reinterpret_cast<const float4*>(part + i);
    for (int z = 1; z < ks; ++z) {
      const float4 v = *reinterpret_cast<const float4*>(part + z * n + i);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    out[i] = from_f<XT>(acc.x); out[i + 1] = from_f<XT>(acc.y);
    out[i + 2] = from_f<XT>(acc.z); out[i + 3] = from_f<XT>(acc.w);
  } else {
    for (int64_t j = i; j < n; ++j) {
      float acc = part[j];
      for (int z = 1; z < ks; ++z) acc += part[z * n + j];
      out[j] = from_f<XT>(acc);
    }
  }
}

// Widen packed affine codes to the register-B kernel's code widths: 2- and
// 3-bit codes to 4-bit, 5- and 6-bit codes to 8-bit (codes, scales and biases
// unchanged, so the product is the one the narrow codes define).  One thread
// per 32-code chunk (BITS words of the LSB-first row stream in, 32 * OB bits
// out); rows of K codes are whole chunks, so the matrix is one chunk sequence.
template <int BITS, int OB>
__global__ __launch_bounds__(256) void widen_codes_kernel(const uint32_t* __restrict__ w, uint32_t* __restrict__ o,
                                                          int64_t nchunks) {
  const int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (c >= nchunks) return;
  uint32_t in[BITS + 1];
#pragma unroll
  for (int i = 0; i < BITS; ++i) in[i] = __builtin_nontemporal_load(w + c * BITS + i);
  in[BITS] = 0;
  uint32_t out[OB] = {};
#pragma unroll
  for (int n = 0; n < 32; ++n) {
    const int pos = BITS * n, wi = pos >> 5, bit = pos & 31;
    const uint32_t v = bit + BITS <= 32 ? __builtin_amdgcn_ubfe(in[wi], bit, BITS)
                                        : __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(in[wi + 1], in[wi], bit), 0, BITS);
    out[(OB * n) >> 5] |= v << ((OB * n) & 31);
  }
  g_u32x4_t* dst = reinterpret_cast<g_u32x4_t*>(o + c * OB);
#pragma unroll
  for (int i = 0; i < OB / 4; ++i) dst[i] = g_u32x4_t{out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]};
}

template <int BITS, int MODE>
constexpr size_t dma_lds_bytes() {
  return DEPTH * DA_STAGE * 2 + DEPTH * DmaCounts<BITS, MODE>::WBYTES + 2 * DEPTH * GBN * 4 +
         2 * DB_STAGE * 2;
}

bool qmm_gemm_supported(const QmmArgs& a) {
  return (a.xdt == BF16 || a.xdt == F16) && a.K % 32 == 0 && (a.transpose || a.N % 32 == 0);
}

namespace {
// Raise a kernel's dynamic-LDS limit once per device; the attribute persists,
// and setting it on every launch costs host time on the launch path.
template <auto KERN>
hipError_t set_lds_once(size_t bytes) {
  static std::atomic<uint64_t> done{0};  // one bit per device id < 64
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 64;
  const uint64_t bit = dev < 64 ? (1ull << dev) : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(KERN),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

// Run `launch(part)` into an fp32 workspace of ks partial outputs and sum
// them into a.out in a fixed order.  The workspace is the stream's split-K
// buffer (workspace.hip), so concurrent calls on other streams get their own.
template <int XT, class F>
hipError_t splitk_run(const QmmArgs& a, int ks, F&& launch) {
  const int64_t n = static_cast<int64_t>(a.nbatch) * a.M * a.N;
  void* ws = nullptr;
  hipError_t e = workspace_get(a.stream, WS_SPLITK, static_cast<size_t>(n) * ks * sizeof(float), &ws);
  if (e != hipSuccess) return e;
  float* part = static_cast<float*>(ws);
  e = launch(part);
  if (e == hipSuccess) {
    const int64_t nb = (n + 1023) / 1024;
    hipLaunchKernelGGL(splitk_reduce_kernel<XT>, dim3(static_cast<unsigned>(nb)), dim3(256), 0, a.stream, part,
                       static_cast<uint16_t*>(a.out), n, ks);
    e = hipGetLastError();
  }
  return e;
}

template <int XT, int MODE, int BITS, int TM, int TN>
hipError_t wr_launch_tile(const QmmArgs& a, int ks, float* part) {
  constexpr int WD = 6;
  const int ntm = (a.M + TM - 1) / TM, ntn = (a.N + TN - 1) / TN;
  const int64_t nblk = static_cast<int64_t>(ntm) * ntn;
  if (nblk > 0x7fffffffLL || a.nbatch > 65535) return hipErrorInvalidConfiguration;
  constexpr auto kern = qmm_gemm_wr_kernel<XT, MODE, BITS, WD, TM, TN>;
  constexpr size_t lds = wr_lds_bytes<BITS>(WD, TM, TN);
  hipError_t e = set_lds_once<kern>(lds);
  if (e != hipSuccess) return e;
  const dim3 grid(static_cast<unsigned>(nblk), static_cast<unsigned>(a.nbatch), static_cast<unsigned>(ks));
  hipLaunchKernelGGL(kern, grid, dim3(2 * TN), lds, a.stream, a, ntm, ntn, part);
  return hipGetLastError();
}

// Tile / split choice for the register-B kernel: 256 x 256 tiles while they
// give most CUs a tile (K split in two or four from 64 tiles at K >= 8192);
// otherwise 128 x 128 tiles with K split over enough
// workgroups to fill the GPU (two per CU when the tiles alone are 128-256).  Split partials are fp32 in the stream's
// split-K workspace (workspace.hip), summed in a fixed order by
// splitk_reduce_kernel, so results do not depend on scheduling.
template <int XT, int MODE, int BITS>
hipError_t wr_launch(const QmmArgs& a, int G) {
  const int64_t big = ((a.M + 255) / 256) * ((a.N + 255) / 256) * a.nbatch;
  if (big >= 192) return wr_launch_tile<XT, MODE, BITS, 256, 256>(a, 1, nullptr);
  // each split keeps whole scale chunks (8 or 16 groups) and 128-code W chunks
  const int gs = MODE == AFFINE ? a.gs : ModeInfo<MODE>::GS;
  const int span = std::max(128, (MODE == AFFINE ? 8 : 16) * gs);
  // 64-191 big tiles over long K: two (96-191) or four (64-95) K ranges of
  // 256 x 256 tiles (the fp32 partial round trip is small next to K >= 8192
  // of MFMA work; against 128 x 128 tiles M = 2048, K = 14336, N = 4096
  // measured 311 -> 264-276 us and M = 1024 159 -> 145 us, while at K = 4096
  // the split measured slower)
  if (big >= 64 && a.K >= 8192) {
    const int kb = big >= 96 ? 2 : 4;
    if (a.K % (span * kb) == 0)
      return splitk_run<XT>(a, kb, [&](float* part) { return wr_launch_tile<XT, MODE, BITS, 256, 256>(a, kb, part); });
  }
  const int64_t small = ((a.M + 127) / 128) * ((a.N + 127) / 128) * a.nbatch;
  int ks = 1;
  while (small * ks < 256 && ks < 16 && a.K % (span * ks * 2) == 0 && a.K / (ks * 2) >= 512) ks *= 2;
  // Exactly one workgroup per CU from >= 128 tiles: one more split puts two
  // on each CU, which measured 8-10% faster at K = N = 4096 for M = 512 and
  // M = 1024 (at M <= 256 and at 1.5 per CU the extra split measured slower).
  if (small >= 128 && small * ks == 256 && ks < 16 && a.K % (span * ks * 2) == 0 && a.K / (ks * 2) >= 512) ks *= 2;
  (void)G;
  if (ks == 1) return wr_launch_tile<XT, MODE, BITS, 128, 128>(a, 1, nullptr);
  return splitk_run<XT>(a, ks, [&](float* part) { return wr_launch_tile<XT, MODE, BITS, 128, 128>(a, ks, part); });
}

template <int XT, int MODE, int BITS>
hipError_t gemm_launch_t(const QmmArgs& a) {
  const int ntm = (a.M + GBM - 1) / GBM, ntn = (a.N + GBN - 1) / GBN;
  const int64_t nblk = static_cast<int64_t>(ntm) * ntn;
  if (nblk <= 0 || a.nbatch <= 0) return hipSuccess;
  if (nblk > 0x7fffffffLL || a.nbatch > 65535) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(nblk), static_cast<unsigned>(a.nbatch));
  const int G = a.K / (MODE == AFFINE ? a.gs : ModeInfo<MODE>::GS);
  const bool dma_ok = a.transpose && a.K % DBK == 0 && (MODE == AFFINE ? G % 2 == 0 : G % 4 == 0);
  constexpr int WD = 6;
  constexpr int GPC = MODE == AFFINE ? 8 : 16;
  const bool wr_ok = dma_ok && (BITS == 4 || BITS == 8) && a.K % (32 * (BITS == 4 ? 4 : 2)) == 0 &&
                     G % GPC == 0;
  if constexpr (BITS == 4 || BITS == 8) {
    if (wr_ok) return wr_launch<XT, MODE, BITS>(a, G);
  } else if constexpr (MODE == AFFINE) {
    // 2 / 3 / 5 / 6-bit codes of one weight matrix: widen them into the
    // stream's code workspace (N K / 2 or N K bytes) and run the register-B
    // kernel on the wide codes
    constexpr int OB = BITS < 4 ? 4 : 8;
    const bool one_w = a.bm.ndim == 0 && a.bm.lhs == nullptr && a.bm.rhs == nullptr;
    if (dma_ok && one_w && a.K % (32 * (OB == 4 ? 4 : 2)) == 0 && G % GPC == 0) {
      const int64_t nchunks = static_cast<int64_t>(a.N) * (a.K / 32);
      if ((nchunks + 255) / 256 > 0x7fffffffLL) return hipErrorInvalidConfiguration;
      void* ws = nullptr;
      hipError_t e = workspace_get(a.stream, WS_CODES, static_cast<size_t>(nchunks) * OB * 4, &ws);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((widen_codes_kernel<BITS, OB>), dim3(static_cast<unsigned>((nchunks + 255) / 256)), dim3(256),
                         0, a.stream, a.w, static_cast<uint32_t*>(ws), nchunks);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      QmmArgs b = a;
      b.w = static_cast<const uint32_t*>(ws);
      b.bits = OB;
      b.w_mat = nchunks * OB;
      return wr_launch<XT, MODE, OB>(b, G);
    }
  }
  if (dma_ok) {
    constexpr auto kern = qmm_gemm_dma8_kernel<XT, MODE, BITS>;
    constexpr size_t lds = dma_lds_bytes<BITS, MODE>();
    hipError_t e = set_lds_once<kern>(lds);
    if (e != hipSuccess) return e;
    // few 256x256 tiles: split K over workgroups (whole scale pairs / quads
    // of groups per split, at least 16 K steps each)
    const int span = (MODE == AFFINE ? 2 : 4) * (MODE == AFFINE ? a.gs : ModeInfo<MODE>::GS);
    int ks = 1;
    while (nblk * a.nbatch * ks < 192 && ks < 16 && a.K % (std::max(span, DBK) * ks * 2) == 0 &&
           a.K / (ks * 2) >= 16 * DBK)
      ks *= 2;
    if (ks > 1) {
      const dim3 g3(grid.x, grid.y, static_cast<unsigned>(ks));
      return splitk_run<XT>(a, ks, [&](float* part) {
        hipLaunchKernelGGL(kern, g3, dim3(512), lds, a.stream, a, ntm, ntn, part);
        return hipGetLastError();
      });
    }
    hipLaunchKernelGGL(kern, grid, dim3(512), lds, a.stream, a, ntm, ntn, nullptr);
  } else if (a.transpose) {
    constexpr auto kern = qmm_gemm_reg_kernel<XT, MODE, BITS, true>;
    hipError_t e = set_lds_once<kern>(REG_LDS_BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(256), REG_LDS_BYTES, a.stream, a, ntm, ntn);
  } else {
    constexpr auto kern = qmm_gemm_reg_kernel<XT, MODE, BITS, false>;
    hipError_t e = set_lds_once<kern>(REG_LDS_BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(256), REG_LDS_BYTES, a.stream, a, ntm, ntn);
  }
  return hipGetLastError();
}

template <int XT>
hipError_t gemm_by_mode(const QmmArgs& a) {
  switch (a.mode) {
    case AFFINE:
      switch (a.bits) {
        case 2: return gemm_launch_t<XT, AFFINE, 2>(a);
        case 3: return gemm_launch_t<XT, AFFINE, 3>(a);
        case 4: return gemm_launch_t<XT, AFFINE, 4>(a);
        case 5: return gemm_launch_t<XT, AFFINE, 5>(a);
        case 6: return gemm_launch_t<XT, AFFINE, 6>(a);
        case 8: return gemm_launch_t<XT, AFFINE, 8>(a);
      }
      break;
    case MXFP4: return gemm_launch_t<XT, MXFP4, 4>(a);
    case MXFP8: return gemm_launch_t<XT, MXFP8, 8>(a);
    case NVFP4: return gemm_launch_t<XT, NVFP4, 4>(a);
  }
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_qmm_gemm(const QmmArgs& a) {
  if (a.xdt == BF16) return gemm_by_mode<BF16>(a);
  if (a.xdt == F16) return gemm_by_mode<F16>(a);
  return hipErrorInvalidValue;
}

}  // namespace iqmm
