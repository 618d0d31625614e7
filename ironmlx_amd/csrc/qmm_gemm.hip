// qmm_gemm.hip — prefill-shaped quantized matmul on CDNA4 matrix cores.
//
// out[M, N] = x[M, K] . deq(W)^T  (transpose)  or  x . deq(W)  (!transpose),
// x bf16 or fp16, fp32 accumulation.  Reference op: mlx/src/ops.rs:695-727
// at prefill (x = [1, L, K], mlx/src/generate/mod.rs:76-80).
//
// Workgroup: 256 threads (4 waves, one per SIMD), output tile 256 x 256,
// K step 64.  Each wave owns a 128 x 128 sub-tile as 4 x 4 blocks of
// v_mfma_f32_32x32x16_{bf16,f16}; the 256 fp32 accumulators per lane live in
// the unified VGPR/AGPR file (one wave per SIMD).
//
// Pipeline (one barrier per K step):
//   - x tiles go global -> LDS directly (global_load_lds_dwordx4, no register
//     staging) into a 3-stage ring, issued two steps ahead;
//   - packed W tiles (8 KiB at 4 bits + scales) are fetched into registers
//     two steps ahead, dequantized one step ahead with the same arithmetic as
//     `dequantize` (rn(s*q + b); s*q is exact for 16-bit scales) and written
//     as x's 16-bit type into a 2-stage ring.
//   3 x 32 KiB (x) + 2 x 32 KiB (W) = the 160 KiB of LDS per CU.  Tiles are
//   stored unpadded with 16-byte granules XOR-swizzled by (row / 2) mod 8, so
//   the 16-byte fragment reads of 32 consecutive rows hit distinct banks.
//   The step ends with s_waitcnt vmcnt(8) (everything but the 8 x loads just
//   issued) and a bare s_barrier, so prefetches stay in flight across it.
//
// Workgroups are mapped so that consecutive tiles of an XCD share a column
// block of W (its L2 keeps the dequantization inputs hot) and m varies
// fastest.
#include <stdlib.h>

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
// DMA-pipelined kernel (transpose=true).  Every global read -- the x tile, the
// packed W tile, its scales and biases -- is an LDS DMA
// (global_load_lds_dword[x4]) issued DEPTH-1 = 3 K steps ahead into 4-stage
// rings; no global data passes through registers, so the only waits are the
// explicit s_waitcnt before each step's barrier.  Each step one thread
// dequantizes one W row's 32 codes from the packed ring into a 2-stage bf16 /
// fp16 ring (rn(s*q + b), the `dequantize` arithmetic), while the waves run
// the step's MFMAs.  BK = 32; x and dequantized-W rows are 64 bytes (4
// granules), granules XOR-swizzled so the fragment reads of consecutive rows
// hit distinct banks.  One barrier per step: step k's MFMAs run interleaved
// (sched_group_barrier) with the dequantization of step k+1, whose packed W
// was made resident by the wait ending step k-1.
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
__device__ __forceinline__ void dma_x4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma_x1(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(g), "s"(lds) : "memory", "m0");
}

template <int BITS, int MODE>
struct DmaCounts {
  static constexpr int X = 4;                              // x: 16 KiB / 4 waves / 1 KiB
  static constexpr int W = BITS == 4 ? 1 : BITS;           // packed W per wave
  static constexpr int S = MODE == AFFINE ? 2 : 1;         // scales (+ biases)
  static constexpr int PER_STEP = X + W + S;
  static constexpr int WBYTES = GBN * 4 * BITS;            // packed bytes per step
};

template <int XT, int MODE, int BITS>
__global__ __launch_bounds__(256, 1) void qmm_gemm_dma_kernel(QmmArgs a, int ntm, int ntn) {
  using XS = uint16_t;
  using DC = DmaCounts<BITS, MODE>;
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
  const int G = K / gs;
  const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
  const char* sbase = static_cast<const char*>(a.s) + wb * a.s_mat * (AFF ? 2 : 1);
  const char* bbase = AFF ? static_cast<const char*>(a.b) + wb * a.s_mat * 2 : nullptr;

  // LDS map (bytes): x ring | W-packed ring | scale ring | bias ring | deq-W ring
  char* lbase = reinterpret_cast<char*>(glds);
  char* xr = lbase;
  char* wr = xr + DEPTH * DA_STAGE * 2;
  char* sr = wr + DEPTH * DC::WBYTES;
  char* br = sr + DEPTH * GBN * 4;
  uint16_t* dq = reinterpret_cast<uint16_t*>(br + DEPTH * GBN * 4);

  // ---- issue all DMA of K step `ks` into ring slot ks % DEPTH
  auto issue = [&](int ks) {
    const int slot = ks % DEPTH, k0 = ks * DBK;
    // x: 16 rows x 64 B per instruction; wave covers rows [64 wave, +64)
#pragma unroll
    for (int i = 0; i < DC::X; ++i) {
      const int rbase = wave * 64 + i * 16;
      const int row = rbase + (lane >> 2);
      const int g = ((lane & 3) ^ dswzf(row)) & 3;
      const int gm = min(m0 + row, M - 1);
      dma_x4(x + static_cast<int64_t>(gm) * K + k0 + g * 8,
             __builtin_amdgcn_readfirstlane(lds_addr(xr + (slot * DA_STAGE + rbase * DBK) * 2)));
    }
    // packed W: the step's 4*BITS bytes of each of 256 rows
    if constexpr (BITS == 4) {
      const int row = wave * 64 + lane;
      const int gn = min(n0 + row, N - 1);
      dma_x4(w + gn * wpr + (k0 >> 5) * 4,
             __builtin_amdgcn_readfirstlane(lds_addr(wr + slot * DC::WBYTES + wave * 64 * 16)));
    } else {
#pragma unroll
      for (int i = 0; i < BITS; ++i) {
        const int idx = (wave * BITS + i) * 64 + lane;      // word index in the stage
        const int row = idx / BITS, word = idx - row * BITS;
        const int gn = min(n0 + row, N - 1);
        dma_x1(w + gn * wpr + (k0 >> 5) * BITS + word,
               __builtin_amdgcn_readfirstlane(lds_addr(wr + slot * DC::WBYTES + (wave * BITS + i) * 256)));
      }
    }
    // scales (and biases): the aligned dword holding this step's group
    {
      const int row = wave * 64 + lane;
      const int gn = min(n0 + row, N - 1);
      const int g = k0 / gs;
      if constexpr (AFF) {
        const int64_t e = static_cast<int64_t>(gn) * G + (g & ~1);
        dma_x1(sbase + e * 2, __builtin_amdgcn_readfirstlane(lds_addr(sr + slot * GBN * 4 + wave * 256)));
        dma_x1(bbase + e * 2, __builtin_amdgcn_readfirstlane(lds_addr(br + slot * GBN * 4 + wave * 256)));
      } else {
        const int64_t e = static_cast<int64_t>(gn) * G + (g & ~3);
        dma_x1(sbase + e, __builtin_amdgcn_readfirstlane(lds_addr(sr + slot * GBN * 4 + wave * 256)));
      }
    }
  };

  // ---- dequantize step ks (ring slot ks % DEPTH) into deq slot ks & 1; thread = W row
  auto dequant = [&](int ks) {
    const int slot = ks % DEPTH, k0 = ks * DBK;
    const int n = t;
    uint32_t wd[BITS];
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(wr + slot * DC::WBYTES) + n * BITS;
    if constexpr (BITS == 4) {
      const g_u32x4_t v = *reinterpret_cast<const g_u32x4_t*>(wp);
      wd[0] = v.x; wd[1] = v.y; wd[2] = v.z; wd[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < BITS; ++i) wd[i] = wp[i];
    }
    const int g = k0 / gs;
    const uint32_t sw = reinterpret_cast<const uint32_t*>(sr + slot * GBN * 4)[n];
    float s, b = 0.f, s2;
    if constexpr (AFF) {
      const uint16_t sh = static_cast<uint16_t>((g & 1) ? (sw >> 16) : (sw & 0xffffu));
      const uint32_t bw = reinterpret_cast<const uint32_t*>(br + slot * GBN * 4)[n];
      const uint16_t bh = static_cast<uint16_t>((g & 1) ? (bw >> 16) : (bw & 0xffffu));
      s = to_f<XT>(sh);
      b = to_f<XT>(bh);
      s2 = s;
    } else {
      s = fp_scale<MODE>((sw >> (8 * (g & 3))) & 0xffu);
      s2 = MODE == NVFP4 ? fp_scale<MODE>((sw >> (8 * ((g + 1) & 3))) & 0xffu) : s;
    }
    uint32_t o[16];
    dequant32<XT, MODE, BITS>(wd, s, b, s2, o);
    uint16_t* B = dq + (ks & 1) * DB_STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<g_u32x4_t*>(&B[dswz(n, 8 * i)]) =
          g_u32x4_t{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = K / DBK;
  // prologue: steps 0 .. DEPTH-2 in flight; step 0 dequantized; step 1 resident
  for (int ks = 0; ks < DEPTH - 1 && ks < nk; ++ks) issue(ks);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  dequant(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  for (int ks = 0; ks < nk; ++ks) {
    if (ks + DEPTH - 1 < nk) issue(ks + DEPTH - 1);
    const uint16_t* Ast = reinterpret_cast<const uint16_t*>(xr) + (ks % DEPTH) * DA_STAGE;
    const uint16_t* Bst = dq + (ks & 1) * DB_STAGE;
#pragma unroll
    for (int kk = 0; kk < DBK / 16; ++kk) {
      const int kq = kk * 16 + 8 * (lane >> 5);
      g_u32x4_t af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const g_u32x4_t*>(&Ast[dswz(wm * 128 + i * 32 + (lane & 31), kq)]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = *reinterpret_cast<const g_u32x4_t*>(&Bst[dswz(wn * 128 + j * 32 + (lane & 31), kq)]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32<XT>(af[i], bf[j], acc[i][j]);
    }
    if (ks + 1 < nk) dequant(ks + 1);
    // interleave: fragment reads first, then MFMA / VALU / LDS groups
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);   // 8 DS reads (kk = 0 fragments)
#pragma unroll
    for (int g = 0; g < 32; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // 4 VALU
      if (g % 4 == 3) __builtin_amdgcn_sched_group_barrier(0x300, 2, 0);  // DS read/write
    }
    // end of step: everything but the last issued step's DMA is resident
    if (ks + 2 < nk) {
      if (ks + DEPTH - 1 < nk) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(DC::PER_STEP) : "memory");
      else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
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

template <int BITS, int MODE>
constexpr size_t dma_lds_bytes() {
  return DEPTH * DA_STAGE * 2 + DEPTH * DmaCounts<BITS, MODE>::WBYTES + 2 * DEPTH * GBN * 4 +
         2 * DB_STAGE * 2;
}

bool qmm_gemm_supported(const QmmArgs& a) {
  return (a.xdt == BF16 || a.xdt == F16) && a.K % 32 == 0 && (a.transpose || a.N % 32 == 0);
}

namespace {
template <int XT, int MODE, int BITS>
hipError_t gemm_launch_t(const QmmArgs& a) {
  const int ntm = (a.M + GBM - 1) / GBM, ntn = (a.N + GBN - 1) / GBN;
  const int64_t nblk = static_cast<int64_t>(ntm) * ntn;
  if (nblk <= 0 || a.nbatch <= 0) return hipSuccess;
  if (nblk > 0x7fffffffLL || a.nbatch > 65535) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(nblk), static_cast<unsigned>(a.nbatch));
  const int G = a.K / (MODE == AFFINE ? a.gs : ModeInfo<MODE>::GS);
  const bool dma_ok = a.transpose && a.K % DBK == 0 && (MODE == AFFINE ? G % 2 == 0 : G % 4 == 0);
  if (dma_ok) {
    auto kern = qmm_gemm_dma_kernel<XT, MODE, BITS>;
    constexpr size_t lds = dma_lds_bytes<BITS, MODE>();
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, a.stream, a, ntm, ntn);
  } else if (a.transpose) {
    auto kern = qmm_gemm_reg_kernel<XT, MODE, BITS, true>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, REG_LDS_BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(256), REG_LDS_BYTES, a.stream, a, ntm, ntn);
  } else {
    auto kern = qmm_gemm_reg_kernel<XT, MODE, BITS, false>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, REG_LDS_BYTES);
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
