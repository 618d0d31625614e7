// decode_common.h — helpers shared by the decode-width kernels
// (qmm_decode.hip) and their grouped gather_qmm form (qmm_gather.hip).
#pragma once
#include "mfma_common.h"

namespace iqmm {

typedef __attribute__((ext_vector_type(4))) float f32x4d_t;

template <int XT>
__device__ __forceinline__ f32x4d_t mfma16(const g_u32x4_t& a, const g_u32x4_t& b, const f32x4d_t& c) {
  if constexpr (XT == BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(g_bf16x8_t, a),
                                                   __builtin_bit_cast(g_bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(g_f16x8_t, a),
                                                  __builtin_bit_cast(g_f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}
// one LDS DMA instruction: 16 bytes per lane from g to LDS byte m0 + 16 lane
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
// A register load whose completion the caller waits for with vm_wait: the
// compiler takes the output as written when the statement issues, so a kernel
// using it must not spill or move that register before the wait (the build
// rejects such kernels that use scratch), and the caller ties the register to
// its wait with an empty asm statement ("+v").
__device__ __forceinline__ g_u32x4_t gload16(const void* g) {
  g_u32x4_t v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(g) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// x fragment (16 bytes: codes 8p .. 8p + 7 of one row) -> MFMA A operand in
// the pair order (x0,x4) (x1,x5) (x2,x6) (x3,x7) of the unpacked weights
__device__ __forceinline__ g_u32x4_t x_pairs(const g_u32x4_t& v) {
  return g_u32x4_t{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                   __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
}

// The group sums X of one block: XG[i][g] holds, in the MFMA output layout,
// sum x over group g of the block for the rows of m tile i (every column
// equal), computed by MFMAs against a B operand of ones.
template <int XT, int MT, int GB>
__device__ __forceinline__ void block_xsums(f32x4d_t (&XG)[MT][GB], const g_u32x4_t (&A)[MT][4]) {
  constexpr uint32_t ONE2 = XT == BF16 ? 0x3f803f80u : 0x3c003c00u;
  constexpr int JG = 4 / GB;  // MFMAs per group
  const g_u32x4_t ones = {ONE2, ONE2, ONE2, ONE2};
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      XG[i][g] = mfma16<XT>(A[i][g * JG], ones, f32x4d_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int j = 1; j < JG; ++j) XG[i][g] = mfma16<XT>(A[i][g * JG + j], ones, XG[i][g]);
    }
}

// One 128-code block of the factored affine 4-bit product for NT 16-row
// weight tiles and MT 16-row x tiles.  A holds the x operands (x_pairs) of
// the block's four 32-code MFMA slots; the weights are the block's 64-byte
// row pieces in LDS at wst + row * 128 + 16 * ((4 h + q) ^ (row & 7)) (h: the
// block's half of a two-block stage, pieces XOR-swizzled by the row); sw / bw
// hold the scale / bias halves of the wave's K range, hb the first half of
// this block.  Y[tt][i] accumulates sum_g s D + (b - C s) X.
// fac_block_xs takes the block's group sums already computed (block_xsums),
// for kernels that reuse one x block against many weight tiles; fac_block
// computes them itself.
template <int XT, int NT, int MT, int GB, int SW>
__device__ __forceinline__ void fac_block_xs(f32x4d_t (&Y)[NT][MT], const g_u32x4_t (&A)[MT][4],
                                             const f32x4d_t (&XG)[MT][GB], const char* wst, int h, int hb,
                                             const uint32_t (&sw)[NT][SW], const uint32_t (&bw)[NT][SW], int r,
                                             int q) {
  using XS = uint16_t;
  constexpr float CM = XT == BF16 ? 128.f : 1024.f;
  constexpr uint32_t EB = XT == BF16 ? 0x43434343u : 0x64646464u;
  constexpr int JG = 4 / GB;  // MFMAs per group
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int row = 16 * tt + r;
    const g_u32x4_t wv = *reinterpret_cast<const g_u32x4_t*>(wst + row * 128 + 16 * ((4 * h + q) ^ (row & 7)));
    uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
    // 4 x 4 transpose over the lanes q: afterwards wd[j] of lane q is dword q
    // of chunk 4p + j
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
      const int hf = hb + g;
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
}

template <int XT, int NT, int MT, int GB, int SW>
__device__ __forceinline__ void fac_block(f32x4d_t (&Y)[NT][MT], const g_u32x4_t (&A)[MT][4], const char* wst, int h,
                                          int hb, const uint32_t (&sw)[NT][SW], const uint32_t (&bw)[NT][SW], int r,
                                          int q) {
  f32x4d_t XG[MT][GB];
  block_xsums<XT, MT, GB>(XG, A);
  fac_block_xs<XT, NT, MT, GB, SW>(Y, A, XG, wst, h, hb, sw, bw, r, q);
}

// Row segment of a sorted grouped gather found inside the kernel: the first
// batch index i in [0, n] whose expert key is >= e, where the key is the rhs
// index clamped into [-1, E] (the definition of segment_offsets_kernel's
// off[e]).  A wave probes 64 evenly spaced entries per round and keeps the
// interval where the sorted keys cross e: two dependent rounds for 4096
// rows.  Every lane returns the same (wave-uniform) index; a rhs that is not
// sorted as promised gives some index in [0, n], never an out-of-range one.
__device__ __forceinline__ int64_t seg_lower_bound(const void* rhs, int dt, int64_t n, int64_t E, int64_t e,
                                                   int lane) {
  int64_t lo = 0, hi = n;
  while (hi > lo) {
    const int64_t len = hi - lo;
    const int64_t step = (len + 63) / 64;
    const int64_t p = lo + min(static_cast<int64_t>(lane) * step, len - 1);
    int64_t v = load_index(rhs, dt, p);
    v = v < 0 ? int64_t{-1} : v > E ? E : v;
    const uint64_t m = __ballot(v >= e);
    if (m == 0) {
      lo = lo + min(63 * step, len - 1) + 1;  // every probe is below e
    } else {
      const int f = __builtin_ctzll(m);
      const int64_t pf = lo + min(static_cast<int64_t>(f) * step, len - 1);
      hi = pf;
      if (f > 0) lo = lo + min(static_cast<int64_t>(f - 1) * step, len - 1) + 1;
    }
  }
  return lo;
}

// LDS plan of the streaming kernels (qmm_stream.hip, qmm_gather.hip): per
// wave a ring of D weight stages plus double-buffered scale / bias words, and
// the cross-wave partial sums of one tile-block.
template <int NT, int MT, int S, int D, int SW>
struct StreamLds {
  static constexpr int WST = NT * 2048;           // one stage of a wave's weights: NT*16 rows x 128 B
  static constexpr int SCL = NT * 16 * SW * 4;    // a tile-block's scale (or bias) words, one wave
  static constexpr int WAVE = D * WST + 4 * SCL;  // ring + double-buffered scales and biases
  static constexpr int RED = S * NT * MT * 1024;  // cross-wave partial sums of one tile-block
  static constexpr int TOTAL = S * WAVE + RED;
};

template <int NT, int MT, int S, int D, int KB, int GB>
constexpr bool stream_fits() {
  constexpr int SW = KB * GB / 2;
  constexpr int NDW = 2 * NT, NSC = (2 * NT * 16 * (SW / 4) + 63) / 64;
  return KB % 2 == 0 && SW % 4 == 0 && D >= 2 && D <= 3 && StreamLds<NT, MT, S, D, SW>::TOTAL <= 160 * 1024 &&
         (D - 2) * (2 * NDW + NSC) < 64;
}

}  // namespace iqmm
