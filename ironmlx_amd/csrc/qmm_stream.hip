// qmm_stream.hip — affine 4-bit quantized matmul at decode widths on wide
// matrices (transpose, 1 <= M <= 32, K = 4096, gs 32 / 64), the batched decode
// step of mlx/src/nn/linear.rs:51-63 with x = [B, 1, K] for the projections
// with many output rows (gate / up, the fused gate_up SwiGLU, fused q/k/v).
//
// Same factored arithmetic as qmm_decode.hip (fac_block: the weights enter
// v_mfma_f32_16x16x32 as C + n halves, per-group rescale s D + (b - C s) X),
// organised to overlap loads with compute.  A workgroup of S waves splits K
// into S ranges of KB 128-code blocks; each wave loads the x fragments of its
// range for all M rows ONCE, permuted into MFMA A operands held in registers
// (with their per-group sums, where the registers allow), and then streams a sequence of tile-blocks (NT 16-row weight tiles; a gate
// tile and its up tile for the SwiGLU) through a ring of D stages in its own
// slice of LDS, filled by LDS DMA (8 rows x 128 B per instruction, pieces
// XOR-swizzled by the row); each tile-block's scale and bias words come with
// its first stage (16-byte DMA pieces into a double buffer).  The ring runs
// across tile-blocks, so while a wave computes one stage the next D - 1 are in
// flight, also across tile boundaries.  After each tile-block the S partial
// sums meet in LDS (two barriers) and the workgroup stores the NC outputs.
// Workgroup g takes tile-blocks g, g + G, g + 2G, ... (G = min(tile-blocks,
// CUs)), so each CU streams several tile-blocks back to back.
#include "launch.h"
#include "mfma_common.h"
#include "decode_common.h"

namespace iqmm {
namespace {

template <int XT, int NT, int MT, int GB, int S, int D, int KB, bool GLU>
__global__ __launch_bounds__(64 * S) void qmm_stream_kernel(QmmArgs a, int ntb) {
  static_assert(!GLU || NT == 2, "GLU pairs one gate tile with its up tile");
  static_assert(stream_fits<NT, MT, S, D, KB, GB>(), "LDS / vmcnt budget");
  constexpr int NS = KB / 2;                 // stages per tile-block
  constexpr int SW = KB * GB / 2;            // scale words per row in a wave's K range
  using L = StreamLds<NT, MT, S, D, SW>;
  constexpr int NDW = 2 * NT;                // weight DMA per stage
  constexpr int PSC = NT * 16 * (SW / 4);    // 16-byte scale pieces per tile-block (biases as many)
  constexpr int NSC = (2 * PSC + 63) / 64;   // scale + bias DMA with the first stage
  constexpr int NC = GLU ? 8 * NT : 16 * NT; // output columns per tile-block
  using XS = uint16_t;
  __shared__ __attribute__((aligned(1024))) char lds[L::TOTAL];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int M = a.M, N = a.N, K = a.K;
  const int r = lane & 15, q = lane >> 4;
  const int pb = KB * wave;  // first 128-code block of this wave
  const int gshift = __builtin_ctz(a.gs);
  const int64_t wrow = K / 2, srow = (K >> gshift) * 2;
  const char* w = reinterpret_cast<const char*>(a.w);
  const char* sp = static_cast<const char*>(a.s);
  const char* bp = static_cast<const char*>(a.b);
  XS* out = static_cast<XS*>(a.out);

  // x operands of the wave's K range for all M rows (rows past M repeat the
  // last row; their outputs are not stored)
  g_u32x4_t A[KB][MT][4];
  {
    const char* xb = static_cast<const char*>(a.x);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const char* xr = xb + static_cast<int64_t>(min(16 * i + r, M - 1)) * K * 2 + pb * 256 + 16 * q;
#pragma unroll
      for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) A[b][i][j] = x_pairs(*reinterpret_cast<const g_u32x4_t*>(xr + b * 256 + 64 * j));
    }
  }
  // the compiler's own loads are complete before the counted DMA starts
  __builtin_amdgcn_s_waitcnt(0);
  // group sums of the wave's x blocks, the same for every tile-block: kept in
  // registers where they fit (one m tile at gs 64 / 128), else recomputed
  // per tile-block by fac_block
  constexpr bool PRE = MT * GB <= 2;
  f32x4d_t XS_[PRE ? KB : 1][MT][GB];
  if constexpr (PRE) {
#pragma unroll
    for (int b = 0; b < KB; ++b) block_xsums<XT, MT, GB>(XS_[b], A[b]);
  }

  const int G = gridDim.x;
  const int nit = (ntb - static_cast<int>(blockIdx.x) + G - 1) / G;  // >= 1: G <= ntb
  const int total = nit * NS;
  auto wrow_of = [&](int tb, int row) {  // tile-block row -> weight row
    const int tt = row >> 4, rr = row & 15, n0 = tb * NC;
    return GLU ? static_cast<int64_t>(tt) * N + min(n0 + rr, N - 1) : static_cast<int64_t>(min(n0 + row, N - 1));
  };
  const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds_u32(lds)) + wave * L::WAVE;
  const char* lds_w = lds + wave * L::WAVE;
  // stage u = (tile-block iteration it, stage st) into ring slot u % D
  auto issue = [&](int it, int st) {
    const int tb = static_cast<int>(blockIdx.x) + G * it;
    const int slot = (it * NS + st) % D;
#pragma unroll
    for (int u = 0; u < NDW; ++u) {
      const int row = 8 * u + (lane >> 3);
      dma16(w + wrow_of(tb, row) * wrow + pb * 64 + st * 128 + 16 * ((lane & 7) ^ (row & 7)),
            lds_wave + slot * L::WST + u * 1024);
    }
    if (st == 0) {
      // piece p: scales (p < PSC) then biases; row p' / (SW / 4), 16-byte part p' % (SW / 4)
      const uint32_t sbase = lds_wave + D * L::WST + (it & 1) * 2 * L::SCL;
#pragma unroll
      for (int v = 0; v < NSC; ++v) {
        const int p = 64 * v + lane;
        if (p < 2 * PSC) {
          const int which = p >= PSC, pp = p - which * PSC;
          const int row = pp / (SW / 4), part = pp % (SW / 4);
          dma16((which ? bp : sp) + wrow_of(tb, row) * srow + pb * GB * 2 + part * 16, sbase + v * 1024);
        }
      }
    }
  };
  f32x4d_t Y[NT][MT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int i = 0; i < MT; ++i) Y[tt][i] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  // prologue: the first D - 1 stages
#pragma unroll
  for (int u = 0; u < D - 1; ++u)
    if (u < total) issue(u / NS, u % NS);
  uint32_t sw[NT][SW], bw[NT][SW];
  float* red = reinterpret_cast<float*>(lds + S * L::WAVE);
  for (int it = 0; it < nit; ++it) {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      const int u = it * NS + st;
      // stages issued after u: min(D - 2, total - 1 - u); each carries NDW
      // DMA, plus NSC for the first stage of a tile-block
      const int later = min(D - 2, total - 1 - u);
      if (later >= 1) {
        if ((st + 1) % NS == 0) vm_wait<(D >= 3 ? NDW + NSC : 0)>();
        else vm_wait<(D >= 3 ? NDW : 0)>();
      } else {
        vm_wait<0>();
      }
      if (st == 0) {
        // this tile-block's scale / bias words, from the buffer of its parity
        const char* sb = lds_w + D * L::WST + (it & 1) * 2 * L::SCL;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
          for (int h = 0; h < SW; ++h) {
            sw[tt][h] = *reinterpret_cast<const uint32_t*>(sb + ((tt * 16 + r) * SW + h) * 4);
            bw[tt][h] = *reinterpret_cast<const uint32_t*>(sb + L::SCL + ((tt * 16 + r) * SW + h) * 4);
          }
      }
      if (u + D - 1 < total) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // slot (u - 1) % D has been read
        issue((u + D - 1) / NS, (st + D - 1) % NS);
      }
      const char* wst = lds_w + (u % D) * L::WST;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (PRE)
          fac_block_xs<XT, NT, MT, GB, SW>(Y, A[2 * st + h], XS_[2 * st + h], wst, h, (2 * st + h) * GB, sw, bw, r, q);
        else
          fac_block<XT, NT, MT, GB, SW>(Y, A[2 * st + h], wst, h, (2 * st + h) * GB, sw, bw, r, q);
      }
    }
    // the S partial sums of tile-block it meet in LDS
    const int n0 = (static_cast<int>(blockIdx.x) + G * it) * NC;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          red[((wave * NT + tt) * MT + i) * 256 + (4 * q + v) * 16 + r] = Y[tt][i][v];
          Y[tt][i][v] = 0.f;
        }
    __syncthreads();
    for (int idx = t; idx < M * NC; idx += 64 * S) {
      const int m = idx / NC, nn = idx % NC;
      const int i = m >> 4, mr = m & 15;
      if (n0 + nn >= N) continue;
      if constexpr (GLU) {
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int w2 = 0; w2 < S; ++w2) acc[hh] += red[((w2 * NT + hh) * MT + i) * 256 + mr * 16 + nn];
        out[static_cast<int64_t>(m) * N + n0 + nn] = swiglu_out<XT>(acc[0], acc[1]);
      } else {
        const int tt = nn >> 4;
        float acc = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < S; ++w2) acc += red[((w2 * NT + tt) * MT + i) * 256 + mr * 16 + (nn & 15)];
        out[static_cast<int64_t>(m) * N + n0 + nn] = from_f<XT>(acc);
      }
    }
    __syncthreads();  // the partials are read before the next tile-block's are written
  }
}

int cu_count() {
  static int n[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (n[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    n[dev] = c;
  }
  return n[dev];
}

template <int XT, int NT, int MT, int GB, int S, int D, int KB, bool GLU>
hipError_t stream_go(const QmmArgs& a) {
  if constexpr (!stream_fits<NT, MT, S, D, KB, GB>() || (GLU && NT != 2)) {
    return hipErrorInvalidValue;
  } else {
    constexpr int NC = GLU ? 8 * NT : 16 * NT;
    const int ntb = (a.N + NC - 1) / NC;
    const int grid = ntb < cu_count() ? ntb : cu_count();
    hipLaunchKernelGGL((qmm_stream_kernel<XT, NT, MT, GB, S, D, KB, GLU>), dim3(grid), dim3(64 * S), 0, a.stream, a,
                       ntb);
    return hipGetLastError();
  }
}

// eight waves of four blocks (K = 4096), three stages in flight; one tile per
// tile-block, or the gate tile and its up tile for the SwiGLU
template <int XT, int GB, bool GLU>
hipError_t stream_launch(const QmmArgs& a) {
  if constexpr (GLU) {
    return stream_go<XT, 2, 1, GB, 8, 3, 4, true>(a);  // M <= 16 (qmm_stream_supported)
  } else {
    return a.M > 16 ? stream_go<XT, 1, 2, GB, 8, 3, 4, false>(a) : stream_go<XT, 1, 1, GB, 8, 3, 4, false>(a);
  }
}

}  // namespace

bool qmm_stream_supported(const QmmArgs& a) {
  const bool mapped = a.bm.ndim != 0 || a.bm.lhs != nullptr || a.bm.rhs != nullptr;
  return a.transpose && a.mode == AFFINE && a.bits == 4 && (a.xdt == BF16 || a.xdt == F16) && a.M >= 1 &&
         a.M <= 32 && a.K == 4096 && a.nbatch == 1 && !mapped && a.N >= 1 && (a.gs == 32 || a.gs == 64) &&
         (reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 16 == 0 && a.b != nullptr &&
         // two m tiles of the SwiGLU or of gs 32 exceed the register file
         !(a.M > 16 && (a.glu || a.gs == 32)) &&
         // measured on MI355X (bf16, gs 64, K = 4096, group sums of x kept in
         // registers): ahead of the decode-width kernel where each CU streams
         // several tile-blocks -- the fused gate_up SwiGLU (2 x 14336 rows,
         // M = 4 / 16: 21.7 / 24.3 -> 18.9 / 20.9 us), very wide matrices
         // (N = 128256, M = 8: 87.5 -> 63.6 us), and 6144 .. 14336 rows at
         // M <= 12 (N = 14336, M = 8: 12.4 -> 11.7 us; N = 10240, M = 4:
         // 10.8 -> 9.1 us); at M = 16 behind or even at 6144 and 14336 rows
         // (8.5 vs 9.5 us; kernel average 13.1 vs 13.5 us)
         (a.glu || static_cast<int64_t>(a.N) >= 65536 || (a.N >= 6144 && a.M <= 12));
}

hipError_t launch_qmm_stream(const QmmArgs& a) {
  if (a.glu) {
    if (a.gs == 32) return a.xdt == BF16 ? stream_launch<BF16, 4, true>(a) : stream_launch<F16, 4, true>(a);
    return a.xdt == BF16 ? stream_launch<BF16, 2, true>(a) : stream_launch<F16, 2, true>(a);
  }
  if (a.gs == 32) return a.xdt == BF16 ? stream_launch<BF16, 4, false>(a) : stream_launch<F16, 4, false>(a);
  return a.xdt == BF16 ? stream_launch<BF16, 2, false>(a) : stream_launch<F16, 2, false>(a);
}

}  // namespace iqmm
