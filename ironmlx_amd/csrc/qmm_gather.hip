// qmm_gather.hip — sorted grouped gather_qmm (affine 4-bit, gs 32 / 64 / 128)
// with the factored MFMA arithmetic of qmm_decode.hip: gather_decode_kernel
// (one 64-column block of one expert per workgroup) and gather_stream_kernel
// (few rows per expert: each expert's weights streamed past x rows fetched
// once per pass).
#include <algorithm>
#include <type_traits>

#include "launch.h"
#include "mfma_common.h"
#include "decode_common.h"

namespace iqmm {
namespace {

// Sorted grouped gather_qmm (sorted_indices; the MoE layer of
// mlx/src/nn/moe.rs:84-170 over the stacked experts of
// mlx/src/model/qwen35.rs:653-775) with the factored arithmetic of
// qmm_decode.hip.  Workgroup (column block, expert e) takes the expert's rows
// [off[e], off[e + 1]) of the flattened batch (x rows gathered through lhs),
// in passes of up to 16 MTMAX rows.  Its S waves split K; each wave streams
// its KB blocks of the NT weight tiles through its own LDS ring by LDS DMA
// (8 rows x 128 B per instruction, as in qmm_decode.hip) with D stages of two
// blocks in flight, and x straight into registers (16 rows x 64 B), or, with
// XL, also through the ring (2 rows x 512 B).  The scale / bias words of the
// wave's range are read once for every pass.  Rows whose lhs index is out of
// range are written as NaN; workgroup e = E (one past the experts) writes NaN
// for batch entries outside every expert's segment.
template <int NT, int MT, int S, int D, bool XL, int KB>
constexpr int gat_lds_bytes() {
  constexpr int ring = D < KB / 2 ? D : KB / 2;  // stages allocated
  constexpr int wave = ring * (NT * 2048 + (XL ? MT * 8192 : 0));
  constexpr int red = S > 1 ? S * NT * MT * 1024 : 0;
  return S * wave > red ? S * wave : red;
}
template <int NT, int MT, int S, int D, bool XL, int KB>
constexpr bool gat_fits() {
  return gat_lds_bytes<NT, MT, S, D, XL, KB>() <= 160 * 1024 && D <= 3 && (D - 1) * (2 * NT + 8 * MT) < 64;
}

template <int XT, int NT, int GB, int S, int D, int KB, bool XL, bool GLU, int MTMAX>
__global__ __launch_bounds__(64 * S) void gather_decode_kernel(QmmArgs a, int64_t nflat, const int64_t* off) {
  static_assert(!GLU || NT % 2 == 0, "GLU pairs gate tiles with up tiles");
  static_assert(KB % 2 == 0, "stages of two blocks");
  constexpr int NC = GLU ? 8 * NT : 16 * NT;
  using XS = uint16_t;
  constexpr int SW = (KB * GB + 1) / 2;
  constexpr int NS = KB / 2;
  constexpr int WSTAGE = NT * 16 * 128;
  constexpr int XSTAGE = XL ? MTMAX * 16 * 512 : 0;
  constexpr int SSTAGE = WSTAGE + XSTAGE;
  constexpr int WAVE_LDS = (D < NS ? D : NS) * SSTAGE;
  constexpr int LDS = gat_lds_bytes<NT, MTMAX, S, D, XL, KB>();
  static_assert(gat_fits<NT, MTMAX, S, D, XL, KB>(), "LDS / vmcnt budget");
  constexpr int NDW = 2 * NT;
  __shared__ __attribute__((aligned(1024))) char lds[LDS];
  // per pass row: element offset of its x row, and of its output row (one's
  // complement when the row's lhs index is out of range: written as NaN)
  __shared__ int64_t prow_x[16 * MTMAX], prow_o[16 * MTMAX];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int Mx = a.M, N = a.N, K = a.K;
  // one-dimensional grid of gx (E + 1) workgroups (E = a.bm.nw), dispatched
  // round robin over the 8 XCDs (workgroup L on XCD L % 8); renumbered so that
  // each XCD takes a contiguous range of (expert, column block) pairs and the
  // column blocks of one expert share their gathered x rows in one L2
  const int gx = (N + NC - 1) / NC;
  const int64_t total = gridDim.x;
  const int64_t L = blockIdx.x, per = total / 8;
  const int64_t F = L < 8 * per ? (L % 8) * per + L / 8 : L;
  const int n0 = static_cast<int>(F % gx) * NC;
  const int64_t e = F / gx;
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
  auto wrow_of = [&](int row) {
    const int tt = row >> 4, rr = row & 15;
    return GLU ? static_cast<int64_t>(tt / (NT / 2)) * N + min(n0 + 16 * (tt % (NT / 2)) + rr, N - 1)
               : static_cast<int64_t>(min(n0 + row, N - 1));
  };
  const char* wsrc[NDW];
#pragma unroll
  for (int u = 0; u < NDW; ++u) {
    const int row = 8 * u + (lane >> 3);
    wsrc[u] = w + wrow_of(row) * wrow + pb * 64 + 16 * ((lane & 7) ^ (row & 7));
  }
  uint32_t sw[NT][SW], bw[NT][SW];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int64_t n = wrow_of(16 * tt + r);
    const char* s0 = sp + n * srow + pb * GB * 2;
    const char* b0 = bp + n * srow + pb * GB * 2;
#pragma unroll
    for (int h = 0; h < SW; ++h) {
      sw[tt][h] = *reinterpret_cast<const uint32_t*>(s0 + 4 * h);
      bw[tt][h] = *reinterpret_cast<const uint32_t*>(b0 + 4 * h);
    }
  }
  const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds_u32(lds)) + wave * WAVE_LDS;
  const char* lds_w = lds + wave * WAVE_LDS;
  auto pass = [&](auto mt_c, int64_t r0) {
    constexpr int MT = decltype(mt_c)::value;
    // rows past the segment repeat its last row; their outputs are not stored
    if (t < 16 * MT) {
      const int64_t rr = min(r0 + t, rows_total - 1);
      const int64_t b = blo + rr / Mx, mrow = rr % Mx;
      const int64_t xm = a.bm.lhs ? load_index(a.bm.lhs, a.bm.lhs_dt, b) : b;
      const bool ok = xm >= 0 && xm < a.bm.nx;
      prow_x[t] = (ok ? xm : 0) * a.x_mat + mrow * K;
      prow_o[t] = ok ? (b * Mx + mrow) * N : ~((b * Mx + mrow) * N);
    }
    __syncthreads();
    auto xrow_ptr = [&](int64_t, int m) { return reinterpret_cast<const char*>(x + prow_x[m]); };
    constexpr int NDX = XL ? 8 * MT : 0;
    constexpr int NRX = XL ? 0 : 8 * MT;
    constexpr int PER = NDW + NDX + NRX;
    static_assert((D - 1) * PER < 64, "vmcnt range");
    const char* xsrc[XL ? NDX : 1];
    const char* xr[XL ? 1 : MT];
    if constexpr (XL) {
#pragma unroll
      for (int u = 0; u < NDX; ++u) {
        const int row = 2 * u + (lane >> 5);
        xsrc[u] = xrow_ptr(r0, row) + pb * 256 + 16 * ((lane & 31) ^ (row & 15));
      }
    } else {
#pragma unroll
      for (int i = 0; i < MT; ++i) xr[i] = xrow_ptr(r0, 16 * i + r) + pb * 256 + 16 * q;
    }
    // the compiler's own loads (scales, indices) are complete before the
    // counted loads of the K loop start
    __builtin_amdgcn_s_waitcnt(0);
    g_u32x4_t xreg[XL ? 1 : D][2][MT][4];
    auto issue = [&](int st, int slot) {
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
    auto compute = [&](int slot, int h, int b) {
      g_u32x4_t A[MT][4];
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (XL) {
            const int m = 16 * i + r, p = 16 * h + 4 * j + q;
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
      const int later = st + D <= NS ? D - 1 : NS - 1 - st;
      if (later == 2) vm_wait<(D >= 3 ? 2 * PER : 0)>();
      else if (later == 1) vm_wait<PER>();
      else vm_wait<0>();
      if constexpr (!XL) {
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
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(st + D, slot);
      }
    }
    // row rr = r0 + m of the expert, column col
    auto store = [&](int m, int col, float g, float u) {
      const int64_t o = prow_o[m];
      const auto v = GLU ? swiglu_out<XT>(g, u) : from_f<XT>(g);
      if (o >= 0) out[o + col] = v;
      else out[~o + col] = from_f<XT>(__builtin_nanf(""));
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
            if (rr < rows_total && col < N) store(16 * i + 4 * q + v, col, Y[tt][i][v], GLU ? Y[tt + NT / 2][i][v] : 0.f);
          }
      __syncthreads();  // the ring and row tables are refilled by the next pass
    } else {
      __syncthreads();  // every wave's ring reads are done before the partials overwrite LDS
      float* red = reinterpret_cast<float*>(lds);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int v = 0; v < 4; ++v) red[((wave * NT + tt) * MT + i) * 256 + (4 * q + v) * 16 + r] = Y[tt][i][v];
      __syncthreads();
      for (int idx = t; idx < 16 * MT * NC; idx += 64 * S) {
        const int m = idx / NC, nn = idx % NC;
        const int i = m >> 4, mr = m & 15;
        const int64_t rr = r0 + m;
        if (rr >= rows_total || n0 + nn >= N) continue;
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int hh = 0; hh < (GLU ? 2 : 1); ++hh) {
          const int tt = GLU ? hh * (NT / 2) + (nn >> 4) : (nn >> 4);
#pragma unroll
          for (int w2 = 0; w2 < S; ++w2) acc[hh] += red[((w2 * NT + tt) * MT + i) * 256 + mr * 16 + (nn & 15)];
        }
        store(m, n0 + nn, acc[0], acc[1]);
      }
      __syncthreads();  // the partials are read before the next pass refills the ring
    }
  };
  if constexpr (MTMAX == 2) {
    for (int64_t r0 = 0; r0 < rows_total; r0 += 32) {
      if (rows_total - r0 > 16) pass(std::integral_constant<int, 2>{}, r0);
      else pass(std::integral_constant<int, 1>{}, r0);
    }
  } else {
    for (int64_t r0 = 0; r0 < rows_total; r0 += 16) pass(std::integral_constant<int, 1>{}, r0);
  }
}

// Sorted grouped gather_qmm streamed per expert (the MoE layer of
// mlx/src/nn/moe.rs:84-170 over mlx/src/model/qwen35.rs:653-775's stacked
// experts): workgroup (expert e, part z of Z) takes tile-blocks z, z + Z, ...
// of expert e's N weight rows for each 16-row pass over the expert's rows.
// Per pass, each of its S waves loads the x operands of its K range (KB
// 128-code blocks) for the pass's rows ONCE -- gathered through the row
// table, held in registers with their group sums -- and then streams its
// tile-blocks (one 16-row weight tile, or a gate tile with its up tile for the
// SwiGLU) through a D-stage LDS ring by LDS DMA, as qmm_stream_kernel does; the
// S partial sums of each tile-block meet in LDS and the workgroup stores the
// pass's rows.  Against gather_decode_kernel (one 64-column block per
// workgroup), the x rows are fetched and converted once per pass instead of
// once per column block.  Each workgroup finds its expert's row segment in the
// sorted rhs itself (seg_lower_bound: two dependent probe rounds for 4096
// rows), so no offsets pre-pass runs.  Workgroups e = E write NaN for batch
// entries outside every expert's segment; rows whose lhs index is out of range
// are NaN.
template <int XT, int NT, int GB, int S, int D, int KB, bool GLU>
__global__ __launch_bounds__(64 * S) void gather_stream_kernel(QmmArgs a, int64_t nflat, int Z) {
  constexpr int MT = 1;
  static_assert(!GLU || NT == 2, "GLU pairs one gate tile with its up tile");
  static_assert(stream_fits<NT, MT, S, D, KB, GB>(), "LDS / vmcnt budget");
  constexpr int NS = KB / 2;                  // stages per tile-block
  constexpr int SW = KB * GB / 2;             // scale words per row in a wave's K range
  using L = StreamLds<NT, MT, S, D, SW>;
  constexpr int NDW = 2 * NT;                 // weight DMA per stage
  constexpr int PSC = NT * 16 * (SW / 4);     // 16-byte scale pieces per tile-block (biases as many)
  constexpr int NSC = (2 * PSC + 63) / 64;    // scale + bias DMA with the first stage
  constexpr int NC = GLU ? 8 * NT : 16 * NT;  // output columns per tile-block
  using XS = uint16_t;
  __shared__ __attribute__((aligned(1024))) char lds[L::TOTAL];
  __shared__ int64_t prow_x[16], prow_o[16];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int Mx = a.M, N = a.N, K = a.K;
  const int r = lane & 15, q = lane >> 4;
  const int pb = KB * wave;
  const int64_t e = blockIdx.x / Z;
  const int z = static_cast<int>(blockIdx.x - e * Z);
  XS* out = static_cast<XS*>(a.out);
  if (e == a.bm.nw) {
    if (z != 0) return;
    // offsets are clamped into [0, nflat]: indices that are not sorted as
    // promised give wrong rows, never out-of-range accesses
    const int64_t o0 = seg_lower_bound(a.bm.rhs, a.bm.rhs_dt, nflat, a.bm.nw, 0, lane);
    const int64_t oE = seg_lower_bound(a.bm.rhs, a.bm.rhs_dt, nflat, a.bm.nw, e, lane);
    const int64_t first_valid = min(max(o0, int64_t{0}), nflat);
    const int64_t end_valid = min(max(oE, first_valid), nflat);
    const int64_t nbad = first_valid + (nflat - end_valid);
    for (int64_t i = t; i < nbad * Mx * N; i += 64 * S) {
      const int64_t rr = i / N, n = i % N;
      const int64_t bi = rr / Mx, mrow = rr % Mx;
      const int64_t b = bi < first_valid ? bi : end_valid + (bi - first_valid);
      out[(b * Mx + mrow) * N + n] = from_f<XT>(__builtin_nanf(""));
    }
    return;
  }
  // the expert's row segment, searched in the sorted rhs by every wave (no
  // offsets pre-pass)
  const int64_t oe = seg_lower_bound(a.bm.rhs, a.bm.rhs_dt, nflat, a.bm.nw, e, lane);
  const int64_t oe1 = seg_lower_bound(a.bm.rhs, a.bm.rhs_dt, nflat, a.bm.nw, e + 1, lane);
  const int64_t blo = min(max(oe, int64_t{0}), nflat);
  const int64_t bhi = min(max(oe1, blo), nflat);
  if (blo >= bhi) return;  // workgroup-uniform
  const int64_t rows_total = (bhi - blo) * Mx;
  const int gshift = __builtin_ctz(a.gs);
  const int64_t wrow = K / 2, srow = (K >> gshift) * 2;
  const char* w = reinterpret_cast<const char*>(a.w + e * a.w_mat);
  const char* sp = reinterpret_cast<const char*>(static_cast<const XS*>(a.s) + e * a.s_mat);
  const char* bp = reinterpret_cast<const char*>(static_cast<const XS*>(a.b) + e * a.s_mat);
  const XS* x = static_cast<const XS*>(a.x);
  const int ntb = (N + NC - 1) / NC;
  const int nit = z < ntb ? (ntb - z + Z - 1) / Z : 0;
  if (nit == 0) return;  // workgroup-uniform
  const int total = nit * NS;
  auto wrow_of = [&](int tb, int row) {  // tile-block row -> weight row of the expert
    const int tt = row >> 4, rr = row & 15, n0 = tb * NC;
    return GLU ? static_cast<int64_t>(tt) * N + min(n0 + rr, N - 1) : static_cast<int64_t>(min(n0 + row, N - 1));
  };
  const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds_u32(lds)) + wave * L::WAVE;
  const char* lds_w = lds + wave * L::WAVE;
  float* red = reinterpret_cast<float*>(lds + S * L::WAVE);
  auto issue = [&](int it, int st) {
    const int tb = z + Z * it;
    const int slot = (it * NS + st) % D;
#pragma unroll
    for (int u = 0; u < NDW; ++u) {
      const int row = 8 * u + (lane >> 3);
      dma16(w + wrow_of(tb, row) * wrow + pb * 64 + st * 128 + 16 * ((lane & 7) ^ (row & 7)),
            lds_wave + slot * L::WST + u * 1024);
    }
    if (st == 0) {
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
  for (int64_t r0 = 0; r0 < rows_total; r0 += 16) {
    // row table of the pass: rows past the segment repeat its last row (their
    // outputs are not stored)
    if (t < 16) {
      const int64_t rr = min(r0 + t, rows_total - 1);
      const int64_t b = blo + rr / Mx, mrow = rr % Mx;
      const int64_t xm = a.bm.lhs ? load_index(a.bm.lhs, a.bm.lhs_dt, b) : b;
      const bool ok = xm >= 0 && xm < a.bm.nx;
      prow_x[t] = (ok ? xm : 0) * a.x_mat + mrow * K;
      prow_o[t] = ok ? (b * Mx + mrow) * N : ~((b * Mx + mrow) * N);
    }
    __syncthreads();
    g_u32x4_t A[KB][MT][4];
    {
      const char* xr = reinterpret_cast<const char*>(x + prow_x[r]) + pb * 256 + 16 * q;
#pragma unroll
      for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) A[b][0][j] = x_pairs(*reinterpret_cast<const g_u32x4_t*>(xr + b * 256 + 64 * j));
    }
    // the compiler's own loads are complete before the counted DMA starts
    __builtin_amdgcn_s_waitcnt(0);
    constexpr bool PRE = MT * GB <= 2;
    f32x4d_t XS_[PRE ? KB : 1][MT][GB];
    if constexpr (PRE) {
#pragma unroll
      for (int b = 0; b < KB; ++b) block_xsums<XT, MT, GB>(XS_[b], A[b]);
    }
    f32x4d_t Y[NT][MT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) Y[tt][0] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < D - 1; ++u)
      if (u < total) issue(u / NS, u % NS);
    uint32_t sw[NT][SW], bw[NT][SW];
    for (int it = 0; it < nit; ++it) {
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const int u = it * NS + st;
        const int later = min(D - 2, total - 1 - u);
        if (later >= 1) {
          if ((st + 1) % NS == 0) vm_wait<(D >= 3 ? NDW + NSC : 0)>();
          else vm_wait<(D >= 3 ? NDW : 0)>();
        } else {
          vm_wait<0>();
        }
        if (st == 0) {
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
            fac_block_xs<XT, NT, MT, GB, SW>(Y, A[2 * st + h], XS_[2 * st + h], wst, h, (2 * st + h) * GB, sw, bw, r,
                                             q);
          else
            fac_block<XT, NT, MT, GB, SW>(Y, A[2 * st + h], wst, h, (2 * st + h) * GB, sw, bw, r, q);
        }
      }
      // the S partial sums of tile-block it meet in LDS
      const int n0 = (z + Z * it) * NC;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          red[(wave * NT + tt) * 256 + (4 * q + v) * 16 + r] = Y[tt][0][v];
          Y[tt][0][v] = 0.f;
        }
      __syncthreads();
      for (int idx = t; idx < 16 * NC; idx += 64 * S) {
        const int m = idx / NC, nn = idx % NC;
        if (r0 + m >= rows_total || n0 + nn >= N) continue;
        float acc[2] = {0.f, 0.f};
#pragma unroll
        for (int hh = 0; hh < (GLU ? 2 : 1); ++hh) {
          const int tt = GLU ? hh : (nn >> 4);
#pragma unroll
          for (int w2 = 0; w2 < S; ++w2) acc[hh] += red[(w2 * NT + tt) * 256 + m * 16 + (nn & 15)];
        }
        const int64_t o = prow_o[m];
        const auto v = GLU ? swiglu_out<XT>(acc[0], acc[1]) : from_f<XT>(acc[0]);
        if (o >= 0) out[o + n0 + nn] = v;
        else out[~o + n0 + nn] = from_f<XT>(__builtin_nanf(""));
      }
      __syncthreads();  // the partials (and, after the last, the row table) are read before they are rewritten
    }
  }
}

struct GatCfg {
  int nt, s, d, kb;
  bool xl;
  int mt;
};

// Measured (256 experts, top 8, q4 gs 64, bf16, T = 64 / 512): four 16-row
// tiles per workgroup, x in registers, passes of 16 rows (two-tile MT passes
// need more registers than the extra weight re-reads cost: T = 512 gate
// 83.6 -> 65.1 us); K = 2048 (gate) four waves of four blocks, K = 512
// (down) two waves of two.  A wave's K range is at most four blocks (two at
// gs 32, whose scale words take twice the registers), so that the kernel
// stays below the VGPR limit next to its x ring; other K take the generic
// grouped kernel.
GatCfg gather_choose(const QmmArgs& a) {
  const int P = a.K >> 7;
  const int kb = a.gs == 32 ? 2 : 4;  // blocks per wave
  GatCfg c{0, 0, 0, 0, false, 1};
  if (P == 4) c = GatCfg{4, 2, 2, 2, false, 1};
  else if (P == 8) c = GatCfg{4, 4, 2, 2, false, 1};
  else if (P == 16 || (P == 32 && kb == 4)) c = GatCfg{4, P / kb, 2, kb, false, 1};
  else if (P == 2 && a.gs != 32) c = GatCfg{4, 1, 2, 2, false, 1};
  return c;
}

// instantiations whose register use reaches the VGPR limit (scale words of
// long K ranges at gs 32) are never produced by gather_choose
template <int GB, int S, int KB>
constexpr bool gat_regs_ok() {
  return !(GB == 4 && (KB >= 4 || S == 1));
}

template <int XT, int GB, bool GLU, int NT, int S, int D, int KB, bool XL, int MT>
hipError_t gat_go(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  if constexpr ((GLU && NT % 2 != 0) || KB % 2 != 0 || !gat_fits<NT, MT, S, D, XL, KB>() || !gat_regs_ok<GB, S, KB>()) {
    return hipErrorInvalidValue;
  } else {
    constexpr int NC = GLU ? 8 * NT : 16 * NT;
    const dim3 grid(static_cast<unsigned>((a.N + NC - 1) / NC * (E + 1)));
    hipLaunchKernelGGL((gather_decode_kernel<XT, NT, GB, S, D, KB, XL, GLU, MT>), grid, dim3(64 * S), 0, a.stream, a,
                       nflat, off);
    return hipGetLastError();
  }
}

#define IQMM_GAT_CONFIGS(X)                                                                             \
  X(4, 2, 2, 2, false, 1) X(4, 4, 2, 2, false, 1) X(4, 4, 2, 4, false, 1) X(4, 8, 2, 2, false, 1)      \
  X(4, 8, 2, 4, false, 1) X(4, 1, 2, 2, false, 1)

bool gat_instantiated(const GatCfg& c, int gs) {
  bool ok = false;
#define IQMM_GAT_K(NT_, S_, D_, KB_, XL_, MT_)                                                                 \
  ok = ok || (c.nt == NT_ && c.s == S_ && c.d == D_ && c.kb == KB_ && c.xl == XL_ && c.mt == MT_ &&              \
              gat_fits<NT_, MT_, S_, D_, XL_, KB_>() &&                                                        \
              (gs == 32 ? gat_regs_ok<4, S_, KB_>() : gs == 64 ? gat_regs_ok<2, S_, KB_>() : gat_regs_ok<1, S_, KB_>()));
  IQMM_GAT_CONFIGS(IQMM_GAT_K)
#undef IQMM_GAT_K
  return ok;
}

template <int XT, int GB, bool GLU>
hipError_t gather_dec_go(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  const GatCfg c = gather_choose(a);
#define IQMM_GAT(NT_, S_, D_, KB_, XL_, MT_)                                                              \
  if (c.nt == NT_ && c.s == S_ && c.d == D_ && c.kb == KB_ && c.xl == XL_ && c.mt == MT_)                \
    return gat_go<XT, GB, GLU, NT_, S_, D_, KB_, XL_, MT_>(a, nflat, E, off);
  IQMM_GAT_CONFIGS(IQMM_GAT)
#undef IQMM_GAT
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


int gat_cu_count() {
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

// two 16-row weight tiles per tile-block: a gate tile and its up tile, or two
// consecutive tiles (one tile: T = 512 gate 2048 -> 512 62-63 us, two: 60.7 us)
template <int XT, int GB, bool GLU, int S>
hipError_t gstream_go(const QmmArgs& a, int64_t nflat, int64_t E) {
  constexpr int NT = 2, D = 3, KB = 4;
  if constexpr (!stream_fits<NT, 1, S, D, KB, GB>()) {
    return hipErrorInvalidValue;
  } else {
    constexpr int NC = GLU ? 8 * NT : 16 * NT;
    const int ntb = (a.N + NC - 1) / NC;
    // about eight waves per CU over the experts: Z workgroups per expert
    const int64_t want = (8LL * gat_cu_count() + E * S - 1) / (E * S);
    const int Z = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(want, ntb)));
    const int64_t nblk = (E + 1) * Z;
    if (nblk > 0x7fffffffLL) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((gather_stream_kernel<XT, NT, GB, S, D, KB, GLU>), dim3(static_cast<unsigned>(nblk)),
                       dim3(64 * S), 0, a.stream, a, nflat, Z);
    return hipGetLastError();
  }
}

template <int XT, int GB, bool GLU>
hipError_t gstream_s(const QmmArgs& a, int64_t nflat, int64_t E) {
  switch (a.K / 512) {
    case 1: return gstream_go<XT, GB, GLU, 1>(a, nflat, E);
    case 2: return gstream_go<XT, GB, GLU, 2>(a, nflat, E);
    case 4: return gstream_go<XT, GB, GLU, 4>(a, nflat, E);
    default: return gstream_go<XT, GB, GLU, 8>(a, nflat, E);
  }
}

template <int XT>
hipError_t gstream_xt(const QmmArgs& a, int64_t nflat, int64_t E) {
  // gs 64 only (gather_stream_supported): at gs 32 the scale words of two
  // tiles exceed the register budget
  return a.glu ? gstream_s<XT, 2, true>(a, nflat, E) : gstream_s<XT, 2, false>(a, nflat, E);
}

}  // namespace

bool gather_stream_supported(const QmmArgs& a) {
  return a.transpose && a.mode == AFFINE && a.bits == 4 && (a.xdt == BF16 || a.xdt == F16) &&
         a.gs == 64 && a.bm.rhs != nullptr && a.N >= 1 &&
         (a.K == 512 || a.K == 1024 || a.K == 2048 || a.K == 4096) && (a.K / a.gs) % 8 == 0 && a.b != nullptr &&
         (reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 16 == 0;
}

hipError_t launch_gather_stream(const QmmArgs& a, int64_t nflat, int64_t E) {
  return a.xdt == BF16 ? gstream_xt<BF16>(a, nflat, E) : gstream_xt<F16>(a, nflat, E);
}


bool gather_decode_supported(const QmmArgs& a) {
  if (!(a.transpose && a.mode == AFFINE && a.bits == 4 && (a.xdt == BF16 || a.xdt == F16) && a.K % 128 == 0 &&
        a.N >= 1 && a.bm.rhs != nullptr))
    return false;
  if (a.gs != 32 && a.gs != 64 && a.gs != 128) return false;
  const GatCfg c = gather_choose(a);
  if (c.kb == 0 || c.s * c.kb * 128 != a.K || !gat_instantiated(c, a.gs)) return false;
  return (reinterpret_cast<uintptr_t>(a.s) | reinterpret_cast<uintptr_t>(a.b)) % 4 == 0 && ((a.K / a.gs) * 2) % 4 == 0;
}

hipError_t launch_gather_decode(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off) {
  if (a.glu) return a.xdt == BF16 ? gather_dec_gs<BF16, true>(a, nflat, E, off) : gather_dec_gs<F16, true>(a, nflat, E, off);
  return a.xdt == BF16 ? gather_dec_gs<BF16, false>(a, nflat, E, off) : gather_dec_gs<F16, false>(a, nflat, E, off);
}

}  // namespace iqmm
