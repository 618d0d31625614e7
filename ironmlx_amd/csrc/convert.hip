// convert.hip — dequantize and quantize on the GPU.
//
// dequantize (mlx/src/ops.rs:653-686; caller mlx/src/nn/embedding.rs:62-72):
//   one thread per packed word (dequant_words_kernel: 2 / 4 / 8-bit codes and
//   the fp modes, rows of whole 32-code chunks) or per 32-code chunk
//   (dequant_kernel: 3 / 5 / 6-bit codes and other rows), bit-exact either
//   way; with an index array, output row i is table row idx[i] (the embedding
//   lookup without dequantizing the whole table):
//   affine  v = rn(rn(s * q) + b)  (multiply and add rounded separately),
//   fp      v = rn(elem(q) * scale), then RNE to the output dtype.
// swiglu rows: the elementwise SwiGLU step of a fused gate_up product
//   (mlx/src/nn/mlp.rs:27-33), rounded like the unfused composition.
// quantize (mlx_quantize; makes the packed inputs):
//   one thread per quantization group, same arithmetic as MLX's per-group
//   rule (see oracle/iqmm_oracle.c for the restated rule), so codes, scales
//   and biases are bit-identical to the CPU restatement.  Divisions are IEEE
//   correctly rounded (hipcc's default for fp32 '/').
#include "launch.h"

namespace iqmm {

#pragma clang fp contract(off)

template <int SDT, int ODT, int MODE, int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(ConvArgs a, int64_t nchunks) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (id >= nchunks) return;
  using OS = typename Store<ODT>::T;
  constexpr bool AFF = MODE == AFFINE;
  const int K = a.K;
  const int cpr = (K + 31) >> 5;                 // chunks per row
  const int64_t orow = id / cpr;                 // output row
  const int c = static_cast<int>(id - orow * cpr);
  const int k0 = c * 32;
  const int ncode = min(32, K - k0);
  OS* dst = static_cast<OS*>(a.out) + orow * K + k0;
  // row gather: output row i takes table row idx[i] (negative from the end)
  int64_t row = orow;
  if (a.idx != nullptr) {
    row = load_index(a.idx, a.idx_dt, orow);
    if (row < 0) row += a.table_rows;
    if (row < 0 || row >= a.table_rows) {
      for (int j = 0; j < ncode; ++j) dst[j] = from_f<ODT>(__builtin_nanf(""));
      return;
    }
  }
  const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
  const uint32_t* src = a.w + row * wpr + static_cast<int64_t>(c) * BITS;
  uint32_t wd[BITS];
  if (ncode == 32) {
    load_chunk<BITS>(wd, src);
  } else {
    const int nw = (ncode * BITS + 31) / 32;
#pragma unroll
    for (int i = 0; i < BITS; ++i) wd[i] = i < nw ? src[i] : 0u;
  }
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const int G = K / gs;
  // a 32-code chunk lies in one group (affine and MX group sizes are multiples
  // of 32); nvfp4's 16-code groups give two per chunk: scales load once per chunk
  const int64_t g0 = row * G + k0 / gs;
  float s0, b0 = 0.f, s1;
  if constexpr (AFF) {
    using SS = typename Store<SDT>::T;
    s0 = s1 = to_f<SDT>(static_cast<const SS*>(a.s)[g0]);
    b0 = to_f<SDT>(static_cast<const SS*>(a.b)[g0]);
  } else {
    const uint8_t* s8 = static_cast<const uint8_t*>(a.s);
    s0 = fp_scale<MODE>(s8[g0]);
    s1 = (MODE == NVFP4 && k0 + 16 < K) ? fp_scale<MODE>(s8[g0 + 1]) : s0;
  }
  OS vals[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const uint32_t q = chunk_code<BITS>(wd, j);
    float v;
    if constexpr (AFF) {
      const float p = s0 * static_cast<float>(q);
      v = p + b0;
    } else {
      v = fp_elem<MODE>(q) * (j < 16 ? s0 : s1);
    }
    vals[j] = from_f<ODT>(v);
  }
  if (ncode == 32 && sizeof(OS) == 2) {
    uint4* d4 = reinterpret_cast<uint4*>(dst);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t u[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        u[j] = static_cast<uint32_t>(vals[8 * i + 2 * j]) |
               (static_cast<uint32_t>(vals[8 * i + 2 * j + 1]) << 16);
      d4[i] = make_uint4(u[0], u[1], u[2], u[3]);
    }
  } else {
    for (int j = 0; j < ncode; ++j) dst[j] = vals[j];
  }
}

// Row-segment dequantize (affine 2-, 4- and 8-bit codes; mxfp4, nvfp4,
// mxfp8).  Block b takes segment b % segs of output row b / segs; thread t
// takes packed words w0 + t + 256 u (U per thread, all loads issued before any
// arithmetic) and writes each word's 32 / BITS values as one contiguous
// store of 8 to 64 bytes, so a wave's store instruction covers one contiguous
// span (dequant_kernel's one-chunk-per-thread layout writes each thread's
// piece 16 bytes at a time, 64 bytes apart across lanes).  A word's codes lie
// in one group (groups are 16 codes or more).  Same arithmetic as
// dequant_kernel: s * q (exact in fp32) + b, or the fp element times its
// scale, rounded once to the output type.
template <int SDT, int ODT, int MODE, int BITS, int U>
__global__ __launch_bounds__(256) void dequant_words_kernel(ConvArgs a, int segs) {
  constexpr bool AFF = MODE == AFFINE;
  using SS = typename Store<AFF ? SDT : U8>::T;
  using OS = typename Store<ODT>::T;
  constexpr int CPW = 32 / BITS;  // codes per word
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const int K = a.K, W = K / CPW, G = K / gs;
  const int gshift = __builtin_ctz(gs);
  const int64_t orow = blockIdx.x / segs;
  const int w0 = static_cast<int>(blockIdx.x - orow * segs) * 256 * U + static_cast<int>(threadIdx.x);
  OS* dst = static_cast<OS*>(a.out) + orow * K;
  int64_t row = orow;
  if (a.idx != nullptr) {
    row = load_index(a.idx, a.idx_dt, orow);
    if (row < 0) row += a.table_rows;
    if (row < 0 || row >= a.table_rows) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int wi = w0 + 256 * u;
        if (wi < W)
          for (int j = 0; j < CPW; ++j) dst[wi * CPW + j] = from_f<ODT>(__builtin_nanf(""));
      }
      return;
    }
  }
  const uint32_t* src = a.w + row * W;
  const SS* sp = static_cast<const SS*>(a.s) + row * G;
  const SS* bp = AFF ? static_cast<const SS*>(a.b) + row * G : nullptr;
  uint32_t wd[U];
  SS sv[U], bv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int wi = min(w0 + 256 * u, W - 1);
    wd[u] = __builtin_nontemporal_load(src + wi);
    sv[u] = sp[(wi * CPW) >> gshift];
    if constexpr (AFF) bv[u] = bp[(wi * CPW) >> gshift];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int wi = w0 + 256 * u;
    if (wi >= W) break;
    float s0, b0 = 0.f;
    if constexpr (AFF) {
      s0 = to_f<SDT>(sv[u]);
      b0 = to_f<SDT>(bv[u]);
    } else {
      s0 = fp_scale<MODE>(sv[u]);
    }
    uint32_t o[CPW * sizeof(OS) / 4];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const uint32_t q = (wd[u] >> (j * BITS)) & ((1u << BITS) - 1);
      float v;
      if constexpr (AFF) {
        const float p = s0 * static_cast<float>(q);
        v = p + b0;
      } else {
        v = fp_elem<MODE>(q) * s0;
      }
      const OS e = from_f<ODT>(v);
      if constexpr (sizeof(OS) == 4) {
        o[j] = __builtin_bit_cast(uint32_t, e);
      } else {
        if (j % 2 == 0) o[j / 2] = static_cast<uint32_t>(e);
        else o[j / 2] |= static_cast<uint32_t>(e) << 16;
      }
    }
    OS* d = dst + wi * CPW;
    constexpr int NB = CPW * static_cast<int>(sizeof(OS));  // bytes per word's values
    if constexpr (NB == 8) {
      *reinterpret_cast<uint2*>(d) = make_uint2(o[0], o[1]);
    } else {
#pragma unroll
      for (int h = 0; h < NB / 16; ++h)
        reinterpret_cast<uint4*>(d)[h] = make_uint4(o[4 * h], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);
    }
  }
}

// round-to-nearest-even onto the element grid with saturation, written as the
// same grid search as the CPU restatement so ties and zero signs agree
template <int MODE>
__device__ __forceinline__ uint32_t nearest_code(float v) {
  constexpr int NPOS = MODE == MXFP8 ? 127 : 8;
  constexpr uint32_t SIGN = MODE == MXFP8 ? 0x80u : 0x8u;
  const float top = fp_elem<MODE>(NPOS - 1);
  float av = fminf(fabsf(v), top);
  if (__builtin_isnan(v)) return 0u;
  uint32_t best = 0;
  float gb = 0.f;
  for (int c = 1; c < NPOS; ++c) {
    const float g = fp_elem<MODE>(static_cast<uint32_t>(c));
    const float dg = fabsf(av - g), db = fabsf(av - gb);
    if (dg < db || (dg == db && (c & 1) == 0 && (best & 1u) == 1u)) {
      best = static_cast<uint32_t>(c);
      gb = g;
    }
  }
  const bool neg = v < 0.f || (v == 0.f && __builtin_signbit(v));
  return (neg && best != 0u) ? (best | SIGN) : best;
}

template <int WDT, int MODE, int BITS>
__global__ __launch_bounds__(256) void quant_kernel(ConvArgs a, int64_t ngroups) {
  const int64_t id = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (id >= ngroups) return;
  using WS = typename Store<WDT>::T;
  const int K = a.K;
  constexpr bool AFF = MODE == AFFINE;
  const int gs = AFF ? a.gs : ModeInfo<MODE>::GS;
  const int G = K / gs;
  const int64_t row = id / G;
  const int g = static_cast<int>(id - row * G);
  const WS* src = static_cast<const WS*>(a.src) + row * K + static_cast<int64_t>(g) * gs;
  const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
  // a group of gs codes fills gs*BITS/32 whole words (gs*BITS is a multiple of 32)
  uint32_t* dstw = a.wq + row * wpr + static_cast<int64_t>(g) * gs * BITS / 32;
  const int nwords = gs * BITS / 32;

  if constexpr (AFF) {
    const float n_bins = static_cast<float>((1 << BITS) - 1), eps = 1e-7f;
    float wmax = -__builtin_inff(), wmin = __builtin_inff();
    for (int j = 0; j < gs; ++j) {
      const float v = to_f<WDT>(src[j]);
      wmax = fmaxf(wmax, v);
      wmin = fminf(wmin, v);
    }
    const bool mask = fabsf(wmin) > fabsf(wmax);
    float scale = fmaxf((wmax - wmin) / n_bins, eps);
    scale = mask ? scale : -scale;
    const float edge = mask ? wmin : wmax;
    const float q0 = rintf(edge / scale);
    float bias = 0.f;
    if (q0 != 0.f) {
      scale = edge / q0;
      bias = edge;
    }
    for (int wi = 0; wi < nwords; ++wi) {
      // codes overlapping word wi: bits [32wi, 32wi+32)
      uint32_t word = 0;
      const int jlo = (32 * wi) / BITS, jhi = min(gs - 1, (32 * wi + 31) / BITS);
      for (int j = jlo; j <= jhi; ++j) {
        float q = rintf((to_f<WDT>(src[j]) - bias) / scale);
        q = fminf(fmaxf(q, 0.f), n_bins);
        const uint32_t qi = static_cast<uint32_t>(q);
        const int bit = j * BITS - 32 * wi;
        word |= bit >= 0 ? (qi << bit) : (qi >> (-bit));
      }
      dstw[wi] = word;
    }
    using SS = typename Store<WDT>::T;
    static_cast<SS*>(a.sq)[id] = from_f<WDT>(scale);
    static_cast<SS*>(a.bq)[id] = from_f<WDT>(bias);
  } else {
    float amax = 0.f;
    for (int j = 0; j < gs; ++j) amax = fmaxf(amax, fabsf(to_f<WDT>(src[j])));
    uint32_t sc;
    float sdec;
    if constexpr (MODE == NVFP4) {
      sc = nearest_code<MXFP8>(amax / 6.0f);   // e4m3 block scale
      sdec = e4m3_to_f(sc);
    } else {
      constexpr int emax_elem = MODE == MXFP8 ? 8 : 2;
      int ex = 0;
      if (amax > 0.f) frexpf(amax, &ex);
      int e = amax > 0.f ? (ex - 1) - emax_elem : -127;
      e = e < -127 ? -127 : (e > 127 ? 127 : e);
      sc = static_cast<uint32_t>(e + 127);
      sdec = ldexpf(1.0f, e);
    }
    for (int wi = 0; wi < nwords; ++wi) {
      uint32_t word = 0;
      const int per = 32 / BITS;
      for (int j = 0; j < per; ++j) {
        const float v = sdec > 0.f ? to_f<WDT>(src[wi * per + j]) / sdec : 0.f;
        word |= nearest_code<MODE>(v) << (j * BITS);
      }
      dstw[wi] = word;
    }
    static_cast<uint8_t*>(a.sq)[id] = static_cast<uint8_t>(sc);
  }
}

namespace {
template <int SDT, int ODT>
hipError_t deq_by_mode(const ConvArgs& a, int64_t nchunks, dim3 grid) {
#define IQMM_D(MODE, BITS) \
  hipLaunchKernelGGL((dequant_kernel<SDT, ODT, MODE, BITS>), grid, dim3(256), 0, a.stream, a, nchunks); \
  return hipGetLastError()
  switch (a.mode) {
    case AFFINE:
      switch (a.bits) {
        case 2: IQMM_D(AFFINE, 2);
        case 3: IQMM_D(AFFINE, 3);
        case 4: IQMM_D(AFFINE, 4);
        case 5: IQMM_D(AFFINE, 5);
        case 6: IQMM_D(AFFINE, 6);
        case 8: IQMM_D(AFFINE, 8);
      }
      break;
    case MXFP4: IQMM_D(MXFP4, 4);
    case MXFP8: IQMM_D(MXFP8, 8);
    case NVFP4: IQMM_D(NVFP4, 4);
  }
#undef IQMM_D
  return hipErrorInvalidValue;
}

template <int ODT>
hipError_t deq_by_sdt(const ConvArgs& a, int64_t nchunks, dim3 grid) {
  if (a.mode != AFFINE) return deq_by_mode<U8, ODT>(a, nchunks, grid);
  switch (a.sdt) {
    case F32: return deq_by_mode<F32, ODT>(a, nchunks, grid);
    case F16: return deq_by_mode<F16, ODT>(a, nchunks, grid);
    case BF16: return deq_by_mode<BF16, ODT>(a, nchunks, grid);
  }
  return hipErrorInvalidValue;
}

template <int WDT>
hipError_t quant_by_mode(const ConvArgs& a, int64_t ngroups, dim3 grid) {
#define IQMM_Q(MODE, BITS) \
  hipLaunchKernelGGL((quant_kernel<WDT, MODE, BITS>), grid, dim3(256), 0, a.stream, a, ngroups); \
  return hipGetLastError()
  switch (a.mode) {
    case AFFINE:
      switch (a.bits) {
        case 2: IQMM_Q(AFFINE, 2);
        case 3: IQMM_Q(AFFINE, 3);
        case 4: IQMM_Q(AFFINE, 4);
        case 5: IQMM_Q(AFFINE, 5);
        case 6: IQMM_Q(AFFINE, 6);
        case 8: IQMM_Q(AFFINE, 8);
      }
      break;
    case MXFP4: IQMM_Q(MXFP4, 4);
    case MXFP8: IQMM_Q(MXFP8, 8);
    case NVFP4: IQMM_Q(NVFP4, 4);
  }
#undef IQMM_Q
  return hipErrorInvalidValue;
}
}  // namespace

template <int SDT, int ODT, int MODE, int BITS>
hipError_t deq_words_go(const ConvArgs& a) {
  constexpr int U = 2;
  const int W = a.K * BITS / 32;
  const int segs = (W + 256 * U - 1) / (256 * U);
  const int64_t nblk = a.rows * segs;
  if (nblk > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((dequant_words_kernel<SDT, ODT, MODE, BITS, U>), dim3(static_cast<unsigned>(nblk)), dim3(256), 0,
                     a.stream, a, segs);
  return hipGetLastError();
}

template <int SDT, int ODT>
hipError_t deq_words(const ConvArgs& a) {
  switch (a.mode) {
    case MXFP4: return deq_words_go<U8, ODT, MXFP4, 4>(a);
    case NVFP4: return deq_words_go<U8, ODT, NVFP4, 4>(a);
    case MXFP8: return deq_words_go<U8, ODT, MXFP8, 8>(a);
  }
  switch (a.bits) {
    case 2: return deq_words_go<SDT, ODT, AFFINE, 2>(a);
    case 4: return deq_words_go<SDT, ODT, AFFINE, 4>(a);
    default: return deq_words_go<SDT, ODT, AFFINE, 8>(a);
  }
}

template <int ODT>
hipError_t deq_words_sdt(const ConvArgs& a) {
  if (a.mode != AFFINE) return deq_words<U8, ODT>(a);
  switch (a.sdt) {
    case F32: return deq_words<F32, ODT>(a);
    case F16: return deq_words<F16, ODT>(a);
    default: return deq_words<BF16, ODT>(a);
  }
}

hipError_t launch_dequantize(const ConvArgs& a) {
  const int64_t nchunks = a.rows * ((a.K + 31) / 32);
  if (nchunks == 0) return hipSuccess;
  // whole words of one group each (affine 2 / 4 / 8-bit, the fp modes): the
  // row-segment kernel (128256 x 4096 q4 table into bf16: 364 -> 237 us,
  // 3.7 -> 5.7 TB/s); 3 / 5 / 6-bit codes keep the chunk kernel
  const bool words = a.mode != AFFINE || a.bits == 2 || a.bits == 4 || a.bits == 8;
  const int gsz = a.mode == AFFINE ? a.gs : a.mode == NVFP4 ? 16 : 32;
  if (words && a.K % gsz == 0 && a.K % 32 == 0) {
    switch (a.odt) {
      case F32: return deq_words_sdt<F32>(a);
      case F16: return deq_words_sdt<F16>(a);
      case BF16: return deq_words_sdt<BF16>(a);
    }
    return hipErrorInvalidValue;
  }
  const int64_t nblk = (nchunks + 255) / 256;
  if (nblk > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  dim3 grid(static_cast<unsigned>(nblk));
  switch (a.odt) {
    case F32: return deq_by_sdt<F32>(a, nchunks, grid);
    case F16: return deq_by_sdt<F16>(a, nchunks, grid);
    case BF16: return deq_by_sdt<BF16>(a, nchunks, grid);
  }
  return hipErrorInvalidValue;
}

// SwiGLU epilogue of a fused gate_up product: gu [rows, 2n] -> out [rows, n]
template <int DT>
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const typename Store<DT>::T* gu,
                                                          typename Store<DT>::T* out, int64_t rows,
                                                          int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * n) return;
  const int64_t r = i / n, c = i - r * n;
  const typename Store<DT>::T* src = gu + r * 2 * n;
  out[i] = swiglu_out<DT>(to_f<DT>(src[c]), to_f<DT>(src[n + c]));
}

// x / scales / biases of a mixed-dtype call, upcast to float32 (exact)
__global__ __launch_bounds__(256) void cast_f32_kernel(const uint16_t* src, int sdt, float* dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
    dst[i] = sdt == F16 ? h_to_f(src[i]) : bf16_to_f(src[i]);
}

hipError_t launch_cast_f32(const void* src, int sdt, float* dst, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  if (sdt != F16 && sdt != BF16) return hipErrorInvalidValue;
  const int64_t nb = (n + 255) / 256;
  const unsigned grid = static_cast<unsigned>(nb < 65536 ? nb : 65536);
  hipLaunchKernelGGL(cast_f32_kernel, dim3(grid), dim3(256), 0, st, static_cast<const uint16_t*>(src), sdt, dst, n);
  return hipGetLastError();
}

hipError_t launch_swiglu_rows(const void* gu, void* out, int64_t rows, int64_t n, int dt,
                              hipStream_t st) {
  const int64_t tot = rows * n;
  if (tot == 0) return hipSuccess;
  const int64_t nblk = (tot + 255) / 256;
  if (nblk > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(nblk));
  switch (dt) {
    case F32:
      hipLaunchKernelGGL(swiglu_rows_kernel<F32>, grid, dim3(256), 0, st, static_cast<const float*>(gu),
                         static_cast<float*>(out), rows, n);
      break;
    case F16:
      hipLaunchKernelGGL(swiglu_rows_kernel<F16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(gu),
                         static_cast<uint16_t*>(out), rows, n);
      break;
    case BF16:
      hipLaunchKernelGGL(swiglu_rows_kernel<BF16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(gu),
                         static_cast<uint16_t*>(out), rows, n);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_quantize(const ConvArgs& a) {
  const int gs = a.gs;
  const int64_t ngroups = a.rows * (a.K / gs);
  if (ngroups == 0) return hipSuccess;
  const int64_t nblk = (ngroups + 255) / 256;
  if (nblk > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  dim3 grid(static_cast<unsigned>(nblk));
  switch (a.sdt) {  // sdt carries the source (w) dtype for quantize
    case F32: return quant_by_mode<F32>(a, ngroups, grid);
    case F16: return quant_by_mode<F16>(a, ngroups, grid);
    case BF16: return quant_by_mode<BF16>(a, ngroups, grid);
  }
  return hipErrorInvalidValue;
}

}  // namespace iqmm
