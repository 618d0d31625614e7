/*
 * iqmm_oracle.c — CPU restatement of MLX's quantized-matmul semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in ironmlx_amd/csrc.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it; the product path never does.
 *
 * What it restates.  ironmlx reaches the quantized path through
 *   mlx/src/ops.rs:653-686  dequantize        -> mlx_dequantize
 *   mlx/src/ops.rs:695-727  quantized_matmul  -> mlx_quantized_matmul
 *   mlx/src/nn/moe.rs:55-183 the per-expert loop a gather_qmm replaces
 * The arithmetic itself lives in MLX v0.31.1 (mlx-sys/build.rs:39), which is
 * not vendored (vendor/mlx-c is an empty submodule, .gitmodules:1-3).  The
 * rules below are MLX's published semantics, restated from its documentation
 * and source as remembered; points that only an MLX import could confirm are
 * marked [UPSTREAM-UNVERIFIED].
 *
 *  - Packing: each row of a quantized matrix is an LSB-first bit stream of
 *    `bits`-wide codes stored in little-endian uint32 words.  For bits in
 *    {2,4,8} this is "value j of a word at bit j*bits"; for bits 3/5/6 codes
 *    straddle word boundaries (MLX packs 3/6-bit as 8/4 codes per 3 bytes,
 *    which is the same bit stream) [UPSTREAM-UNVERIFIED for 3/5/6].
 *  - Affine dequant: w = fp32(s*q) + b, rounded once to fp32 after each of the
 *    multiply and the add (no fusion), then rounded RNE to the output dtype.
 *    For fp16/bf16 scales s*q is exact, so fused and unfused agree.
 *  - mxfp8: e4m3fn codes (4 per word) * 2^(e-127), e = one uint8 per 32.
 *    mxfp4: e2m1 codes (8 per word) * 2^(e-127), one uint8 per 32.
 *    nvfp4: e2m1 codes (8 per word) * e4m3fn scale, one uint8 per 16.
 *  - Matmul: out[m,n] = sum_k x[m,k] * w[n,k] (transpose) or x[m,k]*w[k,n]
 *    with dequantized fp32 weights, accumulated in fp32 (the tolerance
 *    contract names fp32 accumulation; MLX's CPU kernel accumulates in the
 *    input type [UPSTREAM-UNVERIFIED]), rounded once to the output dtype.
 *  - Affine quantize (MLX's per-group rule): scale=max((max-min)/(2^b-1),1e-7),
 *    signed toward the larger-magnitude edge, q0=rint(edge/scale), and when
 *    q0!=0 the scale is snapped to edge/q0 and bias=edge.
 *    q = clamp(rint((w-bias)/scale), 0, 2^b-1) [UPSTREAM-UNVERIFIED: eps and
 *    the edge snap].
 *  - FP quantize: OCP MX v1.0 shared exponent floor(log2(amax)) - emax_elem
 *    for mxfp4/mxfp8, NVIDIA's amax/6 e4m3 block scale for nvfp4; element
 *    conversion RNE with saturation [UPSTREAM-UNVERIFIED: MLX's exact scale
 *    selection].
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { IQO_F32 = 0, IQO_F16 = 1, IQO_BF16 = 2 };
enum { IQO_AFFINE = 0, IQO_MXFP4 = 1, IQO_MXFP8 = 2, IQO_NVFP4 = 3 };

/* ------------------------------------------------------------------ */
/* scalar conversions, written from the IEEE-754 / OCP definitions      */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float iqo_bf16_to_float(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t iqo_float_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;                       /* round to nearest, ties to even */
  return (uint16_t)(u >> 16);
}

float iqo_half_to_float(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) {
    /* zero / subnormal: m * 2^-24 is exact in fp32 */
    float v = (float)m * 5.9604644775390625e-08f;
    return s ? -v : v;
  }
  if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
  return u2f(s | ((e + 112) << 23) | (m << 13));
}

uint16_t iqo_float_to_half(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00;           /* NaN */
  if (a >= 0x477ff000u) return sign | 0x7c00;          /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                               /* below 2^-14: subnormal */
    /* value in units of 2^-24, rounded to nearest even */
    uint32_t e = a >> 23;
    if (e < 102) return sign;                           /* < 2^-25: rounds to 0 */
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126 - e;                           /* 2^(e-127)*mant/2^23 / 2^-24 */
    uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return sign | (uint16_t)q;
  }
  uint32_t e = (a >> 23) - 112, mant = a & 0x7fffffu;
  uint32_t q = (e << 10) | (mant >> 13), rem = mant & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++;  /* carry may bump exponent: correct */
  return sign | (uint16_t)q;
}

/* e4m3fn: bias 7, no infinities, S.1111.111 is NaN, max 448 */
float iqo_e4m3_to_float(uint8_t c) {
  int s = c >> 7, e = (c >> 3) & 0xf, m = c & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return s ? -v : v;
}
/* e2m1: bias 1, values {0,.5,1,1.5,2,3,4,6} */
float iqo_e2m1_to_float(uint8_t c) {
  int s = (c >> 3) & 1, e = (c >> 1) & 3, m = c & 1;
  float v = e == 0 ? 0.5f * m : ldexpf((float)(2 + m), e - 2);
  return s ? -v : v;
}
/* e8m0: 2^(e-127), 255 is NaN */
float iqo_e8m0_to_float(uint8_t c) {
  if (c == 255) return NAN;
  return ldexpf(1.0f, (int)c - 127);
}

/* round-to-nearest-even onto a small float grid with saturation.  The grid is
 * enumerated from the decoder, so encode is the exact inverse of decode. */
static uint8_t nearest_code(float v, float (*dec)(uint8_t), int ncodes_pos, uint8_t sign_bit) {
  float a = fminf(fabsf(v), dec((uint8_t)(ncodes_pos - 1)));   /* saturate */
  uint8_t best = 0;
  if (isnan(v)) return 0;
  for (int c = 1; c < ncodes_pos; ++c) {
    float g = dec((uint8_t)c), gb = dec(best);
    if (isnan(g)) continue;
    float dg = fabsf(a - g), db = fabsf(a - gb);
    /* ties go to the code with even mantissa LSB */
    if (dg < db || (dg == db && (c & 1) == 0 && (best & 1) == 1)) best = (uint8_t)c;
  }
  return (v < 0 || (v == 0 && signbit(v))) && best != 0 ? (uint8_t)(best | sign_bit) : best;
}
uint8_t iqo_float_to_e4m3(float v) { return nearest_code(v, iqo_e4m3_to_float, 127, 0x80); }
uint8_t iqo_float_to_e2m1(float v) { return nearest_code(v, iqo_e2m1_to_float, 8, 0x8); }

static inline float load_f(const void* p, int dt, int64_t i) {
  switch (dt) {
    case IQO_F32: return ((const float*)p)[i];
    case IQO_F16: return iqo_half_to_float(((const uint16_t*)p)[i]);
    default: return iqo_bf16_to_float(((const uint16_t*)p)[i]);
  }
}
static inline void store_f(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case IQO_F32: ((float*)p)[i] = v; break;
    case IQO_F16: ((uint16_t*)p)[i] = iqo_float_to_half(v); break;
    default: ((uint16_t*)p)[i] = iqo_float_to_bf16(v); break;
  }
}

/* value rounded to dt and read back as float */
static inline float load_round(float v, int dt) {
  switch (dt) {
    case IQO_F32: return v;
    case IQO_F16: return iqo_half_to_float(iqo_float_to_half(v));
    default: return iqo_bf16_to_float(iqo_float_to_bf16(v));
  }
}

/* ------------------------------------------------------------------ */
/* bit stream                                                          */
/* ------------------------------------------------------------------ */
/* code j of a row that starts at word pointer `row` */
static inline uint32_t get_code(const uint32_t* row, int64_t j, int bits) {
  uint64_t bit = (uint64_t)j * bits;
  uint64_t w = bit >> 5;
  uint32_t sh = bit & 31;
  uint64_t v = row[w] >> sh;
  if (sh + bits > 32) v |= (uint64_t)row[w + 1] << (32 - sh);
  return (uint32_t)v & ((1u << bits) - 1);
}
static inline void put_code(uint32_t* row, int64_t j, int bits, uint32_t q) {
  uint64_t bit = (uint64_t)j * bits;
  uint64_t w = bit >> 5;
  uint32_t sh = bit & 31;
  row[w] |= q << sh;
  if (sh + bits > 32) row[w + 1] |= q >> (32 - sh);
}

void iqo_pack(const uint32_t* codes, int64_t rows, int64_t K, int bits, uint32_t* out) {
  int64_t wpr = K * bits / 32;
  memset(out, 0, sizeof(uint32_t) * rows * wpr);
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < K; ++j) put_code(out + r * wpr, j, bits, codes[r * K + j]);
}
void iqo_unpack(const uint32_t* w, int64_t rows, int64_t K, int bits, uint32_t* codes) {
  int64_t wpr = K * bits / 32;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < K; ++j) codes[r * K + j] = get_code(w + r * wpr, j, bits);
}

/* element decode of code q for a given mode */
static inline float decode_elem(uint32_t q, int mode) {
  return mode == IQO_MXFP8 ? iqo_e4m3_to_float((uint8_t)q) : iqo_e2m1_to_float((uint8_t)q);
}
static inline float decode_scale(uint8_t c, int mode) {
  return mode == IQO_NVFP4 ? iqo_e4m3_to_float(c) : iqo_e8m0_to_float(c);
}

/* ------------------------------------------------------------------ */
/* dequantize: w [rows, K*bits/32] -> out [rows, K]                    */
/* ------------------------------------------------------------------ */
int iqo_dequantize(const uint32_t* w, const void* scales, const void* biases, int sdt,
                   int64_t rows, int64_t K, int gs, int bits, int mode, void* out, int odt) {
  int64_t wpr = K * bits / 32, G = K / gs;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint32_t* row = w + r * wpr;
    for (int64_t k = 0; k < K; ++k) {
      uint32_t q = get_code(row, k, bits);
      float v;
      if (mode == IQO_AFFINE) {
        float s = load_f(scales, sdt, r * G + k / gs), b = load_f(biases, sdt, r * G + k / gs);
        float p = s * (float)q;   /* -ffp-contract=off: separate roundings */
        v = p + b;
      } else {
        float s = decode_scale(((const uint8_t*)scales)[r * G + k / gs], mode);
        v = decode_elem(q, mode) * s;
      }
      store_f(out, odt, r * K + k, v);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* quantized matmul (2-D).                                              */
/*   transpose=1: x [M,K], w [N, K*bits/32], s/b [N, K/gs]              */
/*   transpose=0: x [M,K], w [K, N*bits/32], s/b [K, N/gs]              */
/* ------------------------------------------------------------------ */
int iqo_qmm(const void* x, int xdt, int64_t M, int64_t K, const uint32_t* w,
            const void* scales, const void* biases, int sdt, int64_t N, int transpose,
            int gs, int bits, int mode, void* out, int odt, int nthreads) {
  /* dequantize the weight to fp32 once, then an fp32-accumulating product */
  int64_t rows = transpose ? N : K, cols = transpose ? K : N;
  float* wd = (float*)malloc(sizeof(float) * rows * cols);
  float* xf = (float*)malloc(sizeof(float) * M * K);
  if (!wd || !xf) { free(wd); free(xf); return 1; }
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
  iqo_dequantize(w, scales, biases, sdt, rows, cols, gs, bits, mode, wd, IQO_F32);
  for (int64_t i = 0; i < M * K; ++i) xf[i] = load_f(x, xdt, i);
  if (transpose) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; ++m)
      for (int64_t n = 0; n < N; ++n) {
        const float* xr = xf + m * K;
        const float* wr = wd + n * K;
        float acc = 0.f;
        for (int64_t k = 0; k < K; ++k) acc += xr[k] * wr[k];
        store_f(out, odt, m * N + n, acc);
      }
  } else {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
      float* acc = (float*)calloc(N, sizeof(float));
      for (int64_t k = 0; k < K; ++k) {
        float xv = xf[m * K + k];
        const float* wr = wd + k * N;
        for (int64_t n = 0; n < N; ++n) acc[n] += xv * wr[n];
      }
      for (int64_t n = 0; n < N; ++n) store_f(out, odt, m * N + n, acc[n]);
      free(acc);
    }
  }
  free(wd);
  free(xf);
  return 0;
}

/* GEMV in the streaming form a CPU backend uses: for each output row the
 * packed codes are decoded group by group and dotted with x on the fly, no
 * dequantized copy.  Same result contract as iqo_qmm (fp32 accumulate);
 * this is the timed CPU baseline. */
int iqo_qmv_affine(const void* x, int xdt, int64_t M, int64_t K, const uint32_t* w,
                   const void* scales, const void* biases, int sdt, int64_t N, int gs, int bits,
                   void* out, int odt, int nthreads) {
  int64_t wpr = K * bits / 32, G = K / gs;
  float* xf = (float*)malloc(sizeof(float) * M * K);
  if (!xf) return 1;
  for (int64_t i = 0; i < M * K; ++i) xf[i] = load_f(x, xdt, i);
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const uint32_t* row = w + n * wpr;
      const float* xr = xf + m * K;
      float acc = 0.f;
      for (int64_t g = 0; g < G; ++g) {
        float s = load_f(scales, sdt, n * G + g), b = load_f(biases, sdt, n * G + g);
        for (int64_t k = g * gs; k < (g + 1) * gs; ++k) {
          float p = s * (float)get_code(row, k, bits);
          acc += xr[k] * (p + b);
        }
      }
      store_f(out, odt, m * N + n, acc);
    }
  free(xf);
  return 0;
}

/* ------------------------------------------------------------------ */
/* quantize                                                             */
/* ------------------------------------------------------------------ */
/* w [rows, K] -> wq [rows, K*bits/32], scales/biases [rows, K/gs] in sdt */
int iqo_affine_quantize(const void* w, int wdt, int64_t rows, int64_t K, int gs, int bits,
                        uint32_t* wq, void* scales, void* biases, int sdt) {
  int64_t wpr = K * bits / 32, G = K / gs;
  float n_bins = (float)((1 << bits) - 1), eps = 1e-7f;
  memset(wq, 0, sizeof(uint32_t) * rows * wpr);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < G; ++g) {
      int64_t base = r * K + g * gs;
      float wmax = -INFINITY, wmin = INFINITY;
      for (int j = 0; j < gs; ++j) {
        float v = load_f(w, wdt, base + j);
        wmax = fmaxf(wmax, v);
        wmin = fminf(wmin, v);
      }
      int mask = fabsf(wmin) > fabsf(wmax);
      float scale = fmaxf((wmax - wmin) / n_bins, eps);
      scale = mask ? scale : -scale;
      float edge = mask ? wmin : wmax;
      float q0 = rintf(edge / scale);
      float bias = 0.f;
      if (q0 != 0.f) {
        scale = edge / q0;
        bias = edge;
      }
      for (int j = 0; j < gs; ++j) {
        float v = load_f(w, wdt, base + j);
        float q = rintf((v - bias) / scale);
        q = fminf(fmaxf(q, 0.f), n_bins);
        put_code(wq + r * wpr, g * gs + j, bits, (uint32_t)q);
      }
      store_f(scales, sdt, r * G + g, scale);
      store_f(biases, sdt, r * G + g, bias);
    }
  }
  return 0;
}

/* mode in {MXFP4, MXFP8, NVFP4}; scales uint8 [rows, K/gs] */
int iqo_fp_quantize(const void* w, int wdt, int64_t rows, int64_t K, int mode, uint32_t* wq,
                    uint8_t* scales) {
  int gs = mode == IQO_NVFP4 ? 16 : 32, bits = mode == IQO_MXFP8 ? 8 : 4;
  int64_t wpr = K * bits / 32, G = K / gs;
  memset(wq, 0, sizeof(uint32_t) * rows * wpr);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < G; ++g) {
      int64_t base = r * K + g * gs;
      float amax = 0.f;
      for (int j = 0; j < gs; ++j) amax = fmaxf(amax, fabsf(load_f(w, wdt, base + j)));
      uint8_t sc;
      float sdec;
      if (mode == IQO_NVFP4) {
        sc = iqo_float_to_e4m3(amax / 6.0f);
        sdec = iqo_e4m3_to_float(sc);
      } else {
        int emax_elem = mode == IQO_MXFP8 ? 8 : 2;
        int ex = 0;
        if (amax > 0.f) frexpf(amax, &ex);           /* amax = f*2^ex, f in [0.5,1) */
        int e = amax > 0.f ? (ex - 1) - emax_elem : -127;
        if (e < -127) e = -127;
        if (e > 127) e = 127;
        sc = (uint8_t)(e + 127);
        sdec = ldexpf(1.0f, e);
      }
      for (int j = 0; j < gs; ++j) {
        float v = sdec > 0.f ? load_f(w, wdt, base + j) / sdec : 0.f;
        uint32_t q = mode == IQO_MXFP8 ? iqo_float_to_e4m3(v) : iqo_float_to_e2m1(v);
        put_code(wq + r * wpr, g * gs + j, bits, q);
      }
      scales[r * G + g] = sc;
    }
  }
  return 0;
}

/* array conversions (used by the Python wrapper for speed) */
void iqo_from_float_array(const float* in, int64_t n, int dt, void* out) {
  for (int64_t i = 0; i < n; ++i) store_f(out, dt, i, in[i]);
}
void iqo_to_float_array(const void* in, int64_t n, int dt, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = load_f(in, dt, i);
}

/* ------------------------------------------------------------------ */
/* SwiGLU and MoE routing (mlx/src/nn/mlp.rs:27-33,                    */
/* mlx/src/nn/activations.rs:7-10, mlx/src/nn/moe.rs:67-168)           */
/* ------------------------------------------------------------------ */

/* exp(x) by Cody-Waite reduction x = n ln2 + r (|r| <= ln2 / 2, ln2 split
 * into a 16-bit head and a tail so n * head is exact) and the degree-7
 * Taylor polynomial of e^r in Horner form with explicit fmaf, then a 2^n
 * scale.  Every step is a correctly rounded IEEE operation, so the library's
 * device copy of these steps gives bit-identical results.  MLX's own exp is
 * not available here: this function is pinned against float64 exp (<= 2 ulp)
 * by the tests, not against MLX. */
float iqo_expf(float x) {
  if (x != x) return x;
  if (x > 88.7228394f) return INFINITY;
  if (x < -103.972084f) return 0.0f;
  const float n = rintf(x * 1.44269502f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860682e-6f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

/* silu(g) * u of stored (rounded) gate / up values, each elementwise op
 * rounded to dt: s = rn(1 / (1 + exp(-g))), a = rn(g * s), out = rn(a * u). */
static float swiglu1(float g, float u, int dt) {
  const float gr = load_round(g, dt), ur = load_round(u, dt);
  const float sg = load_round(1.0f / (1.0f + iqo_expf(-gr)), dt);
  const float a = load_round(gr * sg, dt);
  return a * ur;
}

/* gu [rows, 2I] (gate | up) -> out [rows, I] */
void iqo_swiglu(const void* gu, int dt, int64_t rows, int64_t I, void* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < I; ++c)
      store_f(out, dt, r * I + c, swiglu1(load_f(gu, dt, r * 2 * I + c), load_f(gu, dt, r * 2 * I + I + c), dt));
}

/* Router of one token set: softmax over E experts in fp32, the sum taken in
 * the library's fixed order (64 lane partial sums over e = lane + 64 j in j
 * order, then a butterfly over lane distances 32, 16, .., 1), probabilities
 * rounded to dt; the k largest by a stable descending sort (ties: lower id,
 * as a stable argsort of -p, moe.rs:72-73); with norm, rn(p / rn(sum of the
 * k in slot order)) (moe.rs:76-82). */
void iqo_moe_route(const void* logits, int dt, int64_t T, int64_t E, int k, int norm, float* scores,
                   int32_t* experts) {
  float* p = (float*)malloc(sizeof(float) * (size_t)E);
  int32_t* ord = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  float part[64];
  for (int64_t t = 0; t < T; ++t) {
    float m = -INFINITY;
    for (int64_t e = 0; e < E; ++e) {
      p[e] = load_f(logits, dt, t * E + e);
      m = fmaxf(m, p[e]);
    }
    for (int l = 0; l < 64; ++l) part[l] = 0.0f;
    for (int64_t e = 0; e < E; ++e) {
      p[e] = iqo_expf(p[e] - m);
      part[e % 64] = part[e % 64] + p[e];
    }
    for (int off = 32; off > 0; off >>= 1) {
      float nx[64];
      for (int l = 0; l < 64; ++l) nx[l] = part[l] + part[l ^ off];
      memcpy(part, nx, sizeof(nx));
    }
    const float s = part[0];
    for (int64_t e = 0; e < E; ++e) p[e] = load_round(p[e] / s, dt);
    /* stable insertion sort of ids by descending p */
    for (int64_t e = 0; e < E; ++e) {
      int64_t j = e;
      while (j > 0 && p[ord[j - 1]] < p[e]) { ord[j] = ord[j - 1]; --j; }
      ord[j] = (int32_t)e;
    }
    float tot = 0.0f;
    for (int i = 0; i < k; ++i) tot = tot + p[ord[i]];
    for (int i = 0; i < k; ++i) {
      float v = p[ord[i]];
      if (norm) v = load_round(v / load_round(tot, dt), dt);
      scores[t * k + i] = v;
      experts[t * k + i] = ord[i];
    }
  }
  free(p);
  free(ord);
}

/* Stable sort of the n (token, slot) rows by expert; ids outside [0, E)
 * after all valid ones; offsets[e] = first row of expert e, offsets[E] =
 * number of valid rows (moe.rs:92-104 builds the same per-expert lists). */
void iqo_moe_sort(const int32_t* experts, int64_t n, int k, int E, int32_t* tokens, int32_t* sorted,
                  int32_t* inverse, int32_t* offsets) {
  int64_t pos = 0;
  for (int e = 0; e <= E; ++e) {
    offsets[e] = (int32_t)pos;
    for (int64_t r = 0; r < n; ++r) {
      const int32_t x = experts[r];
      const int valid = x >= 0 && x < E;
      if ((e < E && valid && x == e) || (e == E && !valid)) {
        tokens[pos] = (int32_t)(r / k);
        sorted[pos] = x;
        inverse[r] = (int32_t)pos;
        ++pos;
      }
    }
  }
}

/* out[t, :] = sum over t's slots with a valid expert, in ascending expert
 * order, of float(y[inverse[slot], :]) * score: the first product as is, each
 * further one added in fp32 (moe.rs:146-168). */
void iqo_moe_combine(const void* y, int dt, int64_t D, const int32_t* inverse, const int32_t* experts,
                     const float* scores, int64_t T, int k, int E, float* out) {
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t d = 0; d < D; ++d) {
      float acc = 0.0f;
      int first = 1;
      for (int e = 0; e < E; ++e)
        for (int s = 0; s < k; ++s)
          if (experts[t * k + s] == e) {
            const float v = load_f(y, dt, (int64_t)inverse[t * k + s] * D + d) * scores[t * k + s];
            acc = first ? v : acc + v;
            first = 0;
          }
      out[t * D + d] = acc;
    }
  }
}
